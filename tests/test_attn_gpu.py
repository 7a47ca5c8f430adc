"""GPU parity of the KV-cache write (bit-exact codes and scales) and of the
attention decode (fp32 summation order differs from the CPU: bar
max|out_gpu - out_cpu| / max|out_cpu| <= 1e-4) against the oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import libinferbit_amd as L
    L.ops.init(0)
    return L.ops


def alloc(bits, cap, n_kv, hd):
    from oracle import pyoracle as O
    rb = O.kv_row_bytes(bits, n_kv, hd)
    k = torch.zeros(cap * rb, dtype=torch.uint8, device="cuda")
    v = torch.zeros(cap * rb, dtype=torch.uint8, device="cuda")
    ks = torch.zeros(cap * n_kv, dtype=torch.float32, device="cuda")
    vs = torch.zeros(cap * n_kv, dtype=torch.float32, device="cuda")
    return k, v, ks, vs


CASES = [  # n_heads, n_kv, head_dim, positions
    (32, 4, 64, 40),      # TinyLlama attention shape
    (32, 8, 128, 37),     # Mistral attention shape
    (4, 4, 16, 9),
    (8, 2, 32, 65),
    (2, 1, 256, 33),
]


@pytest.mark.parametrize("bits", [32, 8, 4])
@pytest.mark.parametrize("n_heads,n_kv,hd,T", CASES)
def test_kv_write_and_attention_vs_oracle(ops, oracle_lib, bits, n_heads, n_kv, hd, T):
    print(f"case attn bits={bits} heads={n_heads}/{n_kv} hd={hd} T={T}", flush=True)
    rng = np.random.default_rng(n_heads * 1000 + hd + T + bits)
    cache = oracle_lib.kv_alloc(bits, T, n_kv, hd)
    gk, gv, gks, gvs = alloc(bits, T, n_kv, hd)
    for t in range(T):
        k = rng.standard_normal(n_kv * hd).astype(np.float32) * (1 + t % 3)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        if t == 3:
            k[:hd] = 0.0                                    # all-zero head: scale floor
        oracle_lib.kv_write(cache, t, k, v, n_kv, hd, bits)
        ops.kv_cache_write(gk, gv, gks, gvs, t, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                           n_kv, hd, bits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(gk.cpu().numpy(), cache[0])
    np.testing.assert_array_equal(gv.cpu().numpy(), cache[1])
    if bits < 16:
        np.testing.assert_array_equal(gks.cpu().numpy().view(np.uint32), cache[2].view(np.uint32))
        np.testing.assert_array_equal(gvs.cpu().numpy().view(np.uint32), cache[3].view(np.uint32))
    for pos in sorted({0, 1, T // 2, T - 1}):
        q = rng.standard_normal(n_heads * hd).astype(np.float32)
        out = torch.empty(n_heads * hd, device="cuda")
        ops.attn_decode(out, torch.from_numpy(q).cuda(), gk, gv, gks, gvs, pos, n_heads, n_kv, hd, bits)
        torch.cuda.synchronize()
        ref = oracle_lib.attn_decode(q, cache, pos, n_heads, n_kv, hd, bits)
        got = out.cpu().numpy()
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err <= 1e-4, (pos, err)


@pytest.mark.parametrize("bits", [8, 4, 32])
def test_attention_long_context_mistral(ops, oracle_lib, bits):
    """Mistral layer shape at 4096 cached positions."""
    n_heads, n_kv, hd, T = 32, 8, 128, 4096
    print(f"case attn-long bits={bits}", flush=True)
    rng = np.random.default_rng(bits)
    K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    cache = oracle_lib.kv_alloc(bits, T, n_kv, hd)
    for t in range(T):
        oracle_lib.kv_write(cache, t, K[t], V[t], n_kv, hd, bits)
    gk = torch.from_numpy(cache[0]).cuda()
    gv = torch.from_numpy(cache[1]).cuda()
    gks = torch.from_numpy(cache[2]).cuda()
    gvs = torch.from_numpy(cache[3]).cuda()
    q = rng.standard_normal(n_heads * hd).astype(np.float32) * 2
    out = torch.empty(n_heads * hd, device="cuda")
    ops.attn_decode(out, torch.from_numpy(q).cuda(), gk, gv, gks, gvs, T - 1, n_heads, n_kv, hd, bits)
    torch.cuda.synchronize()
    ref = oracle_lib.attn_decode(q, cache, T - 1, n_heads, n_kv, hd, bits)
    err = np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 1e-4, err


def test_attention_bad_arguments(ops):
    import libinferbit_amd as L
    t = torch.zeros(64, device="cuda")
    with pytest.raises(L.IbhError):
        ops.attn_decode(t, t, t, t, t, t, 0, 6, 4, 16, 8)       # heads not a multiple of kv heads
    with pytest.raises(L.IbhError):
        ops.attn_decode(t, t, t, t, None, None, 0, 4, 4, 16, 8)  # int8 cache needs scales


@pytest.mark.parametrize("bits,n_heads,n_kv,hd,T", [(8, 32, 8, 128, 4096), (4, 32, 8, 128, 4000),
                                                  (32, 32, 4, 64, 2048), (8, 32, 4, 64, 131), (32, 8, 8, 128, 65)])
def test_attention_one_launch_matches_chunk_merge(ops, oracle_lib, bits, n_heads, n_kv, hd, T):
    """The one-launch split kernel (per-KV-head arrival counters, merge by
    the last chunk) against the chunk + merge kernels and the oracle; each
    configuration twice in a row, bit-identical (the counters reset)."""
    import libinferbit_amd as L
    print(f"case attn-split bits={bits} heads={n_heads}/{n_kv} hd={hd} T={T}", flush=True)
    rng = np.random.default_rng(T + hd + bits)
    K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    cache = oracle_lib.kv_alloc(bits, T, n_kv, hd)
    for t in range(T):
        oracle_lib.kv_write(cache, t, K[t], V[t], n_kv, hd, bits)
    g = [torch.from_numpy(a).cuda() for a in cache]
    q = torch.from_numpy(rng.standard_normal(n_heads * hd).astype(np.float32) * 2).cuda()

    def run():
        out = torch.empty(n_heads * hd, device="cuda")
        ops.attn_decode(out, q, g[0], g[1], g[2], g[3], T - 1, n_heads, n_kv, hd, bits)
        torch.cuda.synchronize()
        return out.cpu().numpy()
    a, b = run(), run()
    try:
        L.lib().ibh_attn_set_split(0)
        c = run()
    finally:
        L.lib().ibh_attn_set_split(1)
    np.testing.assert_array_equal(a, b)
    ref = oracle_lib.attn_decode(q.cpu().numpy(), cache, T - 1, n_heads, n_kv, hd, bits)
    assert np.abs(a - ref).max() / np.abs(ref).max() <= 1e-4
    assert np.abs(a - c).max() / np.abs(c).max() <= 1e-5

