"""The exact-order attention (the x86 head loop, src/forward.c:463-504) in its
two score layouts: the KV-head-grouped kernel (one coalesced key tile in LDS
shared by the group's query heads) must give the same bits as the per-head
kernel, for fp32 / int8 / int4 caches, head_dim 64 and 128, groups of 1-8,
through ibh_host_attn (host cache, device mirror)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    import libinferbit_amd as L
    L.ops.init(0)
    return L.lib()


def cache(rng, bits, T, n_kv, hd):
    kv_dim = n_kv * hd
    if bits == 32:
        return [rng.standard_normal((T, kv_dim)).astype(np.float32) for _ in range(2)] + [None, None]
    if bits == 8:
        k, v = (rng.integers(-127, 128, (T, kv_dim), dtype=np.int8) for _ in range(2))
    else:
        k, v = (rng.integers(0, 256, (T, (kv_dim + 1) // 2), dtype=np.uint8) for _ in range(2))
    ks, vs = ((rng.uniform(0.005, 0.03, (T, n_kv))).astype(np.float32) for _ in range(2))
    return [k, v, ks, vs]


def run(lib, key, arrs, T, bits, q, n_heads, n_kv, hd):
    k, v, ks, vs = arrs
    out = np.zeros(n_heads * hd, np.float32)
    p = lambda a: None if a is None else a.ctypes.data
    rc = lib.ibh_host_attn(C.c_void_p(key), p(k), p(v), p(ks), p(vs), T, T - 1, bits, q.ctypes.data, out.ctypes.data,
                           n_heads, n_kv, hd)
    assert rc == 0, lib.ibh_last_error()
    return out


@pytest.mark.parametrize("bits", [32, 8, 4])
@pytest.mark.parametrize("hd,n_heads,n_kv,T", [(64, 32, 4, 300), (128, 32, 8, 700), (128, 8, 8, 65), (64, 16, 2, 129),
                                               (128, 16, 16, 64)])
def test_grouped_scores_bit_identical(lib, bits, hd, n_heads, n_kv, T):
    print(f"case exact attention bits={bits} hd={hd} heads={n_heads}/{n_kv} T={T}", flush=True)
    rng = np.random.default_rng(bits * 1000 + hd + T)
    arrs = cache(rng, bits, T, n_kv, hd)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    key = 0x1000 + bits * 10 + hd
    try:
        lib.ibh_attn_exact_set_grouped(0)
        a = run(lib, key, arrs, T, bits, q, n_heads, n_kv, hd)
        lib.ibh_host_kv_release(C.c_void_p(key))
        lib.ibh_attn_exact_set_grouped(1)
        b = run(lib, key, arrs, T, bits, q, n_heads, n_kv, hd)
    finally:
        lib.ibh_attn_exact_set_grouped(1)
        lib.ibh_host_kv_release(C.c_void_p(key))
    assert np.isfinite(a).all()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def scores_case(rng, kind, T, n_kv, hd):
    """fp32 K/V rows whose scores stress the exact softmax sum: random,
    flat (every e_t = 1: the sum is an integer), few distinct values (long
    runs of equal terms: many round-to-even ties), peaky (terms spanning
    many binades, underflow to 0), and a sum that crosses many binades."""
    kv_dim = n_kv * hd
    v = rng.standard_normal((T, kv_dim)).astype(np.float32)
    if kind == "random":
        k = rng.standard_normal((T, kv_dim)).astype(np.float32)
    elif kind == "flat":
        k = np.zeros((T, kv_dim), np.float32)
    elif kind == "few":
        k = rng.choice(np.array([-1.0, -0.5, 0.0, 0.25], np.float32), (T, kv_dim))
    elif kind == "peaky":
        k = (rng.standard_normal((T, kv_dim)) * 6).astype(np.float32)
    else:  # "ramp": scores rise along t, so the partial sums climb through many binades
        k = np.outer(np.linspace(-4, 0.5, T), np.ones(kv_dim)).astype(np.float32)
    return [k, v, None, None]


@pytest.mark.parametrize("kind", ["random", "flat", "few", "peaky", "ramp"])
@pytest.mark.parametrize("hd,n_heads,n_kv,T", [(128, 32, 8, 4176), (64, 32, 4, 111), (128, 8, 8, 8000), (64, 8, 2, 1)])
def test_exact_attention_matches_oracle_bits(lib, oracle_lib, kind, hd, n_heads, n_kv, T):
    """Same bits as the oracle's restatement of the x86 head loop (serial
    dot, max, expf, serial sum, serial P.V): the device sums the softmax
    denominator by binade jumps and must still equal the serial sum."""
    print(f"case exact attention vs oracle kind={kind} hd={hd} heads={n_heads}/{n_kv} T={T}", flush=True)
    rng = np.random.default_rng([len(kind), ord(kind[0]), hd, T])
    arrs = scores_case(rng, kind, T, n_kv, hd)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    if kind == "few":
        q = np.abs(q).round(1).astype(np.float32)
    key = 0x2000 + hd + T
    try:
        got = run(lib, key, arrs, T, 32, q, n_heads, n_kv, hd)
    finally:
        lib.ibh_host_kv_release(C.c_void_p(key))
    ref = oracle_lib.attn_decode(q, [arrs[0], arrs[1], np.zeros(1, np.float32), np.zeros(1, np.float32)], T - 1,
                                 n_heads, n_kv, hd, 32)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
