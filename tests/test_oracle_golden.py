"""The C restatement (oracle/ib_oracle.c) against the golden vectors the
compiled reference wrote (tests/golden/gen_golden.py), bit for bit, and
against closed forms that do not depend on the reference at all."""
import numpy as np
import pytest

from conftest import int4g_case, load_golden, pq_case

SHAPES = ["64x256", "37x200", "16x4100", "8x4096"]


def f16(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("tag", SHAPES)
@pytest.mark.parametrize("bits", [8, 4, 2])
def test_quantizers_match_reference(oracle_lib, tag, bits):
    q = load_golden("quant.npz")
    if f"w{bits}_{tag}" not in q.files:
        pytest.skip("shape not a whole number of bytes at this width")
    w, s = oracle_lib.quantize(bits, q[f"W_{tag}"])
    same_bits(w, q[f"w{bits}_{tag}"])
    same_bits(s, q[f"s{bits}_{tag}"])


@pytest.mark.parametrize("tag", SHAPES)
@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("order", ["avx2", "scalar"])
def test_matvec_matches_reference(oracle_lib, tag, bits, order):
    q, mv = load_golden("quant.npz"), load_golden("matvec.npz")
    if f"w{bits}_{tag}" not in q.files:
        pytest.skip("shape not a whole number of bytes at this width")
    y = oracle_lib.matmul(bits, q[f"w{bits}_{tag}"], f16(q[f"s{bits}_{tag}"]), mv[f"x_{tag}"],
                          order=1 if order == "avx2" else 0)
    same_bits(y, mv[f"y{bits}_{order}_{tag}"])


@pytest.mark.parametrize("tag", SHAPES)
def test_w4a8_matches_reference(oracle_lib, tag):
    q, mv, g = load_golden("quant.npz"), load_golden("matvec.npz"), load_golden("w4a8.npz")
    qx, sa = oracle_lib.quantize_act(mv[f"x_{tag}"])
    same_bits(qx, g[f"qx_{tag}"])
    same_bits(sa, g[f"sa_{tag}"])
    for order, name in ((1, "avx2"), (0, "scalar")):
        y = oracle_lib.matmul_w4a8(q[f"w4_{tag}"], f16(q[f"s4_{tag}"]), qx, sa, order)
        same_bits(y, g[f"y_{name}_{tag}"])


def test_act_quantizer_edges(oracle_lib):
    g = load_golden("w4a8.npz")
    qx, sa = oracle_lib.quantize_act(g["x_edge"])
    same_bits(qx, g["qx_edge"])
    same_bits(sa, g["sa_edge"])
    assert sa[0] == np.float32(1e-10) and not qx[:128].any()


@pytest.mark.parametrize("MN", ["48x256", "33x384"])
@pytest.mark.parametrize("B", [1, 2, 5, 8])
def test_batched_match_reference(oracle_lib, MN, B):
    d = load_golden("batch.npz")
    tag = f"{MN}_b{B}"
    M = int(MN.split("x")[0])
    y8 = oracle_lib.matmul_int8_batch(d[f"w8_{MN}"], f16(d[f"s8_{MN}"]), d[f"X_{tag}"], M + 3)
    same_bits(y8, d[f"y8_{tag}"])
    y4 = oracle_lib.matmul_w4a8_batch(d[f"w4_{MN}"], f16(d[f"s4_{MN}"]), d[f"QX_{tag}"], d[f"SA_{tag}"], M + 3)
    same_bits(y4, d[f"y4_{tag}"])


@pytest.mark.parametrize("name", ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40"])
def test_pq_matches_reference(oracle_lib, name):
    d = load_golden("pq.npz")
    t = pq_case(d, name)
    same_bits(oracle_lib.pq_matmul(t, t["x"]), t["y"])
    same_bits(oracle_lib.pq_matmul(t, t["xs"]), t["ys"])
    same_bits(oracle_lib.pq_reconstruct(t), t["W"])


# ── closed forms (independent of the reference build) ─────────────────────

@pytest.mark.parametrize("bits", [8, 4, 2])
def test_one_hot_picks_code_times_scale(oracle_lib, bits):
    rng = np.random.default_rng(3)
    M, N = 9, 64
    W = (rng.standard_normal((M, N)) * 0.02).astype(np.float32)
    w, s = oracle_lib.quantize(bits, W)
    sc = f16(s)
    for j in (0, 1, 2, 3, 17, N - 1):
        x = np.zeros(N, np.float32)
        x[j] = 1.0
        y = oracle_lib.matmul(bits, w, sc, x, order=1)
        if bits == 8:
            code = w[:, j].astype(np.float32)
        elif bits == 4:
            code = ((w[:, j // 2] >> (4 * (j % 2))) & 15).astype(np.float32) - 8
        else:
            code = ((w[:, j // 4] >> (2 * (j % 4))) & 3).astype(np.float32) - 1
        np.testing.assert_array_equal(y, code * sc)


def test_quantizer_roundtrip_bound(oracle_lib):
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((16, 128)) * 0.02).astype(np.float32)
    for bits, qmax in ((8, 127), (4, 7)):
        w, s = oracle_lib.quantize(bits, W)
        sc = f16(s)
        if bits == 4:
            lo, hi = (w & 15).astype(np.int32) - 8, (w >> 4).astype(np.int32) - 8
            codes = np.stack([lo, hi], -1).reshape(16, 128)
        else:
            codes = w.astype(np.int32)
        assert np.abs(codes).max() <= qmax
        deq = codes * sc[:, None]
        # the scale is truncated toward zero, so the error bound is one step
        assert np.all(np.abs(deq - W) <= sc[:, None] * 1.0001 + 1e-7)


def test_w4a8_on_int8_grid_is_exact(oracle_lib):
    """With x already on the int8 grid of its group scale, W4A8 equals the
    exact integer dot times scales (single group so no fold rounding)."""
    rng = np.random.default_rng(11)
    M, N = 7, 128
    w = rng.integers(0, 256, (M, N // 2), dtype=np.uint8)
    q = rng.integers(-127, 128, N).astype(np.int8)
    sa = np.array([0.5], np.float32)
    sw = np.ones(M, np.float32)
    y = oracle_lib.matmul_w4a8(w, sw, q, sa, 1)
    codes = np.stack([(w & 15).astype(np.int64) - 8, (w >> 4).astype(np.int64) - 8], -1).reshape(M, N)
    np.testing.assert_array_equal(y, (codes @ q.astype(np.int64)).astype(np.float32) * 0.5)


def test_attention_single_position_returns_v0(oracle_lib):
    rng = np.random.default_rng(2)
    n_heads, n_kv, hd = 8, 2, 16
    for bits in (32, 8, 4):
        cache = oracle_lib.kv_alloc(bits, 4, n_kv, hd)
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        oracle_lib.kv_write(cache, 0, k, v, n_kv, hd, bits)
        q = rng.standard_normal(n_heads * hd).astype(np.float32)
        out = oracle_lib.attn_decode(q, cache, 0, n_heads, n_kv, hd, bits)
        # softmax of one score is exactly 1, so out = dequantized v
        if bits == 32:
            vd = v
        else:
            sc = cache[3][:n_kv]
            if bits == 8:
                codes = cache[1][: n_kv * hd].view(np.int8).astype(np.float32)
            else:
                b = cache[1][: n_kv * hd // 2]
                codes = np.stack([(b & 15).astype(np.float32) - 8, (b >> 4).astype(np.float32) - 8], -1).ravel()
            vd = (codes.reshape(n_kv, hd) * sc[:, None]).ravel().astype(np.float32)
        for h in range(n_heads):
            kh = h // (n_heads // n_kv)
            np.testing.assert_array_equal(out[h * hd:(h + 1) * hd], vd[kh * hd:(kh + 1) * hd])


def test_attention_identical_keys_is_mean_of_values(oracle_lib):
    rng = np.random.default_rng(4)
    n_heads, n_kv, hd, T = 4, 4, 32, 9
    cache = oracle_lib.kv_alloc(32, T, n_kv, hd)
    k = rng.standard_normal(n_kv * hd).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    for t in range(T):
        oracle_lib.kv_write(cache, t, k, V[t], n_kv, hd, 32)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    out = oracle_lib.attn_decode(q, cache, T - 1, n_heads, n_kv, hd, 32)
    np.testing.assert_allclose(out, V.mean(0), rtol=1e-5, atol=1e-6)


def test_attention_matches_fp64_softmax(oracle_lib):
    rng = np.random.default_rng(6)
    n_heads, n_kv, hd, T = 8, 2, 64, 37
    cache = oracle_lib.kv_alloc(32, T, n_kv, hd)
    K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    for t in range(T):
        oracle_lib.kv_write(cache, t, K[t], V[t], n_kv, hd, 32)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    out = oracle_lib.attn_decode(q, cache, T - 1, n_heads, n_kv, hd, 32)
    ref = np.zeros(n_heads * hd)
    for h in range(n_heads):
        kh = h // (n_heads // n_kv)
        s = K[:, kh * hd:(kh + 1) * hd].astype(np.float64) @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
        a = np.exp(s - s.max())
        a /= a.sum()
        ref[h * hd:(h + 1) * hd] = a @ V[:, kh * hd:(kh + 1) * hd]
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


def test_kv_int8_quantization_rule(oracle_lib):
    hd, n_kv = 8, 1
    cache = oracle_lib.kv_alloc(8, 1, n_kv, hd)
    k = np.array([1, -2, 0.5, 0, 127, -127, 63.5, -63.5], np.float32)
    oracle_lib.kv_write(cache, 0, k, k, n_kv, hd, 8)
    assert cache[2][0] == np.float32(1.0)
    np.testing.assert_array_equal(cache[0][:8].view(np.int8), [1, -2, 1, 0, 127, -127, 64, -64])


def test_pq_one_hot_codebook_closed_form(oracle_lib):
    """K=1 codebooks of all ones: every row equals row_scale * sum(x)."""
    M, Cc, G = 5, 4, 8
    N = Cc * G
    one = np.full((1, G // 2), 1.0, np.float16).view(np.uint16)
    t = dict(M=M, N=N, G=G, K=1, n_levels=1, n_outlier=0, C=Cc, cb1l=one, cb1r=one,
             i1l=np.zeros((M, Cc), np.uint8), i1r=np.zeros((M, Cc), np.uint8),
             row_scale=np.array([1, 2, 0.5, 4, -1], np.float16).view(np.uint16))
    x = np.arange(N, dtype=np.float32) / 8
    y = oracle_lib.pq_matmul(t, x)
    np.testing.assert_allclose(y, np.array([1, 2, 0.5, 4, -1]) * x.sum(), rtol=1e-6)


def test_pq_matches_materialized_fp64(oracle_lib):
    d = load_golden("pq.npz")
    for name in ("l1", "l2u8", "out8"):
        t = pq_case(d, name)
        W = oracle_lib.pq_reconstruct(t).astype(np.float64)
        y = oracle_lib.pq_matmul(t, t["x"])
        ref = W @ t["x"].astype(np.float64)
        # reconstruct rounds weights to fp16; the LUT path keeps fp32
        assert np.abs(y - ref).max() <= 2e-3 * np.abs(ref).max()


def test_fp16_conversions(oracle_lib):
    import ctypes
    L = oracle_lib.lib()
    for h in (0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x3c00, 0x7bff, 0x7c00, 0xfc00, 0xc000):
        assert np.float32(L.or_fp16_to_fp32(h)).tobytes() == np.array([h], np.uint16).view(
            np.float16).astype(np.float32).tobytes()
    for f in (1.0, -2.5, 65504.0, 1e-3, 3.14159, 6.1e-5, 1e-8, 70000.0):
        assert L.or_fp32_to_fp16_rne(ctypes.c_float(f)) == int(np.array([f], np.float32).astype(
            np.float16).view(np.uint16)[0])
        # truncation never rounds up in magnitude
        t = L.or_fp32_to_fp16_trunc(ctypes.c_float(f))
        tv = np.array([t], np.uint16).view(np.float16).astype(np.float32)[0]
        assert abs(tv) <= abs(np.float32(f)) or np.isinf(tv)


INT4G = ["g32", "g128awq", "g64awq", "g128out", "g96", "g2", "g128big", "g256"]


@pytest.mark.parametrize("name", INT4G)
def test_int4g_matches_reference(oracle_lib, name):
    """ib_pq_session_matmul on INT4 group-scale tensors, with and without the
    IB_ACT_SPARSE_REL skip mask, bit for bit."""
    d = load_golden("int4g.npz")
    t = int4g_case(d, name)
    same_bits(oracle_lib.int4g_matmul(t, t["x"]), t["y"])
    same_bits(oracle_lib.int4g_matmul(t, t["x"], float(d["skip_rel"])), t["ys"])


def _int4g_dense(t):
    q = np.asarray(t["q"])
    M, N = q.shape[0], q.shape[1] * 2
    n = np.empty((M, N), np.float64)
    n[:, 0::2] = (q & 15).astype(np.float64) - 8
    n[:, 1::2] = (q >> 4).astype(np.float64) - 8
    G = N // t["s"].shape[1]
    W = n * np.repeat(f16(t["s"]).astype(np.float64), G, axis=1)
    if t.get("outl_idx") is not None:
        for m in range(M):
            for k, j in enumerate(t["outl_idx"][m]):
                W[m, j] += f16(t["outl_val"][m, k])
    return W


@pytest.mark.parametrize("name", INT4G)
def test_int4g_matches_materialized_fp64(oracle_lib, name):
    """y = W (x * inv_act) with W[m, j] = (nibble - 8) * scale[m, j // G] plus
    the outlier values, in fp64: pins the nibble order, the -8 bias, the
    group index, the AWQ pre-scale and the sidecar independently of the
    reference."""
    t = int4g_case(load_golden("int4g.npz"), name)
    xk = t["x"].astype(np.float64)
    if t["inv_act"] is not None:
        xk = xk * t["inv_act"].astype(np.float32).astype(np.float64)
    ref = _int4g_dense(t) @ xk
    y = oracle_lib.int4g_matmul(t, t["x"])
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


def test_int4g_skip_mask_drops_whole_groups(oracle_lib):
    """With the skip mask on, y equals the unmasked matvec over x with the
    qualifying groups set to zero (and only those): threshold <= is inclusive."""
    rng = np.random.default_rng(5)
    M, N, G = 9, 256, 32
    t = dict(q=rng.integers(0, 256, (M, N // 2), dtype=np.uint8),
             s=np.asarray(rng.uniform(0.01, 0.1, (M, N // G)), np.float16).view(np.uint16))
    x = rng.standard_normal(N).astype(np.float32)
    x[0] = 4.0
    x[32:64] = 0.0                     # max 0 <= thr: skipped
    x[64:96] = np.float32(0.5 * 4.0) * np.sign(x[64:96])   # exactly 0.5 * max: skipped at rel 0.5
    x[96:128] *= 1e-3
    y = oracle_lib.int4g_matmul(t, x, 0.5)
    xz = x.copy()
    gmax = np.abs(x.reshape(-1, G)).max(1)
    for g in range(N // G):
        if gmax[g] <= np.float32(0.5) * np.float32(4.0):
            xz[g * G:(g + 1) * G] = 0
    assert (gmax <= 2.0).sum() >= 3
    same_bits(y, oracle_lib.int4g_matmul(t, xz))


def test_int4g_live_reference(oracle_lib):
    """The compiled reference (oracle/_ref/libref_int4g.so), when present,
    agrees bit for bit on a fresh random tensor with AWQ and outliers."""
    from oracle import refbind as R
    import os
    if not os.path.exists(R.REF_INT4G):
        pytest.skip("oracle/_ref/libref_int4g.so not built (make -C oracle ref)")
    from gen_golden import make_int4g
    rng = np.random.default_rng(77)
    t = make_int4g(rng, 31, 1024, 128, 1, 6)
    x = rng.standard_normal(1024).astype(np.float32)
    same_bits(oracle_lib.int4g_matmul(t, x), R.int4g_matmul(t, x))


@pytest.mark.parametrize("name", ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40", "g4", "g32", "g4l2"])
def test_pq_streaming_matches_reference(oracle_lib, name):
    """ib_pq_matmul_fp32_streaming_cached (the PQ session's default), bit for bit."""
    d = load_golden("pqs.npz")
    src = d if f"{name}.M" in d.files else load_golden("pq.npz")
    t = pq_case(src, name)
    same_bits(oracle_lib.pq_matmul_streaming(t, t["x"]), d[f"{name}.y"])
    if f"{name}.ys" in d.files:
        same_bits(oracle_lib.pq_matmul_streaming(t, t["xs"]), d[f"{name}.ys"])



def test_pq_streaming_keeps_every_chunk(oracle_lib):
    """On x whose first half is scaled by 1e-4 the skipping variant drops
    those chunks (its result equals the matvec over the second half only)
    while the streaming variant keeps them (it does not)."""
    t = pq_case(load_golden("pq.npz"), "l1")
    xs = t["xs"].copy()
    half = xs.copy()
    half[: t["N"] // 2] = 0
    y_skip, y_half = oracle_lib.pq_matmul(t, xs), oracle_lib.pq_matmul(t, half)
    np.testing.assert_allclose(y_skip, y_half, rtol=0, atol=1e-6 * np.abs(y_half).max())
    y_str = oracle_lib.pq_matmul_streaming(t, xs)
    assert np.abs(y_str - y_half).max() > 1e-6 * np.abs(y_half).max()


PQV_NAMES = ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40", "pyr16", "pyr8"]
PQV_POLICIES = {"l1only": (1, 0.0, 0.0), "l2skip05": (2, 0.5, 0.0), "l2skip5": (2, 5.0, 0.0),
                "sparse": (3, 0.0, 1e-2), "int8": (4, 0.0, 0.0)}


def pqv_case(name):
    d = load_golden("pqv.npz")
    src = d if f"{name}.M" in d.files else load_golden("pq.npz")
    return d, pq_case(src, name)


@pytest.mark.parametrize("name", PQV_NAMES)
@pytest.mark.parametrize("pol", list(PQV_POLICIES))
def test_pq_policy_variants_match_reference(oracle_lib, name, pol):
    """The PQ session's policy variants, bit for bit against the compiled reference."""
    d, t = pqv_case(name)
    v, st, at = PQV_POLICIES[pol]
    same_bits(oracle_lib.pq_matmul_variant(t, t["x"], v, st, at), d[f"{name}.{pol}.y"])
    same_bits(oracle_lib.pq_matmul_variant(t, t["xs"], v, st, at), d[f"{name}.{pol}.ys"])


def test_pq_policy_variant_properties(oracle_lib):
    """Closed forms: L1_ONLY equals the streaming result of the tensor with
    its level 2 removed; L2SKIP at threshold 0 and SPARSE at threshold 0
    equal STREAMING; INT8 stays within the int8 quantisation error."""
    d, t = pqv_case("l2u8")
    x = t["x"]
    one = {k: v for k, v in t.items() if k not in ("cb2l", "cb2r", "i2l", "i2r")}
    one["n_levels"], one["K_l2"] = 1, 0
    same_bits(oracle_lib.pq_matmul_variant(t, x, 1), oracle_lib.pq_matmul_streaming(one, x))
    ys = oracle_lib.pq_matmul_streaming(t, x)
    np.testing.assert_allclose(oracle_lib.pq_matmul_variant(t, x, 2, 0.0), ys, rtol=0, atol=1e-6 * np.abs(ys).max())
    np.testing.assert_allclose(oracle_lib.pq_matmul_variant(t, x, 3, 0.0, 0.0), ys, rtol=0,
                               atol=1e-6 * np.abs(ys).max())
    y8 = oracle_lib.pq_matmul_variant(t, x, 4)
    assert 0 < np.abs(y8 - ys).max() <= 0.05 * np.abs(ys).max()


TOPK_CASES = [("head1", 1), ("head1", 8), ("head1", 40), ("head2", 3), ("head2", 64), ("small", 12)]


@pytest.mark.parametrize("name,k", TOPK_CASES)
def test_pq_lm_head_topk_matches_reference(oracle_lib, name, k):
    d = load_golden("pqtopk.npz")
    t = pq_case(d, name)
    lg, ids = oracle_lib.pq_lm_head_topk(t, t["x"], k)
    same_bits(lg, d[f"{name}.k{k}.logits"])
    same_bits(ids, d[f"{name}.k{k}.ids"])


def test_pq_topk_is_the_subset_of_largest_coarse_logits(oracle_lib):
    """Properties: the ids are the K largest level-1 logits; the logits are
    the subset matvec of those ids, sorted descending; K = M returns every
    row."""
    d = load_golden("pqtopk.npz")
    t = pq_case(d, "head2")
    coarse = oracle_lib.pq_matmul_variant(t, t["x"], 1)
    lg, ids = oracle_lib.pq_lm_head_topk(t, t["x"], 64)
    assert set(ids.tolist()) == set(np.argsort(-coarse, kind="stable")[:64].tolist())
    same_bits(lg, oracle_lib.pq_matmul_subset(t, t["x"], ids))
    assert (np.diff(lg) <= 0).all()
    W = oracle_lib.pq_reconstruct(t).astype(np.float64)
    np.testing.assert_allclose(lg, (W @ t["x"].astype(np.float64))[ids], rtol=0, atol=2e-3 * np.abs(lg).max())
    small = pq_case(d, "small")
    lg, ids = oracle_lib.pq_lm_head_topk(small, small["x"], 12)
    assert sorted(ids.tolist()) == list(range(12))


PQQ8_NAMES = ["l1", "l2", "out8", "out40l2", "g4", "g32", "g6"]


@pytest.mark.parametrize("name", PQQ8_NAMES)
def test_pq_q8lut_matches_reference(oracle_lib, name):
    """ib_pq_matmul_fp32_q8lut, bit for bit against the reference's outputs."""
    d = load_golden("pqq8.npz")
    t = pq_case(d, name)
    same_bits(oracle_lib.pq_matmul_q8lut(t, t["x"]), d[f"{name}.y"])


@pytest.mark.parametrize("name", PQQ8_NAMES)
def test_pq_q8lut_error_bound(oracle_lib, name):
    """Independent of the restatement: the int8 tables move each chunk term
    by at most half a step of its (chunk, side) scale, so
    |y - W x| <= |row_scale| * sum_c sum_side (max_k |T| / 254) per level
    (+ fp32 slack), with W x in float64 from the materialised matrix and
    T in float64 from the codebooks."""
    d = load_golden("pqq8.npz")
    t = pq_case(d, name)
    x = t["x"].astype(np.float64)
    W = oracle_lib.pq_reconstruct(t).astype(np.float64)
    y = oracle_lib.pq_matmul_q8lut(t, t["x"]).astype(np.float64)
    exact = W @ x
    G, C, hf = t["G"], t["C"], t["G"] // 2
    mask = np.ones(t["N"], bool)
    if t["n_outlier"]:
        mask[np.asarray(t["ocols"])] = False
    inner = np.nonzero(mask)[0]
    bound = 0.0
    for lev in range(t["n_levels"]):
        for side, key in enumerate(("cb1l", "cb1r") if lev == 0 else ("cb2l", "cb2r")):
            cb = np.asarray(t[key]).view(np.float16).astype(np.float64).reshape(-1, hf)
            for c in range(C):
                xs = x[inner[c * G + side * hf: c * G + side * hf + hf]]
                bound += np.abs(cb @ xs).max() / 254.0
    rs = np.abs(np.asarray(t["row_scale"]).view(np.float16).astype(np.float64))
    slack = 1e-5 * np.abs(exact).max() + 1e-6
    if t["n_outlier"] >= 32:      # the int8 outlier dot adds its own half step per column
        oc = np.asarray(t["ocols"])
        os_ = np.asarray(t["oscale"]).view(np.float16).astype(np.float64)
        slack += np.abs(t["oside"]).max() * np.abs(x[oc] * os_).max() / 254.0 * t["n_outlier"]
    assert np.all(np.abs(y - exact) <= rs * bound + slack)


# ── decode-layer helpers (or_rmsnorm, or_rope, or_silu_mul) ──────────────────
LAYER_N = [1, 7, 64, 2051]


@pytest.mark.parametrize("n", LAYER_N)
def test_rmsnorm_matches_reference(oracle_lib, n):
    """avx2_rmsnorm (src/kernels/avx2.c:153-188) wrote these: 8-lane FMA sum of
    squares, fold, FMA tail, (x*scale)*w -- bit for bit, odd lengths too."""
    d = load_golden("layer.npz")
    same_bits(oracle_lib.rmsnorm(d[f"rms{n}.x"], d[f"rms{n}.w"], 1e-5), d[f"rms{n}.y"])


@pytest.mark.parametrize("n", LAYER_N)
def test_silu_mul_matches_reference(oracle_lib, n):
    """avx2_silu_mul (src/kernels/avx2.c:233-251), bit for bit."""
    d = load_golden("layer.npz")
    same_bits(oracle_lib.silu_mul(d[f"silu{n}.g"], d[f"silu{n}.u"]), d[f"silu{n}.y"])


@pytest.mark.parametrize("i", range(5))
def test_rope_matches_reference(oracle_lib, i):
    """avx2_rope (src/kernels/avx2.c:256-273): head dims 6..128, positions 0..4095,
    theta 500..1e6, bit for bit."""
    d = load_golden("layer.npz")
    hd, pos, theta = d[f"rope{i}.arg"]
    q, k = oracle_lib.rope(d[f"rope{i}.q"], d[f"rope{i}.k"], int(hd), int(pos), float(theta))
    same_bits(q, d[f"rope{i}.qo"])
    same_bits(k, d[f"rope{i}.ko"])


def test_layer_helpers_closed_forms(oracle_lib):
    """Properties fixed by the mathematics, independent of the reference:
    rmsnorm of a constant vector is w * c / sqrt(c^2 + eps); RoPE at position
    0 is the identity and at any position keeps each pair's norm and rotates
    pair i by pos * theta^(-2i/hd); silu(0) = 0 and silu(g) -> g for large g."""
    n = 33
    x = np.full(n, 2.5, np.float32)
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    y = oracle_lib.rmsnorm(x, w, 1e-5)
    np.testing.assert_allclose(y, w * 2.5 / np.sqrt(2.5 ** 2 + 1e-5), rtol=2e-7)
    rng = np.random.default_rng(3)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    q0, k0 = oracle_lib.rope(q, k, 64, 0, 10000.0)
    same_bits(q0, q)
    same_bits(k0, k)
    pos = 37
    q1, _ = oracle_lib.rope(q, k, 64, pos, 10000.0)
    for i in range(0, 64, 2):
        ang = pos * 10000.0 ** (-i / 64)
        c, s = np.cos(ang), np.sin(ang)
        want = (q[i] * c - q[i + 1] * s, q[i] * s + q[i + 1] * c)
        np.testing.assert_allclose(q1[i:i + 2], want, rtol=0, atol=2e-5)
        np.testing.assert_allclose(np.hypot(*q1[i:i + 2]), np.hypot(q[i], q[i + 1]), rtol=1e-5)
    g = np.array([0.0, 30.0, -30.0, 1.0], np.float32)
    y = oracle_lib.silu_mul(g, np.ones(4, np.float32))
    assert y[0] == 0.0 and abs(y[1] - 30.0) < 1e-5 and abs(y[2]) < 1e-10
    np.testing.assert_allclose(y[3], 1.0 / (1.0 + np.exp(-1.0)), rtol=1e-6)
