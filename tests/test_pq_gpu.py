"""GPU parity of the PQ LUT matvec against the reference-written golden
vectors and the oracle.  The chunk sum is associated differently from the
CPU's serial loop: bar max|y_gpu - y_cpu| / max|y_cpu| <= 1e-4."""
import numpy as np
import pytest
import torch

from conftest import load_golden, pq_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import libinferbit_amd as L
    L.ops.init(0)
    return L.ops


def run(ops, t, x):
    d = ops.PqDeviceTensor(t)
    out = torch.empty(t["M"], device="cuda")
    d.matmul(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda(), out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def relerr(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


@pytest.mark.parametrize("name", ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40"])
def test_pq_golden(ops, name):
    print(f"case pq {name}", flush=True)
    t = pq_case(load_golden("pq.npz"), name)
    assert relerr(run(ops, t, t["x"]), t["y"]) <= 1e-4
    assert relerr(run(ops, t, t["xs"]), t["ys"]) <= 1e-4       # chunk-skipping case


def test_pq_mistral_ffn_shape(ops, oracle_lib):
    """M=4096, N=14336, G=16, K=256, one level, no outliers."""
    from gen_golden import make_pq
    rng = np.random.default_rng(5)
    t = make_pq(rng, 4096, 896, 16, 256, 1, 0, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    assert relerr(run(ops, t, x), oracle_lib.pq_matmul(t, x)) <= 1e-4


def test_pq_zero_input(ops, oracle_lib):
    from gen_golden import make_pq
    t = make_pq(np.random.default_rng(1), 64, 16, 16, 256, 1, 0, 8)
    x = np.zeros(t["N"], np.float32)
    np.testing.assert_array_equal(run(ops, t, x), oracle_lib.pq_matmul(t, x))


def run_streaming(ops, t, x):
    d = ops.PqDeviceTensor(t)
    out = torch.empty(t["M"], device="cuda")
    d.matmul_streaming(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda(), out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("name", ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40", "g4", "g32", "g4l2"])
def test_pq_streaming_golden(ops, name):
    """ib_pq_matmul_fp32_streaming_cached (the PQ session's default): no chunk skipping."""
    print(f"case pq streaming {name}", flush=True)
    d = load_golden("pqs.npz")
    src = d if f"{name}.M" in d.files else load_golden("pq.npz")
    t = pq_case(src, name)
    assert relerr(run_streaming(ops, t, t["x"]), d[f"{name}.y"]) <= 1e-4
    if f"{name}.ys" in d.files:
        assert relerr(run_streaming(ops, t, t["xs"]), d[f"{name}.ys"]) <= 1e-4


def test_pq_streaming_mistral_shape(ops, oracle_lib):
    from gen_golden import make_pq
    rng = np.random.default_rng(6)
    t = make_pq(rng, 4096, 896, 16, 256, 1, 0, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    x[: t["N"] // 3] *= 1e-3
    assert relerr(run_streaming(ops, t, x), oracle_lib.pq_matmul_streaming(t, x)) <= 1e-4


def test_pq_streaming_rejects_wide_chunks(ops):
    from gen_golden import make_pq
    from libinferbit_amd import IbhError
    t = make_pq(np.random.default_rng(1), 16, 4, 64, 16, 1, 0, 0)
    with pytest.raises(IbhError):
        run_streaming(ops, t, np.zeros(t["N"], np.float32))


def run_q8lut(ops, t, x):
    d = ops.PqDeviceTensor(t)
    out = torch.empty(t["M"], device="cuda")
    d.matmul_q8lut(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda(), out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("name", ["l1", "l2", "out8", "out40l2", "g4", "g32", "g6"])
def test_pq_q8lut_golden(ops, name):
    """ib_pq_matmul_fp32_q8lut: the int8 codes equal the reference's, the
    gather sums in another order."""
    print(f"case pq q8lut {name}", flush=True)
    d = load_golden("pqq8.npz")
    t = pq_case(d, name)
    assert relerr(run_q8lut(ops, t, t["x"]), d[f"{name}.y"]) <= 1e-4


def test_pq_q8lut_mistral_shape(ops, oracle_lib):
    from gen_golden import make_pq
    rng = np.random.default_rng(61)
    t = make_pq(rng, 4096, 896, 16, 256, 2, 256, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    assert relerr(run_q8lut(ops, t, x), oracle_lib.pq_matmul_q8lut(t, x)) <= 1e-4


def test_pq_q8lut_rejects_unreadable_level2(ops):
    from gen_golden import make_pq
    from libinferbit_amd import IbhError
    t = make_pq(np.random.default_rng(2), 16, 4, 16, 64, 2, 256, 0)     # K_l2 != K
    with pytest.raises(IbhError):
        run_q8lut(ops, t, np.zeros(t["N"], np.float32))


PQV_NAMES = ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40", "pyr16", "pyr8"]
PQV_POLICIES = {"l1only": (1, 0.0, 0.0), "l2skip05": (2, 0.5, 0.0), "l2skip5": (2, 5.0, 0.0),
                "sparse": (3, 0.0, 1e-2), "int8": (4, 0.0, 0.0)}


def run_policy(ops, t, x, v, st, at):
    d = ops.PqDeviceTensor(t)
    out = torch.empty(t["M"], device="cuda")
    d.matmul_policy(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda(), out, v, st, at)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("name", PQV_NAMES)
@pytest.mark.parametrize("pol", list(PQV_POLICIES))
def test_pq_policy_golden(ops, name, pol):
    """The PQ session's policy variants against the reference's outputs."""
    print(f"case pq policy {name} {pol}", flush=True)
    d = load_golden("pqv.npz")
    src = d if f"{name}.M" in d.files else load_golden("pq.npz")
    t = pq_case(src, name)
    v, st, at = PQV_POLICIES[pol]
    assert relerr(run_policy(ops, t, t["x"], v, st, at), d[f"{name}.{pol}.y"]) <= 1e-4
    assert relerr(run_policy(ops, t, t["xs"], v, st, at), d[f"{name}.{pol}.ys"]) <= 1e-4


@pytest.mark.parametrize("v,st,at", [(1, 0, 0), (2, 0.5, 0), (3, 0, 1e-3), (4, 0, 0)])
def test_pq_policy_mistral_shape(ops, oracle_lib, v, st, at):
    from gen_golden import make_pq
    print(f"case pq policy mistral v={v}", flush=True)
    rng = np.random.default_rng(8)
    t = make_pq(rng, 4096, 896, 16, 256, 2, 256, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    x[: t["N"] // 3] *= 1e-4
    assert relerr(run_policy(ops, t, x, v, st, at), oracle_lib.pq_matmul_variant(t, x, v, st, at)) <= 1e-4


@pytest.mark.parametrize("name,k", [("head1", 1), ("head1", 8), ("head1", 40), ("head2", 3), ("head2", 64),
                                    ("small", 12)])
def test_pq_lm_head_topk_golden(ops, name, k):
    print(f"case pq topk {name} k={k}", flush=True)
    d = load_golden("pqtopk.npz")
    t = pq_case(d, name)
    lg, ids = ops.PqDeviceTensor(t).lm_head_topk(torch.from_numpy(t["x"]).cuda(), k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), d[f"{name}.k{k}.ids"])
    want = d[f"{name}.k{k}.logits"]
    assert float(np.abs(lg.cpu().numpy().astype(np.float64) - want).max() / np.abs(want).max()) <= 1e-4


def test_pq_lm_head_topk_vocab_shape(ops, oracle_lib):
    """A 32000-row head (Llama vocabulary) over hidden 4096, two levels."""
    from gen_golden import make_pq
    rng = np.random.default_rng(12)
    t = make_pq(rng, 32000, 256, 16, 256, 2, 256, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    want_lg, want_ids = oracle_lib.pq_lm_head_topk(t, x, 50)
    lg, ids = ops.PqDeviceTensor(t).lm_head_topk(torch.from_numpy(x).cuda(), 50)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    assert float(np.abs(lg.cpu().numpy().astype(np.float64) - want_lg).max() / np.abs(want_lg).max()) <= 1e-4


@pytest.mark.parametrize("k", [1, 8, 16, 17])
def test_pq_lm_head_topk_two_pass(ops, oracle_lib, k):
    """Heads of 4096 rows and more with K <= 16 select in two passes (each
    block of 1024 rows keeps its K best, then one block selects among the
    candidates); K = 17 takes the one-pass select.  Ids equal the oracle's,
    also with many exactly tied rows (duplicated index rows)."""
    from gen_golden import make_pq
    rng = np.random.default_rng(100 + k)
    t = make_pq(rng, 32000, 64, 16, 64, 1, 0, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    d = ops.PqDeviceTensor(t)
    want_lg, want_ids = oracle_lib.pq_lm_head_topk(t, x, k)
    lg, ids = d.lm_head_topk(torch.from_numpy(x).cuda(), k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    assert float(np.abs(lg.cpu().numpy().astype(np.float64) - want_lg).max() / np.abs(want_lg).max()) <= 1e-4
    # ties: the best row copied into rows spread over several blocks
    best = int(want_ids[0])
    t2 = dict(t)
    for key in ("i1l", "i1r"):
        a = np.array(t[key])
        for r in (5, 3000, 17001, 31999):
            a[r] = a[best]
        t2[key] = a
    rs = np.array(t["row_scale"])
    for r in (5, 3000, 17001, 31999):
        rs[r] = rs[best]
    t2["row_scale"] = rs
    want_lg2, want_ids2 = oracle_lib.pq_lm_head_topk(t2, x, k)
    lg2, ids2 = ops.PqDeviceTensor(t2).lm_head_topk(torch.from_numpy(x).cuda(), k)
    torch.cuda.synchronize()
    got = ids2.cpu().numpy()
    # equal refined logits: the oracle keeps the reference's heap order, the
    # GPU row order; compare as sets per equal value and the values exactly
    assert sorted(got.tolist()) == sorted(want_ids2.tolist())
    assert float(np.abs(lg2.cpu().numpy().astype(np.float64) - want_lg2).max() / np.abs(want_lg2).max()) <= 1e-4


@pytest.mark.parametrize("heavy", [False, True])
@pytest.mark.parametrize("shape", [(4096, 896, 16, 256, 0), (300, 130, 16, 256, 0), (1000, 64, 8, 128, 40),
                                   (257, 200, 4, 64, 8), (513, 97, 16, 256, 33)])
def test_pq_one_launch_matches_three_kernels(ops, oracle_lib, shape, heavy):
    """The one-launch kernel (tables on the matrix cores, per-row fixed-point
    words) against the three-kernel path and the oracle, on ragged row
    tiles and slabs, with and without outliers, x N(0,1) and heavy-tailed
    (Student t, 1.5 dof: the fixed-point scale follows max|x|); each call
    twice, so the words' reset between calls is exercised."""
    from gen_golden import make_pq
    M, C, G, K, no = shape
    print(f"case pq one-launch {shape} heavy={heavy}", flush=True)
    rng = np.random.default_rng(M + C)
    t = make_pq(rng, M, C, G, K, 1, 0, no)
    x = (rng.standard_t(1.5, t["N"]) if heavy else rng.standard_normal(t["N"])).astype(np.float32)
    ref = oracle_lib.pq_matmul(t, x)
    lib = ops.lib()
    try:
        lib.ibh_pq_set_fused(0)
        three = run(ops, t, x)
    finally:
        lib.ibh_pq_set_fused(1)
    one = run(ops, t, x)
    again = run(ops, t, x)
    np.testing.assert_array_equal(one, again)
    assert relerr(one, ref) <= 1e-4
    assert relerr(one, three) <= 1e-5


def test_pq_one_launch_nonfinite_x(ops, oracle_lib):
    """A non-finite x on the one-launch path: every row NaN (the CPU gives
    +-Inf or NaN there), and the next finite call is right again."""
    from gen_golden import make_pq
    rng = np.random.default_rng(11)
    t = make_pq(rng, 4096, 896, 16, 256, 1, 0, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    for bad in (np.inf, np.nan):
        xb = x.copy()
        xb[123] = bad
        y = run(ops, t, xb)
        assert np.isnan(y).all()
        assert not np.isfinite(oracle_lib.pq_matmul(t, xb)).all()
    assert relerr(run(ops, t, x), oracle_lib.pq_matmul(t, x)) <= 1e-4


def test_pq_workspace_needs_stamp(ops, oracle_lib):
    """A caller workspace that ibh_pq_workspace_init did not prepare: NaN rows
    and IBH_DEVERR_PQ_WS, never a silent sum into unknown words; prepared,
    the same memory gives the right result."""
    import ctypes
    from gen_golden import make_pq
    rng = np.random.default_rng(12)
    t = make_pq(rng, 4096, 896, 16, 256, 1, 0, 0)
    x = rng.standard_normal(t["N"]).astype(np.float32)
    d = ops.PqDeviceTensor(t)
    lib = ops.lib()
    assert lib.ibh_device_errors(1) == 0
    ws = torch.full((d.ws.numel(),), 7, dtype=torch.uint8, device="cuda")   # garbage, no stamp
    xd = torch.from_numpy(x).cuda()
    out = torch.empty(t["M"], device="cuda")
    assert lib.ibh_pq_matmul(ctypes.byref(d.s), xd.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), None) == 0
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    assert lib.ibh_device_errors(1) == 2
    assert lib.ibh_device_errors(0) == 0
    assert lib.ibh_pq_workspace_init(ws.data_ptr(), ws.numel(), None) == 0
    assert lib.ibh_pq_matmul(ctypes.byref(d.s), xd.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), None) == 0
    torch.cuda.synchronize()
    assert relerr(out.cpu().numpy(), oracle_lib.pq_matmul(t, x)) <= 1e-4
    assert lib.ibh_device_errors(0) == 0
