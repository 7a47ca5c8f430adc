"""GPU parity of the IBF v5 INT4 group-scale matvec (ib_pq_session_matmul's
INT4 backend) against the reference-written golden vectors and the oracle.
The GPU sums in another order than the CPU's serial group loop (and reads x
as three int8 digit planes, |error| <= max|xk| * 2^-22 per element, on the
matrix-core path): bar max|y_gpu - y_cpu| / max|y_cpu| <= 1e-4."""
import numpy as np
import pytest
import torch

from conftest import int4g_case, load_golden

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ops():
    import libinferbit_amd as L
    L.ops.init(0)
    return L.ops


def run(ops, t, x, rel=0.0):
    d = ops.Int4gDeviceTensor(t)
    out = torch.full((d.M,), float("nan"), device="cuda")
    d.matmul(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda(), out, rel)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def relerr(a, b):
    assert np.isfinite(a).all()
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("name", ["g32", "g128awq", "g64awq", "g128out", "g96", "g2", "g128big", "g256"])
def test_int4g_golden(ops, name):
    print(f"case int4g golden {name}", flush=True)
    d = load_golden("int4g.npz")
    t = int4g_case(d, name)
    assert relerr(run(ops, t, t["x"]), t["y"]) <= TOL
    assert relerr(run(ops, t, t["x"], float(d["skip_rel"])), t["ys"]) <= TOL


# (M, N, G, AWQ, outliers per row): Mistral/TinyLlama projection shapes on the
# matrix-core path (N = 5632 ends inside a 1 KiB step), the any-G fallback
# (G = 32, 64), a row too long for the LDS digit planes (N = 24576) and
# rows wide enough that a plain launch needs more waves per row (N = 5632).
SHAPES = [(14336, 4096, 128, 1, 4), (4096, 14336, 128, 1, 0), (2048, 5632, 128, 1, 2), (5632, 2048, 128, 0, 0),
          (1024, 4096, 256, 1, 3), (512, 20480, 128, 0, 1), (300, 4096, 64, 1, 3), (77, 2048, 32, 0, 0),
          (64, 24576, 128, 1, 2), (3, 96, 32, 1, 1), (2048, 5632, 128, 0, 0), (256, 5632, 128, 0, 3),
          # the quad-layout kernel with row counts that are not whole quads or
          # blocks, ragged K-ranges (5632 columns) with G = 256, and the
          # outlier sidecar at its limit (32 per row) and one past it
          (1001, 4096, 128, 1, 3), (13, 2048, 128, 0, 2), (333, 5632, 128, 1, 5), (100, 5632, 256, 1, 1),
          (64, 4096, 128, 1, 32), (64, 4096, 128, 1, 33)]


@pytest.mark.parametrize("M,N,G,awq,K", SHAPES)
def test_int4g_shapes(ops, oracle_lib, M, N, G, awq, K):
    from gen_golden import make_int4g
    print(f"case int4g shape {M}x{N} G={G} awq={awq} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N)
    t = make_int4g(rng, M, N, G, awq, K)
    x = rng.standard_normal(N).astype(np.float32)
    x[rng.integers(0, N, 8)] *= 30.0                 # a few large channels
    assert relerr(run(ops, t, x), oracle_lib.int4g_matmul(t, x)) <= TOL


def test_int4g_skip_mask_full_size(ops, oracle_lib):
    """IB_ACT_SPARSE_REL > 0 at the Mistral down_proj shape: a third of the
    groups fall under the threshold and are left out exactly as on the CPU."""
    from gen_golden import make_int4g
    rng = np.random.default_rng(9)
    M, N, G = 4096, 14336, 128
    t = make_int4g(rng, M, N, G, 1, 2)
    x = rng.standard_normal(N).astype(np.float32)
    x[np.repeat(rng.random(N // G) < 0.33, G)] *= 1e-2
    rel = 0.01
    y = run(ops, t, x, rel)
    assert relerr(y, oracle_lib.int4g_matmul(t, x, rel)) <= TOL
    assert relerr(oracle_lib.int4g_matmul(t, x), oracle_lib.int4g_matmul(t, x, rel)) > 10 * TOL


def test_int4g_zero_input_is_zero(ops, oracle_lib):
    from gen_golden import make_int4g
    for (M, N, G) in [(256, 4096, 128), (40, 192, 64)]:
        t = make_int4g(np.random.default_rng(2), M, N, G, 1, 3)
        y = run(ops, t, np.zeros(N, np.float32))
        np.testing.assert_array_equal(y, np.zeros(M, np.float32))


def test_int4g_batched_equals_single(ops):
    from gen_golden import make_int4g
    rng = np.random.default_rng(4)
    for (M, N, G) in [(1000, 4096, 128), (50, 640, 64)]:
        t = make_int4g(rng, M, N, G, 1, 2)
        d = ops.Int4gDeviceTensor(t)
        X = torch.from_numpy(rng.standard_normal((3, N)).astype(np.float32)).cuda()
        for rel in (0.0, 0.05):
            Y = torch.empty(3, M, device="cuda")
            d.matmul_batched(X, Y, rel)
            for b in range(3):
                y = torch.empty(M, device="cuda")
                d.matmul(X[b].contiguous(), y, rel)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(Y[b].cpu().numpy(), y.cpu().numpy())


def test_int4g_rejects_bad_tensors(ops):
    from libinferbit_amd import IbhError
    rng = np.random.default_rng(1)
    x = torch.zeros(96, device="cuda")
    out = torch.zeros(4, device="cuda")
    t = dict(q=rng.integers(0, 256, (4, 48), dtype=np.uint8), s=np.zeros((4, 32), np.uint16))   # G = 3 (odd)
    with pytest.raises(IbhError):
        ops.Int4gDeviceTensor(t).matmul(x, out)
    t = dict(q=rng.integers(0, 256, (4, 48), dtype=np.uint8), s=np.zeros((4, 5), np.uint16))    # 96 % 5 != 0
    with pytest.raises(IbhError):
        ops.Int4gDeviceTensor(t).matmul(x, out)
