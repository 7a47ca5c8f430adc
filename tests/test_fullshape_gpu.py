"""Full-shape parity with every row distinct: the headline matvec shapes
(14336x4096 and 4096x14336, INT8 / INT4 / INT2 with fp32 x), W4A8 batched at
B = 8, and the config-5 prefill GEMM over all 14336 rows for a sample of its
512 tokens.  Weights come from the library's N(0, 0.02) generator and the
reference quantizer (ibh_quantize_rows, byte-identical to quantize.c); every
output row is compared with the oracle.  Bars as in test_gemv_gpu: fp32
activations max|d| / max|y| <= 1e-4, W4A8 bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ops():
    import libinferbit_amd as L
    L.ops.init(0)
    return L.ops


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def f16(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def relerr(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def distinct(bits, M, N, seed):
    """M distinct rows: N(0, 0.02) from the library generator, quantized."""
    from libinferbit_amd import ibf
    w = ibf.fill_normal(M * N, seed, 0.02).reshape(M, N)
    return ibf.quantize(bits, w)


@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("M,N", [(14336, 4096), (4096, 14336)])
def test_matvec_full_shape_distinct_rows(ops, oracle_lib, bits, M, N):
    print(f"case fullshape matvec bits={bits} M={M} N={N}", flush=True)
    w, s = distinct(bits, M, N, 1000 + bits)
    assert len(np.unique(w[:, :64], axis=0)) > M // 2          # rows are not tiled copies
    rng = np.random.default_rng(bits + M)
    for x in (rng.standard_normal(N).astype(np.float32),
              (rng.standard_normal(N) * np.exp(rng.standard_normal(N) * 2)).astype(np.float32)):   # heavy-tailed
        out = torch.empty(M, dtype=torch.float32, device="cuda")
        ops.parallel_matmul(out, dev(w), dev(s.view(np.int16)), dev(x), M, N, bits)
        torch.cuda.synchronize()
        y = out.cpu().numpy()
        ref = oracle_lib.matmul(bits, w, f16(s), x, order=1)
        assert relerr(y, ref) <= TOL


def test_w4a8_batch8_full_shape_distinct_rows(ops, oracle_lib):
    print("case fullshape w4a8 B=8", flush=True)
    M, N, B = 14336, 4096, 8
    w, s = distinct(4, M, N, 77)
    rng = np.random.default_rng(8)
    X = rng.standard_normal((B, N)).astype(np.float32)
    QS = [oracle_lib.quantize_act(X[b]) for b in range(B)]
    QX, SA = np.stack([a for a, _ in QS]), np.stack([b for _, b in QS])
    out = torch.empty(B * M, dtype=torch.float32, device="cuda")
    ops.matmul_w4a8_batch(out, dev(w), dev(s.view(np.int16)), dev(QX), dev(SA), M, N, B, M)
    torch.cuda.synchronize()
    ref = oracle_lib.matmul_w4a8_batch(w, f16(s), QX, SA, M)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), ref.reshape(-1).view(np.uint32))


def test_gemm_config5_all_rows(ops, oracle_lib):
    """M=14336, N=4096, B=512 tokens: every row of 16 sampled tokens against
    the oracle's matmul_int8_batch."""
    print("case fullshape gemm config5", flush=True)
    M, N, B = 14336, 4096, 512
    w, s = distinct(8, M, N, 5)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((B, N)).astype(np.float32)
    out = torch.empty(B * M, dtype=torch.float32, device="cuda")
    ops.gemm_int8(out, dev(w), dev(s.view(np.int16)), dev(x), M, N, B, M)
    torch.cuda.synchronize()
    y = out.cpu().numpy().reshape(B, M)
    toks = np.sort(rng.choice(B, 16, replace=False))
    ref = oracle_lib.matmul_int8_batch(w, f16(s), x[toks]).reshape(len(toks), M)
    assert relerr(y[toks], ref) <= TOL
