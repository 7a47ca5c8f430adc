"""Prefill INT8 GEMM (ibh_gemm_int8) against the scalar matmul_int8_batch
restatement (small shapes, every element) and against float64 on sampled
rows at the BASELINE config-5 shape (M=14336, N=4096, B=512).  Bar:
max|y - ref| / max|ref| <= 1e-4 (fp32 accumulate)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import libinferbit_amd as L
    L.ops.init(0)
    return L.ops


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def relerr(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def run(ops, w, s, x, M_stride=None):
    M, N = w.shape
    B = x.shape[0]
    ms = M if M_stride is None else M_stride
    out = torch.full((B * ms,), 7.0, dtype=torch.float32, device="cuda")
    ops.gemm_int8(out, dev(w), dev(s.view(np.int16)), dev(x), M, N, B, ms)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# (16384, 64, 400) takes the 256-row tile (more than 256 blocks at 224 rows),
# every other case the 224-row tile.
@pytest.mark.parametrize("M,N,B", [(128, 64, 64), (300, 256, 70), (37, 192, 5), (1000, 2048, 130), (256, 4096, 1),
                                   (16384, 64, 400)])
def test_gemm_small_vs_oracle(ops, oracle_lib, M, N, B):
    print(f"case gemm M={M} N={N} B={B}", flush=True)
    rng = np.random.default_rng(M + N + B)
    w, s = oracle_lib.quantize(8, (rng.standard_normal((M, N)) * 0.02).astype(np.float32))
    x = rng.standard_normal((B, N)).astype(np.float32)
    ref = oracle_lib.matmul_int8_batch(w, oracle_lib.fp16_to_fp32(s), x)
    assert relerr(run(ops, w, s, x), ref) <= 1e-4


def test_gemm_m_stride(ops, oracle_lib):
    rng = np.random.default_rng(3)
    M, N, B, ms = 100, 128, 9, 130
    w, s = oracle_lib.quantize(8, (rng.standard_normal((M, N)) * 0.02).astype(np.float32))
    x = rng.standard_normal((B, N)).astype(np.float32)
    y = run(ops, w, s, x, ms).reshape(B, ms)
    assert np.all(y[:, M:] == 7.0)                                 # untouched
    ref = oracle_lib.matmul_int8_batch(w, oracle_lib.fp16_to_fp32(s), x, ms).reshape(B, ms)
    assert relerr(y[:, :M], ref[:, :M]) <= 1e-4


def test_gemm_prefill_config5(ops, oracle_lib):
    """M=14336, N=4096, B=512 tokens, x N(0,1): sampled rows against float64."""
    print("case gemm config5", flush=True)
    rng = np.random.default_rng(5)
    M, N, B = 14336, 4096, 512
    base = (rng.standard_normal((256, N)) * 0.02).astype(np.float32)
    wb, sb = oracle_lib.quantize(8, base)
    w, s = np.tile(wb, (M // 256, 1)), np.tile(sb, M // 256)
    x = rng.standard_normal((B, N)).astype(np.float32)
    y = run(ops, w, s, x).reshape(B, M)
    rows = rng.choice(M, 96, replace=False)
    ref = (x.astype(np.float64) @ w[rows].astype(np.float64).T) * oracle_lib.fp16_to_fp32(s[rows]).astype(np.float64)
    assert relerr(y[:, rows], ref) <= 1e-4


def test_gemm_rejects_bad_shape(ops):
    from libinferbit_amd import IbhError
    w = torch.zeros(64 * 100, dtype=torch.int8, device="cuda")
    s = torch.zeros(64, dtype=torch.float16, device="cuda")
    x = torch.zeros(4 * 100, device="cuda")
    out = torch.zeros(4 * 64, device="cuda")
    with pytest.raises(IbhError):
        ops.gemm_int8(out, w, s, x, 64, 100, 4, 64)               # N % 64 != 0
