"""ibh_matmul_w4a8_x_noalloc (the allocation-free W4A8 decode entry) against
ibh_matmul_w4a8_x with caller workspace: bit-identical outputs on two calls
in a row, the second with a smaller input, and the size limit rejected."""
import ctypes

import numpy as np
import pytest
import torch

import libinferbit_amd as L
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu


def _case(rng, M, N):
    W = (rng.standard_normal((M, N)) * 0.02).astype(np.float32)
    w, s = O.quantize(4, W)
    x = rng.standard_normal(N).astype(np.float32)
    return (torch.from_numpy(w).cuda(), torch.from_numpy(s.view(np.int16)).cuda(), torch.from_numpy(x).cuda(),
            w, s, x)


def _noalloc(out, w, s, x, M, N):
    return L.lib().ibh_matmul_w4a8_x_noalloc(out.data_ptr(), w.data_ptr(), s.data_ptr(), 0, x.data_ptr(), M, N,
                                              torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_workspace_entry():
    L.ops.init(0)
    rng = np.random.default_rng(7)
    for M, N in [(1024, 4096), (300, 1280)]:          # second call: smaller input
        wd, sd, xd, w, s, x = _case(rng, M, N)
        y_ref = torch.empty(M, device="cuda")
        qws = torch.empty(N, dtype=torch.int8, device="cuda")
        sws = torch.empty((N + 127) // 128, device="cuda")
        L.ops.matmul_w4a8_x(y_ref, wd, sd, xd, M, N, qws, sws)
        y = torch.full((M,), float("nan"), device="cuda")
        assert _noalloc(y, wd, sd, xd, M, N) == 0, L.lib().ibh_last_error()
        torch.cuda.synchronize()
        a, b = y.cpu().numpy(), y_ref.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"M={M} N={N}"
        # and the oracle (reference rules), bit for bit
        qx, sa = O.quantize_act(x)
        ref = O.matmul_w4a8(w, s.view(np.float16).astype(np.float32), qx, sa, 1)
        assert np.array_equal(a.view(np.uint32), ref.view(np.uint32)), f"oracle M={M} N={N}"


def test_noalloc_rejects_oversize():
    L.ops.init(0)
    N = 65536 + 256
    y = torch.empty(4, device="cuda")
    w = torch.zeros((4, N // 2), dtype=torch.uint8, device="cuda")
    s = torch.zeros(4, dtype=torch.int16, device="cuda")
    x = torch.zeros(N, device="cuda")
    rc = _noalloc(y, w, s, x, 4, N)
    assert rc == -5
    assert b"65536" in L.lib().ibh_last_error()
