"""Host-side mirror of the reference's matvec operator entry points.

Names and argument meaning follow the reference (src/threading.c,
src/kernels/scalar.c, src/inferbit_internal.h:199-277): ``out`` first, then
weights, scales, activations, then sizes.  Operands are torch tensors
resident on the GPU; work is enqueued on torch's current stream so
torch.cuda events time it.  Errors raise IbhError (the library's negative
INFERBIT_ERROR_* code plus its message).
"""
from __future__ import annotations

import torch

import ctypes

import numpy as np

from ._lib import Int4gTensor, PqPolicy, PqTensor, check, lib

SCALE_F16, SCALE_F32 = 0, 1


def _ptr(t: torch.Tensor):
    if not t.is_cuda:
        raise ValueError("libinferbit_amd ops take GPU tensors")
    if not t.is_contiguous():
        raise ValueError("operand must be contiguous")
    return t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _scale_kind(s: torch.Tensor) -> int:
    if s.dtype in (torch.float16, torch.int16, torch.uint16):
        return SCALE_F16
    if s.dtype == torch.float32:
        return SCALE_F32
    raise TypeError(f"scales must be fp16 bits or fp32, got {s.dtype}")


def init(device: int = 0) -> None:
    check(lib().ibh_init(device), "ibh_init")


def parallel_matmul(out, w, scales, x, M: int, N: int, bits: int) -> None:
    """ib_parallel_matmul (src/threading.c:244-258): out[M] = W[M,N] x[N] * scales."""
    check(lib().ibh_matmul(_ptr(out), _ptr(w), _ptr(scales), _scale_kind(scales), _ptr(x), M, N, bits,
                           _stream()), "ibh_matmul")


def quantize_input_int8_g128(x, q, s, N: int) -> int:
    """ib_quantize_input_int8_g128 (src/threading.c:401-432); returns the group count."""
    check(lib().ibh_quantize_act_g128(_ptr(x), _ptr(q), _ptr(s), N, _stream()), "ibh_quantize_act_g128")
    return (N + 127) // 128


def parallel_matmul_w4a8(out, w, scales_w, qx, scales_a, M: int, N: int) -> None:
    """ib_parallel_matmul_w4a8 (src/threading.c:283-294), x86 AVX2 kernel semantics."""
    check(lib().ibh_matmul_w4a8(_ptr(out), _ptr(w), _ptr(scales_w), _scale_kind(scales_w), _ptr(qx),
                                _ptr(scales_a), M, N, _stream()), "ibh_matmul_w4a8")


def matmul_w4a8_x(out, w, scales_w, x, M: int, N: int, qx_ws, sa_ws) -> None:
    """tensor_matmul's INT4 branch (src/forward.c:158-172): quantize x, then W4A8."""
    check(lib().ibh_matmul_w4a8_x(_ptr(out), _ptr(w), _ptr(scales_w), _scale_kind(scales_w), _ptr(x), M, N,
                                  _ptr(qx_ws), _ptr(sa_ws), _stream()), "ibh_matmul_w4a8_x")


def matmul_w4a8_batch(out, w, scales_w, qx, scales_a, M: int, N: int, B: int, M_stride: int) -> None:
    """ib_kern.matmul_w4a8_batch (src/kernels/scalar.c:86-124)."""
    check(lib().ibh_matmul_w4a8_batch(_ptr(out), _ptr(w), _ptr(scales_w), _scale_kind(scales_w), _ptr(qx),
                                      _ptr(scales_a), M, N, B, M_stride, _stream()), "ibh_matmul_w4a8_batch")


def matmul_int8_batch(out, w, scales_w, x, M: int, N: int, B: int, M_stride: int) -> None:
    """ib_kern.matmul_int8_batch (src/kernels/scalar.c:70-84)."""
    check(lib().ibh_matmul_int8_batch(_ptr(out), _ptr(w), _ptr(scales_w), _scale_kind(scales_w), _ptr(x), M,
                                      N, B, M_stride, _stream()), "ibh_matmul_int8_batch")


def gemm_int8(out, w, scales, x, M: int, N: int, B: int, M_stride: int, ws=None) -> None:
    """Prefill INT8 GEMM, matmul_int8_batch semantics at any B (src/kernels/scalar.c:70-84)."""
    if ws is None:
        ws = torch.empty(lib().ibh_gemm_int8_workspace_bytes(N, B), dtype=torch.uint8, device=out.device)
    check(lib().ibh_gemm_int8(_ptr(out), _ptr(w), _ptr(scales), _scale_kind(scales), _ptr(x), M, N, B, M_stride,
                              _ptr(ws), ws.numel(), _stream()), "ibh_gemm_int8")


def _optptr(t):
    return None if t is None else _ptr(t)


def kv_cache_write(kdata, vdata, kscales, vscales, pos: int, k, v, n_kv: int, head_dim: int, kv_bits: int) -> None:
    """kv_cache_write (src/forward.c:352-413) into device cache tensors."""
    check(lib().ibh_kv_write(_ptr(kdata), _ptr(vdata), _optptr(kscales), _optptr(vscales), pos, _ptr(k), _ptr(v),
                             n_kv, head_dim, kv_bits, _stream()), "ibh_kv_write")


def attn_decode(out, q, kdata, vdata, kscales, vscales, pos: int, n_heads: int, n_kv: int, head_dim: int,
                kv_bits: int) -> None:
    """ib_attn_head_task for all heads of a layer (src/forward.c:449-504)."""
    check(lib().ibh_attn_decode(_ptr(out), _ptr(q), _ptr(kdata), _ptr(vdata), _optptr(kscales), _optptr(vscales),
                                pos, n_heads, n_kv, head_dim, kv_bits, None, 0, _stream()), "ibh_attn_decode")


class PqDeviceTensor:
    """A PQ tensor (ib_pq_tensor layout, src/pq_decode.h:39-87) uploaded to the
    GPU once.  `t` maps the reference field names used by the oracle
    (cb1l, cb1r, cb2l, cb2r, i1l, i1r, i2l, i2r, row_scale, ocols, oside,
    oscale) and sizes (M, N, G, K, K_l2, n_levels, n_outlier, C,
    l2_idx_bytes) to numpy arrays / ints."""

    _MAP = {"cb1l": "codebook_l1_l", "cb1r": "codebook_l1_r", "cb2l": "codebook_l2_l", "cb2r": "codebook_l2_r",
            "i1l": "indices_l1_l", "i1r": "indices_l1_r", "i2l": "indices_l2_l", "i2r": "indices_l2_r",
            "row_scale": "row_scale", "ocols": "outlier_cols", "oside": "outlier_sidecar",
            "oscale": "outlier_scale"}

    def __init__(self, t: dict):
        import torch
        self.keep = []
        s = PqTensor()
        for n in ("M", "N", "G", "K", "n_levels", "n_outlier", "C"):
            setattr(s, n, int(t[n]))
        s.K_l2 = int(t.get("K_l2", 0))
        s.l2_idx_bytes = int(t.get("l2_idx_bytes", 1))
        s.format = int(t.get("format", 0))
        for k, f in self._MAP.items():
            a = t.get(k)
            if a is not None:
                d = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
                self.keep.append(d)
                setattr(s, f, d.data_ptr())
        if s.n_outlier > 0:
            mask = np.ones(s.N, bool)
            mask[np.asarray(t["ocols"])] = False
            inner = np.nonzero(mask)[0].astype(np.int32)
            d = torch.from_numpy(inner.view(np.uint8).copy()).cuda()
            self.keep.append(d)
            s.inner_cols = d.data_ptr()
        self.s = s
        self.M = s.M
        # a workspace of its own (tables, slab partials), allocated once
        self.ws = torch.empty(max(1, lib().ibh_pq_workspace_bytes(ctypes.byref(s))), dtype=torch.uint8,
                              device="cuda")
        check(lib().ibh_pq_workspace_init(_ptr(self.ws), self.ws.numel(), _stream()), "ibh_pq_workspace_init")
        self._topk_ws = {}

    def matmul(self, x, out) -> None:
        """ib_pq_matmul_fp32 (src/pq_decode.c:1684)."""
        check(lib().ibh_pq_matmul(ctypes.byref(self.s), _ptr(x), _ptr(out), _ptr(self.ws), self.ws.numel(),
                                  _stream()), "ibh_pq_matmul")

    def matmul_policy(self, x, out, variant: int, skip_threshold: float = 0.0, act_threshold: float = 0.0) -> None:
        """ib_pq_session_matmul with an ib_pq_policy (src/pq_decode.c:4464-4491)."""
        p = PqPolicy(variant, skip_threshold, act_threshold)
        check(lib().ibh_pq_matmul_policy(ctypes.byref(self.s), _ptr(x), _ptr(out), ctypes.byref(p), _ptr(self.ws),
                                         self.ws.numel(), _stream()), "ibh_pq_matmul_policy")

    def matmul_q8lut(self, x, out) -> None:
        """ib_pq_matmul_fp32_q8lut (src/pq_decode.c:2451-2561)."""
        check(lib().ibh_pq_matmul_q8lut(ctypes.byref(self.s), _ptr(x), _ptr(out), _ptr(self.ws), self.ws.numel(),
                                        _stream()), "ibh_pq_matmul_q8lut")

    def lm_head_topk(self, x, k_top: int):
        """ib_pq_lm_head_topk (src/pq_decode.c:2259-2346): (logits [k], ids [k]) on the GPU."""
        need = lib().ibh_pq_topk_workspace_bytes(ctypes.byref(self.s), k_top)
        ws = self._topk_ws.get(k_top)
        if ws is None:
            # prepared once, kept for later calls with the same K_top
            ws = torch.empty(max(1, need), dtype=torch.uint8, device="cuda")
            check(lib().ibh_pq_workspace_init(_ptr(ws), ws.numel(), _stream()), "ibh_pq_workspace_init")
            self._topk_ws[k_top] = ws
        lg = torch.empty(k_top, device="cuda")
        ids = torch.empty(k_top, dtype=torch.int32, device="cuda")
        check(lib().ibh_pq_lm_head_topk(ctypes.byref(self.s), _ptr(x), k_top, _ptr(lg), _ptr(ids), _ptr(ws), need,
                                        _stream()), "ibh_pq_lm_head_topk")
        return lg, ids

    def matmul_streaming(self, x, out) -> None:
        """ib_pq_matmul_fp32_streaming_cached (src/pq_decode.c:2987): every chunk."""
        check(lib().ibh_pq_matmul_streaming(ctypes.byref(self.s), _ptr(x), _ptr(out), _ptr(self.ws),
                                            self.ws.numel(), _stream()), "ibh_pq_matmul_streaming")


class Int4gDeviceTensor:
    """An IBF v5 INT4 group-scale tensor (struct ib_int4_tensor,
    src/pq_decode.c:3474-3482) uploaded to the GPU once.  `t` maps q
    (uint8 [M, N/2]), s (fp16 bits [M, N/G]) and the optional inv_act
    (fp32 [N]), outl_idx / outl_val (uint16 / fp16 bits [M, K_out]) to numpy
    arrays (None or absent = not present)."""

    def __init__(self, t: dict):
        self.keep = []
        s = Int4gTensor()
        q = np.ascontiguousarray(t["q"], np.uint8)
        sc = np.ascontiguousarray(t["s"], np.uint16)
        s.M, s.N = q.shape[0], q.shape[1] * 2
        s.G = s.N // sc.shape[1]
        for f in ("q", "s", "inv_act", "outl_idx", "outl_val"):
            a = t.get(f)
            if a is not None:
                d = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
                self.keep.append(d)
                setattr(s, f, d.data_ptr())
        s.K_out = 0 if t.get("outl_idx") is None else int(np.asarray(t["outl_idx"]).shape[1])
        self.s = s
        self.M, self.N = s.M, s.N

    def matmul(self, x, out, act_sparse_rel: float = 0.0) -> None:
        """ib_pq_session_matmul on this tensor (src/pq_decode.c:4442-4452)."""
        check(lib().ibh_int4g_matmul(ctypes.byref(self.s), _ptr(x), _ptr(out), act_sparse_rel, None, 0, _stream()),
              "ibh_int4g_matmul")

    def matmul_batched(self, x, out, act_sparse_rel: float = 0.0) -> None:
        """ib_pq_session_matmul_batched (src/pq_decode.c:4501-4539): x [B, N], out [B, M]."""
        B = x.shape[0]
        check(lib().ibh_int4g_matmul_batched(ctypes.byref(self.s), B, _ptr(x), _ptr(out), act_sparse_rel, None, 0,
                                             _stream()), "ibh_int4g_matmul_batched")
