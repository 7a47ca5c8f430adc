"""ctypes bindings of the C restatement in ``oracle/ib_oracle.c``.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Arrays are numpy;
every wrapper allocates its outputs and returns them.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_lib", "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
I = C.c_int


def _declare(L):
    sigs = {
        "or_fp16_to_fp32": (C.c_float, [C.c_uint16]),
        "or_fp32_to_fp16_trunc": (C.c_uint16, [C.c_float]),
        "or_fp32_to_fp16_rne": (C.c_uint16, [C.c_float]),
        "or_quantize_int8": (None, [P, P, P, I, I]),
        "or_quantize_int4": (None, [P, P, P, I, I]),
        "or_quantize_int2": (None, [P, P, P, I, I]),
        "or_quantize_act_g128": (I, [P, P, P, I]),
        "or_matmul_int8": (None, [P, P, P, P, I, I, I]),
        "or_matmul_int4": (None, [P, P, P, P, I, I, I]),
        "or_matmul_int2": (None, [P, P, P, P, I, I]),
        "or_matmul_w4a8": (None, [P, P, P, P, P, I, I, I]),
        "or_matmul_int8_batch": (None, [P, P, P, P, I, I, I, I]),
        "or_matmul_w4a8_batch": (None, [P, P, P, P, P, I, I, I, I]),
        "or_kv_write": (None, [P, P, P, P, I, P, P, I, I, I]),
        "or_attn_decode": (None, [P, P, P, P, P, P, P, I, I, I, I, I]),
        "or_softmax": (None, [P, I]),
        "or_rmsnorm": (None, [P, P, P, C.c_float, I]),
        "or_rope": (None, [P, P, I, I, C.c_float]),
        "or_silu_mul": (None, [P, P, P, I]),
        "or_pq_matmul": (I, [P, P, P]),
        "or_pq_matmul_streaming": (I, [P, P, P]),
        "or_pq_matmul_q8lut": (I, [P, P, P]),
        "or_pq_matmul_variant": (I, [P, P, P, I, C.c_float, C.c_float, I]),
        "or_pq_matmul_subset": (I, [P, P, P, I, P]),
        "or_pq_lm_head_topk": (I, [P, P, I, P, P]),
        "or_pq_reconstruct": (I, [P, P]),
        "or_expf_batch": (None, [P, P, C.c_size_t]),
        "or_int4g_matmul": (I, [P, P, P, P, P, I, I, I, I, P, C.c_float, P]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def packed_cols(bits: int, N: int) -> int:
    return {8: N, 4: N // 2, 2: N // 4}[bits]


def quantize(bits: int, W):
    """Row-wise weight quantization -> (packed uint8/int8 [M, row_bytes], fp16 bits uint16 [M])."""
    W = _c(W, np.float32)
    M, N = W.shape
    s = np.zeros(M, np.uint16)
    if bits == 8:
        w = np.zeros((M, N), np.int8)
        lib().or_quantize_int8(_p(w), _p(s), _p(W), M, N)
    else:
        w = np.zeros((M, packed_cols(bits, N)), np.uint8)
        getattr(lib(), f"or_quantize_int{bits}")(_p(w), _p(s), _p(W), M, N)
    return w, s


def fp16_to_fp32(h):
    h = np.asarray(h, np.uint16)
    return np.array([lib().or_fp16_to_fp32(int(v)) for v in h.ravel()], np.float32).reshape(h.shape)


def quantize_act(x):
    x = _c(x, np.float32)
    N = x.shape[0]
    q = np.zeros(N, np.int8)
    s = np.zeros((N + 127) // 128, np.float32)
    lib().or_quantize_act_g128(_p(x), _p(q), _p(s), N)
    return q, s


def matmul(bits: int, w, scales, x, order: int = 1):
    """ib_kern.matmul_int{8,4,2} semantics; scales fp32 [M]."""
    M = w.shape[0]
    N = x.shape[0]
    out = np.zeros(M, np.float32)
    w = np.ascontiguousarray(w)
    sc, x = _c(scales, np.float32), _c(x, np.float32)
    if bits == 2:
        lib().or_matmul_int2(_p(out), _p(w), _p(sc), _p(x), M, N)
    else:
        getattr(lib(), f"or_matmul_int{bits}")(_p(out), _p(w), _p(sc), _p(x), M, N, order)
    return out


def matmul_w4a8(w, sw, qx, sa, order: int = 1):
    M = w.shape[0]
    N = qx.shape[0]
    out = np.zeros(M, np.float32)
    lib().or_matmul_w4a8(_p(out), _p(np.ascontiguousarray(w)), _p(_c(sw, np.float32)),
                         _p(_c(qx, np.int8)), _p(_c(sa, np.float32)), M, N, order)
    return out


def matmul_int8_batch(w, sw, X, M_stride=None):
    M, N = w.shape
    B = X.shape[0]
    ms = M if M_stride is None else M_stride
    out = np.zeros(B * ms, np.float32)
    lib().or_matmul_int8_batch(_p(out), _p(np.ascontiguousarray(w)), _p(_c(sw, np.float32)),
                               _p(_c(X, np.float32)), M, N, B, ms)
    return out


def matmul_w4a8_batch(w, sw, QX, SA, M_stride=None):
    M = w.shape[0]
    B, N = QX.shape
    ms = M if M_stride is None else M_stride
    out = np.zeros(B * ms, np.float32)
    lib().or_matmul_w4a8_batch(_p(out), _p(np.ascontiguousarray(w)), _p(_c(sw, np.float32)),
                               _p(_c(QX, np.int8)), _p(_c(SA, np.float32)), M, N, B, ms)
    return out


def kv_row_bytes(bits: int, n_kv: int, hd: int) -> int:
    kv_dim = n_kv * hd
    return {32: 4 * kv_dim, 16: 4 * kv_dim, 8: kv_dim, 4: (kv_dim + 1) // 2}[bits]


def kv_alloc(bits: int, cap: int, n_kv: int, hd: int):
    rb = kv_row_bytes(bits, n_kv, hd)
    k = np.zeros(cap * rb, np.uint8)
    v = np.zeros(cap * rb, np.uint8)
    ks = np.zeros(cap * n_kv, np.float32)
    vs = np.zeros(cap * n_kv, np.float32)
    return k, v, ks, vs


def kv_write(cache, pos, k, v, n_kv, hd, bits):
    kd, vd, ks, vs = cache
    lib().or_kv_write(_p(kd), _p(vd), _p(ks), _p(vs), pos, _p(_c(k, np.float32)),
                      _p(_c(v, np.float32)), n_kv, hd, bits)


def attn_decode(q, cache, pos, n_heads, n_kv, hd, bits):
    kd, vd, ks, vs = cache
    out = np.zeros(n_heads * hd, np.float32)
    att = np.zeros(pos + 1, np.float32)
    lib().or_attn_decode(_p(out), _p(att), _p(_c(q, np.float32)), _p(kd), _p(vd), _p(ks), _p(vs),
                         pos, n_heads, n_kv, hd, bits)
    return out


def softmax(x):
    d = _c(x, np.float32).copy()
    lib().or_softmax(_p(d), d.shape[0])
    return d


def rmsnorm(x, w, eps):
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.zeros_like(x)
    lib().or_rmsnorm(_p(out), _p(x), _p(w), C.c_float(eps), x.shape[0])
    return out


def rope(q, k, hd, pos, theta):
    q, k = _c(q, np.float32).copy(), _c(k, np.float32).copy()
    lib().or_rope(_p(q), _p(k), hd, pos, C.c_float(theta))
    return q, k


def silu_mul(g, u):
    g, u = _c(g, np.float32), _c(u, np.float32)
    out = np.zeros_like(g)
    lib().or_silu_mul(_p(out), _p(g), _p(u), g.shape[0])
    return out


class _PQ(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("M", "N", "G", "K", "K_l2", "n_levels", "n_outlier", "C",
                                       "l2_idx_bytes")] + \
               [(n, C.c_void_p) for n in ("cb1l", "cb1r", "cb2l", "cb2r", "i1l", "i1r", "i2l", "i2r",
                                          "row_scale", "ocols", "oside", "oscale")]


def _pq_struct(t: dict):
    s = _PQ()
    for n in ("M", "N", "G", "K", "n_levels", "n_outlier", "C"):
        setattr(s, n, int(t[n]))
    s.K_l2 = int(t.get("K_l2", 0))
    s.l2_idx_bytes = int(t.get("l2_idx_bytes", 1))
    keep = []
    for n in ("cb1l", "cb1r", "cb2l", "cb2r", "i1l", "i1r", "i2l", "i2r", "row_scale", "ocols", "oside",
              "oscale"):
        a = t.get(n)
        if a is not None:
            a = np.ascontiguousarray(a)
            keep.append(a)
            setattr(s, n, a.ctypes.data)
    return s, keep


def pq_matmul(t: dict, x):
    s, keep = _pq_struct(t)
    x = _c(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    lib().or_pq_matmul(C.byref(s), _p(x), _p(out))
    return out


def pq_matmul_streaming(t: dict, x):
    """ib_pq_matmul_fp32_streaming_cached (the session's default PQ variant)."""
    s, keep = _pq_struct(t)
    x = _c(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    assert lib().or_pq_matmul_streaming(C.byref(s), _p(x), _p(out)) == 0
    return out


def pq_matmul_q8lut(t: dict, x):
    """ib_pq_matmul_fp32_q8lut (int8-quantised tables)."""
    s, keep = _pq_struct(t)
    x = _c(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    assert lib().or_pq_matmul_q8lut(C.byref(s), _p(x), _p(out)) == 0
    return out


def pq_matmul_variant(t: dict, x, variant: int, skip_threshold=0.0, act_threshold=0.0):
    """The PQ session's policy variants (0 streaming, 1 l1-only, 2 l2skip,
    3 sparse, 4 int8); t["format"] == 4 marks a pyramid tensor."""
    s, keep = _pq_struct(t)
    x = _c(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    assert lib().or_pq_matmul_variant(C.byref(s), _p(x), _p(out), variant, C.c_float(skip_threshold),
                                      C.c_float(act_threshold), int(t.get("format", 0) == 4)) == 0
    return out


def pq_matmul_subset(t: dict, x, rows):
    s, keep = _pq_struct(t)
    x = _c(x, np.float32)
    rows = _c(rows, np.int32)
    out = np.zeros(len(rows), np.float32)
    assert lib().or_pq_matmul_subset(C.byref(s), _p(x), _p(rows), len(rows), _p(out)) == 0
    return out


def pq_lm_head_topk(t: dict, x, k: int):
    s, keep = _pq_struct(t)
    x = _c(x, np.float32)
    lg, ids = np.zeros(k, np.float32), np.zeros(k, np.int32)
    assert lib().or_pq_lm_head_topk(C.byref(s), _p(x), k, _p(lg), _p(ids)) == 0
    return lg, ids


def pq_reconstruct(t: dict):
    s, keep = _pq_struct(t)
    out = np.zeros((t["M"], t["N"]), np.float32)
    lib().or_pq_reconstruct(C.byref(s), _p(out))
    return out


def expf(x):
    """glibc expf elementwise (the reference's libm)."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_expf_batch(_p(x), _p(y), C.c_size_t(x.size))
    return y


def _opt(a, dt):
    return None if a is None else _c(a, dt)


def int4g_matmul(t: dict, x, act_sparse_rel: float = 0.0):
    """ib_pq_session_matmul on an INT4 group-scale tensor ``t`` (keys q, s,
    inv_act, outl_idx, outl_val; the optional ones may be None)."""
    q, s = _c(t["q"], np.uint8), _c(t["s"], np.uint16)
    M, N = q.shape[0], q.shape[1] * 2
    G = N // s.shape[1]
    ia = _opt(t.get("inv_act"), np.float32)
    oi, ov = _opt(t.get("outl_idx"), np.uint16), _opt(t.get("outl_val"), np.uint16)
    K = 0 if oi is None else oi.shape[1]
    x = _c(x, np.float32)
    out = np.zeros(M, np.float32)
    rc = lib().or_int4g_matmul(_p(q), _p(s), None if ia is None else _p(ia), None if oi is None else _p(oi),
                               None if ov is None else _p(ov), M, N, G, K, _p(x), C.c_float(act_sparse_rel), _p(out))
    assert rc == 0
    return out
