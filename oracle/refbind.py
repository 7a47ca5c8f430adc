"""ctypes bindings of the reference library compiled from its own sources.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  ``oracle/Makefile``
(target ``ref``) builds ``oracle/_ref/libinferbit_ref.so`` from the files
under the reference tree; this module calls its exported entry points
(``ib_quantize_int*``, the ``ib_kern`` dispatch table, the W4A8 activation
quantizer, the PQ matmul/reconstruct) to write golden vectors and to
cross-check ``oracle/ib_oracle.c``.

Struct layouts mirror ``src/inferbit_internal.h:199-277`` (``ib_kernels``)
and ``src/pq_decode.h:39-87`` (``ib_pq_tensor``).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB = os.path.join(_HERE, "_ref", "libinferbit_ref.so")
REF_INT4G = os.path.join(_HERE, "_ref", "libref_int4g.so")

P = C.c_void_p
I = C.c_int

_MV = C.CFUNCTYPE(None, P, P, P, P, I, I)                     # matmul_int{4,8,2}
_W4A8 = C.CFUNCTYPE(None, P, P, P, P, P, I, I)
_W4A8B = C.CFUNCTYPE(None, P, P, P, P, P, I, I, I, I)
_I8B = C.CFUNCTYPE(None, P, P, P, P, I, I, I, I)


class IbKernels(C.Structure):
    _fields_ = [
        ("matmul_int4", _MV),
        ("matmul_int8", _MV),
        ("matmul_int2", _MV),
        ("rmsnorm", C.CFUNCTYPE(None, P, P, P, C.c_float, I)),
        ("rope", C.CFUNCTYPE(None, P, P, I, I, C.c_float)),
        ("softmax", C.CFUNCTYPE(None, P, I)),
        ("silu_mul", C.CFUNCTYPE(None, P, P, P, I)),
        ("matmul_w4a8", _W4A8),
        ("matmul_w4a8_batch", _W4A8B),
        ("matmul_int8_batch", _I8B),
    ]


class IbPqTensor(C.Structure):
    _fields_ = [(n, I) for n in ("M", "N", "G", "K", "K_l2", "n_levels", "rotate", "n_outlier",
                                 "format")] + \
               [(n, P) for n in ("codebook_l1_l", "codebook_l1_r", "codebook_l2_l", "codebook_l2_r",
                                 "indices_l1_l", "indices_l1_r", "indices_l2_l", "indices_l2_r")] + \
               [("C", I), ("l2_idx_bytes", I), ("l2_packed_bits", I),
                ("row_scale", P), ("outlier_cols", P), ("outlier_sidecar", P), ("outlier_scale", P),
                ("_arena", P), ("_arena_size", C.c_size_t), ("_mmap_base", P),
                ("_mmap_size", C.c_size_t), ("_owns_mmap", I)]


IB_SIMD_NONE, IB_SIMD_AVX2 = 0, 1

_lib = None


def available() -> bool:
    return os.path.exists(REF_LIB)


def lib():
    global _lib
    if _lib is None:
        _lib = C.CDLL(REF_LIB)
        for q in ("ib_quantize_int8", "ib_quantize_int4", "ib_quantize_int2"):
            getattr(_lib, q).argtypes = [P, P, P, C.c_char_p, I, I]
            getattr(_lib, q).restype = None
        _lib.ib_quantize_input_int8_g128.argtypes = [P, P, P, I]
        _lib.ib_quantize_input_int8_g128.restype = I
        _lib.ib_init_kernels.argtypes = [I]
        _lib.ib_detect_simd.restype = I
        _lib.ib_pq_matmul_fp32.argtypes = [P, P, P]
        _lib.ib_pq_reconstruct_fp32.argtypes = [P, P]
        _lib.ib_pq_lut_cache_create.argtypes = [P, P]
        _lib.ib_pq_lut_cache_free.argtypes = [P]
        _lib.ib_pq_lut_cache_free.restype = None
        _lib.ib_pq_matmul_fp32_streaming_cached.argtypes = [P, P, P, P]
        _lib.ib_pq_matmul_fp32_l1_only.argtypes = [P, P, P]
        _lib.ib_pq_matmul_fp32_q8lut.argtypes = [P, P, P, P]
        _lib.ib_pq_matmul_fp32_streaming_sparse.argtypes = [P, P, P, C.c_float]
        _lib.ib_pq_matmul_fp32_streaming_l2skip_cached.argtypes = [P, P, P, P, C.c_float]
        _lib.ib_pq_lut_cache_quantize_int8.argtypes = [P]
        _lib.ib_pq_matmul_fp32_streaming_int8_cached.argtypes = [P, P, P, P]
        _lib.ib_pq_matmul_fp32_subset.argtypes = [P, P, P, I, P]
        _lib.ib_pq_lm_head_topk.argtypes = [P, P, I, P, P]
        _lib.ib_pq_load_single.argtypes = [C.c_char_p, P]
        _lib.ib_pq_load_single.restype = I
        _lib.ib_pq_free.argtypes = [P]
        _lib.ib_pq_free.restype = None
    return _lib


def pq_load_single(path: str) -> IbPqTensor:
    """ib_pq_load_single (src/pq_decode.c:726-744): the reference's own
    loader fills an ib_pq_tensor whose arrays live in its arena."""
    s = IbPqTensor()
    rc = lib().ib_pq_load_single(path.encode(), C.byref(s))
    if rc != 0:
        raise RuntimeError(f"ib_pq_load_single({path}) = {rc}")
    return s


def pq_free(s: IbPqTensor) -> None:
    lib().ib_pq_free(C.byref(s))


def pq_matmul_struct(s: IbPqTensor, x):
    """ib_pq_matmul_fp32 on a loaded tensor."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(s.M, np.float32)
    assert lib().ib_pq_matmul_fp32(C.byref(s), _p(x), _p(out)) == 0
    return out


def kernels(level: int) -> IbKernels:
    """Fill the global table for ``level`` and return a snapshot of it."""
    L = lib()
    L.ib_init_kernels(level)
    k = IbKernels.in_dll(L, "ib_kern")
    snap = IbKernels()
    C.pointer(snap)[0] = k
    return snap


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def quantize(bits: int, W):
    W = np.ascontiguousarray(W, np.float32)
    M, N = W.shape
    s = np.zeros(M, np.uint16)
    cols = {8: N, 4: N // 2, 2: N // 4}[bits]
    w = np.zeros((M, cols), np.int8 if bits == 8 else np.uint8)
    getattr(lib(), f"ib_quantize_int{bits}")(_p(w), _p(s), _p(W), b"F32", M, N)
    return w, s


def quantize_act(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.shape[0], np.int8)
    s = np.zeros((x.shape[0] + 127) // 128, np.float32)
    lib().ib_quantize_input_int8_g128(_p(x), _p(q), _p(s), x.shape[0])
    return q, s


def matmul(tab: IbKernels, bits: int, w, sc, x):
    w = np.ascontiguousarray(w)
    sc = np.ascontiguousarray(sc, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(w.shape[0], np.float32)
    getattr(tab, f"matmul_int{bits}")(_p(out), _p(w), _p(sc), _p(x), w.shape[0], x.shape[0])
    return out


def matmul_w4a8(tab: IbKernels, w, sw, qx, sa):
    out = np.zeros(w.shape[0], np.float32)
    tab.matmul_w4a8(_p(out), _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(sw, np.float32)),
                    _p(np.ascontiguousarray(qx, np.int8)), _p(np.ascontiguousarray(sa, np.float32)),
                    w.shape[0], qx.shape[0])
    return out


def matmul_int8_batch(tab: IbKernels, w, sw, X, M_stride):
    B, N = X.shape
    out = np.zeros(B * M_stride, np.float32)
    tab.matmul_int8_batch(_p(out), _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(sw, np.float32)),
                          _p(np.ascontiguousarray(X, np.float32)), w.shape[0], N, B, M_stride)
    return out


def matmul_w4a8_batch(tab: IbKernels, w, sw, QX, SA, M_stride):
    B, N = QX.shape
    out = np.zeros(B * M_stride, np.float32)
    tab.matmul_w4a8_batch(_p(out), _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(sw, np.float32)),
                          _p(np.ascontiguousarray(QX, np.int8)), _p(np.ascontiguousarray(SA, np.float32)),
                          w.shape[0], N, B, M_stride)
    return out


def call_f32(tab: IbKernels, name: str, *args):
    return getattr(tab, name)(*args)


def _pq(t: dict):
    s = IbPqTensor()
    for n in ("M", "N", "G", "K", "n_levels", "n_outlier", "C"):
        setattr(s, n, int(t[n]))
    s.K_l2 = int(t.get("K_l2", 0))
    s.l2_idx_bytes = int(t.get("l2_idx_bytes", 1))
    s.format = int(t["format"]) if "format" in t else (1 if t["n_levels"] == 1 else 3)
    keep = []
    m = {"cb1l": "codebook_l1_l", "cb1r": "codebook_l1_r", "cb2l": "codebook_l2_l",
         "cb2r": "codebook_l2_r", "i1l": "indices_l1_l", "i1r": "indices_l1_r", "i2l": "indices_l2_l",
         "i2r": "indices_l2_r", "row_scale": "row_scale", "ocols": "outlier_cols",
         "oside": "outlier_sidecar", "oscale": "outlier_scale"}
    for k, f in m.items():
        a = t.get(k)
        if a is not None:
            a = np.ascontiguousarray(a)
            keep.append(a)
            setattr(s, f, a.ctypes.data)
    return s, keep


def pq_matmul(t: dict, x):
    s, keep = _pq(t)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    rc = lib().ib_pq_matmul_fp32(C.byref(s), _p(x), _p(out))
    assert rc == 0
    return out


def pq_matmul_streaming(t: dict, x):
    """ib_pq_lut_cache_create + ib_pq_matmul_fp32_streaming_cached (the PQ
    session's default variant, src/pq_decode.c:2987)."""
    s, keep = _pq(t)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    cache = C.c_void_p()
    assert lib().ib_pq_lut_cache_create(C.byref(s), C.byref(cache)) == 0
    try:
        assert lib().ib_pq_matmul_fp32_streaming_cached(C.byref(s), cache, _p(x), _p(out)) == 0
    finally:
        lib().ib_pq_lut_cache_free(cache)
    return out


def pq_matmul_q8lut(t: dict, x):
    """ib_pq_matmul_fp32_q8lut, single-threaded (src/pq_decode.c:2451-2561)."""
    s, keep = _pq(t)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    assert lib().ib_pq_matmul_fp32_q8lut(C.byref(s), _p(x), _p(out), None) == 0
    return out


def pq_matmul_variant(t: dict, x, variant: int, skip_threshold=0.0, act_threshold=0.0):
    """What ib_pq_session_matmul runs for each ib_pq_policy variant
    (src/pq_decode.c:4468-4491)."""
    s, keep = _pq(t)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(t["M"], np.float32)
    L = lib()
    if variant == 1:
        assert L.ib_pq_matmul_fp32_l1_only(C.byref(s), _p(x), _p(out)) == 0
        return out
    if variant == 3:
        assert L.ib_pq_matmul_fp32_streaming_sparse(C.byref(s), _p(x), _p(out), C.c_float(act_threshold)) == 0
        return out
    cache = C.c_void_p()
    assert L.ib_pq_lut_cache_create(C.byref(s), C.byref(cache)) == 0
    try:
        if variant == 0:
            assert L.ib_pq_matmul_fp32_streaming_cached(C.byref(s), cache, _p(x), _p(out)) == 0
        elif variant == 2:
            assert L.ib_pq_matmul_fp32_streaming_l2skip_cached(C.byref(s), cache, _p(x), _p(out),
                                                              C.c_float(skip_threshold)) == 0
        elif variant == 4:
            assert L.ib_pq_lut_cache_quantize_int8(cache) == 0
            assert L.ib_pq_matmul_fp32_streaming_int8_cached(C.byref(s), cache, _p(x), _p(out)) == 0
    finally:
        L.ib_pq_lut_cache_free(cache)
    return out


def pq_matmul_subset(t: dict, x, rows):
    s, keep = _pq(t)
    x = np.ascontiguousarray(x, np.float32)
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros(len(rows), np.float32)
    assert lib().ib_pq_matmul_fp32_subset(C.byref(s), _p(x), _p(rows), len(rows), _p(out)) == 0
    return out


def pq_lm_head_topk(t: dict, x, k: int):
    s, keep = _pq(t)
    x = np.ascontiguousarray(x, np.float32)
    lg, ids = np.zeros(k, np.float32), np.zeros(k, np.int32)
    assert lib().ib_pq_lm_head_topk(C.byref(s), _p(x), k, _p(lg), _p(ids)) == 0
    return lg, ids


def pq_reconstruct(t: dict):
    s, keep = _pq(t)
    out = np.zeros((t["M"], t["N"]), np.float32)
    rc = lib().ib_pq_reconstruct_fp32(C.byref(s), _p(out))
    assert rc == 0
    return out


_i4 = None


def _int4g_lib():
    global _i4
    if _i4 is None:
        _i4 = C.CDLL(REF_INT4G)
        _i4.ref_int4g_matmul.argtypes = [P, P, P, P, P, I, I, I, I, P, P]
        _i4.ref_int4g_matmul.restype = I
        _i4.ref_sample_from_logits.argtypes = [P, I, C.c_float, I, C.c_float, P]
        _i4.ref_sample_from_logits.restype = I
    return _i4


def sample_from_logits(logits, temperature, top_k, top_p, state: int):
    """The reference's full-vocabulary pick (src/pq_decode.c:5363-5436) from
    xorshift64 state ``state``; returns (token, advanced state)."""
    lg = np.ascontiguousarray(logits, np.float32)
    st = np.array([state], np.uint64)
    tok = _int4g_lib().ref_sample_from_logits(_p(lg), lg.size, temperature, top_k, top_p, _p(st))
    return tok, int(st[0])


def int4g_matmul(t: dict, x):
    """The reference's INT4 group-scale session matmul (oracle/ref_int4g.c).
    IB_ACT_SPARSE_REL is read by the reference once per process, so a caller
    that wants the skip mask sets it before the first call (in a subprocess)."""
    _int4g_lib()
    q, s = np.ascontiguousarray(t["q"], np.uint8), np.ascontiguousarray(t["s"], np.uint16)
    M, N = q.shape[0], q.shape[1] * 2
    G = N // s.shape[1]
    opt = lambda a, dt: None if a is None else np.ascontiguousarray(a, dt)
    ia, oi, ov = opt(t.get("inv_act"), np.float32), opt(t.get("outl_idx"), np.uint16), opt(t.get("outl_val"), np.uint16)
    K = 0 if oi is None else oi.shape[1]
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(M, np.float32)
    pp = lambda a: None if a is None else _p(a)
    assert _i4.ref_int4g_matmul(_p(q), _p(s), pp(ia), pp(oi), pp(ov), M, N, G, K, _p(x), _p(out)) == 0
    return out
