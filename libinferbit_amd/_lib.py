"""ctypes loader for libibhip.so with the signatures of include/ibhip.h."""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libibhip.so")
_lib = None

P = C.c_void_p
I = C.c_int
SZ = C.c_size_t

# name -> (restype, argtypes); must match include/ibhip.h
SIGNATURES = {
    "ibh_init": (I, [I]),
    "ibh_last_error": (C.c_char_p, []),
    "ibh_version": (C.c_char_p, []),
    "ibh_default_stream": (P, []),
    "ibh_synchronize": (I, [P]),
    "ibh_device_malloc": (I, [C.POINTER(P), SZ]),
    "ibh_device_free": (I, [P]),
    "ibh_memcpy_h2d": (I, [P, P, SZ, P]),
    "ibh_memcpy_d2h": (I, [P, P, SZ, P]),
    "ibh_memcpy_d2d": (I, [P, P, SZ, P]),
    "ibh_matmul": (I, [P, P, P, I, P, I, I, I, P]),
    "ibh_set_tile_config": (I, [I, I, I, I]),
    "ibh_probe": (I, [I, P, SZ, P]),
    "ibh_probe_read": (I, [I, I, I, I, P, SZ, P]),
    "ibh_probe_read_write": (I, [I, I, I, I, P, SZ, P, I, P]),
    "ibh_probe_chain": (I, [I, I, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "ibh_matmul_w4a8_x_noalloc": (I, [P, P, P, I, P, I, I, P]),
    "ibh_quantize_act_g128": (I, [P, P, P, I, P]),
    "ibh_matmul_w4a8": (I, [P, P, P, I, P, P, I, I, P]),
    "ibh_matmul_w4a8_x": (I, [P, P, P, I, P, I, I, P, P, P]),
    "ibh_matmul_w4a8_batch": (I, [P, P, P, I, P, P, I, I, I, I, P]),
    "ibh_matmul_int8_batch": (I, [P, P, P, I, P, I, I, I, I, P]),
    "ibh_gemm_int8_workspace_bytes": (SZ, [I, I]),
    "ibh_gemm_int8": (I, [P, P, P, I, P, I, I, I, I, P, SZ, P]),
    "ibh_kv_write": (I, [P, P, P, P, I, P, P, I, I, I, P]),
    "ibh_attn_workspace_bytes": (SZ, [I, I, I]),
    "ibh_attn_decode": (I, [P, P, P, P, P, P, I, I, I, I, I, P, SZ, P]),
    "ibh_attn_exact_set_grouped": (I, [I]),
    "ibh_attn_set_split": (I, [I]),
    "ibh_pq_workspace_bytes": (SZ, [P]),
    "ibh_pq_workspace_init": (I, [P, SZ, P]),
    "ibh_pq_matmul_fp32_host": (I, [P, P, P]),
    "ibh_pq_host_release": (None, [P]),
    "ibh_pq_matmul_policy_host": (I, [P, P, P, P]),
    "ibh_int4g_matmul_host": (I, [P, P, P]),
    "ibh_int4g_host_release": (None, [P]),
    "ibh_device_errors": (I, [I]),
    "ibh_pq_matmul": (I, [P, P, P, P, SZ, P]),
    "ibh_pq_set_fused": (I, [I]),
    "ibh_pq_matmul_streaming": (I, [P, P, P, P, SZ, P]),
    "ibh_pq_matmul_policy": (I, [P, P, P, P, P, SZ, P]),
    "ibh_pq_matmul_q8lut": (I, [P, P, P, P, SZ, P]),
    "ibh_pq_topk_workspace_bytes": (SZ, [P, I]),
    "ibh_pq_lm_head_topk": (I, [P, P, I, P, P, P, SZ, P]),
    "ibh_int4g_workspace_bytes": (SZ, [P]),
    "ibh_int4g_matmul": (I, [P, P, P, C.c_float, P, SZ, P]),
    "ibh_int4g_matmul_batched": (I, [P, I, P, P, C.c_float, P, SZ, P]),
    "ibh_v5_open": (I, [C.c_char_p, P]),
    "ibh_v5_close": (None, [P]),
    "ibh_v5_dims": (I, [P, P]),
    "ibh_v5_tensor_info": (I, [P, C.c_char_p, P, P, P]),
    "ibh_v5_set_default_policy": (I, [P, P]),
    "ibh_v5_set_policy": (I, [P, C.c_char_p, P]),
    "ibh_v5_session_matmul": (I, [P, C.c_char_p, P, P, P]),
    "ibh_v5_kv_create": (I, [P, I, P]),
    "ibh_v5_kv_free": (None, [P]),
    "ibh_v5_kv_clear": (None, [P]),
    "ibh_v5_kv_length": (I, [P]),
    "ibh_v5_forward_step": (I, [P, P, I, I, P]),
    "ibh_v5_forward_step_to_hidden": (I, [P, P, I, I, P]),
    "ibh_v5_generate_greedy": (I, [P, P, P, I, I, I, P, P]),
    "ibh_v5_generate_sample": (I, [P, P, P, I, I, I, P, P, P]),
    "ibh_v5_sample_from_logits": (I, [P, I, P, P]),
    "ibh_model_load": (I, [C.c_char_p, I, P]),
    "ibh_model_free": (None, [P]),
    "ibh_model_dims": (I, [P, P]),
    "ibh_model_forward": (I, [P, P, I, P, I]),
    "ibh_model_generate_greedy": (I, [P, P, I, P, I]),
    "ibh_model_set_exact": (I, [P, I]),
    "ibh_model_kv_length": (I, [P]),
    "ibh_model_kv_clear": (I, [P]),
    "ibh_model_kv_truncate": (I, [P, I]),
    "ibh_model_kv_prefill": (I, [P, P, P, I]),
    "ibh_model_decode_steps": (I, [P, I]),
    "ibh_model_synchronize": (I, [P]),
    "ibh_model_forward_positions": (I, [P, P, I, P, I]),
    "ibh_prompt_lookup_search": (I, [P, I, I, I, P]),
    "ibh_model_generate": (I, [P, P, I, P, I, P]),
    "ibh_default_sample_params": (None, []),   # struct return: restype set below
    "ibh_model_generate_lookup": (I, [P, P, I, P, I, I, I]),
    "ibh_model_generate_draft": (I, [P, P, P, I, P, I, I]),
    "ibh_packed_row_bytes": (SZ, [I, I]),
    "ibh_quantize_rows": (I, [I, P, I, I, P, P]),
    "ibh_fill_normal": (I, [P, SZ, C.c_uint64, C.c_uint64, C.c_float]),
    "ibh_expf_host": (None, [P, P, SZ]),
    "ib_init_kernels_hip": (None, [P]),
    "ibh_register_host_weights": (I, [P, SZ, C.POINTER(P)]),
    "ibh_unregister_host_weights": (None, [P]),
    "ibh_host_attn": (I, [P, P, P, P, P, I, I, I, P, P, I, I, I]),
    "ibh_host_kv_release": (None, [P]),
}


class IbhError(RuntimeError):
    def __init__(self, code: int, where: str):
        msg = lib().ibh_last_error()
        super().__init__(f"{where} failed with code {code}: {msg.decode() if msg else 'no message'}")
        self.code = code


def lib_path() -> str:
    return _LIB_PATH


def loaded() -> bool:
    return _lib is not None


def lib():
    """Load libibhip.so; raise if it has not been built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"libinferbit_amd: {_LIB_PATH} is missing -- build it with "
                "`python -m libinferbit_amd.build` (hipcc, gfx950). There is no CPU fallback.")
        L = C.CDLL(_LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        L.ibh_default_sample_params.restype = SampleParams
        _lib = L
    return _lib


def check(rc: int, where: str) -> None:
    if rc != 0:
        raise IbhError(rc, where)


class PqTensor(C.Structure):
    """ibh_pq_tensor (include/ibhip.h)."""
    _fields_ = [(n, I) for n in ("M", "N", "G", "K", "K_l2", "n_levels", "n_outlier", "C", "l2_idx_bytes")] + \
               [(n, P) for n in ("codebook_l1_l", "codebook_l1_r", "codebook_l2_l", "codebook_l2_r",
                                 "indices_l1_l", "indices_l1_r", "indices_l2_l", "indices_l2_r", "row_scale",
                                 "outlier_cols", "outlier_sidecar", "outlier_scale", "inner_cols")] + \
               [("format", I)]


class PqSampleParams(C.Structure):
    """ib_pq_sample_params (src/pq_decode.h:499-504)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("seed", C.c_uint32)]


class PqPolicy(C.Structure):
    """ibh_pq_policy (include/ibhip.h)."""
    _fields_ = [("variant", I), ("skip_threshold", C.c_float), ("act_threshold", C.c_float)]


class Int4gTensor(C.Structure):
    """ibh_int4g_tensor (include/ibhip.h)."""
    _fields_ = [(n, P) for n in ("q", "s", "inv_act", "outl_idx", "outl_val")] + \
               [(n, I) for n in ("M", "N", "G", "K_out")]


class SampleParams(C.Structure):
    """ibh_sample_params (include/ibhip.h) = inferbit_sample_params."""
    _fields_ = [("temperature", C.c_float), ("top_k", I), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("max_tokens", I), ("seed", I)]
