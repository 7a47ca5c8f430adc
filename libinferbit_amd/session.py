"""The IBF v5 PQ session on the GPU: twins of the reference's session API
(src/pq_decode.h:345-506: ib_pq_session_open / _set_policy /
_set_default_policy / _matmul / _tensor_shape, ib_pq_kv_cache_create /
_clear / _length, ib_pq_forward_step, ib_pq_forward_step_to_hidden,
ib_pq_generate_greedy).  Host numpy arrays in and out for the step and
generate calls; device tensors for `matmul`.  Errors raise IbhError."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import PqPolicy, PqSampleParams, check, lib

DIM_NAMES = ("num_layers", "hidden_size", "num_heads", "num_kv_heads", "head_dim", "intermediate_size",
             "vocab_size", "fused_qkv", "fused_gateup")
KINDS = ("pq", "int4", "fp16")

VARIANT_STREAMING, VARIANT_L1_ONLY, VARIANT_L2SKIP, VARIANT_SPARSE, VARIANT_INT8 = range(5)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class KvCache:
    """ib_pq_kv_cache (src/pq_decode.c:4740-4852): fp32 K/V in HBM."""

    def __init__(self, session: "PqSession", max_seq: int):
        h = ctypes.c_void_p()
        check(lib().ibh_v5_kv_create(session._h, max_seq, ctypes.byref(h)), "ibh_v5_kv_create")
        self._h = h
        self.session = session   # the cache must not outlive its session
        self.max_seq = max_seq

    def clear(self) -> None:
        lib().ibh_v5_kv_clear(self._h)

    def __len__(self) -> int:
        return lib().ibh_v5_kv_length(self._h)

    def close(self) -> None:
        if self._h:
            lib().ibh_v5_kv_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PqSession:
    def __init__(self, path: str):
        """ib_pq_session_open (src/pq_decode.c:4111-4362), data region in HBM."""
        h = ctypes.c_void_p()
        check(lib().ibh_v5_open(path.encode(), ctypes.byref(h)), "ibh_v5_open")
        self._h = h
        d = np.zeros(9, np.int32)
        check(lib().ibh_v5_dims(self._h, _ptr(d)), "ibh_v5_dims")
        self.dims = dict(zip(DIM_NAMES, (int(v) for v in d)))

    def close(self) -> None:
        if self._h:
            lib().ibh_v5_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor_info(self, name: str):
        """(backend, M, N) of a matrix, as ib_pq_session_tensor_shape finds it."""
        k, m, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().ibh_v5_tensor_info(self._h, name.encode(), ctypes.byref(k), ctypes.byref(m), ctypes.byref(n)),
              "ibh_v5_tensor_info")
        return KINDS[k.value], m.value, n.value

    def set_default_policy(self, variant: int, skip_threshold: float = 0.0, act_threshold: float = 0.0) -> None:
        p = PqPolicy(variant, skip_threshold, act_threshold)
        check(lib().ibh_v5_set_default_policy(self._h, ctypes.byref(p)), "ibh_v5_set_default_policy")

    def set_policy(self, name: str, variant: int, skip_threshold: float = 0.0, act_threshold: float = 0.0) -> None:
        p = PqPolicy(variant, skip_threshold, act_threshold)
        check(lib().ibh_v5_set_policy(self._h, name.encode(), ctypes.byref(p)), "ibh_v5_set_policy")

    def matmul(self, name: str, x, out) -> None:
        """ib_pq_session_matmul on device tensors x [N] -> out [M]."""
        import torch
        check(lib().ibh_v5_session_matmul(self._h, name.encode(), ctypes.c_void_p(x.data_ptr()),
                                          ctypes.c_void_p(out.data_ptr()),
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "ibh_v5_session_matmul")

    def kv_cache(self, max_seq: int) -> KvCache:
        return KvCache(self, max_seq)

    def forward_step(self, kv: KvCache, token: int, pos: int) -> np.ndarray:
        """ib_pq_forward_step: logits [vocab] of `token` at `pos`."""
        out = np.empty(self.dims["vocab_size"], np.float32)
        check(lib().ibh_v5_forward_step(self._h, kv._h, token, pos, _ptr(out)), "ibh_v5_forward_step")
        return out

    def forward_step_to_hidden(self, kv: KvCache, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.dims["hidden_size"], np.float32)
        check(lib().ibh_v5_forward_step_to_hidden(self._h, kv._h, token, pos, _ptr(out)),
              "ibh_v5_forward_step_to_hidden")
        return out

    def generate_greedy(self, kv: KvCache, prompt, max_new: int, eos: int = -1) -> np.ndarray:
        """ib_pq_generate_greedy (src/pq_decode.c:5297-5346)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(max_new, 1), np.int32)
        n = ctypes.c_int()
        check(lib().ibh_v5_generate_greedy(self._h, kv._h, _ptr(p), len(p), max_new, eos, _ptr(out),
                                           ctypes.byref(n)), "ibh_v5_generate_greedy")
        return out[:n.value]

    def generate_sample(self, kv: KvCache, prompt, max_new: int, temperature: float = 1.0, top_k: int = 40,
                        top_p: float = 0.9, seed: int = 0, eos: int = -1) -> np.ndarray:
        """ib_pq_generate_sample (src/pq_decode.c:5480-5561)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(max_new, 1), np.int32)
        n = ctypes.c_int()
        sp = PqSampleParams(temperature, top_k, top_p, seed)
        check(lib().ibh_v5_generate_sample(self._h, kv._h, _ptr(p), len(p), max_new, eos, ctypes.byref(sp),
                                           _ptr(out), ctypes.byref(n)), "ibh_v5_generate_sample")
        return out[:n.value]
