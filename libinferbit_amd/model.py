"""Device-resident decode of an IBF v1 model: twins of the reference's public
model API (include/inferbit.h: inferbit_load, inferbit_forward,
inferbit_generate at temperature 0, inferbit_kv_length / _clear / _truncate).
Host numpy arrays in and out; errors raise IbhError."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import SampleParams, check, lib

DIM_NAMES = ("num_layers", "hidden_size", "num_heads", "num_kv_heads", "head_dim", "intermediate_size",
             "vocab_size", "max_context_length", "kv_bits", "capacity", "eos_token_id", "positions", "exact")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class Model:
    def __init__(self, path: str, context_length: int = 0):
        """inferbit_load (src/ibf_loader.c:300-546) with the weight region uploaded to HBM."""
        h = ctypes.c_void_p()
        check(lib().ibh_model_load(path.encode(), context_length, ctypes.byref(h)), "ibh_model_load")
        self._h = h
        d = np.zeros(13, np.int32)
        check(lib().ibh_model_dims(self._h, _ptr(d)), "ibh_model_dims")
        self.dims = dict(zip(DIM_NAMES, (int(v) for v in d)))

    def close(self) -> None:
        if self._h:
            lib().ibh_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, tokens) -> np.ndarray:
        """inferbit_forward (src/generate.c:225-241): logits of the last token."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.dims["vocab_size"], np.float32)
        check(lib().ibh_model_forward(self._h, _ptr(t), len(t), _ptr(out), len(out)), "ibh_model_forward")
        return out

    def generate(self, tokens, max_out: int) -> np.ndarray:
        """inferbit_generate with temperature 0 (src/generate.c:243-300)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(max_out, np.int32)
        n = lib().ibh_model_generate_greedy(self._h, _ptr(t), len(t), _ptr(out), max_out)
        if n < 0:
            check(n, "ibh_model_generate_greedy")
        return out[:n]

    def generate_sampled(self, tokens, max_out: int, temperature: float = 1.0, top_k: int = 40, top_p: float = 0.9,
                         repeat_penalty: float = 1.0, seed: int = -1) -> np.ndarray:
        """inferbit_generate with sampling parameters (src/generate.c:243-302)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(max_out, np.int32)
        p = SampleParams(temperature, top_k, top_p, repeat_penalty, max_out, seed)
        n = lib().ibh_model_generate(self._h, _ptr(t), len(t), _ptr(out), max_out, ctypes.byref(p))
        if n < 0:
            check(n, "ibh_model_generate")
        return out[:n]

    def forward_positions(self, tokens) -> np.ndarray:
        """ib_forward_positions (src/forward.c:904-939): logits [n, vocab] of
        every position of `tokens` (n <= 32) in one batched pass."""
        t = np.ascontiguousarray(tokens, np.int32)
        V = self.dims["vocab_size"]
        out = np.empty((len(t), V), np.float32)
        check(lib().ibh_model_forward_positions(self._h, _ptr(t), len(t), _ptr(out), V),
              "ibh_model_forward_positions")
        return out

    def generate_lookup(self, tokens, max_out: int, ngram: int, k: int) -> np.ndarray:
        """inferbit_generate at temperature 0 with inferbit_set_prompt_lookup(ngram, k)
        (src/generate.c:305-409)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(max_out, np.int32)
        n = lib().ibh_model_generate_lookup(self._h, _ptr(t), len(t), _ptr(out), max_out, ngram, k)
        if n < 0:
            check(n, "ibh_model_generate_lookup")
        return out[:n]

    def generate_draft(self, draft: "Model", tokens, max_out: int, draft_k: int = 4) -> np.ndarray:
        """inferbit_generate at temperature 0 with inferbit_set_draft_model(draft, draft_k)
        (src/generate.c:411-520)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(max_out, np.int32)
        n = lib().ibh_model_generate_draft(self._h, draft._h, _ptr(t), len(t), _ptr(out), max_out, draft_k)
        if n < 0:
            check(n, "ibh_model_generate_draft")
        return out[:n]

    def kv_prefill(self, k: np.ndarray, v: np.ndarray) -> None:
        """Append positions to every layer's KV cache; k, v fp32 [layers][n_pos][kv_dim]."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert k.shape == v.shape and k.ndim == 3
        check(lib().ibh_model_kv_prefill(self._h, _ptr(k), _ptr(v), k.shape[1]), "ibh_model_kv_prefill")

    def set_exact(self, exact: bool) -> None:
        """Bit-identical-to-CPU kernels (default) or the fast tolerance-bound ones."""
        check(lib().ibh_model_set_exact(self._h, int(exact)), "ibh_model_set_exact")
        self.dims["exact"] = int(exact)

    def kv_length(self) -> int:
        return lib().ibh_model_kv_length(self._h)

    def kv_clear(self) -> None:
        check(lib().ibh_model_kv_clear(self._h), "ibh_model_kv_clear")

    def kv_truncate(self, n: int) -> None:
        check(lib().ibh_model_kv_truncate(self._h, n), "ibh_model_kv_truncate")

    def decode_steps(self, n: int) -> None:
        check(lib().ibh_model_decode_steps(self._h, n), "ibh_model_decode_steps")

    def synchronize(self) -> None:
        check(lib().ibh_model_synchronize(self._h), "ibh_model_synchronize")
