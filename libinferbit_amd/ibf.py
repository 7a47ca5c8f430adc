"""IBF v1 files: packed-weight producers and a synthetic-model writer.

The file layout is the one src/ibf_loader.c:1-12 reads and src/convert.c:718-842
writes: a 32-byte preamble ("INFERBIT", version 1, JSON header size, flags,
12 reserved bytes), the UTF-8 JSON header, then the weight region at the next
64-byte boundary.  Tensor offsets in the JSON are relative to that region.
Packed tensors are per-row quantized with the quantize.c rules
(``ibh_quantize_rows``), norms are fp16.

``write_synthetic`` builds random-init decoders of a given shape (there are
no checkpoints offline): weights N(0, std) from the library's counter-based
generator, seeded per tensor from (seed, tensor name), so a model is
reproducible from its config alone.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

from ._lib import check, lib

ALIGN = 64

# Decoder shapes of the benchmark configurations.  Bits per tensor follow the
# reference converter's defaults (attention q/k/v, embeddings and LM head at
# the sensitive 8 bits; o_proj and the MLP at 4 bits).
TINYLLAMA = dict(name="tinyllama-1.1b-shape", num_layers=22, hidden_size=2048, num_heads=32, num_kv_heads=4,
                 head_dim=64, intermediate_size=5632, vocab_size=32000, max_context_length=2048,
                 rope_theta=10000.0, norm_epsilon=1e-5, kv_bits=32)
MISTRAL = dict(name="mistral-7b-shape", num_layers=32, hidden_size=4096, num_heads=32, num_kv_heads=8,
               head_dim=128, intermediate_size=14336, vocab_size=32000, max_context_length=4352,
               rope_theta=10000.0, norm_epsilon=1e-5, kv_bits=8)
DEFAULT_BITS = dict(q_proj=8, k_proj=8, v_proj=8, o_proj=4, gate_proj=4, up_proj=4, down_proj=4,
                    token_embedding=8, head=8)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def fill_normal(n: int, seed: int, std: float = 1.0, first: int = 0, out: np.ndarray | None = None) -> np.ndarray:
    out = np.empty(n, np.float32) if out is None else out[:n]
    check(lib().ibh_fill_normal(_ptr(out), n, seed & (2**64 - 1), first, std), "ibh_fill_normal")
    return out


def quantize(bits: int, w: np.ndarray):
    """ib_quantize_int{8,4,2} (src/quantize.c:75-239): (packed bytes [rows][row_bytes], fp16-bit scales)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    rb = lib().ibh_packed_row_bytes(bits, cols)
    packed = np.empty((rows, rb), np.uint8)
    scales = np.empty(rows, np.uint16)
    check(lib().ibh_quantize_rows(bits, _ptr(w), rows, cols, _ptr(packed), _ptr(scales)), "ibh_quantize_rows")
    return packed, scales


def tensor_seed(seed: int, name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & (2**64 - 1)
    return (h ^ (seed * 0x9E3779B97F4A7C15)) & (2**64 - 1)


def _align(x: int) -> int:
    return (x + ALIGN - 1) // ALIGN * ALIGN


def write_synthetic(path: str, cfg: dict, seed: int = 0, std: float = 0.02, bits: dict | None = None) -> dict:
    """Write a random-init decoder of shape `cfg` (keys as TINYLLAMA) to `path`.
    Returns the JSON header written."""
    bits = dict(DEFAULT_BITS, **(bits or {}))
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    KV = cfg["num_kv_heads"] * cfg["head_dim"]
    plan = []   # (name, key, rows, cols, bits or 16 for a norm)
    for layer in range(cfg["num_layers"]):
        p = f"layers.{layer}."
        for key, r, c in (("q_proj", H, H), ("k_proj", KV, H), ("v_proj", KV, H), ("o_proj", H, H),
                          ("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)):
            plan.append((p + key, key, r, c, bits[key]))
        plan.append((p + "input_norm", "input_norm", H, 1, 16))
        plan.append((p + "post_attn_norm", "post_attn_norm", H, 1, 16))
    plan.append(("token_embedding", "token_embedding", V, H, bits["token_embedding"]))
    plan.append(("output.norm", "norm", H, 1, 16))
    plan.append(("output.head", "head", V, H, bits["head"]))

    metas, off = {}, 0
    for name, key, r, c, b in plan:
        wsize = r * 2 if b == 16 else r * c * b // 8
        m = {"offset": off, "size": wsize, "shape": [r, c] if c > 1 else [r], "bits": b,
             "scale_offset": 0, "scale_size": 0, "has_bias": False}
        off = _align(off + wsize)
        if b != 16:
            m["scale_offset"], m["scale_size"] = off, r * 2
            off = _align(off + r * 2)
        metas[name] = m
    total = off

    layers = []
    for layer in range(cfg["num_layers"]):
        p = f"layers.{layer}."
        w = {k: metas[p + k] for k in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                       "down_proj", "input_norm", "post_attn_norm")}
        layers.append({"index": layer, "weights": w, "sparsity_mask": {"offset": 0, "size": 0}})
    header = {
        "version": 1,
        "model": {"architecture": "llama", "name": cfg.get("name", "synthetic")},
        "architecture": {k: cfg[k] for k in ("num_layers", "hidden_size", "num_heads", "num_kv_heads", "head_dim",
                                             "intermediate_size", "vocab_size", "max_context_length",
                                             "rope_theta", "norm_epsilon")}
        | {"norm_type": "rmsnorm", "activation": "silu", "tie_word_embeddings": False,
           "bos_token_id": 1, "eos_token_id": 2},
        "quantization": {"default_bits": 4, "sensitive_bits": 8, "sparsity": 0.0, "block_size": 8},
        "kv_cache": {"bits": cfg["kv_bits"]},
        "data": {"weight_data_size": total, "alignment": ALIGN},
        "layers": layers,
        "embeddings": {"token_embedding": metas["token_embedding"]},
        "output": {"norm": metas["output.norm"], "head": metas["output.head"]},
    }
    js = json.dumps(header, separators=(",", ":")).encode()
    base = _align(32 + len(js))
    scratch = np.empty(max(r * c for _, _, r, c, b in plan if b != 16), np.float32)   # reused: no page faults
    with open(path, "wb") as f:
        f.write(b"INFERBIT" + np.array([1, len(js), 0], np.uint32).tobytes() + bytes(12))
        f.write(js)
        f.truncate(base + total)
        for name, key, r, c, b in plan:
            m = metas[name]
            f.seek(base + m["offset"])
            if b == 16:
                f.write(np.ones(r, np.float16).tobytes())
                continue
            packed, scales = quantize(b, fill_normal(r * c, tensor_seed(seed, name), std, out=scratch).reshape(r, c))
            f.write(packed.tobytes())
            f.seek(base + m["scale_offset"])
            f.write(scales.tobytes())
    return header
