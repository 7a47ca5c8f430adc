"""Writer of IBF v5 files (the PQ-session format, src/pq_decode.c:257-259,
391-555, 685-849): a 32-byte preamble ("INFERBIT", uint32 version 5,
uint32 JSON size), the JSON header {weight_data_start, tensors, raw_tensors,
config}, then the data blocks at weight_data_start + offset.

`tensors` are product-quantised matrices (format pq2d_v1_l1 / pq2d_v1_l1_l2,
blocks codebook_l1_l/_r, indices_l1_l/_r, row_scale, level-2 and outlier
blocks); `raw_tensors` are typed arrays, among them the INT4 group-scale
pairs <base>__i4_q / __i4_s (+ __act_scale, __i4_outl_idx / _val), fp16
matrices <base>__fp16w, norm weights and the token embedding.

`write_synthetic_v5` builds a seeded random decoder of a given shape with a
chosen backend per projection (no reference counterpart: the reference's
converter needs a checkpoint)."""
from __future__ import annotations

import json

import numpy as np

MAGIC = b"INFERBIT"
VERSION = 5
PREAMBLE = 32


def _f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


class V5Writer:
    def __init__(self, config: dict):
        self.config = dict(config)
        self.tensors, self.raw = {}, {}
        self.blobs, self.size = [], 0

    def _blob(self, arr) -> dict:
        b = np.ascontiguousarray(arr).tobytes()
        pad = (-self.size) % 64
        if pad:
            self.blobs.append(b"\0" * pad)
            self.size += pad
        off = self.size
        self.blobs.append(b)
        self.size += len(b)
        return {"offset": off, "size": len(b)}

    def raw_tensor(self, name: str, arr: np.ndarray, dtype: str):
        d = self._blob(arr)
        d.update(dtype=dtype, shape=list(np.asarray(arr).shape))
        self.raw[name] = d

    def pq_tensor(self, name: str, t: dict, rotate: bool = False, l2_packed_bits: int = 0):
        """t: the oracle's PQ dict (M, N, G, K, n_levels, K_l2, n_outlier,
        cb1l, cb1r, i1l, i1r, row_scale[, cb2l, cb2r, i2l, i2r, ocols, oside, oscale]).
        Two-byte level-2 indices (l2_idx_bytes 2), or a K_l2 outside {16, 64,
        K} (which pq2d_v1_l1_l2 refuses, src/pq_decode.c:425-426), make a
        pyramid tensor (pq2d_v1_pyramid).  l2_packed_bits > 0 stores those indices
        bit-packed LSB-first per row, ceil(C * bits / 8) bytes a row, which
        the loader unpacks to uint16 (src/pq_decode.c:431-446, 504-528)."""
        K2 = int(t.get("K_l2") or t["K"])
        pyramid = t["n_levels"] == 2 and (int(t.get("l2_idx_bytes", 1)) == 2 or K2 not in (16, 64, int(t["K"])))
        fmt = "pq2d_v1_l1" if t["n_levels"] == 1 else ("pq2d_v1_pyramid" if pyramid else "pq2d_v1_l1_l2")
        m = {"format": fmt, "shape": [int(t["M"]), int(t["N"])], "G": int(t["G"]), "K": int(t["K"]),
             "n_levels": int(t["n_levels"])}
        if rotate:
            m["rotate"] = True
        if l2_packed_bits:
            assert pyramid, "bit-packed level-2 indices are a pyramid-format option"
            m["l2_packed_bits"] = int(l2_packed_bits)
        if t.get("K_l2"):
            m["K_l2"] = int(t["K_l2"])
        if t.get("n_outlier"):
            m["outlier"] = {"n_cols": int(t["n_outlier"])}
        blocks = [("codebook_l1_l", "cb1l"), ("codebook_l1_r", "cb1r"), ("indices_l1_l", "i1l"),
                  ("indices_l1_r", "i1r"), ("row_scale", "row_scale")]
        if t["n_levels"] == 2:
            blocks += [("codebook_l2_l", "cb2l"), ("codebook_l2_r", "cb2r"), ("indices_l2_l", "i2l"),
                       ("indices_l2_r", "i2r")]
        if t.get("n_outlier"):
            blocks += [("outlier_cols", "ocols"), ("outlier_sidecar", "oside"), ("outlier_scale", "oscale")]
        for key, k in blocks:
            a = t[k]
            if l2_packed_bits and k in ("i2l", "i2r"):
                a = _pack_bits(np.ascontiguousarray(a).view(np.uint16).reshape(int(t["M"]), int(t["C"])),
                               l2_packed_bits)
            m[key] = self._blob(a)
        self.tensors[name] = m

    def write(self, path: str):
        hdr = {"weight_data_start": 0, "tensors": self.tensors, "raw_tensors": self.raw, "config": self.config}
        js = json.dumps(hdr, separators=(",", ":")).encode()
        reserve = len(js) + 64
        start = (PREAMBLE + reserve + 4095) // 4096 * 4096
        hdr["weight_data_start"] = start
        js = json.dumps(hdr, separators=(",", ":")).encode()
        assert len(js) <= reserve
        js = js + b" " * (reserve - len(js))
        pre = MAGIC + np.array([VERSION, reserve], np.uint32).tobytes()
        pre = pre + b"\0" * (PREAMBLE - len(pre))
        with open(path, "wb") as f:
            f.write(pre)
            f.write(js)
            f.write(b"\0" * (start - PREAMBLE - reserve))
            for b in self.blobs:
                f.write(b)


def _pack_bits(v: np.ndarray, bits: int) -> np.ndarray:
    """Rows of values < 2^bits packed LSB-first, each row ceil(C*bits/8) bytes."""
    M, C = v.shape
    per = (C * bits + 7) // 8
    bitsarr = ((v[:, :, None].astype(np.uint32) >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.uint8)
    flat = bitsarr.reshape(M, C * bits)
    pad = np.zeros((M, per * 8), np.uint8)
    pad[:, :C * bits] = flat
    return np.packbits(pad.reshape(M, per, 8), axis=2, bitorder="little").reshape(M, per)


def _pq(rng, M, N, G=16, K=256, levels=1, K2=0, n_outlier=0, cb_std=0.05):
    """Random PQ tensor dict (the oracle's field names).  K2 == 16 packs the
    level-2 indices two per byte, low nibble first (pq_l2_idx_at)."""
    C = (N - n_outlier) // G
    assert C * G == N - n_outlier
    h = G // 2
    t = dict(M=M, N=N, G=G, K=K, n_levels=levels, n_outlier=n_outlier, C=C, K_l2=K2 if levels == 2 else 0)
    t["cb1l"] = _f16(rng.standard_normal((K, h)) * cb_std)
    t["cb1r"] = _f16(rng.standard_normal((K, h)) * cb_std)
    t["i1l"] = rng.integers(0, K, (M, C), dtype=np.uint8)
    t["i1r"] = rng.integers(0, K, (M, C), dtype=np.uint8)
    t["row_scale"] = _f16(1 + 0.1 * rng.standard_normal(M))
    if levels == 2:
        t["cb2l"] = _f16(rng.standard_normal((K2, h)) * cb_std * 0.25)
        t["cb2r"] = _f16(rng.standard_normal((K2, h)) * cb_std * 0.25)
        for k in ("i2l", "i2r"):
            i2 = rng.integers(0, K2, (M, C), dtype=np.uint8)
            if K2 == 16:
                pad = np.zeros((M, C + (C & 1)), np.uint8)
                pad[:, :C] = i2
                i2 = (pad[:, 0::2] | (pad[:, 1::2] << 4)).astype(np.uint8)
            t[k] = i2
    if n_outlier:
        t["ocols"] = np.sort(rng.choice(N, n_outlier, replace=False)).astype(np.int32)
        t["oside"] = rng.integers(-127, 128, (M, n_outlier), dtype=np.int8)
        t["oscale"] = _f16(rng.uniform(0.5, 1.5, n_outlier) * cb_std / 64)
    return t


def write_synthetic_v5(path: str, cfg: dict, seed: int = 0, backend=None, awq: bool = False, outliers: int = 0,
                       head: str = "pq", levels: int = 1, k2: int = 256, pq_outliers: int = 0,
                       pq_act_scale: bool = False, fused: bool = False, embed: str = "f16", i4_group: int = 0):
    """A random decoder in IBF v5.  cfg: num_layers, hidden_size, num_heads,
    num_kv_heads, head_dim, intermediate_size, vocab_size (+ rms_norm_eps,
    rope_theta).  backend maps projection names (q_proj, k_proj, v_proj,
    o_proj, gate_proj, up_proj, down_proj) to "int4g" (group 128 scales,
    optional AWQ inv_act and fp16 outliers), "pq" or "fp16"; default int4g.
    The LM head is a PQ tensor ("pq", the greedy path's top-K head needs
    one) or int4g / fp16.  PQ tensors: `levels` 1 or 2 (K_l2 = k2),
    `pq_outliers` outlier columns, `pq_act_scale` an <name>__act_scale
    vector.  `fused` writes L{i}_qkv_proj / L{i}_gateup_proj instead of the
    separate projections; `embed` is "f16", "f32" or "pq"; `i4_group` the
    INT4 scale group (0: 128 when it divides N, else 32)."""
    rng = np.random.default_rng(seed)
    backend = dict(backend or {})
    H, L = cfg["hidden_size"], cfg["num_layers"]
    nh, nkv = cfg["num_heads"], cfg["num_kv_heads"]
    hd = cfg.get("head_dim", H // nh)
    I, V = cfg["intermediate_size"], cfg["vocab_size"]
    config = dict(num_layers=L, hidden_size=H, num_heads=nh, num_kv_heads=nkv, head_dim=hd, intermediate_size=I,
                  vocab_size=V, rms_norm_eps=cfg.get("rms_norm_eps", 1e-5), rope_theta=cfg.get("rope_theta", 10000.0))
    w = V5Writer(config)
    if embed == "pq":
        w.pq_tensor("tok_embed", _pq(rng, V, H, levels=levels, K2=k2, n_outlier=pq_outliers, cb_std=1.0))
    elif embed == "f32":
        w.raw_tensor("tok_embed", rng.standard_normal((V, H)).astype(np.float32), "float32")
    else:
        w.raw_tensor("tok_embed", _f16(rng.standard_normal((V, H))), "float16")

    def matrix(name, M, N, kind):
        if kind == "pq":
            w.pq_tensor(name, _pq(rng, M, N, levels=levels, K2=k2 if levels == 2 else 0, n_outlier=pq_outliers))
            if pq_act_scale:
                w.raw_tensor(name + "__act_scale", np.exp(rng.normal(0, 0.3, N)).astype(np.float32), "float32")
        elif kind == "fp16":
            w.raw_tensor(name + "__fp16w", _f16(rng.standard_normal((M, N)) / np.sqrt(N)), "float16")
        else:
            G = i4_group or (128 if N % 128 == 0 else 32)
            w.raw_tensor(name + "__i4_q", rng.integers(0, 256, (M, N // 2), dtype=np.uint8), "uint8")
            w.raw_tensor(name + "__i4_s", _f16(rng.uniform(0.5, 1.5, (M, N // G)) / (4 * np.sqrt(N))), "float16")
            if awq:
                w.raw_tensor(name + "__act_scale", np.exp(rng.normal(0, 0.3, N)).astype(np.float32), "float32")
            if outliers:
                idx = np.stack([rng.choice(N, outliers, replace=False) for _ in range(M)]).astype(np.uint16)
                w.raw_tensor(name + "__i4_outl_idx", idx, "uint16")
                w.raw_tensor(name + "__i4_outl_val", _f16(rng.normal(0, 0.05, (M, outliers))), "float16")

    shapes = {"q_proj": (nh * hd, H), "k_proj": (nkv * hd, H), "v_proj": (nkv * hd, H), "o_proj": (H, nh * hd),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    for l in range(L):
        w.raw_tensor(f"L{l}_input_norm", (1 + 0.1 * rng.standard_normal(H)).astype(np.float32), "float32")
        w.raw_tensor(f"L{l}_post_attn_norm", (1 + 0.1 * rng.standard_normal(H)).astype(np.float32), "float32")
        for p, (M, N) in shapes.items():
            if fused and p in ("q_proj", "k_proj", "v_proj", "gate_proj", "up_proj"):
                continue
            matrix(f"L{l}_{p}", M, N, backend.get(p, "int4g"))
        if fused:
            matrix(f"L{l}_qkv_proj", nh * hd + 2 * nkv * hd, H, backend.get("qkv_proj", "int4g"))
            matrix(f"L{l}_gateup_proj", 2 * I, H, backend.get("gateup_proj", "int4g"))
    w.raw_tensor("final_norm", (1 + 0.1 * rng.standard_normal(H)).astype(np.float32), "float32")
    matrix("lm_head", V, H, head)
    w.write(path)
    return config
