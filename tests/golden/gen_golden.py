"""Writes the golden vectors in this directory from the REFERENCE library.

The reference library is compiled from the reference sources by
``make -C oracle ref`` (oracle/_ref/libinferbit_ref.so); this script calls its
exported entry points through ctypes (oracle/refbind.py) on seeded inputs and
stores inputs and outputs as .npz fixtures (data only).  Run from the repo
root:  python tests/golden/gen_golden.py

Contents (every array is what the reference produced, except the inputs):
  quant.npz    ib_quantize_int{8,4,2} on fp32 W            (src/quantize.c)
  matvec.npz   ib_kern.matmul_int{8,4,2}, x86 (avx2) and scalar tables
  w4a8.npz     ib_quantize_input_int8_g128 + matmul_w4a8 (avx2/scalar)
  batch.npz    matmul_int8_batch / matmul_w4a8_batch with M_stride > M
  pq.npz       ib_pq_matmul_fp32 / ib_pq_reconstruct_fp32 on small tensors
  pqs.npz      ib_pq_lut_cache_create + ib_pq_matmul_fp32_streaming_cached
               (the PQ session's default variant) on the pq.npz cases and on
               G = 4 / 32 cases
  pqv.npz      the PQ session's policy variants (l1_only, l2skip_cached,
               streaming_sparse, streaming_int8_cached) on the pq.npz cases and
               on pyramid-format tensors
  pqtopk.npz   ib_pq_lm_head_topk (l1-only logits, top-K, subset refinement)
  pqq8.npz     ib_pq_matmul_fp32_q8lut (int8-quantised tables)
  int4g.npz    ib_pq_session_matmul on IBF v5 INT4 group-scale tensors
               (oracle/_ref/libref_int4g.so): y without, ys with the
               IB_ACT_SPARSE_REL skip mask (set in a child process, since the
               reference reads it once per process)

  python tests/golden/gen_golden.py int4g   writes int4g.npz only;
  python tests/golden/gen_golden.py pqs     writes pqs.npz only;
  python tests/golden/gen_golden.py pqv     writes pqv.npz only;
  python tests/golden/gen_golden.py pqtopk  writes pqtopk.npz only;
  python tests/golden/gen_golden.py pqq8    writes pqq8.npz only.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import refbind as R  # noqa: E402

SHAPES = [(64, 256), (37, 200), (16, 4100), (8, 4096)]


def f16bits(a):
    return np.asarray(a, np.float16).view(np.uint16)


def fp16_to_f32(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def gen_quant_matvec(out):
    rng = np.random.default_rng(20240601)
    q, mv, w4 = {}, {}, {}
    avx, sca = R.kernels(R.IB_SIMD_AVX2), R.kernels(R.IB_SIMD_NONE)
    for (M, N) in SHAPES:
        tag = f"{M}x{N}"
        W = (rng.standard_normal((M, N)) * 0.02).astype(np.float32)
        W[0, :] = 0.0                                  # all-zero row: scale floor
        W[1, 5] = 3.0                                  # outlier row
        x = rng.standard_normal(N).astype(np.float32)
        q[f"W_{tag}"] = W
        mv[f"x_{tag}"] = x
        for bits in (8, 4, 2):
            if bits == 2 and N % 4:
                continue
            w, s = R.quantize(bits, W)
            q[f"w{bits}_{tag}"], q[f"s{bits}_{tag}"] = w, s
            sc = fp16_to_f32(s)
            mv[f"y{bits}_avx2_{tag}"] = R.matmul(avx, bits, w, sc, x)
            mv[f"y{bits}_scalar_{tag}"] = R.matmul(sca, bits, w, sc, x)
        qx, sa = R.quantize_act(x)
        w4[f"qx_{tag}"], w4[f"sa_{tag}"] = qx, sa
        wq, s = q[f"w4_{tag}"], q[f"s4_{tag}"]
        w4[f"y_avx2_{tag}"] = R.matmul_w4a8(avx, wq, fp16_to_f32(s), qx, sa)
        w4[f"y_scalar_{tag}"] = R.matmul_w4a8(sca, wq, fp16_to_f32(s), qx, sa)
    # activation-quantizer edge cases: zero group, tiny group, ties at .5
    xe = np.zeros(300, np.float32)
    xe[128:256] = 1e-12
    xe[256:] = np.linspace(-1, 1, 44, dtype=np.float32)
    xe[260] = 127.0 / 254.0
    qx, sa = R.quantize_act(xe)
    w4["x_edge"], w4["qx_edge"], w4["sa_edge"] = xe, qx, sa
    np.savez_compressed(os.path.join(out, "quant.npz"), **q)
    np.savez_compressed(os.path.join(out, "matvec.npz"), **mv)
    np.savez_compressed(os.path.join(out, "w4a8.npz"), **w4)


def gen_batch(out):
    rng = np.random.default_rng(7)
    tab = R.kernels(R.IB_SIMD_AVX2)
    d = {}
    for (M, N) in [(48, 256), (33, 384)]:
        W = (rng.standard_normal((M, N)) * 0.02).astype(np.float32)
        w8, s8 = R.quantize(8, W)
        w4, s4 = R.quantize(4, W)
        for B in (1, 2, 5, 8):
            tag = f"{M}x{N}_b{B}"
            X = rng.standard_normal((B, N)).astype(np.float32)
            QS = [R.quantize_act(X[b]) for b in range(B)]
            QX = np.stack([a for a, _ in QS])
            SA = np.stack([b for _, b in QS])
            ms = M + 3
            d[f"X_{tag}"], d[f"QX_{tag}"], d[f"SA_{tag}"] = X, QX, SA
            d[f"y8_{tag}"] = R.matmul_int8_batch(tab, w8, fp16_to_f32(s8), X, ms)
            d[f"y4_{tag}"] = R.matmul_w4a8_batch(tab, w4, fp16_to_f32(s4), QX, SA, ms)
        d[f"w8_{M}x{N}"], d[f"s8_{M}x{N}"] = w8, s8
        d[f"w4_{M}x{N}"], d[f"s4_{M}x{N}"] = w4, s4
    np.savez_compressed(os.path.join(out, "batch.npz"), **d)


def make_pq(rng, M, Cc, G, K, nl, K2, no, l2b=1):
    N = Cc * G + no
    h = G // 2
    t = dict(M=M, N=N, G=G, K=K, n_levels=nl, n_outlier=no, C=Cc, K_l2=K2 if nl == 2 else 0, l2_idx_bytes=l2b)
    t["cb1l"] = f16bits(rng.standard_normal((K, h)) * 0.02)
    t["cb1r"] = f16bits(rng.standard_normal((K, h)) * 0.02)
    t["i1l"] = rng.integers(0, K, (M, Cc), dtype=np.uint8)
    t["i1r"] = rng.integers(0, K, (M, Cc), dtype=np.uint8)
    t["row_scale"] = f16bits(1 + 0.1 * rng.standard_normal(M))
    if nl == 2:
        t["cb2l"] = f16bits(rng.standard_normal((K2, h)) * 0.005)
        t["cb2r"] = f16bits(rng.standard_normal((K2, h)) * 0.005)
        if K2 == 16:
            st = (Cc + 1) // 2
            t["i2l"] = rng.integers(0, 256, (M, st), dtype=np.uint8)
            t["i2r"] = rng.integers(0, 256, (M, st), dtype=np.uint8)
        elif l2b == 2:
            t["i2l"] = rng.integers(0, K2, (M, Cc), dtype=np.uint16).view(np.uint8)
            t["i2r"] = rng.integers(0, K2, (M, Cc), dtype=np.uint16).view(np.uint8)
        else:
            t["i2l"] = rng.integers(0, K2, (M, Cc), dtype=np.uint8)
            t["i2r"] = rng.integers(0, K2, (M, Cc), dtype=np.uint8)
    if no:
        t["ocols"] = np.sort(rng.choice(N, no, replace=False)).astype(np.int32)
        t["oside"] = rng.integers(-127, 128, (M, no), dtype=np.int8)
        t["oscale"] = f16bits(np.abs(rng.standard_normal(no)) * 0.01 + 0.001)
    return t


PQ_CASES = {
    "l1": (64, 16, 16, 256, 1, 0, 0),
    "l2p16": (33, 20, 16, 256, 2, 16, 0),
    "l2u8": (40, 12, 16, 64, 2, 256, 0),
    "l2u16": (40, 12, 8, 256, 2, 512, 0, 2),
    "out8": (48, 16, 16, 256, 1, 0, 8),
    "out40": (48, 16, 16, 256, 1, 0, 40),
}


def gen_pq(out):
    rng = np.random.default_rng(99)
    d = {}
    for name, args in PQ_CASES.items():
        t = make_pq(rng, *args)
        x = rng.standard_normal(t["N"]).astype(np.float32)
        xs = x.copy()
        xs[: t["N"] // 2] *= 1e-4                    # chunk-skipping case
        for k, v in t.items():
            d[f"{name}.{k}"] = np.asarray(v)
        d[f"{name}.x"], d[f"{name}.xs"] = x, xs
        d[f"{name}.y"] = R.pq_matmul(t, x)
        d[f"{name}.ys"] = R.pq_matmul(t, xs)
        d[f"{name}.W"] = R.pq_reconstruct(t)
    np.savez_compressed(os.path.join(out, "pq.npz"), **d)


# cases of pqs.npz beyond pq.npz's: (M, C, G, K, levels, K_l2, outliers)
PQS_EXTRA = {
    "g4": (40, 24, 4, 256, 1, 0, 0),
    "g32": (36, 10, 32, 256, 2, 256, 5),
    "g4l2": (20, 16, 4, 64, 2, 16, 3),
}


def gen_pqs(out):
    d = {}
    pq = np.load(os.path.join(out, "pq.npz"))
    for name in PQ_CASES:
        t = {k[len(name) + 1:]: (int(pq[k]) if pq[k].ndim == 0 else pq[k]) for k in pq.files
             if k.startswith(name + ".")}
        d[f"{name}.y"] = R.pq_matmul_streaming(t, t["x"])
        d[f"{name}.ys"] = R.pq_matmul_streaming(t, t["xs"])
    rng = np.random.default_rng(1234)
    for name, args in PQS_EXTRA.items():
        t = make_pq(rng, *args)
        x = rng.standard_normal(t["N"]).astype(np.float32)
        for k, v in t.items():
            d[f"{name}.{k}"] = np.asarray(v)
        d[f"{name}.x"] = x
        d[f"{name}.y"] = R.pq_matmul_streaming(t, x)
    np.savez_compressed(os.path.join(out, "pqs.npz"), **d)


# (variant, skip_threshold, act_threshold) per policy case of pqv.npz
PQV_POLICIES = {"l1only": (1, 0.0, 0.0), "l2skip05": (2, 0.5, 0.0), "l2skip5": (2, 5.0, 0.0),
                "sparse": (3, 0.0, 1e-2), "int8": (4, 0.0, 0.0)}
# pyramid tensors: (M, C, G, K, levels, K_l2 = K * K_inner, outliers)
PQV_PYRAMID = {"pyr16": (50, 12, 16, 16, 2, 256, 3), "pyr8": (40, 10, 8, 8, 2, 64, 0)}


def gen_pqv(out):
    d = {}
    pq = np.load(os.path.join(out, "pq.npz"))
    cases = {}
    for name in PQ_CASES:
        cases[name] = {k[len(name) + 1:]: (int(pq[k]) if pq[k].ndim == 0 else pq[k]) for k in pq.files
                       if k.startswith(name + ".")}
    rng = np.random.default_rng(777)
    for name, args in PQV_PYRAMID.items():
        t = make_pq(rng, *args)
        t["format"] = 4
        t["x"] = rng.standard_normal(t["N"]).astype(np.float32)
        t["xs"] = t["x"].copy()
        t["xs"][: t["N"] // 2] *= 1e-3
        for k, v in t.items():
            d[f"{name}.{k}"] = np.asarray(v)
        cases[name] = t
    for name, t in cases.items():
        for pol, (v, st, at) in PQV_POLICIES.items():
            d[f"{name}.{pol}.y"] = R.pq_matmul_variant(t, t["x"], v, st, at)
            d[f"{name}.{pol}.ys"] = R.pq_matmul_variant(t, t["xs"], v, st, at)
    np.savez_compressed(os.path.join(out, "pqv.npz"), **d)


# top-K head cases: (M, C, G, K, levels, K_l2, outliers), K_top values
PQTOPK = {"head1": ((2000, 24, 16, 256, 1, 0, 0), (1, 8, 40)),
          "head2": ((1500, 16, 16, 64, 2, 256, 6), (3, 64)),
          "small": ((12, 8, 8, 16, 2, 16, 0), (12,))}


def gen_pqtopk(out):
    d = {}
    rng = np.random.default_rng(4242)
    for name, (args, ks) in PQTOPK.items():
        t = make_pq(rng, *args)
        t["x"] = rng.standard_normal(t["N"]).astype(np.float32)
        for k, v in t.items():
            d[f"{name}.{k}"] = np.asarray(v)
        for kt in ks:
            lg, ids = R.pq_lm_head_topk(t, t["x"], kt)
            d[f"{name}.k{kt}.logits"], d[f"{name}.k{kt}.ids"] = lg, ids
    np.savez_compressed(os.path.join(out, "pqtopk.npz"), **d)


# name: (M, N, G, AWQ inv_act, outliers per row)
INT4G_CASES = {
    "g32": (64, 256, 32, 0, 0),
    "g128awq": (100, 512, 128, 1, 3),
    "g64awq": (33, 384, 64, 1, 0),
    "g128out": (17, 2048, 128, 0, 5),
    "g96": (5, 96, 96, 1, 2),
    "g2": (8, 40, 2, 0, 1),
    "g128big": (48, 4096, 128, 1, 4),
    "g256": (20, 1536, 256, 1, 2),
}
INT4G_SKIP_REL = 1e-2


def make_int4g(rng, M, N, G, awq, K):
    t = dict(q=rng.integers(0, 256, (M, N // 2), dtype=np.uint8),
             s=f16bits(rng.uniform(0.002, 0.05, (M, N // G))))
    if awq:
        t["inv_act"] = np.exp(rng.normal(0, 0.5, N)).astype(np.float32)
    if K:
        t["outl_idx"] = np.stack([rng.choice(N, K, replace=False) for _ in range(M)]).astype(np.uint16)
        t["outl_val"] = f16bits(rng.normal(0, 1, (M, K)))
    return t


def int4g_inputs():
    rng = np.random.default_rng(4104)
    d = {}
    for name, (M, N, G, awq, K) in INT4G_CASES.items():
        t = make_int4g(rng, M, N, G, awq, K)
        x = rng.standard_normal(N).astype(np.float32)
        small = np.repeat(rng.random(N // G) < 0.3, G)         # whole groups near zero
        x[small] *= 3e-3
        for k, v in t.items():
            d[f"{name}.{k}"] = v
        d[f"{name}.x"] = x
    return d


def int4g_outputs(d):
    out = {}
    for name in INT4G_CASES:
        t = {k[len(name) + 1:]: d[k] for k in d if k.startswith(name + ".")}
        out[f"{name}.y"] = R.int4g_matmul(t, t["x"])
    return out


def gen_int4g(out):
    import subprocess
    import tempfile
    d = int4g_inputs()
    d.update(int4g_outputs(d))
    with tempfile.TemporaryDirectory() as tmp:
        f = os.path.join(tmp, "skip.npz")
        subprocess.run([sys.executable, os.path.abspath(__file__), "int4g-skip-child", f], check=True,
                       env=dict(os.environ, IB_ACT_SPARSE_REL=repr(INT4G_SKIP_REL)))
        ys = np.load(f)
        for name in INT4G_CASES:
            d[f"{name}.ys"] = ys[f"{name}.y"]
    d["skip_rel"] = np.float32(INT4G_SKIP_REL)
    np.savez_compressed(os.path.join(out, "int4g.npz"), **d)


# q8lut cases: (M, C, G, K, levels, K_l2, outliers); level 2 needs K_l2 == K
PQQ8 = {"l1": (64, 16, 16, 256, 1, 0, 0), "l2": (40, 12, 16, 256, 2, 256, 0),
        "out8": (48, 16, 16, 256, 1, 0, 8), "out40l2": (30, 10, 16, 64, 2, 64, 40),
        "g4": (40, 24, 4, 256, 1, 0, 0), "g32": (36, 10, 32, 256, 1, 0, 5), "g6": (20, 9, 6, 32, 2, 32, 0)}


def gen_pqq8(out):
    d = {}
    rng = np.random.default_rng(8080)
    for name, args in PQQ8.items():
        t = make_pq(rng, *args)
        x = rng.standard_normal(t["N"]).astype(np.float32)
        x[rng.integers(0, t["N"], 3)] *= 20.0
        for k, v in t.items():
            d[f"{name}.{k}"] = np.asarray(v)
        d[f"{name}.x"] = x
        d[f"{name}.y"] = R.pq_matmul_q8lut(t, x)
    np.savez_compressed(os.path.join(out, "pqq8.npz"), **d)


# decode-layer helpers: the reference's own table entries (x86 AVX2 table,
# src/kernels/avx2.c:153-273), odd lengths, several positions and thetas
LAYER_N = [1, 7, 64, 2051]
LAYER_ROPE = [(64, 0, 10000.0), (64, 5, 10000.0), (128, 4095, 10000.0), (128, 77, 1000000.0), (6, 3, 500.0)]


def gen_layer(out):
    tab = R.kernels(R.IB_SIMD_AVX2)
    rng = np.random.default_rng(4242)
    d = {}
    for n in LAYER_N:
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        o = np.zeros(n, np.float32)
        R.call_f32(tab, "rmsnorm", R._p(o), R._p(x), R._p(w), np.float32(1e-5), n)
        d[f"rms{n}.x"], d[f"rms{n}.w"], d[f"rms{n}.y"] = x, w, o
        g = (rng.standard_normal(n) * 4).astype(np.float32)
        u = rng.standard_normal(n).astype(np.float32)
        o2 = np.zeros(n, np.float32)
        R.call_f32(tab, "silu_mul", R._p(o2), R._p(g), R._p(u), n)
        d[f"silu{n}.g"], d[f"silu{n}.u"], d[f"silu{n}.y"] = g, u, o2
    for i, (hd, pos, theta) in enumerate(LAYER_ROPE):
        q = rng.standard_normal(hd).astype(np.float32)
        k = rng.standard_normal(hd).astype(np.float32)
        d[f"rope{i}.q"], d[f"rope{i}.k"] = q.copy(), k.copy()
        R.call_f32(tab, "rope", R._p(q), R._p(k), hd, pos, np.float32(theta))
        d[f"rope{i}.qo"], d[f"rope{i}.ko"] = q, k
        d[f"rope{i}.arg"] = np.array([hd, pos, theta], np.float64)
    np.savez_compressed(os.path.join(out, "layer.npz"), **d)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "layer":
        gen_layer(HERE)
        return
    if len(sys.argv) > 2 and sys.argv[1] == "int4g-skip-child":
        np.savez(sys.argv[2], **int4g_outputs(int4g_inputs()))
        return
    if len(sys.argv) > 1 and sys.argv[1] == "int4g":
        gen_int4g(HERE)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "pqs":
        gen_pqs(HERE)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "pqv":
        gen_pqv(HERE)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "pqtopk":
        gen_pqtopk(HERE)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "pqq8":
        gen_pqq8(HERE)
        return
    if not R.available():
        sys.exit("oracle/_ref/libinferbit_ref.so missing: run `make -C oracle ref` first")
    gen_quant_matvec(HERE)
    gen_batch(HERE)
    gen_pq(HERE)
    gen_pqs(HERE)
    gen_pqv(HERE)
    gen_pqtopk(HERE)
    gen_pqq8(HERE)
    gen_int4g(HERE)
    gen_layer(HERE)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
