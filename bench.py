#!/usr/bin/env python3
"""Benchmark of the headline workload on one MI355X.

Workload: INT4 matvec at the Mistral-7B MLP shape,
W 14336x4096 packed int4 with per-row fp16 scales (quantize.c semantics),
x fp32 N(0,1), batch 1 -- ib_parallel_matmul(bits=4) / ib_kern.matmul_int4.
One step = one GEMV over one weight copy.  16 distinct weight copies
(~470 MB) are used round-robin so the 256 MB Infinity Cache cannot serve
repeated reads; inputs are resident in HBM before timing starts.

value = algorithmic bytes per call / average kernel time, in GB/s
(W + 2M fp16 scales + 4N x + 4M y = 29,462,528 B per call).
Extra lines in the same JSON: the W4A8 decode form of the same tensor, the
other matvec configs, the batch sweep, the roofline object, and the CPU
baseline (the reference library compiled from source, timed on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
COPIES = 16


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--quick", action="store_true", help="headline only (for profiling runs)")
    p.add_argument("--no-decode", action="store_true", help="skip the end-to-end decode legs")
    p.add_argument("--only", choices=["headline", "steps", "floor", "gemm", "pq", "pqpol", "int4g", "verify", "v5", "decode-tinyllama",
                            "decode-mistral"],
                   help="run one case and print its JSON (for profiler runs)")
    p.add_argument("--decode-steps", type=int, default=128,
                   help="timed decode steps of --only decode-* (fewer for profiler runs)")
    p.add_argument("--calib-copy", action="store_true",
                   help="first copy a 64 MiB buffer 8 times (the known-size kernel that scales the "
                        "FETCH_SIZE / WRITE_SIZE counters in the traffic passes)")
    return p.parse_args()


CALIB_BYTES = 64 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_int4_14336x4096_traffic.json")


def calib_copy(torch):
    """8 device-to-device copies of CALIB_BYTES (torch's elementwise copy
    kernel): it reads and writes exactly CALIB_BYTES each, which is what the
    traffic passes divide the counters by."""
    a = torch.empty(CALIB_BYTES // 4, device="cuda")
    a.fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(8):
        b.copy_(a)
    torch.cuda.synchronize()


def measured_traffic():
    """HBM bytes per headline launch from the committed FETCH_SIZE/WRITE_SIZE
    passes (profiles/), or None when they have not been recorded."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def matvec_bytes(M, N, bits, w4a8=False):
    wb = M * N * bits // 8
    xb = (N + 4 * ((N + 127) // 128)) if w4a8 else 4 * N
    return wb + 2 * M + xb + 4 * M


def make_weights(oracle, bits, M, N, seed):
    """Every row distinct: W ~ N(0, 0.02) from the library's generator,
    quantized with the quantize.c rules (ibh_quantize_rows, host threads)."""
    from libinferbit_amd import ibf
    W = ibf.fill_normal(M * N, 0x5EED0000 + 97 * seed + bits, std=0.02).reshape(M, N)
    w, s = ibf.quantize(bits, W)
    return (w.view(np.int8) if bits == 8 else w), s


def time_launches(torch, launch, steps, warmup):
    """Average device time per launch over exactly `steps` launches.  The
    launches (weight copy i % COPIES for launch i) are captured into one HIP
    graph of `steps` nodes, so the timed region holds back-to-back kernels
    with no host launch gaps; HIP events on the replay stream bracket it.
    Before it: `warmup` eager launches and one untimed replay of the graph
    (its first replay uploads the graph); a second untimed replay is queued
    just ahead of the timed one, so the start event is stamped when the
    device reaches it rather than while the host is still submitting the
    timed graph."""
    for i in range(max(1, warmup)):
        launch(i)                                   # eager warmup, also validates
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            for i in range(steps):
                launch(i)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g.replay()                                      # untimed, keeps the device busy while the timed one is queued
    e0.record(st)
    g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps * 1e-3   # seconds per launch


def gemv_case(torch, L, oracle, bits, M, N, steps, warmup, w4a8=False, seed=0):
    w, s = make_weights(oracle, bits, M, N, seed)
    wd = torch.from_numpy(w.view(np.uint8).copy()).cuda()
    copies = [wd] + [wd.clone() for _ in range(COPIES - 1)]
    sd = torch.from_numpy(s.view(np.int16).copy()).cuda()
    x = torch.randn(N, generator=torch.Generator().manual_seed(seed + 1)).cuda()
    y = torch.empty(M, device="cuda")
    if w4a8:
        q = torch.empty(N, dtype=torch.int8, device="cuda")
        sa = torch.empty((N + 127) // 128, device="cuda")
        L.ops.quantize_input_int8_g128(x, q, sa, N)

        def launch(i):
            L.ops.parallel_matmul_w4a8(y, copies[i % COPIES], sd, q, sa, M, N)
    else:
        def launch(i):
            L.ops.parallel_matmul(y, copies[i % COPIES], sd, x, M, N, bits)
    t = time_launches(torch, launch, steps, warmup)
    del copies
    nbytes = matvec_bytes(M, N, bits, w4a8)
    return {"M": M, "N": N, "bits": bits, "w4a8": w4a8, "us": round(t * 1e6, 3),
            "bytes": nbytes, "GBps": round(nbytes / t / 1e9, 1),
            "frac_hbm": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}


def steps_case(torch, L, oracle, warmup):
    """The headline kernel timed as in the bench line at several step counts
    K; a least-squares line through (K, total time) separates the per-launch
    time (slope) from what one timed graph window adds once (intercept:
    the gap before a graph's first kernel and the two event markers)."""
    M, N = 14336, 4096
    w, s = make_weights(oracle, 4, M, N, 0)
    wd = torch.from_numpy(w.view(np.uint8).copy()).cuda()
    copies = [wd] + [wd.clone() for _ in range(COPIES - 1)]
    sd = torch.from_numpy(s.view(np.int16).copy()).cuda()
    x = torch.randn(N, generator=torch.Generator().manual_seed(1)).cuda()
    y = torch.empty(M, device="cuda")

    def launch(i):
        L.ops.parallel_matmul(y, copies[i % COPIES], sd, x, M, N, 4)
    ks = (20, 40, 80, 160, 640, 2000)
    per = {k: time_launches(torch, launch, k, warmup) * 1e6 for k in ks}
    slope, icpt = np.polyfit(np.array(ks, dtype=float), np.array([per[k] * k for k in ks]), 1)
    nbytes = matvec_bytes(M, N, 4)
    return {"us_per_launch": {k: round(v, 3) for k, v in per.items()},
            "slope_us": round(float(slope), 3), "intercept_us": round(float(icpt), 2),
            "frac_hbm_at_slope": round(nbytes / (slope * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def floor_case(torch, L, steps, warmup):
    """The per-launch floor (an empty kernel) and a plain streaming read of
    the headline's 29,462,528 bytes (ibh_probe), timed like the matvecs."""
    nbytes = matvec_bytes(14336, 4096, 4)
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(COPIES)]
    st = lambda: torch.cuda.current_stream().cuda_stream
    out = {}
    for mode, name in ((0, "empty_kernel"), (1, "read_29462528_bytes")):
        def launch(i, mode=mode):
            L._lib.check(L.lib().ibh_probe(mode, bufs[i % COPIES].data_ptr(), nbytes, st()), "ibh_probe")
        t = time_launches(torch, launch, steps, warmup)
        out[name] = {"us": round(t * 1e6, 3)}
        if mode == 1:
            out[name].update(GBps=round(nbytes / t / 1e9, 1), frac_hbm=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4))
    return out


def batch_case(torch, L, oracle, B, steps, warmup):
    M, N = 14336, 4096
    w, s = make_weights(oracle, 4, M, N, 3)
    wd = torch.from_numpy(w.copy()).cuda()
    copies = [wd] + [wd.clone() for _ in range(COPIES - 1)]
    sd = torch.from_numpy(s.view(np.int16).copy()).cuda()
    qx = torch.randint(-127, 128, (B, N), dtype=torch.int8).cuda()
    sa = (torch.rand(B, N // 128) * 0.02 + 0.001).cuda()
    y = torch.empty(B * M, device="cuda")

    def launch(i):
        L.ops.matmul_w4a8_batch(y, copies[i % COPIES], sd, qx, sa, M, N, B, M)
    t = time_launches(torch, launch, steps, warmup)
    nbytes = M * N // 2 + 2 * M + B * (N + 4 * (N // 128)) + 4 * B * M
    return {"B": B, "us": round(t * 1e6, 3), "GBps": round(nbytes / t / 1e9, 1)}


def pq_case(torch, L, steps, warmup):
    """PQ LUT matvec at BASELINE configs[5]: M=4096, N=14336, G=16, K=256,
    one level, no outliers (ib_pq_matmul_fp32).  Bytes = both index planes
    + codebooks + row scales + x + y."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    from gen_golden import make_pq
    M, Cc, G, K = 4096, 896, 16, 256
    t = make_pq(np.random.default_rng(9), M, Cc, G, K, 1, 0, 0)
    devs = [L.ops.PqDeviceTensor(t) for _ in range(COPIES)]
    x = torch.randn(t["N"], generator=torch.Generator().manual_seed(2)).cuda()
    y = torch.empty(M, device="cuda")

    def launch(i):
        devs[i % COPIES].matmul(x, y)
    tm = time_launches(torch, launch, steps, warmup)
    nbytes = 2 * M * Cc + 2 * 2 * K * (G // 2) + 2 * M + 4 * t["N"] + 4 * M
    return {"M": M, "N": t["N"], "G": G, "K": K, "us": round(tm * 1e6, 3), "bytes": nbytes,
            "GBps": round(nbytes / tm / 1e9, 1)}


def int4g_case(torch, L, M, N, G, K_out, steps, warmup, awq=True):
    """IBF v5 INT4 group-scale matvec (ib_pq_session_matmul's INT4 backend,
    ibh_int4g_matmul) with AWQ inv_act and K_out fp16 outliers per row.
    Bytes = packed nibbles + fp16 group scales + outlier index/value pairs +
    x + inv_act + y."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    from gen_golden import make_int4g
    t = make_int4g(np.random.default_rng(12), M, N, G, int(awq), K_out)
    devs = [L.ops.Int4gDeviceTensor(t) for _ in range(COPIES)]
    x = torch.randn(N, generator=torch.Generator().manual_seed(4)).cuda()
    y = torch.empty(M, device="cuda")

    def launch(i):
        devs[i % COPIES].matmul(x, y)
    tm = time_launches(torch, launch, steps, warmup)
    nbytes = M * N // 2 + 2 * M * (N // G) + 4 * M * K_out + (8 if awq else 4) * N + 4 * M
    return {"M": M, "N": N, "G": G, "K_out": K_out, "awq": awq, "us": round(tm * 1e6, 3), "bytes": nbytes,
            "GBps": round(nbytes / tm / 1e9, 1), "frac_hbm": round(nbytes / tm / 1e9 / HBM_PEAK_GBS, 4)}


def pq_policy_cases(torch, L, steps, warmup):
    """The PQ session's policy variants (ibh_pq_matmul_policy) and the
    byte-quantised LUT (ibh_pq_matmul_q8lut) at the config-5 FFN shape with
    two levels (K = K_l2 = 256), and the top-K LM head (ibh_pq_lm_head_topk,
    K_top = 50 and the greedy 8) at a 32000 x 4096 head."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    from gen_golden import make_pq
    rng = np.random.default_rng(21)
    t = make_pq(rng, 4096, 896, 16, 256, 2, 256, 0)
    devs = [L.ops.PqDeviceTensor(t) for _ in range(4)]
    x = torch.randn(t["N"], generator=torch.Generator().manual_seed(5)).cuda()
    x[: t["N"] // 4] *= 1e-4
    y = torch.empty(4096, device="cuda")
    out = {}
    for name, (v, st, at) in {"streaming": (0, 0, 0), "l1_only": (1, 0, 0), "l2skip_0.5": (2, 0.5, 0),
                              "sparse_1e-3": (3, 0, 1e-3), "int8": (4, 0, 0)}.items():
        def launch(i, v=v, st=st, at=at):
            devs[i % 4].matmul_policy(x, y, v, st, at)
        out[name] = {"us": round(time_launches(torch, launch, steps, warmup) * 1e6, 2)}

    def launch_q8(i):
        devs[i % 4].matmul_q8lut(x, y)
    out["q8lut"] = {"us": round(time_launches(torch, launch_q8, steps, warmup) * 1e6, 2)}
    th = make_pq(rng, 32000, 256, 16, 256, 2, 256, 0)
    dh = L.ops.PqDeviceTensor(th)
    xh = torch.randn(th["N"], generator=torch.Generator().manual_seed(6)).cuda()
    for _ in range(3):
        dh.lm_head_topk(xh, 50)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(50):
        dh.lm_head_topk(xh, 50)
    torch.cuda.synchronize()
    out["lm_head_topk_32000x4096_k50"] = {"us_per_call_host_clock": round((time.perf_counter() - t0) / 50 * 1e6, 1)}
    t0 = time.perf_counter()
    for _ in range(50):
        dh.lm_head_topk(xh, 8)
    torch.cuda.synchronize()
    out["lm_head_topk_32000x4096_k8"] = {"us_per_call_host_clock": round((time.perf_counter() - t0) / 50 * 1e6, 1)}
    return out


def verify_case(steps):
    """Batched verify (ibh_model_forward_positions) on the TinyLlama
    configuration: milliseconds for B positions in one pass vs B single
    decode steps, both modes."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import gen_decode_golden as G
    from libinferbit_amd.model import Model
    workdir = os.environ.get("IBH_MODEL_DIR", "/tmp/ibh_models")
    os.makedirs(workdir, exist_ok=True)
    path = G.ensure_model("tinyllama", workdir)
    out = {}
    for mode in ("exact", "fast"):
        m = Model(path)
        m.set_exact(mode == "exact")
        m.forward(list(range(1, 33)))
        base = m.kv_length()
        res = {}
        for B in (1, 4, 8, 16):
            toks = list(range(100, 100 + B))
            m.forward_positions(toks)
            m.kv_truncate(base)
            t0 = time.perf_counter()
            for _ in range(steps):
                m.forward_positions(toks)
                m.kv_truncate(base)
            res[f"B{B}_ms"] = round((time.perf_counter() - t0) / steps * 1e3, 3)
        m.close()
        out[mode] = res
    return out


def prefill_gemm_case(torch, L, steps, warmup):
    """INT8 prefill GEMM at BASELINE configs[4]: 512 tokens x 4096 -> 14336
    (ibh_gemm_int8, matmul_int8_batch semantics), x N(0,1).  One step = one
    call (digit planes + GEMM).  Algorithmic work 2*B*M*N = 60.13 GFLOP; the
    int8 matrix cores execute 3x that (three digit planes)."""
    M, N, B = 14336, 4096, 512
    rng = np.random.default_rng(11)
    w = rng.integers(-127, 128, (M, N), dtype=np.int8)
    sc = (np.abs(rng.standard_normal(M)) * 1e-4 + 1e-4).astype(np.float16).view(np.int16)
    wd = [torch.from_numpy(w).cuda() for _ in range(4)]
    sd = torch.from_numpy(sc).cuda()
    x = torch.randn(B, N, generator=torch.Generator().manual_seed(3)).cuda()
    y = torch.empty(B * M, device="cuda")
    ws = torch.empty(L.lib().ibh_gemm_int8_workspace_bytes(N, B), dtype=torch.uint8, device="cuda")

    def launch(i):
        L.ops.gemm_int8(y, wd[i % 4], sd, x, M, N, B, M, ws)
    t = time_launches(torch, launch, steps, warmup)
    flops = 2.0 * B * M * N
    return {"M": M, "N": N, "B": B, "us": round(t * 1e6, 2), "TFLOPs_algorithmic": round(flops / t / 1e12, 1),
            "TOPs_int8_executed": round(3 * flops / t / 1e12, 1),
            "frac_int8_mfma_peak": round(3 * flops / t / 1e12 / 5000.0, 4),
            "frac_int8_peak_algorithmic": round(flops / t / 1e12 / 5000.0, 4)}


def decode_bytes_per_token(cfg, bits, n_pos):
    """Algorithmic HBM bytes of one decode step: every packed weight + scales
    once, the cache rows read by attention, the embedding row, activations
    ignored (< 0.1 %)."""
    H, I, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_layers"]
    KV = cfg["num_kv_heads"] * cfg["head_dim"]
    per_layer = 0
    for key, r, c in (("q_proj", H, H), ("k_proj", KV, H), ("v_proj", KV, H), ("o_proj", H, H),
                      ("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)):
        per_layer += r * c * bits[key] // 8 + 2 * r
    kvb = cfg["kv_bits"]
    row = 4 * KV if kvb >= 16 else (KV if kvb == 8 else (KV + 1) // 2)
    per_layer += 2 * n_pos * (row + (4 * cfg["num_kv_heads"] if kvb < 16 else 0)) + 4 * H   # K+V rows, 2 norms
    head = V * H * bits["head"] // 8 + 2 * V
    return L * per_layer + head + H * bits["token_embedding"] // 8 + 2 * H


def decode_case(name, steps, cpu):
    """Greedy decode tokens/s of a benchmark configuration: the model is
    regenerated from its seed, loaded (weights to HBM once), the prompt run,
    then `steps` decode steps are timed (each one HIP-graph replay; the clock
    covers host enqueue to device completion).  Measured in exact mode (the
    kernels whose token stream equals the CPU reference's, the headline) and
    in fast mode (fp32-tolerance kernels)."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import gen_decode_golden as G
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    case = G.CASES[name]
    workdir = os.environ.get("IBH_MODEL_DIR", "/tmp/ibh_models")
    os.makedirs(workdir, exist_ok=True)
    t = time.time()
    path = G.ensure_model(name, workdir)
    t_write = time.time() - t
    out = {"config": case["cfg"]["name"], "model_write_s": round(t_write, 1)}
    for mode in ("exact", "fast"):
        m = Model(path)
        m.set_exact(mode == "exact")
        if case["kv_pos"]:
            k, v = G.kv_of(case)
            m.kv_prefill(k, v)
            del k, v
        m.generate(G.prompt_of(case), 8)                  # prompt + warmup steps (graph built here)
        m.decode_steps(8)
        m.synchronize()
        n_pos = m.kv_length() + steps // 2                # mean cache length over the timed steps
        t0 = time.perf_counter()
        m.decode_steps(steps)
        m.synchronize()
        dt = time.perf_counter() - t0
        m.close()
        nbytes = decode_bytes_per_token(case["cfg"], ibf.DEFAULT_BITS, n_pos)
        tok_s = steps / dt
        out[mode] = {"tok_s": round(tok_s, 2), "ms_per_token": round(dt / steps * 1e3, 4), "steps": steps,
                     "kv_positions": n_pos, "bytes_per_token": nbytes, "GBps": round(nbytes * tok_s / 1e9, 1),
                     "frac_hbm": round(nbytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)}
    if cpu:
        threads = host_cpu()[0]
        # bounded samples of a few seconds each (TinyLlama ~15 tok/s, Mistral
        # ~2 tok/s on the box's host threads)
        if name == "tinyllama":
            out["cpu_baseline"] = cpu_decode(path, case, 48, [threads])
        else:
            out["cpu_baseline"] = cpu_decode(path, case, 8, [threads])
        try:
            out["dropin"] = dropin_decode(path, case, 32 if name == "tinyllama" else 8)
        except (RuntimeError, subprocess.TimeoutExpired) as e:
            out["dropin"] = {"error": str(e)[-300:]}
    return out


def host_cpu():
    """(threads to use, affinity count, model name).  The GPU box gives one
    GPU a share of 16 host threads (OMP_NUM_THREADS there is 16), whatever the
    affinity mask shows, so worker pools stop at 16."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(aff, share, 16)), aff, model


def _ref_decode(exe, path, threads, n_out, prompt_file, kv_file=None, n_pos=0):
    cmd = [exe, path, str(threads), "0", str(n_out), prompt_file]
    if kv_file:
        cmd += [kv_file, str(n_pos)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(r.stderr[-400:])
    return json.loads(r.stdout.strip().splitlines()[-1])


def cpu_decode(path, case, n_tok, threads_list):
    """The reference CPU decode (oracle/_ref/ref_decode: inferbit_generate,
    greedy) on the benchmark configuration's own workload: its prompt, and for
    the long-context case the KV cache prefilled to kv_pos positions (through
    the reference's kv_cache_write).  A bounded sample: tok/s = n_tok / (time
    of prompt + 1 + n_tok tokens - time of prompt + 1 token)."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import gen_decode_golden as G
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_decode")
    if not os.path.exists(exe):
        return None
    pp = path + ".cpu_prompt.i32"
    G.prompt_of(case).tofile(pp)
    kvp = None
    if case["kv_pos"]:
        kvp = path + ".cpu_kv.f32"
        if not os.path.exists(kvp):
            k, v = G.kv_of(case)
            with open(kvp + ".tmp", "wb") as f:
                f.write(k.tobytes())
                f.write(v.tobytes())
            del k, v
            os.replace(kvp + ".tmp", kvp)
    out = []
    _, aff, model = host_cpu()
    for threads in threads_list:
        n = n_tok[threads] if isinstance(n_tok, dict) else n_tok
        d1 = _ref_decode(exe, path, threads, 1, pp, kvp, case["kv_pos"])
        d2 = _ref_decode(exe, path, threads, 1 + n, pp, kvp, case["kv_pos"])
        dt = d2["seconds"] - d1["seconds"]
        out.append({"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
                    "sample": f"inferbit_generate greedy, the configuration's {case['n_prompt']}-token prompt"
                              + (f" over a KV cache prefilled to {case['kv_pos']} positions" if case["kv_pos"] else "")
                              + f", {n} decode steps timed ({dt:.2f} s) as the difference of two runs",
                    "host": model, "affinity_cpus": aff})
    return out


def dropin_decode(path, case, n_tok):
    """The drop-in path's decode rate: the reference's own inferbit_generate
    (oracle/_ref/dropin_attn: the reference's host code compiled from its
    sources, test infrastructure) with libibhip's dispatch-table entries and
    attention hook swapped in, weights registered once, threads = 1; the
    configuration's prompt (and prefilled KV cache).  Reported beside the
    CPU baseline, not as a product figure: every matvec stages x and y
    through host memory.  tok/s = n_tok / (generate(1 + n_tok) -
    generate(1)), the GPU pass only."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import gen_decode_golden as G
    exe = os.path.join(ROOT, "oracle", "_ref", "dropin_attn")
    if not os.path.exists(exe):
        return None
    pp = path + ".cpu_prompt.i32"
    G.prompt_of(case).tofile(pp)
    extra = []
    if case["kv_pos"]:
        kvp = path + ".cpu_kv.f32"
        if not os.path.exists(kvp):
            k, v = G.kv_of(case)
            with open(kvp + ".tmp", "wb") as f:
                f.write(k.tobytes())
                f.write(v.tobytes())
            del k, v
            os.replace(kvp + ".tmp", kvp)
        extra = [kvp, str(case["kv_pos"])]

    def run(n_out):
        r = subprocess.run([exe, path, "0", str(n_out), pp, "0", "0"] + extra, capture_output=True, text=True,
                           timeout=900)
        if r.returncode != 0:
            raise RuntimeError(r.stderr[-400:])
        d = json.loads(r.stdout.strip().splitlines()[-1])
        if d["attn_fallbacks"] or d["logits_nan"]:
            raise RuntimeError(f"drop-in pass fell back to the CPU: {d}")
        return d

    d1, d2 = run(1), run(1 + n_tok)
    dt = d2["gpu_seconds"] - d1["gpu_seconds"]
    return {"value": round(n_tok / dt, 2), "unit": "tok/s", "kind": "reference host loop on the GPU table",
            "sample": f"inferbit_generate greedy (threads 1) with ib_init_kernels_hip + ibh_register_host_weights "
                      f"+ the ibh_host_attn head-loop hook, {n_tok} decode steps timed ({dt:.2f} s) as the "
                      f"difference of two runs", "attn_calls": d2["attn_calls"]}


V5_TINYLLAMA = dict(num_layers=22, hidden_size=2048, num_heads=32, num_kv_heads=4, head_dim=64,
                    intermediate_size=5632, vocab_size=32000, rope_theta=10000.0)
# head_dim 128 with four query heads per kv head
V5_MISTRAL = dict(num_layers=32, hidden_size=4096, num_heads=32, num_kv_heads=8, head_dim=128,
                  intermediate_size=14336, vocab_size=32000, rope_theta=1000000.0)
V5_CASES = {"tinyllama": (V5_TINYLLAMA, "TinyLlama-1.1B shape", 8),
            "mistral": (V5_MISTRAL, "Mistral-7B shape (head_dim 128)", 4)}


def v5_bytes_per_token(cfg, n_pos, G=128, pq_G=16, pq_K=256):
    """Algorithmic HBM bytes of one v5 greedy step: INT4 nibbles + fp16 group
    scales + fp32 AWQ vector of every projection, the PQ head's indices, row
    scales and codebooks (level-1 logits of every row; the top-8 refinement
    re-reads 8 rows), the fp32 cache rows attention reads, the fp16
    embedding row."""
    H, I, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_layers"]
    KV = cfg["num_kv_heads"] * cfg["head_dim"]
    per_layer = 0
    for r, c in ((H, H), (KV, H), (KV, H), (H, H), (I, H), (I, H), (H, I)):
        per_layer += r * c // 2 + r * (c // G) * 2 + 4 * c
    per_layer += 2 * n_pos * 4 * KV + 2 * 4 * H
    C = H // pq_G
    head = 2 * V * C + 2 * V + 2 * pq_K * (pq_G // 2) * 2
    return L * per_layer + head + 2 * H


def v5_decode_case(steps, cpu, shape="tinyllama"):
    """IBF v5 session greedy decode (ib_pq_generate_greedy) on a synthetic v5
    model of the named shape (TinyLlama-1.1B, or Mistral-7B for head_dim
    128): INT4 group-128 projections with AWQ scales, PQ LM head (G 16,
    K 256), fp16 embedding.  tok/s = steps / (time
    of prompt + steps - time of the prompt alone), each a full
    generate call (device-resident loop of captured steps)."""
    from libinferbit_amd import ibf5
    from libinferbit_amd.session import PqSession
    workdir = os.environ.get("IBH_MODEL_DIR", "/tmp/ibh_models")
    os.makedirs(workdir, exist_ok=True)
    cfg, label, n_cpu = V5_CASES[shape]
    path = os.path.join(workdir, f"v5_{shape}_int4g_awq.ibf")
    t = time.time()
    if not os.path.exists(path):
        ibf5.write_synthetic_v5(path + ".tmp", cfg, seed=7, awq=True)
        os.replace(path + ".tmp", path)
    out = {"config": f"{label}, IBF v5 INT4 g128 + AWQ, PQ head", "model_write_s": round(time.time() - t, 1)}
    S = PqSession(path)
    kv = S.kv_cache(1024)
    prompt = list(range(1, 9))
    S.generate_greedy(kv, prompt, 8)                 # captures the steps
    kv.clear()
    t0 = time.perf_counter()
    S.generate_greedy(kv, prompt, 0)
    t_pre = time.perf_counter() - t0
    kv.clear()
    t0 = time.perf_counter()
    S.generate_greedy(kv, prompt, steps)
    t_all = time.perf_counter() - t0
    dt = t_all - t_pre
    tok_s = steps / dt
    nbytes = v5_bytes_per_token(cfg, len(prompt) + steps // 2)
    out["gpu"] = {"tok_s": round(tok_s, 2), "ms_per_token": round(dt / steps * 1e3, 4), "steps": steps,
                  "prefill_ms": round(t_pre * 1e3, 3), "bytes_per_token": nbytes,
                  "GBps": round(nbytes * tok_s / 1e9, 1), "frac_hbm": round(nbytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)}
    kv.close()
    S.close()
    if cpu:
        exe = os.path.join(ROOT, "oracle", "_ref", "ref_v5")
        if os.path.exists(exe):
            cores = host_cpu()[0]
            pp = path + ".prompt.i32"
            np.asarray(prompt, np.int32).tofile(pp)
            r = subprocess.run([exe, path, "64", str(n_cpu), pp, "greedy"], capture_output=True, text=True,
                               timeout=900, env=dict(os.environ, IB_PQ_THREADS=str(cores)))
            if r.returncode == 0:
                d = json.loads(r.stdout.strip().splitlines()[-1])
                cdt = d["seconds"] - d["prefill_seconds"]
                out["cpu_baseline"] = {"value": round(n_cpu / cdt, 3), "unit": "tok/s", "cores": cores,
                                       "kind": "reference",
                                       "sample": f"ib_pq_generate_greedy, 8-token prompt + {n_cpu} tokens, "
                                                 f"IB_PQ_THREADS={cores}, {cdt:.2f} s after the prompt"}
    return out


def cpu_baseline():
    """The reference library compiled from its own sources (oracle/_ref),
    ib_parallel_matmul INT4 14336x4096 with the x86 AVX2 table, timed on
    this host over rotating weight copies: with the box's thread share and
    with one thread."""
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_harness")
    if not os.path.exists(exe):
        return None
    threads, aff, model = host_cpu()
    copies = 8
    res = {}
    for t, iters in ((threads, 800), (1, 60)):
        r = subprocess.run([exe, "gemv", "4", "14336", "4096", str(t), str(iters), str(copies)],
                           capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            return None
        res[t] = json.loads(r.stdout.strip().splitlines()[-1])
    d, d1 = res[threads], res[1]
    nbytes = matvec_bytes(14336, 4096, 4)
    return {"value": round(nbytes / d["median_s"] / 1e9, 2), "unit": "GB/s", "cores": threads,
            "kind": "reference",
            "sample": f"{800} calls of ib_parallel_matmul(bits=4) 14336x4096 ({d['simd']}), "
                      f"{copies} rotating weight copies, median per call {d['median_s'] * 1e6:.0f} us",
            "one_thread": {"value": round(nbytes / d1["median_s"] / 1e9, 2), "unit": "GB/s",
                           "median_us": round(d1["median_s"] * 1e6, 1), "calls": 60},
            "host": model, "affinity_cpus": aff,
            "threads_note": "worker pools stop at the GPU box's share of 16 host threads"}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)
    import torch
    import libinferbit_amd as L
    from oracle import pyoracle as oracle

    L.ops.init(0)
    if a.calib_copy:
        calib_copy(torch)
    if a.only:
        if a.only == "headline":
            r = gemv_case(torch, L, oracle, 4, 14336, 4096, a.steps, a.warmup)
        elif a.only == "steps":
            r = steps_case(torch, L, oracle, a.warmup)
        elif a.only == "floor":
            r = floor_case(torch, L, a.steps, a.warmup)
        elif a.only == "gemm":
            r = prefill_gemm_case(torch, L, 64, 8)
        elif a.only == "pq":
            r = pq_case(torch, L, max(200, a.steps // 4), 20)
        elif a.only == "pqpol":
            r = pq_policy_cases(torch, L, max(200, a.steps // 4), 20)
        elif a.only == "v5":
            r = {k: v5_decode_case(256, cpu=not a.no_cpu, shape=k) for k in V5_CASES}
        elif a.only == "verify":
            r = verify_case(10)
        elif a.only == "int4g":
            r = {"14336x4096": int4g_case(torch, L, 14336, 4096, 128, 8, a.steps, a.warmup),
                 "4096x14336": int4g_case(torch, L, 4096, 14336, 128, 28, a.steps, a.warmup),
                 "14336x4096_plain": int4g_case(torch, L, 14336, 4096, 128, 0, a.steps, a.warmup, awq=False),
                 "4096x14336_plain": int4g_case(torch, L, 4096, 14336, 128, 0, a.steps, a.warmup, awq=False)}
        else:
            r = decode_case(a.only.split("-", 1)[1], a.decode_steps, cpu=False)
        print(json.dumps({"only": a.only, "result": r}), flush=True)
        return
    print("bench: headline INT4 GEMV 14336x4096", file=sys.stderr, flush=True)
    head = gemv_case(torch, L, oracle, 4, 14336, 4096, a.steps, a.warmup)
    extra = {"floor": floor_case(torch, L, a.steps, a.warmup)}
    if not a.quick:
        for name, (bits, M, N, w4a8) in {
            "int4_4096x14336": (4, 4096, 14336, False),
            "w4a8_14336x4096": (4, 14336, 4096, True),
            "w4a8_4096x14336": (4, 4096, 14336, True),
            "int8_2048x2048": (8, 2048, 2048, False),
            "int8_14336x4096": (8, 14336, 4096, False),
            "int2_14336x4096": (2, 14336, 4096, False),
        }.items():
            print(f"bench: {name}", file=sys.stderr, flush=True)
            extra[name] = gemv_case(torch, L, oracle, bits, M, N, a.steps, a.warmup, w4a8)
        extra["w4a8_batch_sweep_14336x4096"] = [batch_case(torch, L, oracle, B, max(200, a.steps // 4), 20)
                                                for B in (1, 2, 4, 8)]
        print("bench: prefill gemm", file=sys.stderr, flush=True)
        extra["prefill_gemm_int8_512x4096x14336"] = prefill_gemm_case(torch, L, 64, 8)
        print("bench: pq_4096x14336", file=sys.stderr, flush=True)
        extra["pq_4096x14336_G16_K256"] = pq_case(torch, L, max(200, a.steps // 4), 20)
        print("bench: pq policies + top-K head", file=sys.stderr, flush=True)
        extra["pq_policies_4096x14336_G16_K256_two_level"] = pq_policy_cases(torch, L, max(200, a.steps // 4), 20)
        print("bench: int4g (IBF v5 INT4 group-scale)", file=sys.stderr, flush=True)
        extra["int4g_14336x4096_G128_awq_out8"] = int4g_case(torch, L, 14336, 4096, 128, 8, a.steps, a.warmup)
        extra["int4g_4096x14336_G128_awq_out28"] = int4g_case(torch, L, 4096, 14336, 128, 28, a.steps, a.warmup)
    decode = {}
    if not a.no_decode and not a.quick:
        for name in ("tinyllama", "mistral"):
            print(f"bench: decode {name}", file=sys.stderr, flush=True)
            decode[name] = decode_case(name, 128, cpu=not a.no_cpu)
        print("bench: batched verify (forward_positions)", file=sys.stderr, flush=True)
        decode["tinyllama_forward_positions"] = verify_case(10)
        print("bench: v5 session decode", file=sys.stderr, flush=True)
        decode["v5_tinyllama_int4g"] = v5_decode_case(256, cpu=not a.no_cpu)
        print("bench: v5 session decode, head_dim 128", file=sys.stderr, flush=True)
        decode["v5_mistral_int4g"] = v5_decode_case(256, cpu=not a.no_cpu, shape="mistral")
    cpu = None if a.no_cpu else cpu_baseline()
    out = {
        "metric": "quantized GEMV HBM GB/s (% of peak) + decode tok/s, Mistral-7B-shape INT4, 1 GPU",
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "timing": f"{a.steps} launches in one HIP graph, timed by HIP events; {a.warmup} eager warmup launches "
                  "and one untimed replay before",
        "ms_per_step": round(head["us"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xf32",
        "data": "synthetic: W N(0,0.02), every row distinct, quantized with quantize.c rules, x N(0,1)",
        "config": {"workload": "INT4 matvec 14336x4096 batch 1 (matmul_int4), 16 rotating weight copies",
                   "M": 14336, "N": 4096, "batch": 1, "bits": 4},
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["frac_hbm"], "traffic": measured_traffic(),
                     "kernel": "gemv_tile_x<4,...>", "bytes_per_launch": head["bytes"],
                     "us_per_launch": head["us"]},
        "cpu_baseline": cpu,
        "decode_tok_s": decode.get("mistral", {}).get("exact", {}).get("tok_s"),
        "decode": decode,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
