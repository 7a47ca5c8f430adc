"""The IBF v5 PQ session on the GPU against the reference's own session
(oracle/_ref/ref_v5, built from the reference sources, run live on the same
file): ib_pq_forward_step logits of every prompt position within
max|d| / max|logit| <= 1e-4, the greedy continuation by argmax of those
logits identical, and ib_pq_generate_greedy (top-8 PQ head) identical.

Models are small seeded decoders written by libinferbit_amd.ibf5 covering
each backend of ib_pq_session_matmul (INT4 group scales with and without
AWQ scales and outliers, fp16 matrices, one- and two-level PQ with
outlier columns, 4-bit packed level-2 indices, PQ activation scales), fused
qkv / gateup tensors, fp16 / fp32 / PQ embeddings and the session's PQ
policies."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

REF_V5 = os.path.join(ROOT, "oracle", "_ref", "ref_v5")
REF_V5_NC = os.path.join(ROOT, "oracle", "_ref", "nc", "ref_v5")
CFG = dict(num_layers=2, hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64, intermediate_size=512,
           vocab_size=1000)
ALLPQ = {p: "pq" for p in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")}
CASES = {
    "int4": dict(),
    "int4_awq_outl": dict(awq=True, outliers=3),
    # 40 outliers per row: 4 rows x 40 > 128 sidecar slots, so the fused
    # rmsnorm (q/k/v, gate/up) and silu (down) launches take the per-row loop
    "int4_awq_outl40": dict(awq=True, outliers=40),
    "mixed": dict(backend=dict(gate_proj="pq", up_proj="pq", down_proj="pq", o_proj="fp16"), awq=True),
    "pq_l2_actscale_pqembed": dict(backend=ALLPQ, levels=2, pq_act_scale=True, embed="pq"),
    "pq_outl_k16_f32embed": dict(backend=ALLPQ, levels=2, k2=16, pq_outliers=16, embed="f32"),
    "fused": dict(fused=True, backend=dict(qkv_proj="pq", gateup_proj="int4g")),
}
PROMPT = [5, 17, 300, 42, 7]
N_NEW = 10
TOL = 1e-4


@pytest.fixture(scope="module")
def L():
    import libinferbit_amd as L
    L.ops.init(0)
    return L


def model(tmp_path_factory, name, cfg=CFG, **over):
    from libinferbit_amd import ibf5
    kw = dict(CASES.get(name, {}), **over)
    p = str(tmp_path_factory.mktemp("v5") / f"{name}.ibf")
    ibf5.write_synthetic_v5(p, cfg, seed=3, **kw)
    return p


def ref_run(path, prompt, n_new, mode, tmp, policy=None, max_seq=64, sample=None, binary=REF_V5):
    if not os.path.exists(binary):
        pytest.skip(f"{binary} not built (make -C oracle ref)")
    pp, lp = str(tmp / "p.i32"), str(tmp / "lg.f32")
    np.asarray(prompt, np.int32).tofile(pp)
    env = dict(os.environ, REF_V5_LOGITS=lp)
    if policy is not None:
        env["REF_V5_POLICY"] = ",".join(str(v) for v in policy)
    if sample is not None:
        env["REF_V5_SAMPLE"] = ",".join(str(v) for v in sample)
    r = subprocess.run([binary, path, str(max_seq), str(n_new), pp, mode], capture_output=True, text=True,
                       timeout=300, env=env)
    assert r.returncode == 0, r.stderr
    toks = json.loads(r.stdout.strip().splitlines()[-1])["tokens"]
    lg = np.fromfile(lp, np.float32).reshape(len(prompt), -1) if mode == "steps" else None
    return toks, lg


def relerr(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


def gpu_steps(S, prompt, n_new, max_seq=64, kv=None):
    kv = kv or S.kv_cache(max_seq)
    lg = [S.forward_step(kv, t, i) for i, t in enumerate(prompt)]
    cur, toks = lg[-1], []
    for g in range(n_new):
        best = int(np.argmax(cur))
        toks.append(best)
        if g + 1 < n_new:
            cur = S.forward_step(kv, best, len(prompt) + g)
    assert len(kv) == len(prompt) + n_new - 1
    return toks, np.stack(lg)


@pytest.mark.parametrize("name", list(CASES))
def test_forward_step_and_greedy(L, tmp_path_factory, tmp_path, name):
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, name)
    rt, rl = ref_run(path, PROMPT, N_NEW, "steps", tmp_path)
    S = PqSession(path)
    gt, gl = gpu_steps(S, PROMPT, N_NEW)
    errs = [relerr(gl[i], rl[i]) for i in range(len(PROMPT))]
    print(f"v5 {name}: max rel logit err {max(errs):.3g}", flush=True)
    assert max(errs) <= TOL, (name, errs)
    assert gt == rt, (name, gt, rt)
    rg, _ = ref_run(path, PROMPT, N_NEW, "greedy", tmp_path)
    gg = S.generate_greedy(S.kv_cache(64), PROMPT, N_NEW).tolist()
    assert gg == rg, (name, gg, rg)


# Rows of whole 256-byte steps: every INT4 launch of this shape runs the
# quad-layout group kernel (q/k/v and gate/up with the residual add and
# rmsnorm in front, down with silu * up formed in its prologue).
WIDE = dict(CFG, hidden_size=1024, num_heads=8, num_kv_heads=2, head_dim=128, intermediate_size=2048)


@pytest.mark.parametrize("name,inter", [("int4", 2048), ("int4_awq_outl", 2048), ("int4_awq_outl40", 2048),
                                        ("fused", 2048), ("int4_awq_outl", 5632)])
def test_quad_layout_group_kernel(L, tmp_path_factory, tmp_path, name, inter):
    """AWQ, outliers through the per-wavefront sidecar (3 per row) and the
    per-row loop (40 per row), and the fused q/k/v + gate/up tensors, on the
    quad-layout group kernel; intermediate 5632 (11 steps of 256 bytes)
    takes K-ranges of 4 + 4 + 3 steps in the down projection.  Logits within
    TOL of the reference's and the same tokens; with that kernel switched
    off (the row kernel runs) the same holds."""
    from libinferbit_amd import _lib
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, f"wide_{name}_{inter}", cfg=dict(WIDE, intermediate_size=inter), **CASES[name])
    print(f"case v5 wide {name}", flush=True)
    rt, rl = ref_run(path, PROMPT, 6, "steps", tmp_path)
    for mode in (0, -1):
        assert _lib.lib().ibh_set_tile_config(mode, 0, 0, -1) == 0
        try:
            S = PqSession(path)
            gt, gl = gpu_steps(S, PROMPT, 6)
        finally:
            _lib.lib().ibh_set_tile_config(0, 0, 0, -1)
        errs = [relerr(gl[i], rl[i]) for i in range(len(PROMPT))]
        print(f"v5 wide {name} tile_mode={mode}: max rel logit err {max(errs):.3g}", flush=True)
        assert max(errs) <= TOL, (name, mode, errs)
        assert gt == rt, (name, mode, gt, rt)


POLICIES = {
    "l1_only": (1, 0.0, 0.0),
    "l2skip": (2, 0.5, 0.0),
    "sparse": (3, 0.0, 0.3),
    "int8": (4, 0.0, 0.0),
}


@pytest.mark.parametrize("pol", list(POLICIES))
def test_policies(L, tmp_path_factory, tmp_path, pol):
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "pq_l2_actscale_pqembed")
    p = POLICIES[pol]
    rt, rl = ref_run(path, PROMPT, N_NEW, "steps", tmp_path, policy=p)
    S = PqSession(path)
    S.set_default_policy(*p)
    gt, gl = gpu_steps(S, PROMPT, N_NEW)
    errs = [relerr(gl[i], rl[i]) for i in range(len(PROMPT))]
    # skip decisions compare rounded tables: a decision at its threshold may
    # flip, which moves a logit by one dropped level-2 term
    tol = TOL if pol in ("l1_only", "int8") else 1e-3
    assert max(errs) <= tol, (pol, errs)
    assert gt == rt, (pol, gt, rt)


def test_per_tensor_policy_and_matmul(L, tmp_path_factory, tmp_path):
    """set_policy on one tensor; session matmul of every backend against the
    session's own step (shapes) and the error paths."""
    import torch
    from libinferbit_amd._lib import IbhError
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "mixed")
    S = PqSession(path)
    assert S.tensor_info("L0_q_proj") == ("int4", 256, 256)
    assert S.tensor_info("L0_o_proj") == ("fp16", 256, 256)
    assert S.tensor_info("L0_down_proj") == ("pq", 256, 512)
    with pytest.raises(IbhError):
        S.set_policy("L0_q_proj", 1)       # not a PQ tensor
    with pytest.raises(IbhError):
        S.tensor_info("nope")
    x = torch.randn(512, device="cuda")
    y = torch.empty(256, device="cuda")
    S.matmul("L0_down_proj", x, y)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    S.set_policy("L1_gate_proj", 1)
    rt, _ = ref_run(path, PROMPT, 4, "steps", tmp_path)
    gt, _ = gpu_steps(S, PROMPT, 4)
    assert len(gt) == 4
    kv = S.kv_cache(8)
    with pytest.raises(IbhError):
        S.forward_step(kv, 0, 8)            # position beyond the cache
    with pytest.raises(IbhError):
        S.forward_step(kv, 1000, 0)         # token beyond the vocabulary


def test_cache_limit_stops_generation(L, tmp_path_factory, tmp_path):
    """ib_pq_generate_greedy stops once pos reaches max_seq."""
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "int4")
    rg, _ = ref_run(path, PROMPT, 20, "greedy", tmp_path, max_seq=8)
    S = PqSession(path)
    gg = S.generate_greedy(S.kv_cache(8), PROMPT, 20).tolist()
    assert gg == rg and len(gg) == 8 - len(PROMPT) + 1


def test_eos_cut_and_cache_length(L, tmp_path_factory, tmp_path):
    """Generation stops at the first eos (kept in the output); the cache holds
    the prompt plus every token before it; a second call on a cleared cache
    replays the same captured steps to the same tokens."""
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "mixed")
    rg, _ = ref_run(path, PROMPT, 40, "greedy", tmp_path)
    S = PqSession(path)
    kv = S.kv_cache(64)
    assert S.generate_greedy(kv, PROMPT, 40).tolist() == rg
    assert len(kv) == len(PROMPT) + 40
    for cut in (0, 3, 21):
        eos = rg[cut]
        first = rg.index(eos)
        kv.clear()
        got = S.generate_greedy(kv, PROMPT, 40, eos=eos).tolist()
        assert got == rg[:first + 1], (cut, got)
        assert len(kv) == len(PROMPT) + first


def test_policy_change_recaptures(L, tmp_path_factory, tmp_path):
    """A policy change after steps were captured applies to the next step."""
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "pq_l2_actscale_pqembed")
    S = PqSession(path)
    kv = S.kv_cache(64)
    t0, l0 = gpu_steps(S, PROMPT, 3, kv=kv)
    r0, rl0 = ref_run(path, PROMPT, 3, "steps", tmp_path)
    assert t0 == r0 and relerr(l0[-1], rl0[-1]) <= TOL
    S.set_default_policy(1)
    t1, l1 = gpu_steps(S, PROMPT, 3, kv=kv)
    r1, rl1 = ref_run(path, PROMPT, 3, "steps", tmp_path, policy=(1, 0.0, 0.0))
    assert t1 == r1 and relerr(l1[-1], rl1[-1]) <= TOL
    assert relerr(l1[-1], l0[-1]) > 1e-3      # the level-2 terms are gone


def test_grouped_int4_launch_matches_single(L, tmp_path_factory, monkeypatch):
    """q/k/v and gate/up run as one matrix-core launch per set and silu * up
    is formed inside the down launch; IBH_V5_NO_GROUP=1 runs one launch per
    matrix and a separate silu.  The per-row arithmetic is the same except
    the silu exponential (hardware exp in the fused launch, the glibc-exact
    one in the separate kernel): logits agree to 1e-5."""
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "int4_awq_outl")
    S = PqSession(path)
    _, a = gpu_steps(S, PROMPT, 2)
    monkeypatch.setenv("IBH_V5_NO_GROUP", "1")
    S1 = PqSession(path)
    _, b = gpu_steps(S1, PROMPT, 2)
    assert relerr(a, b) <= 1e-5


@pytest.mark.parametrize("split_env", ["", "1"])
def test_long_prompt_attention_splits(L, tmp_path_factory, tmp_path, monkeypatch, split_env):
    """A 300-token prompt in a 600-position cache: the fused attention spreads
    the positions over three splits merged in-kernel (and, with
    IBH_V5_SPLIT_ATTN=1, the rope + split-K attention kernels run instead);
    logits and tokens as the reference's."""
    from libinferbit_amd.session import PqSession
    if split_env:
        monkeypatch.setenv("IBH_V5_SPLIT_ATTN", split_env)
    path = model(tmp_path_factory, "fused")
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, CFG["vocab_size"], 300)]
    rt, rl = ref_run(path, prompt, 6, "steps", tmp_path, max_seq=600)
    S = PqSession(path)
    gt, gl = gpu_steps(S, prompt, 6, max_seq=600)
    errs = [relerr(gl[i], rl[i]) for i in (0, 1, 150, 255, 256, 299)]
    assert max(errs) <= TOL, errs
    assert gt == rt
    rg, _ = ref_run(path, prompt, 12, "greedy", tmp_path, max_seq=600)
    assert S.generate_greedy(S.kv_cache(600), prompt, 12).tolist() == rg


@pytest.mark.parametrize("heads,kv_heads,hd", [(8, 1, 64), (4, 4, 128), (16, 4, 32)])
def test_head_geometries(L, tmp_path_factory, tmp_path, heads, kv_heads, hd):
    """Eight query heads per kv head, head_dim 128 without GQA, and
    head_dim 32 (the rope + split-K attention kernels)."""
    from libinferbit_amd.session import PqSession
    cfg = dict(CFG, hidden_size=heads * hd, num_heads=heads, num_kv_heads=kv_heads, head_dim=hd)
    path = model(tmp_path_factory, f"geo{heads}_{kv_heads}_{hd}", cfg=cfg, backend=dict(o_proj="pq"))
    prompt = [int(t) for t in np.random.default_rng(heads).integers(0, CFG["vocab_size"], 40)]
    rt, rl = ref_run(path, prompt, 5, "steps", tmp_path, max_seq=300)
    S = PqSession(path)
    gt, gl = gpu_steps(S, prompt, 5, max_seq=300)
    assert max(relerr(gl[i], rl[i]) for i in range(len(prompt))) <= TOL
    assert gt == rt


SAMPLES = {
    "topk40_p09": (0.8, 40, 0.9, 7),
    "topk256_T1": (1.0, 256, 0.0, 123),
    "topk8_T0": (0.0, 8, 0.9, 5),
    "full_p09": (0.8, 0, 0.9, 7),
    "full_T12": (1.2, 0, 0.0, 99),
    "k300_full": (0.7, 300, 0.95, 0),
}


@pytest.mark.parametrize("name", list(SAMPLES))
def test_generate_sample(L, tmp_path_factory, tmp_path, name):
    """ib_pq_generate_sample: the top-K PQ head (0 < top_k <= 256) or the
    full logits (top_k 0 or > 256), the reference's xorshift64 stream and
    softmax / top-p / inverse-CDF pick; token streams equal."""
    from libinferbit_amd.session import PqSession
    T, k, p, seed = SAMPLES[name]
    path = model(tmp_path_factory, "mixed")
    rg, _ = ref_run(path, PROMPT, 24, "sample", tmp_path, sample=(T, k, p, seed))
    S = PqSession(path)
    kv = S.kv_cache(64)
    got = S.generate_sample(kv, PROMPT, 24, temperature=T, top_k=k, top_p=p, seed=seed).tolist()
    assert got == rg, (name, got, rg)
    assert len(kv) == len(PROMPT) + 24


@pytest.mark.parametrize("mode", ["IB_PQ_KV_FP16", "IB_PQ_KV_INT8"])
@pytest.mark.parametrize("name,n_prompt", [("mixed", 5), ("fused", 150)])
def test_kv_storage_modes(L, tmp_path_factory, tmp_path, monkeypatch, mode, name, n_prompt):
    """The reference's fp16 and int8 (one scale per position over kv_dim)
    cache storage, selected by the same environment switches; logits and
    tokens as the reference's under the same switch."""
    from libinferbit_amd.session import PqSession
    monkeypatch.setenv(mode, "1")
    path = model(tmp_path_factory, name)
    prompt = PROMPT if n_prompt == 5 else [int(t) for t in np.random.default_rng(9).integers(0, 1000, n_prompt)]
    rt, rl = ref_run(path, prompt, 6, "steps", tmp_path, max_seq=256)
    S = PqSession(path)
    gt, gl = gpu_steps(S, prompt, 6, max_seq=256)
    assert max(relerr(gl[i], rl[i]) for i in range(len(prompt))) <= TOL
    assert gt == rt
    rg, _ = ref_run(path, prompt, 10, "greedy", tmp_path, max_seq=256)
    assert S.generate_greedy(S.kv_cache(256), prompt, 10).tolist() == rg


def test_kv_pyramid_without_codebooks_is_fp32(L, tmp_path_factory, tmp_path, monkeypatch):
    """IB_PQ_KV_PYRAMID on a file without K/V codebooks: the reference keeps
    fp32 rows, so does the GPU cache (same logits as without the switch)."""
    from libinferbit_amd.session import PqSession
    path = model(tmp_path_factory, "int4")
    monkeypatch.setenv("IB_PQ_KV_PYRAMID", "1")
    rt, rl = ref_run(path, PROMPT, 4, "steps", tmp_path)
    S = PqSession(path)
    gt, gl = gpu_steps(S, PROMPT, 4)
    assert gt == rt and max(relerr(gl[i], rl[i]) for i in range(len(PROMPT))) <= TOL


def test_long_context_odd_vocab_small_groups(L, tmp_path_factory, tmp_path):
    """A 1500-token prompt over 24 attention splits, rope_theta 5e5,
    rms_norm_eps 1e-6, an odd vocabulary and INT4 groups of 64 (the
    wavefront-per-row INT4 kernel)."""
    from libinferbit_amd.session import PqSession
    cfg = dict(CFG, vocab_size=1237, rope_theta=500000.0, rms_norm_eps=1e-6)
    path = model(tmp_path_factory, "long_g64", cfg=cfg, i4_group=64, awq=True, outliers=2)
    prompt = [int(t) for t in np.random.default_rng(15).integers(0, 1237, 1500)]
    rt, rl = ref_run(path, prompt, 4, "steps", tmp_path, max_seq=1600)
    S = PqSession(path)
    gt, gl = gpu_steps(S, prompt, 4, max_seq=1600)
    errs = [relerr(gl[i], rl[i]) for i in (0, 63, 64, 700, 1499)]
    assert max(errs) <= TOL, errs
    assert gt == rt


@pytest.mark.parametrize("mode", ["", "IB_PQ_KV_FP16", "IB_PQ_KV_INT8"])
@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (4, 4)])
def test_head_dim_128_long_prompt(L, tmp_path_factory, tmp_path, monkeypatch, mode, heads, kv_heads):
    """head_dim 128 over a 320-token prompt (several attention splits, so the
    next-tile prefetch and the cross-split merge run), four query heads per
    kv head and no GQA, with fp32, fp16 and int8 cache storage.

    fp32 storage is held to TOL.  fp16 and int8 storage round every cached
    value, so a one-ulp difference upstream flips an element by a whole
    quantization step whenever it lands on a rounding boundary (int8: 1/127
    of the position's max|k|), and those flips accumulate over the prompt.
    The reference shows the same magnification against itself: the same
    sources built with -ffp-contract=off (oracle/_ref/nc/ref_v5, which
    changes nothing but the rounding of a*b+c) differ from the -mfma build by
    up to 9.6e-5 (fp16) and 1.7e-3 (int8) on these cases, 1.7e-6 with fp32
    storage.  So with quantized storage the GPU is held to TOL plus twice the
    reference's own distance between its two builds, and the tokens must
    match exactly."""
    from libinferbit_amd.session import PqSession
    if mode:
        monkeypatch.setenv(mode, "1")
    hd = 128
    cfg = dict(CFG, hidden_size=heads * hd, num_heads=heads, num_kv_heads=kv_heads, head_dim=hd)
    path = model(tmp_path_factory, f"hd128_{heads}_{kv_heads}", cfg=cfg, backend=dict(o_proj="pq"))
    print(f"case v5 hd128 heads={heads}/{kv_heads} {mode or 'fp32'}", flush=True)
    prompt = [int(t) for t in np.random.default_rng(heads + kv_heads).integers(0, CFG["vocab_size"], 320)]
    rt, rl = ref_run(path, prompt, 4, "steps", tmp_path, max_seq=400)
    S = PqSession(path)
    gt, gl = gpu_steps(S, prompt, 4, max_seq=400)
    err = max(relerr(gl[i], rl[i]) for i in range(len(prompt)))
    bound = TOL
    if mode:
        nt, nl = ref_run(path, prompt, 4, "steps", tmp_path, max_seq=400, binary=REF_V5_NC)
        assert nt == rt
        bound += 2 * max(relerr(nl[i], rl[i]) for i in range(len(prompt)))
    print(f"v5 hd128 heads={heads}/{kv_heads} {mode or 'fp32'}: max rel logit err {err:.3g} (bound {bound:.3g})",
          flush=True)
    assert err <= bound
    assert gt == rt
