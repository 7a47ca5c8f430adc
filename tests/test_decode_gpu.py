"""GPU decode (device-resident forward + greedy generate) against the
reference library's CPU decode.

* Small synthetic models: the reference's own `ref_decode` (oracle/_ref,
  built from the reference sources) runs live on the same file.  Exact mode
  (the default) must give bit-identical logits and identical greedy token
  streams; fast mode must give logits within max|d| / max|logit| <= 1e-4.
* Benchmark configurations (TinyLlama-1.1B and Mistral-7B shapes): the
  models are regenerated from their seeds (SHA-256 checked against the
  fixture) and the GPU token streams must equal the reference's streams
  recorded in tests/golden/decode.json by tests/golden/gen_decode_golden.py.
"""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, ROOT

pytestmark = pytest.mark.gpu

REF_DECODE = os.path.join(ROOT, "oracle", "_ref", "ref_decode")
MODEL_DIR = os.environ.get("IBH_MODEL_DIR", "/tmp/ibh_models")


@pytest.fixture(scope="module")
def L():
    import libinferbit_amd as L
    L.ops.init(0)
    return L


def tiny_cfg(**kw):
    from libinferbit_amd import ibf
    c = dict(ibf.TINYLLAMA, num_layers=2, hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64,
             intermediate_size=512, vocab_size=1000, max_context_length=160)
    c.update(kw)
    return c


def ref_run(path, prompt, n_out, tmp, kv=None, env=None):
    if not os.path.exists(REF_DECODE):
        pytest.skip("oracle/_ref/ref_decode not built (make -C oracle ref)")
    pp, lp = str(tmp / "p.i32"), str(tmp / "lg.f32")
    np.asarray(prompt, np.int32).tofile(pp)
    cmd = [REF_DECODE, path, "1", "0", str(n_out), pp]
    if kv is not None:
        kp = str(tmp / "kv.f32")
        with open(kp, "wb") as f:
            f.write(np.ascontiguousarray(kv[0], np.float32).tobytes())
            f.write(np.ascontiguousarray(kv[1], np.float32).tobytes())
        cmd += [kp, str(kv[0].shape[1])]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, REF_DECODE_LOGITS=lp, **(env or {})))
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])["tokens"], np.fromfile(lp, np.float32)


def relerr(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


TINY = {
    "fp32kv": dict(kv_bits=32),
    "int8kv": dict(kv_bits=8),
    "int4kv": dict(kv_bits=4),
    "mlp_int2": dict(kv_bits=8, bits=dict(gate_proj=2, up_proj=2, down_proj=2, o_proj=8)),
    "all_int8": dict(kv_bits=8, bits=dict(o_proj=8, gate_proj=8, up_proj=8, down_proj=8)),
    "int4_emb_head": dict(kv_bits=8, bits=dict(token_embedding=4, head=4)),
}


def same_bits(a, b):
    np.testing.assert_array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("name", list(TINY))
def test_tiny_model_matches_reference(L, tmp_path, name):
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    spec = dict(TINY[name])
    bits = spec.pop("bits", None)
    print(f"case decode tiny {name}", flush=True)
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(**spec), seed=11, bits=bits)
    prompt = [5, 17, 300, 42, 999, 0, 7]
    ref_tokens, ref_logits = ref_run(path, prompt, 40, tmp_path)
    m = Model(path)
    assert m.dims["exact"] == 1
    same_bits(m.forward(prompt), ref_logits)
    m.kv_clear()
    assert m.generate(prompt, 40).tolist() == ref_tokens
    m.kv_clear()
    m.set_exact(False)
    assert relerr(m.forward(prompt), ref_logits) <= 1e-4
    m.close()


@pytest.mark.parametrize("hidden,heads,kv", [(2048, 32, 4), (1024, 16, 16), (512, 8, 1)])
def test_wider_models_bit_exact(L, tmp_path, hidden, heads, kv):
    """Hidden sizes and GQA groups of the benchmark shapes (hidden 2048 with a
    group of 8 is TinyLlama's), 3 layers, W4A8 MLP: logits bit-identical."""
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    print(f"case decode wide hidden={hidden} heads={heads}/{kv}", flush=True)
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(num_layers=3, hidden_size=hidden, num_heads=heads, num_kv_heads=kv,
                                       intermediate_size=2816, kv_bits=8), seed=21)
    prompt = list(range(3, 60, 3))
    ref_tokens, ref_logits = ref_run(path, prompt, 20, tmp_path)
    m = Model(path)
    same_bits(m.forward(prompt), ref_logits)
    m.kv_clear()
    assert m.generate(prompt, 20).tolist() == ref_tokens
    m.close()


def test_tiny_kv_prefill_matches_reference(L, tmp_path):
    """KV prefilled through the kv_cache_write rule, then decode (the config-4 recipe)."""
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    for kvb in (8, 4):
        print(f"case decode tiny kv prefill bits={kvb}", flush=True)
        cfg = tiny_cfg(kv_bits=kvb)
        path = str(tmp_path / f"m{kvb}.ibf")
        ibf.write_synthetic(path, cfg, seed=5)
        shape = (cfg["num_layers"], 100, cfg["num_kv_heads"] * cfg["head_dim"])
        k = ibf.fill_normal(int(np.prod(shape)), 1).reshape(shape)
        v = ibf.fill_normal(int(np.prod(shape)), 2).reshape(shape)
        ref_tokens, ref_logits = ref_run(path, [77], 30, tmp_path, kv=(k, v))
        m = Model(path)
        m.kv_prefill(k, v)
        assert m.kv_length() == 100
        same_bits(m.forward([77]), ref_logits)
        m.kv_truncate(100)
        assert m.generate([77], 30).tolist() == ref_tokens
        m.close()


def test_w4a8_disabled_matches_reference(L, tmp_path, monkeypatch):
    """IB_W4A8=0 (forward.c:14-21) routes INT4 tensors through the fp32-activation matvec."""
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(kv_bits=8), seed=3)
    ref_tokens, ref_logits = ref_run(path, [1, 2, 3], 30, tmp_path, env={"IB_W4A8": "0"})
    monkeypatch.setenv("IB_W4A8", "0")
    m = Model(path)
    same_bits(m.forward([1, 2, 3]), ref_logits)
    m.kv_clear()
    assert m.generate([1, 2, 3], 30).tolist() == ref_tokens
    m.close()


def test_graph_replay_equals_eager(L, tmp_path, monkeypatch):
    """The captured per-token graph gives bit-identical logits to eager launches,
    replay after replay, in both modes."""
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(kv_bits=8), seed=4)
    prompt = list(range(10, 30))
    for exact in (True, False):
        monkeypatch.delenv("IBH_DECODE_EAGER", raising=False)
        g = Model(path)
        g.set_exact(exact)
        a = [g.forward([t]) for t in prompt]
        monkeypatch.setenv("IBH_DECODE_EAGER", "1")
        e = Model(path)
        e.set_exact(exact)
        b = [e.forward([t]) for t in prompt]
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
        g.close()
        e.close()


def test_model_api_errors(L, tmp_path):
    from libinferbit_amd import IbhError, ibf
    from libinferbit_amd.model import Model
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(kv_bits=8, max_context_length=16), seed=4)
    m = Model(path)
    with pytest.raises(IbhError):
        m.forward([1000])                       # token out of range
    with pytest.raises(IbhError):
        m.forward(list(range(17)))              # context exceeded
    m.forward(list(range(16)))
    assert m.kv_length() == 16
    with pytest.raises(IbhError):
        m.forward([1])                          # no room left
    with pytest.raises(IbhError):
        m.generate([1], 2)
    m.close()
    bad = tmp_path / "bad.ibf"
    bad.write_bytes(b"NOTANIBF" + bytes(100))
    with pytest.raises(IbhError):
        Model(str(bad))


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for b in iter(lambda: f.read(1 << 24), b""):
            h.update(b)
    return h.hexdigest()


def _golden_case(name):
    p = os.path.join(GOLDEN, "decode.json")
    if not os.path.exists(p):
        pytest.skip("tests/golden/decode.json not generated")
    d = json.load(open(p))
    if name not in d:
        pytest.skip(f"no {name} entry in decode.json")
    return d[name]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", ["tinyllama", "mistral"])
def test_benchmark_config_tokens_match_reference(L, name):
    import sys
    sys.path.insert(0, GOLDEN)
    import gen_decode_golden as G
    from libinferbit_amd.model import Model
    g = _golden_case(name)
    os.makedirs(MODEL_DIR, exist_ok=True)
    print(f"case decode {name}: writing model", flush=True)
    path = G.ensure_model(name, MODEL_DIR)
    assert _sha256(path) == g["model_sha256"], "synthetic model bytes differ from the fixture's"
    print(f"case decode {name}: decoding", flush=True)
    case = G.CASES[name]
    m = Model(path)
    if case["kv_pos"]:
        k, v = G.kv_of(case)
        m.kv_prefill(k, v)
        del k, v
    got = m.generate(np.asarray(g["prompt"], np.int32), g["n_out"])
    m.close()
    assert got.tolist() == g["tokens"]


def _fast_vs_exact(name, n_steps=None):
    """Fast-mode decode of a benchmark config, teacher-forced along the
    reference's token stream next to the exact-mode model (whose logits are
    bit-identical to the CPU's): per step the fast argmax, the exact top-2
    gap and max|logit_fast - logit_exact|."""
    import sys
    sys.path.insert(0, GOLDEN)
    import gen_decode_golden as G
    from libinferbit_amd.model import Model
    g = _golden_case(name)
    os.makedirs(MODEL_DIR, exist_ok=True)
    path = G.ensure_model(name, MODEL_DIR)
    assert _sha256(path) == g["model_sha256"], "synthetic model bytes differ from the fixture's"
    case = G.CASES[name]
    me, mf = Model(path), Model(path)
    mf.set_exact(False)
    if case["kv_pos"]:
        k, v = G.kv_of(case)
        me.kv_prefill(k, v)
        mf.kv_prefill(k, v)
        del k, v
    ref = g["tokens"][:n_steps] if n_steps else g["tokens"]
    feed = list(g["prompt"])
    rows = []
    for i in range(len(ref)):
        le, lf = me.forward(feed), mf.forward(feed)
        top = np.argsort(-le.astype(np.float64), kind="stable")[:2]
        rows.append(dict(step=i, exact=int(np.argmax(le)), fast=int(np.argmax(lf)), ref=ref[i],
                         gap=float(le[top[0]] - le[top[1]]), err=float(np.abs(lf - le).max()),
                         scale=float(np.abs(le).max())))
        feed = [int(np.argmax(le))]
    me.close()
    mf.close()
    return rows


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["tinyllama", "mistral"])
def test_benchmark_config_fast_mode_tokens(L, name):
    """Fast mode (fp32-tolerance kernels) on configs 3 and 4, teacher-forced
    along the reference's recorded stream.  Reported: every step where the
    fast argmax leaves the stream, with the CPU's (= exact mode's) top-2
    logit gap there.  With INT4 layers in W4A8 form (the reference's default,
    forward.c:14-21) the activations of o/gate/up/down are re-quantized to
    int8 per 128-group with round-to-nearest: an fp32-rounding difference
    upstream can move a value across a rounding boundary, which changes one
    code by 1/127 of its group's max -- a step, not a drift, so fast and
    exact logits differ by far more than 1e-4 (measured up to ~7 %) and the
    streams part at near-ties.  Asserted: the exact model follows the
    reference stream, and every fast departure sits where the CPU's top-2
    gap is within twice the fast path's logit error at that step."""
    print(f"case decode fast {name}", flush=True)
    rows = _fast_vs_exact(name)
    assert all(r["exact"] == r["ref"] for r in rows), "exact mode left the reference stream"
    flips = [r for r in rows if r["fast"] != r["ref"]]
    worst = max(r["err"] / r["scale"] for r in rows)
    print(f"fast {name}: {len(rows)} steps, {len(flips)} argmax departures, max rel logit err {worst:.3g}",
          flush=True)
    for r in flips:
        print(f"  step {r['step']}: fast {r['fast']} ref {r['ref']} top-2 gap {r['gap']:.6g} "
              f"fast err {r['err']:.3g}", flush=True)
    assert all(r["gap"] <= 2 * r["err"] for r in flips)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["tinyllama", "mistral"])
def test_benchmark_config_fast_mode_without_w4a8(L, name, monkeypatch):
    """The same configs with IB_W4A8=0 (INT4 layers on fp32 activations, no
    re-quantization step): fast logits within 1e-4 of the exact model's at
    every step and the same greedy stream (32 steps)."""
    print(f"case decode fast {name} IB_W4A8=0", flush=True)
    monkeypatch.setenv("IB_W4A8", "0")
    rows = _fast_vs_exact(name, 32)
    worst = max(r["err"] / r["scale"] for r in rows)
    print(f"fast {name} IB_W4A8=0: max rel logit err {worst:.3g}", flush=True)
    assert worst <= 1e-4
    assert all(r["fast"] == r["exact"] for r in rows)
