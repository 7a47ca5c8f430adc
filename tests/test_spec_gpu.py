"""Batched verify (ib_forward_positions) and greedy speculative decoding on
the device-resident model against the reference library's CPU run
(oracle/_ref/ref_decode, built from the reference sources, on the same
synthetic model).  Exact mode: bit-identical per-position logits and
identical token streams; fast mode: logits within 1e-4 of max|logit|."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

REF_DECODE = os.path.join(ROOT, "oracle", "_ref", "ref_decode")


@pytest.fixture(scope="module")
def L():
    import libinferbit_amd as L
    L.ops.init(0)
    return L


def cfg(**kw):
    from libinferbit_amd import ibf
    c = dict(ibf.TINYLLAMA, num_layers=2, hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64,
             intermediate_size=512, vocab_size=1000, max_context_length=256)
    c.update(kw)
    return c


def ref(path, prompt, n_out, tmp, env):
    if not os.path.exists(REF_DECODE):
        pytest.skip("oracle/_ref/ref_decode not built (make -C oracle ref)")
    pp = str(tmp / "p.i32")
    np.asarray(prompt, np.int32).tofile(pp)
    r = subprocess.run([REF_DECODE, path, "1", "0", str(n_out), pp], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, **env))
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])["tokens"]


def ref_positions(path, prompt, split, tmp, vocab):
    lp = str(tmp / "pos.f32")
    ref(path, prompt, 1, tmp, {"REF_POSITIONS": lp, "REF_POSITIONS_SPLIT": str(split)})
    return np.fromfile(lp, np.float32).reshape(len(prompt) - split, vocab)


MODELS = {
    "w4a8_int8kv": dict(kv_bits=8),
    "fp32kv": dict(kv_bits=32),
    "int4kv": dict(kv_bits=4),
    "mlp_int2": dict(kv_bits=8, bits=dict(gate_proj=2, up_proj=2, down_proj=2)),
    "all_int8": dict(kv_bits=8, bits=dict(o_proj=8, gate_proj=8, up_proj=8, down_proj=8)),
    "int4_head": dict(kv_bits=8, bits=dict(token_embedding=4, head=4)),
}


def write(tmp, name, seed=13, **over):
    from libinferbit_amd import ibf
    spec = dict(MODELS[name])
    bits = spec.pop("bits", None)
    spec.update(over)
    path = str(tmp / f"{name}.ibf")
    ibf.write_synthetic(path, cfg(**spec), seed=seed, bits=bits)
    return path


@pytest.mark.parametrize("name", list(MODELS))
@pytest.mark.parametrize("split", [0, 5])
def test_forward_positions_bit_exact(L, tmp_path, name, split):
    from libinferbit_amd.model import Model
    print(f"case forward_positions {name} split={split}", flush=True)
    path = write(tmp_path, name)
    prompt = [5, 17, 300, 42, 999, 0, 7, 7, 123, 64, 2, 500, 11]
    want = ref_positions(path, prompt, split, tmp_path, 1000)
    m = Model(path)
    if split:
        m.forward(prompt[:split])
    got = m.forward_positions(prompt[split:])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert m.kv_length() == len(prompt)
    m.set_exact(False)
    m.kv_clear()
    if split:
        m.forward(prompt[:split])
    fast = m.forward_positions(prompt[split:])
    rows = np.abs(fast.astype(np.float64) - want).max(1) / np.abs(want).max()
    if uses_w4a8(name):
        # W4A8 quantizes activations to int8: an fp32 difference of one ulp
        # can move a code by one step, which moves a logit of this 256-wide
        # model by up to ~1 % (the reference's own batch and single paths
        # differ that way on some positions), and later positions inherit
        # the change through the cache.  Bound: 3e-2, with the first
        # position at fp32 level.
        assert rows[0] <= 1e-4 and rows.max() <= 3e-2, rows
    else:
        assert rows.max() <= 1e-4, rows
    m.close()


def uses_w4a8(name):
    bits = dict(MODELS[name].get("bits") or {})
    mlp4 = all(bits.get(k, 4) == 4 for k in ("gate_proj", "up_proj", "down_proj"))
    return mlp4 or bits.get("head") == 4 or bits.get("o_proj") == 4


def test_forward_positions_limits(L, tmp_path):
    from libinferbit_amd import IbhError
    from libinferbit_amd.model import Model
    m = Model(write(tmp_path, "w4a8_int8kv", max_context_length=40))
    with pytest.raises(IbhError):
        m.forward_positions(list(range(33)))          # > IB_BATCH_MAX
    with pytest.raises(IbhError):
        m.forward_positions([1, 1000])                # token out of range
    m.forward_positions(list(range(32)))
    with pytest.raises(IbhError):
        m.forward_positions(list(range(9)))           # context exceeded
    assert m.kv_length() == 32
    m.close()


@pytest.mark.parametrize("name", ["w4a8_int8kv", "all_int8", "int4kv"])
@pytest.mark.parametrize("ngram,k", [(2, 4), (1, 8), (3, 2)])
def test_prompt_lookup_tokens_match_reference(L, tmp_path, name, ngram, k):
    from libinferbit_amd.model import Model
    print(f"case lookup {name} ngram={ngram} k={k}", flush=True)
    path = write(tmp_path, name, seed=21)
    prompt = [5, 17, 300, 42, 5, 17, 300, 42, 5, 17, 9, 8, 5, 17]
    want = ref(path, prompt, 60, tmp_path, {"REF_LOOKUP": f"{ngram},{k}"})
    m = Model(path)
    got = m.generate_lookup(prompt, 60, ngram, k)
    assert got.tolist() == want
    m.close()


@pytest.mark.parametrize("draft_k", [1, 4, 7])
def test_draft_model_tokens_match_reference(L, tmp_path, draft_k):
    from libinferbit_amd import ibf
    from libinferbit_amd.model import Model
    print(f"case draft k={draft_k}", flush=True)
    main = write(tmp_path, "w4a8_int8kv", seed=31)
    dpath = str(tmp_path / "draft.ibf")
    ibf.write_synthetic(dpath, cfg(num_layers=1, kv_bits=8), seed=31)   # same embeddings/head seed family
    prompt = [3, 14, 15, 92, 65, 35, 89, 79]
    want = ref(main, prompt, 50, tmp_path, {"REF_DRAFT": dpath, "REF_DRAFT_K": str(draft_k)})
    m, d = Model(main), Model(dpath)
    got = m.generate_draft(d, prompt, 50, draft_k)
    assert got.tolist() == want
    m.close()
    d.close()


SAMPLING = [(0.8, 40, 0.9, 1.0, 7), (1.0, 0, 1.0, 1.3, 123), (1.5, 5, 0.5, 1.1, 0), (0.3, 1000, 0.95, 1.0, 99)]


@pytest.mark.parametrize("name", ["w4a8_int8kv", "all_int8"])
@pytest.mark.parametrize("temp,top_k,top_p,pen,seed", SAMPLING)
def test_sampled_tokens_match_reference(L, tmp_path, name, temp, top_k, top_p, pen, seed):
    """inferbit_generate with sampling: same seed, same token stream (exact
    mode gives the CPU's logits bit for bit; sampling runs the reference's
    rules on the host)."""
    from libinferbit_amd.model import Model
    print(f"case sampled {name} T={temp} k={top_k} p={top_p} pen={pen} seed={seed}", flush=True)
    path = write(tmp_path, name, seed=17)
    prompt = [5, 17, 300, 42, 999, 0, 7]
    want = ref(path, prompt, 48, tmp_path, {"REF_SAMPLE": f"{temp},{top_k},{top_p},{pen},{seed}"})
    m = Model(path)
    got = m.generate_sampled(prompt, 48, temp, top_k, top_p, pen, seed)
    assert got.tolist() == want
    m.close()


def test_forward_positions_graph_equals_eager(L, tmp_path, monkeypatch):
    """The captured per-B graph gives the eager launches' logits, call after
    call, at different cache lengths, in both modes."""
    from libinferbit_amd.model import Model
    path = write(tmp_path, "w4a8_int8kv", seed=3)
    for exact in (True, False):
        monkeypatch.delenv("IBH_DECODE_EAGER", raising=False)
        g = Model(path)
        g.set_exact(exact)
        monkeypatch.setenv("IBH_DECODE_EAGER", "1")
        e = Model(path)
        e.set_exact(exact)
        for chunk in ([5, 6, 7, 8], [9, 10, 11, 12], [1, 2], [3, 4, 5, 6]):
            np.testing.assert_array_equal(g.forward_positions(chunk), e.forward_positions(chunk))
        g.close()
        e.close()
