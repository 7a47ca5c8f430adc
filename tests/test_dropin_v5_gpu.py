"""The IBF v5 session drop-in: the reference's own PQ session code
(oracle/_ref/dropin_v5, test infrastructure, oracle/dropin_v5.c) with the
INT4 and PQ branches of ib_pq_session_matmul (src/pq_decode.c:4437-4491) and
session_matmul_with_scratch (:4389-4435) served by ibh_int4g_matmul_host /
ibh_pq_matmul_policy_host on the session's own host tensors -- the lines the
integration patch adds.  ib_pq_generate_greedy (:5297-5346) runs once on the
x86 session and once with the hooks on: the greedy streams must be equal, every
hooked call served by the GPU (no fallback)."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

DROPIN_V5 = os.path.join(ROOT, "oracle", "_ref", "dropin_v5")
CFG = dict(num_layers=2, hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64, intermediate_size=512,
           vocab_size=1000)
ALLPQ = {p: "pq" for p in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")}
CASES = {
    "int4": (CFG, dict()),
    "int4_awq_outl": (CFG, dict(awq=True, outliers=3)),
    "mixed": (CFG, dict(backend=dict(gate_proj="pq", up_proj="pq", down_proj="pq", o_proj="fp16"), awq=True)),
    "pq_l2_actscale": (CFG, dict(backend=ALLPQ, levels=2, pq_act_scale=True)),
    "pq_outl_k16": (CFG, dict(backend=ALLPQ, levels=2, k2=16, pq_outliers=16, embed="f32")),
    "tinyllama_width": (dict(CFG, num_layers=2, hidden_size=2048, num_heads=32, num_kv_heads=4,
                             intermediate_size=5632, vocab_size=32000), dict(awq=True)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_reference_session_generate_on_gpu_matvecs(tmp_path, name):
    from libinferbit_amd import ibf5
    if not os.path.exists(DROPIN_V5):
        pytest.skip(f"{DROPIN_V5} not built (make -C oracle ref)")
    cfg, kw = CASES[name]
    path = str(tmp_path / f"{name}.ibf")
    ibf5.write_synthetic_v5(path, cfg, seed=5, **kw)
    prompt = [5, 17, 300, 42, 7, 99, 3]
    pp = str(tmp_path / "p.i32")
    np.asarray(prompt, np.int32).tofile(pp)
    print(f"case dropin_v5 {name}", flush=True)
    r = subprocess.run([DROPIN_V5, path, "64", "24", pp], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    r = json.loads(r.stdout.strip().splitlines()[-1])
    assert r["fallbacks"] == 0, r
    assert r["int4_calls"] + r["pq_calls"] > 0, r
    if kw.get("backend") is ALLPQ:
        assert r["int4_calls"] == 0 and r["pq_calls"] > 0
    assert r["tokens_equal"] == 1, (r["tokens_cpu"], r["tokens_gpu"])
