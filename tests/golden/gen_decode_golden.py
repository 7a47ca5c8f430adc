"""Writes tests/golden/decode.json: greedy token streams of the REFERENCE
library (oracle/_ref/ref_decode, built by `make -C oracle ref`) on the
synthetic decoders of the benchmark configurations.

The models are not stored: libinferbit_amd.ibf.write_synthetic regenerates
them byte for byte from (config, seed), and the fixture keeps each file's
SHA-256 so a test can tell it decodes the same bytes.  Run from the repo
root:  python tests/golden/gen_decode_golden.py [name ...]

  tinyllama  TinyLlama-1.1B shape, fp32 KV, 32 seeded prompt ids, 256 tokens
  mistral    Mistral-7B shape, INT8 KV prefilled with 4096 positions of
             N(0,1) K/V (kv_cache_write quantisation), then 128 tokens
"""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from libinferbit_amd import ibf  # noqa: E402

CASES = {
    "tinyllama": dict(cfg=ibf.TINYLLAMA, seed=1, n_prompt=32, n_out=256, kv_pos=0),
    "mistral": dict(cfg=ibf.MISTRAL, seed=2, n_prompt=1, n_out=128, kv_pos=4096),
}


def prompt_of(case):
    return np.random.default_rng(case["seed"]).integers(0, case["cfg"]["vocab_size"], case["n_prompt"]).astype(
        np.int32)


def kv_of(case):
    """K and V [layers][kv_pos][kv_dim] as N(0,1) streams of the library generator."""
    c = case["cfg"]
    n = c["num_layers"] * case["kv_pos"] * c["num_kv_heads"] * c["head_dim"]
    shape = (c["num_layers"], case["kv_pos"], c["num_kv_heads"] * c["head_dim"])
    return (ibf.fill_normal(n, ibf.tensor_seed(case["seed"], "kv.k")).reshape(shape),
            ibf.fill_normal(n, ibf.tensor_seed(case["seed"], "kv.v")).reshape(shape))


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(1 << 24)
            if not b:
                return h.hexdigest()
            h.update(b)


def model_path(name, workdir):
    return os.path.join(workdir, f"synthetic_{name}.ibf")


def ensure_model(name, workdir):
    p = model_path(name, workdir)
    if not os.path.exists(p):
        case = CASES[name]
        ibf.write_synthetic(p + ".tmp", case["cfg"], seed=case["seed"])
        os.replace(p + ".tmp", p)
    return p


def run_reference(name, workdir, threads):
    case = CASES[name]
    path = ensure_model(name, workdir)
    pp = os.path.join(workdir, f"{name}_prompt.i32")
    prompt_of(case).tofile(pp)
    cmd = [os.path.join(ROOT, "oracle", "_ref", "ref_decode"), path, str(threads), "0", str(case["n_out"]), pp]
    if case["kv_pos"]:
        kp = os.path.join(workdir, f"{name}_kv.f32")
        k, v = kv_of(case)
        with open(kp, "wb") as f:
            f.write(k.tobytes())
            f.write(v.tobytes())
        del k, v
        cmd += [kp, str(case["kv_pos"])]
    t = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True, check=True)
    out = json.loads(r.stdout.strip().splitlines()[-1])
    out["wall_s"] = time.time() - t
    return out, sha256(path)


def main():
    names = sys.argv[1:] or list(CASES)
    workdir = os.environ.get("IBH_MODEL_DIR", "/tmp/ibh_models")
    os.makedirs(workdir, exist_ok=True)
    dst = os.path.join(HERE, "decode.json")
    data = json.load(open(dst)) if os.path.exists(dst) else {}
    for name in names:
        case = CASES[name]
        out, digest = run_reference(name, workdir, os.cpu_count() or 1)
        data[name] = {"config": case["cfg"], "seed": case["seed"], "prompt": prompt_of(case).tolist(),
                      "kv_pos": case["kv_pos"], "n_out": case["n_out"], "model_sha256": digest,
                      "tokens": out["tokens"], "cpu_seconds": out["seconds"], "cpu_threads": out["threads"]}
        json.dump(data, open(dst, "w"), indent=1)
        print(name, out["n"], "tokens", f"{out['seconds']:.1f}s", flush=True)


if __name__ == "__main__":
    main()
