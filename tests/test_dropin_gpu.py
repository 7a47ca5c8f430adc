"""The drop-in boundary: libibhip.so's table entries swapped into the
reference's own `ib_kern` table, driven by the reference's own host code.

* `oracle/_ref/dropin` (test infrastructure, oracle/dropin.c) runs the
  reference library's inferbit_load / inferbit_forward / inferbit_generate
  (compiled from the reference sources) on its x86 table, then again after
  ib_init_kernels_hip + ibh_register_host_weights, exactly as the patch in
  INTEGRATION.md section 1 does.  The last-token logits must be identical bit
  for bit and the greedy token streams equal.
* The table entries themselves, called through ctypes with HOST pointers the
  way forward.c calls them (src/forward.c:144-246): weights resident
  (registered) and staged (not registered), row-slice pointers inside the
  registered region as ib_parallel_* pass them (src/threading.c:220-242), and
  M_stride > M with the rows outside the slice left untouched.  Each result
  equals the reference's own x86 table entry (oracle/_ref, AVX2 level) bit for
  bit.
"""
import ctypes as C
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, ROOT

pytestmark = pytest.mark.gpu

DROPIN = os.path.join(ROOT, "oracle", "_ref", "dropin")
DROPIN_ATTN = os.path.join(ROOT, "oracle", "_ref", "dropin_attn")
MODEL_DIR = os.environ.get("IBH_MODEL_DIR", "/tmp/ibh_models")


@pytest.fixture(scope="module")
def L():
    import libinferbit_amd as L
    L.ops.init(0)
    return L


@pytest.fixture(scope="module")
def R():
    from oracle import refbind as R
    if not R.available():
        pytest.skip("oracle/_ref not built (make -C oracle ref)")
    return R


def run_dropin(path, prompt, n_out, tmp, cpu_threads=4, ctx=0, exe=DROPIN, env=None):
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (make -C oracle ref)")
    pp = str(tmp / "p.i32")
    np.asarray(prompt, np.int32).tofile(pp)
    r = subprocess.run([exe, path, str(ctx), str(n_out), pp, str(cpu_threads)], capture_output=True, text=True,
                       timeout=600, env=dict(os.environ, **(env or {})))
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


def tiny_cfg(**kw):
    from libinferbit_amd import ibf
    c = dict(ibf.TINYLLAMA, num_layers=2, hidden_size=256, num_heads=4, num_kv_heads=2, head_dim=64,
             intermediate_size=512, vocab_size=1000, max_context_length=160)
    c.update(kw)
    return c


TINY = {
    "fp32kv": dict(kv_bits=32),
    "int8kv": dict(kv_bits=8),
    "mlp_int2": dict(kv_bits=8, bits=dict(gate_proj=2, up_proj=2, down_proj=2, o_proj=8)),
    "all_int8": dict(kv_bits=8, bits=dict(o_proj=8, gate_proj=8, up_proj=8, down_proj=8)),
    "int4_emb_head": dict(kv_bits=8, bits=dict(token_embedding=4, head=4)),
    "wide": dict(kv_bits=32, num_layers=3, hidden_size=1024, num_heads=16, num_kv_heads=4, intermediate_size=2816),
}


@pytest.mark.parametrize("name", list(TINY))
def test_reference_generate_on_gpu_table(tmp_path, name):
    from libinferbit_amd import ibf
    spec = dict(TINY[name])
    bits = spec.pop("bits", None)
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(**spec), seed=21, bits=bits)
    prompt = [3, 17, 200, 45, 999, 1, 0, 512, 77, 640, 12, 5]
    print(f"case dropin {name}", flush=True)
    r = run_dropin(path, prompt, 40, tmp_path)
    assert r["gpu_table"] == 1 and r["logits_nan"] == 0
    assert r["logits_same_bits"] == r["vocab"], r
    assert r["tokens_equal"] == 1, (r["tokens_cpu"], r["tokens_gpu"])


@pytest.mark.timeout(900)
def test_reference_generate_tinyllama_config(tmp_path):
    """Config 3 (TinyLlama shape, 32-token prompt, 256 greedy tokens) through
    the reference's inferbit_generate on the GPU table: the stream must equal
    the one the reference recorded on its own x86 table
    (tests/golden/decode.json)."""
    import sys
    sys.path.insert(0, GOLDEN)
    import gen_decode_golden as G
    g = json.load(open(os.path.join(GOLDEN, "decode.json")))["tinyllama"]
    os.makedirs(MODEL_DIR, exist_ok=True)
    print("case dropin tinyllama: writing model", flush=True)
    path = G.ensure_model("tinyllama", MODEL_DIR)
    print("case dropin tinyllama: generating", flush=True)
    r = run_dropin(path, g["prompt"], g["n_out"], tmp_path, cpu_threads=0)
    assert r["logits_nan"] == 0
    assert r["tokens_gpu"] == g["tokens"]
    print(f"dropin tinyllama: {g['n_out'] / r['gpu_seconds']:.1f} tok/s through the reference host loop", flush=True)


ATTN = {
    "fp32kv": dict(kv_bits=32),
    "int8kv": dict(kv_bits=8),
    "int4kv": dict(kv_bits=4),
    "hd128": dict(kv_bits=8, hidden_size=512, num_heads=4, num_kv_heads=1, head_dim=128, intermediate_size=1024),
}


@pytest.mark.parametrize("lookup", [None, "2,4"])
@pytest.mark.parametrize("name", list(ATTN))
def test_reference_generate_with_device_attention(tmp_path, name, lookup):
    """The reference's forward.c with its head loops offered to ibh_host_attn
    (the device KV mirror): every attention step of the GPU pass runs on the
    device, none falls back, and logits and tokens equal the x86 run.  With
    prompt-lookup speculation the reference verifies drafts in forward_batch
    and rewinds with inferbit_kv_truncate, which the mirror follows."""
    from libinferbit_amd import ibf
    path = str(tmp_path / "m.ibf")
    ibf.write_synthetic(path, tiny_cfg(**ATTN[name]), seed=23)
    prompt = [7, 7, 100, 7, 7, 100, 250, 3, 7, 7, 100, 9]
    print(f"case dropin_attn {name} lookup={lookup}", flush=True)
    r = run_dropin(path, prompt, 48, tmp_path, exe=DROPIN_ATTN, env={"DROPIN_LOOKUP": lookup} if lookup else None)
    assert r["attn_calls"] > 0 and r["attn_fallbacks"] == 0, r
    assert r["logits_same_bits"] == r["vocab"], r
    assert r["tokens_equal"] == 1, (r["tokens_cpu"], r["tokens_gpu"])


def test_host_attn_rejects_bad_arguments(L):
    q = np.zeros(64, np.float32)
    k = np.zeros((4, 64), np.float32)
    assert L.lib().ibh_host_attn(_p(k), _p(k), _p(k), None, None, 4, 4, 32, _p(q), _p(q), 1, 1, 64) != 0
    assert L.lib().ibh_host_attn(_p(k), _p(k), _p(k), None, None, 4, 0, 8, _p(q), _p(q), 1, 1, 64) != 0
    assert L.lib().ibh_last_error()


# ── the table entries, host pointers ─────────────────────────────────────────

def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.fixture(scope="module")
def tabs(L, R):
    cpu = R.kernels(R.IB_SIMD_AVX2)
    gpu = R.IbKernels()
    C.pointer(gpu)[0] = cpu
    L.lib().ib_init_kernels_hip(C.byref(gpu))
    return cpu, gpu


@pytest.fixture(scope="module")
def blob(L, R):
    """A registered host region holding INT8/INT4/INT2 matrices back to back."""
    rng = np.random.default_rng(99)
    mats = {}
    parts = []
    off = 0
    for bits, (M, N) in [(8, (300, 1024)), (4, (520, 2048)), (2, (260, 1024))]:
        W = (rng.standard_normal((M, N)) * 0.02).astype(np.float32)
        w, s = R.quantize(bits, W)
        mats[bits] = (off, w.shape, s.view(np.float16).astype(np.float32), N)
        b = np.ascontiguousarray(w).view(np.uint8).ravel()
        parts.append(b)
        off += b.size + (-b.size) % 64
        parts.append(np.zeros((-b.size) % 64, np.uint8))
    host = np.ascontiguousarray(np.concatenate(parts))
    dev = C.c_void_p()
    assert L.lib().ibh_register_host_weights(_p(host), host.size, C.byref(dev)) == 0
    yield host, mats
    L.lib().ibh_unregister_host_weights(_p(host))


def _mat(host, mats, bits):
    off, shape, sc, N = mats[bits]
    w = np.ndarray(shape, np.int8 if bits == 8 else np.uint8, buffer=host, offset=off)
    return w, sc, N


def _same(a, b):
    np.testing.assert_array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("where", ["resident", "staged", "slice"])
def test_table_matmul_entries(tabs, blob, bits, where):
    cpu, gpu = tabs
    host, mats = blob
    w, sc, N = _mat(host, mats, bits)
    if where == "staged":
        w = w.copy()                       # outside the registered region: uploaded per call
    r0, r1 = (0, w.shape[0]) if where != "slice" else (37, 37 + 101)   # a pool worker's row slice
    x = np.random.default_rng(bits).standard_normal(N).astype(np.float32)
    wr, sr = w[r0:r1], np.ascontiguousarray(sc[r0:r1])
    yc, yg = np.zeros(r1 - r0, np.float32), np.zeros(r1 - r0, np.float32)
    name = f"matmul_int{bits}"
    getattr(cpu, name)(_p(yc), _p(wr), _p(sr), _p(x), r1 - r0, N)
    getattr(gpu, name)(_p(yg), _p(wr), _p(sr), _p(x), r1 - r0, N)
    _same(yg, yc)


@pytest.mark.parametrize("where", ["resident", "staged", "slice"])
def test_table_w4a8_entries(tabs, blob, R, where):
    cpu, gpu = tabs
    host, mats = blob
    w, sw, N = _mat(host, mats, 4)
    if where == "staged":
        w = w.copy()
    r0, r1 = (0, w.shape[0]) if where != "slice" else (64, 64 + 200)
    wr, sr = w[r0:r1], np.ascontiguousarray(sw[r0:r1])
    M = r1 - r0
    x = np.random.default_rng(5).standard_normal(N).astype(np.float32)
    qx, sa = R.quantize_act(x)
    yc, yg = np.zeros(M, np.float32), np.zeros(M, np.float32)
    cpu.matmul_w4a8(_p(yc), _p(wr), _p(sr), _p(qx), _p(sa), M, N)
    gpu.matmul_w4a8(_p(yg), _p(wr), _p(sr), _p(qx), _p(sa), M, N)
    _same(yg, yc)
    # batched entry: B = 3 positions, output rows strided by M_stride > M;
    # rows outside the slice keep their sentinel value
    B, M_stride = 3, M + 17
    X = np.random.default_rng(6).standard_normal((B, N)).astype(np.float32)
    Q = np.zeros((B, N), np.int8)
    S = np.zeros((B, (N + 127) // 128), np.float32)
    for b in range(B):
        Q[b], S[b] = R.quantize_act(X[b])
    oc = np.full(B * M_stride, 7.25, np.float32)
    og = oc.copy()
    cpu.matmul_w4a8_batch(_p(oc), _p(wr), _p(sr), _p(Q), _p(S), M, N, B, M_stride)
    gpu.matmul_w4a8_batch(_p(og), _p(wr), _p(sr), _p(Q), _p(S), M, N, B, M_stride)
    _same(og, oc)
    assert np.all(og.reshape(B, M_stride)[:, M:] == 7.25)


@pytest.mark.parametrize("where", ["resident", "staged", "slice"])
def test_table_int8_batch_entry(tabs, blob, where):
    cpu, gpu = tabs
    host, mats = blob
    w, sc, N = _mat(host, mats, 8)
    if where == "staged":
        w = w.copy()
    r0, r1 = (0, w.shape[0]) if where != "slice" else (100, 180)
    wr, sr = w[r0:r1], np.ascontiguousarray(sc[r0:r1])
    M, B, M_stride = r1 - r0, 5, (r1 - r0) + 3
    X = np.random.default_rng(8).standard_normal((B, N)).astype(np.float32)
    oc = np.full(B * M_stride, -3.5, np.float32)
    og = oc.copy()
    cpu.matmul_int8_batch(_p(oc), _p(wr), _p(sr), _p(X), M, N, B, M_stride)
    gpu.matmul_int8_batch(_p(og), _p(wr), _p(sr), _p(X), M, N, B, M_stride)
    _same(og, oc)
    assert np.all(og.reshape(B, M_stride)[:, M:] == -3.5)


def test_unregister_releases_and_restages(L, tabs, R):
    """After ibh_unregister_host_weights the same host pointer is served by
    the staged path (fresh upload per call) and still gives the same result."""
    cpu, gpu = tabs
    rng = np.random.default_rng(12)
    w, s = R.quantize(8, (rng.standard_normal((64, 512)) * 0.02).astype(np.float32))
    sc = s.view(np.float16).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    dev = C.c_void_p()
    assert L.lib().ibh_register_host_weights(_p(w), w.nbytes, C.byref(dev)) == 0
    y1 = np.zeros(64, np.float32)
    gpu.matmul_int8(_p(y1), _p(w), _p(sc), _p(x), 64, 512)
    L.lib().ibh_unregister_host_weights(_p(w))
    w[:] = -w                                   # the device copy is gone: a stale one would show
    y2, yc = np.zeros(64, np.float32), np.zeros(64, np.float32)
    gpu.matmul_int8(_p(y2), _p(w), _p(sc), _p(x), 64, 512)
    cpu.matmul_int8(_p(yc), _p(w), _p(sc), _p(x), 64, 512)
    _same(y2, yc)
    assert np.all(np.sign(y1[y1 != 0]) == -np.sign(y2[y1 != 0]))


@pytest.mark.timeout(900)
def test_reference_generate_mistral_config_with_device_attention(tmp_path):
    """Config 4 through the reference's own host loop: Mistral-7B shape, INT8
    KV prefilled to 4096 positions by forward.c's kv_cache_write, then greedy
    steps whose matvecs run on the GPU table and whose head loops
    (src/forward.c:596-614) go to ibh_host_attn (head_dim 128, T = 4097 ...).
    The tokens must be the prefix of the stream the reference recorded on its
    own x86 table (tests/golden/decode.json), every attention step on the
    device."""
    import sys
    sys.path.insert(0, GOLDEN)
    import gen_decode_golden as G
    g = json.load(open(os.path.join(GOLDEN, "decode.json")))["mistral"]
    n_out = 8
    os.makedirs(MODEL_DIR, exist_ok=True)
    print("case dropin_attn mistral: writing model and KV", flush=True)
    path = G.ensure_model("mistral", MODEL_DIR)
    case = G.CASES["mistral"]
    kp = str(tmp_path / "kv.f32")
    k, v = G.kv_of(case)
    with open(kp, "wb") as f:
        f.write(k.tobytes())
        f.write(v.tobytes())
    del k, v
    print("case dropin_attn mistral: generating", flush=True)
    if not os.path.exists(DROPIN_ATTN):
        pytest.skip(f"{DROPIN_ATTN} not built (make -C oracle ref)")
    pp = str(tmp_path / "p.i32")
    np.asarray(g["prompt"], np.int32).tofile(pp)
    r = subprocess.run([DROPIN_ATTN, path, "0", str(n_out), pp, "0", "0", kp, str(g["kv_pos"])],
                       capture_output=True, text=True, timeout=800)
    assert r.returncode == 0, r.stderr
    r = json.loads(r.stdout.strip().splitlines()[-1])
    assert r["logits_nan"] == 0
    assert r["attn_calls"] > 0 and r["attn_fallbacks"] == 0, r
    assert r["tokens_gpu"] == g["tokens"][:n_out]
    print(f"dropin_attn mistral: {n_out / r['gpu_seconds']:.2f} tok/s through the reference host loop", flush=True)
