"""The PQ twin with the reference's own interface: ibh_pq_matmul_fp32_host
takes the ib_pq_tensor that the reference's loader filled
(ib_pq_load_single, src/pq_decode.c:726-744) by pointer, as
ib_pq_matmul_fp32 (src/pq_decode.h:197) does, and must agree with it:
max|y_gpu - y_cpu| / max|y_cpu| <= 1e-4 (fp32 accumulate, other order)."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import load_golden, pq_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    import libinferbit_amd as L
    L.ops.init(0)
    return L


@pytest.fixture(scope="module")
def ref():
    from oracle import refbind
    if not refbind.available():
        pytest.skip("reference library not built")
    return refbind


def relerr(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def write_single(path, t, **kw):
    from libinferbit_amd.ibf5 import V5Writer
    w = V5Writer({})
    w.pq_tensor("w", t, **kw)
    w.write(path)


def twin(L, s, x):
    out = np.full(s.M, np.nan, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rc = L._lib.lib().ibh_pq_matmul_fp32_host(C.byref(s), x.ctypes.data, out.ctypes.data)
    assert rc == 0, L._lib.lib().ibh_last_error()
    return out


CASES = ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40"]


@pytest.mark.parametrize("name", CASES)
def test_twin_on_reference_loaded_tensor(L, ref, tmp_path, name):
    print(f"case pq host twin {name}", flush=True)
    t = pq_case(load_golden("pq.npz"), name)
    p = str(tmp_path / f"{name}.ibf")
    write_single(p, t, rotate=(name == "l1"))
    s = ref.pq_load_single(p)
    try:
        for x in (t["x"], t["xs"]):
            y = twin(L, s, x)
            assert relerr(y, ref.pq_matmul_struct(s, x)) <= 1e-4
        # second call: the cached device copy
        y2 = twin(L, s, t["x"])
        assert relerr(y2, ref.pq_matmul_struct(s, t["x"])) <= 1e-4
    finally:
        L._lib.lib().ibh_pq_host_release(C.byref(s))
        ref.pq_free(s)


def test_twin_bit_packed_pyramid(L, ref, tmp_path):
    """Pyramid tensor whose level-2 indices are 9-bit packed on disk: the
    loader's uint16 unpack in RAM is what the twin uploads."""
    from gen_golden import make_pq
    t = make_pq(np.random.default_rng(7), 96, 24, 16, 256, 2, 512, 0, 2)
    p = str(tmp_path / "pk.ibf")
    write_single(p, t, l2_packed_bits=9)
    s = ref.pq_load_single(p)
    try:
        assert s.l2_packed_bits == 9 and s.l2_idx_bytes == 2
        x = np.random.default_rng(8).standard_normal(t["N"]).astype(np.float32)
        assert relerr(twin(L, s, x), ref.pq_matmul_struct(s, x)) <= 1e-4
    finally:
        L._lib.lib().ibh_pq_host_release(C.byref(s))
        ref.pq_free(s)


@pytest.mark.parametrize("heavy", [False, True])
def test_twin_config5_shape(L, ref, tmp_path, heavy):
    """BASELINE config 5 (M=4096, N=14336, G=16, K=256, one level) through the
    reference's loader, x N(0,1) and heavy-tailed (Student t, 1.5 dof)."""
    from gen_golden import make_pq
    rng = np.random.default_rng(55)
    t = make_pq(rng, 4096, 896, 16, 256, 1, 0, 0)
    p = str(tmp_path / "c5.ibf")
    write_single(p, t)
    s = ref.pq_load_single(p)
    try:
        x = (rng.standard_t(1.5, t["N"]) if heavy else rng.standard_normal(t["N"])).astype(np.float32)
        assert relerr(twin(L, s, x), ref.pq_matmul_struct(s, x)) <= 1e-4
    finally:
        L._lib.lib().ibh_pq_host_release(C.byref(s))
        ref.pq_free(s)


def test_twin_detects_reloaded_tensor(L, ref, tmp_path):
    """A tensor freed and another loaded (possibly at the same addresses)
    without ibh_pq_host_release: the fingerprint forces a fresh upload."""
    from gen_golden import make_pq
    ya = []
    for seed in (1, 2):
        t = make_pq(np.random.default_rng(seed), 64, 16, 16, 256, 1, 0, 0)
        p = str(tmp_path / f"r{seed}.ibf")
        write_single(p, t)
        s = ref.pq_load_single(p)
        x = np.random.default_rng(9).standard_normal(t["N"]).astype(np.float32)
        y = twin(L, s, x)
        assert relerr(y, ref.pq_matmul_struct(s, x)) <= 1e-4
        ya.append(y)
        ref.pq_free(s)
    assert not np.array_equal(ya[0], ya[1])


def test_twin_uses_registered_region(L, ref, tmp_path):
    """Arrays inside a region registered with ibh_register_host_weights are
    served from that device copy (the mmap case): a tensor whose arrays all
    sit in one host buffer, registered first."""
    from gen_golden import make_pq
    t = make_pq(np.random.default_rng(3), 128, 32, 16, 256, 1, 0, 8)
    keys = ["cb1l", "cb1r", "i1l", "i1r", "row_scale", "ocols", "oside", "oscale"]
    blob = np.zeros(sum((np.asarray(t[k]).nbytes + 63) // 64 * 64 for k in keys), np.uint8)
    offs, o = {}, 0
    for k in keys:
        b = np.ascontiguousarray(t[k]).view(np.uint8).reshape(-1)
        blob[o:o + b.size] = b
        offs[k] = o
        o += (b.size + 63) // 64 * 64
    base = blob.ctypes.data
    lib = L._lib.lib()
    dev = C.c_void_p()
    assert lib.ibh_register_host_weights(C.c_void_p(base), blob.nbytes, C.byref(dev)) == 0
    try:
        s = ref.IbPqTensor()
        for n in ("M", "N", "G", "K", "n_levels", "n_outlier", "C"):
            setattr(s, n, int(t[n]))
        s.l2_idx_bytes = 1
        s.format = 1
        m = {"cb1l": "codebook_l1_l", "cb1r": "codebook_l1_r", "i1l": "indices_l1_l", "i1r": "indices_l1_r",
             "row_scale": "row_scale", "ocols": "outlier_cols", "oside": "outlier_sidecar", "oscale": "outlier_scale"}
        for k, f in m.items():
            setattr(s, f, base + offs[k])
        x = np.random.default_rng(4).standard_normal(t["N"]).astype(np.float32)
        assert relerr(twin(L, s, x), ref.pq_matmul_struct(s, x)) <= 1e-4
        lib.ibh_pq_host_release(C.byref(s))
    finally:
        lib.ibh_unregister_host_weights(C.c_void_p(base))


def test_twin_rejects_bad_tensor(L):
    from oracle.refbind import IbPqTensor
    s = IbPqTensor()
    out = np.zeros(4, np.float32)
    x = np.zeros(4, np.float32)
    assert L._lib.lib().ibh_pq_matmul_fp32_host(C.byref(s), x.ctypes.data, out.ctypes.data) == -1
    assert L._lib.lib().ibh_last_error()
