"""The IBF v5 writer against the reference's own loader (CPU): a single PQ
tensor written by libinferbit_amd.ibf5.V5Writer and read back by
ib_pq_load_single (src/pq_decode.c:726-744) has the shape, flags and arrays
that were written, including level-2 indices stored bit-packed, which the
loader unpacks to uint16 (src/pq_decode.c:504-528, pq_unpack_bits_to_u16)."""
import ctypes as C

import numpy as np
import pytest


@pytest.fixture(scope="module")
def ref():
    from oracle import refbind
    if not refbind.available():
        pytest.skip("reference library not built")
    return refbind


def arr(p, n, dt):
    return np.ctypeslib.as_array(C.cast(p, C.POINTER(dt)), (n,)).copy()


@pytest.mark.parametrize("bits", [0, 9, 10, 16])
def test_pyramid_roundtrip(ref, tmp_path, bits):
    from gen_golden import make_pq
    from libinferbit_amd.ibf5 import V5Writer
    K2 = 512 if bits != 16 else 1024
    t = make_pq(np.random.default_rng(bits), 21, 13, 16, 256, 2, K2, 0, 2)
    w = V5Writer({})
    w.pq_tensor("w", t, rotate=True, l2_packed_bits=bits)
    p = str(tmp_path / "t.ibf")
    w.write(p)
    s = ref.pq_load_single(p)
    try:
        assert (s.M, s.N, s.G, s.K, s.K_l2, s.n_levels, s.C) == (21, 13 * 16, 16, 256, K2, 2, 13)
        assert s.rotate == 1 and s.format == 4 and s.l2_idx_bytes == 2 and s.l2_packed_bits == bits
        n = 21 * 13
        np.testing.assert_array_equal(arr(s.indices_l2_l, n, C.c_uint16), t["i2l"].view(np.uint16).reshape(-1))
        np.testing.assert_array_equal(arr(s.indices_l2_r, n, C.c_uint16), t["i2r"].view(np.uint16).reshape(-1))
        np.testing.assert_array_equal(arr(s.indices_l1_l, n, C.c_uint8), t["i1l"].reshape(-1))
        np.testing.assert_array_equal(arr(s.codebook_l2_r, K2 * 8, C.c_uint16), t["cb2r"].reshape(-1))
    finally:
        ref.pq_free(s)


@pytest.mark.parametrize("name", ["l1", "l2p16", "l2u8", "l2u16", "out8", "out40"])
def test_golden_cases_load_and_multiply(ref, tmp_path, name):
    """Every PQ golden case written as a v5 file loads through the reference
    loader, and its ib_pq_matmul_fp32 equals the golden output the reference
    wrote from the in-memory tensor."""
    from conftest import load_golden, pq_case
    from libinferbit_amd.ibf5 import V5Writer
    t = pq_case(load_golden("pq.npz"), name)
    w = V5Writer({})
    w.pq_tensor("w", t)
    p = str(tmp_path / "t.ibf")
    w.write(p)
    s = ref.pq_load_single(p)
    try:
        np.testing.assert_array_equal(ref.pq_matmul_struct(s, t["x"]), t["y"])
        np.testing.assert_array_equal(ref.pq_matmul_struct(s, t["xs"]), t["ys"])
    finally:
        ref.pq_free(s)
