"""Host-side producers in libibhip.so (no GPU needed): the weight quantizers
(row a10, src/quantize.c:75-239) against the reference-written golden
vectors, the synthetic-data generator, and the IBF v1 writer."""
import json

import numpy as np
import pytest

from conftest import load_golden

SHAPES = ["64x256", "37x200", "16x4100", "8x4096"]


@pytest.fixture(scope="module")
def ibf():
    from libinferbit_amd import ibf
    return ibf


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("bits", [8, 4, 2])
def test_quantize_matches_reference(ibf, shape, bits):
    d = load_golden("quant.npz")
    packed, scales = ibf.quantize(bits, d[f"W_{shape}"])
    np.testing.assert_array_equal(packed.reshape(-1), d[f"w{bits}_{shape}"].view(np.uint8).reshape(-1))
    np.testing.assert_array_equal(scales, d[f"s{bits}_{shape}"].view(np.uint16))


def test_quantize_rejects_partial_bytes(ibf):
    from libinferbit_amd import IbhError
    with pytest.raises(IbhError):
        ibf.quantize(4, np.zeros((2, 7), np.float32))


def test_fill_normal_is_counter_based(ibf):
    a = ibf.fill_normal(1 << 20, 7, 1.0)
    b = ibf.fill_normal(1000, 7, 1.0, first=5000)
    np.testing.assert_array_equal(a[5000:6000], b)
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    assert not np.array_equal(a[:1000], ibf.fill_normal(1000, 8, 1.0))


def test_ibf_writer_layout(ibf, tmp_path):
    cfg = dict(ibf.TINYLLAMA, num_layers=2, hidden_size=128, num_heads=4, num_kv_heads=2, head_dim=32,
               intermediate_size=256, vocab_size=512, max_context_length=64)
    p = tmp_path / "m.ibf"
    hdr = ibf.write_synthetic(str(p), cfg, seed=3)
    raw = p.read_bytes()
    assert raw[:8] == b"INFERBIT"
    ver, hsize, flags = np.frombuffer(raw[8:20], np.uint32)
    assert (ver, flags) == (1, 0)
    assert json.loads(raw[32:32 + hsize]) == json.loads(json.dumps(hdr))
    base = (32 + hsize + 63) // 64 * 64
    assert len(raw) == base + hdr["data"]["weight_data_size"]
    q = hdr["layers"][1]["weights"]["q_proj"]
    w = ibf.fill_normal(128 * 128, ibf.tensor_seed(3, "layers.1.q_proj"), 0.02).reshape(128, 128)
    packed, scales = ibf.quantize(8, w)
    assert raw[base + q["offset"]: base + q["offset"] + q["size"]] == packed.tobytes()
    assert raw[base + q["scale_offset"]: base + q["scale_offset"] + 256] == scales.tobytes()
    n = hdr["output"]["norm"]
    assert np.all(np.frombuffer(raw[base + n["offset"]: base + n["offset"] + 256], np.float16) == 1)


def test_expf_restatement_matches_glibc(oracle_lib):
    """The device expf (ib_expf, also compiled for the host) against glibc
    expf, which the reference's softmax and SiLU call: every 61st float bit
    pattern with |x| <= 110 (36.8 M values) plus the special values.  (An
    exhaustive sweep of all 2.24e9 floats in that range also gives 0
    mismatches; it takes ~90 s and is not part of this suite.)"""
    import ctypes
    from libinferbit_amd._lib import lib
    lo = np.arange(0, 0x42DC0000, 61, dtype=np.uint32)          # 0 .. 110.0
    bits = np.concatenate([lo, lo | np.uint32(0x80000000)])
    x = bits.view(np.float32)
    x = np.concatenate([x, np.array([np.inf, -np.inf, np.nan, 200, -200, 88.72, 88.7228, -103.97, -103.973,
                                     float.fromhex("0x1.04845ep+5"), float.fromhex("-0x1.f8cbb2p+5")], np.float32)])
    ours = np.empty_like(x)
    lib().ibh_expf_host(x.ctypes.data_as(ctypes.c_void_p), ours.ctypes.data_as(ctypes.c_void_p), x.size)
    ref = oracle_lib.expf(x)
    same = (ours.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all(), x[~same][:10]
