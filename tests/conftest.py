import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)   # gen_golden.make_pq builds synthetic PQ tensors


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def pq_case(npz, name):
    """Rebuild a PQ tensor dict (oracle layout) from pq.npz entries 'name.*'."""
    t = {}
    for k in npz.files:
        if k.startswith(name + "."):
            v = npz[k]
            key = k[len(name) + 1:]
            t[key] = int(v) if v.ndim == 0 else v
    return t


INT4G_KEYS = ("q", "s", "inv_act", "outl_idx", "outl_val", "x", "y", "ys")


def int4g_case(npz, name):
    """An INT4 group-scale tensor dict (+ x, y, ys) from int4g.npz entries 'name.*'."""
    return {k: (npz[f"{name}.{k}"] if f"{name}.{k}" in npz.files else None) for k in INT4G_KEYS}


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle
