"""CPU-side checks of the C-ABI library: it loads and exports every symbol
include/ibhip.h declares.  No compute calls (no GPU here)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "ibhip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    names = set(re.findall(r"\b((?:ibh|ib)_[a-z0-9_]+)\s*\(", txt))
    return sorted(n for n in names if not n.startswith("ibh_kernels"))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for must in ("ibh_matmul", "ibh_matmul_w4a8", "ibh_quantize_act_g128", "ib_init_kernels_hip"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    from libinferbit_amd import _lib
    L = ctypes.CDLL(_lib.lib_path())
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from libinferbit_amd import _lib
    assert set(declared_symbols()) <= set(_lib.SIGNATURES), set(declared_symbols()) - set(_lib.SIGNATURES)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from libinferbit_amd import _lib
    monkeypatch.setattr(_lib, "_LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    try:
        _lib.lib()
    except RuntimeError as e:
        assert "no CPU fallback" in str(e)
    else:
        raise AssertionError("expected a loud failure")


def test_prompt_lookup_search_matches_reference():
    """ibh_prompt_lookup_search (host code, no GPU) against the compiled
    reference's ib_prompt_lookup_search on random short histories."""
    import ctypes
    import numpy as np
    from oracle import refbind as R
    if not R.available():
        pytest.skip("reference library not built")
    from libinferbit_amd import _lib
    ours, theirs = _lib.lib(), R.lib()
    theirs.ib_prompt_lookup_search.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_void_p]
    rng = np.random.default_rng(0)
    hits = 0
    for _ in range(2000):
        h = rng.integers(0, 4, rng.integers(0, 30)).astype(np.int32)
        ng, k = int(rng.integers(0, 5)), int(rng.integers(0, 10))
        a, b = np.full(16, -1, np.int32), np.full(16, -1, np.int32)
        na = ours.ibh_prompt_lookup_search(h.ctypes.data_as(ctypes.c_void_p), len(h), ng, k,
                                           a.ctypes.data_as(ctypes.c_void_p))
        nb = theirs.ib_prompt_lookup_search(h.ctypes.data_as(ctypes.c_void_p), len(h), ng, k,
                                            b.ctypes.data_as(ctypes.c_void_p))
        assert na == nb and (a == b).all()
        hits += na > 0
    assert hits > 100
