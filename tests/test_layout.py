"""The struct mirrors of include/ibhip.h against the reference's own headers
(src/inferbit_internal.h:199-277 ib_kernels, src/pq_decode.h:39-87
ib_pq_tensor): tests/layout_check.c static-asserts every field offset and
the sizes; this test compiles it.  Needs the reference tree (present where
the library is built, absent on the GPU box: skipped there)."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")) or shutil.which("gcc") is None,
                    reason="reference headers or gcc absent")
def test_mirrors_match_reference_layout(tmp_path):
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", os.path.join(REPO, "tests", "layout_check.c"),
                        "-I", os.path.join(REPO, "include"), "-I", os.path.join(REF, "src"),
                        "-I", os.path.join(REF, "include"), "-o", str(tmp_path / "l.o")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_ctypes_pq_mirror_matches_header():
    """The ctypes mirror the tests use has the header's field order."""
    import ctypes as C
    from oracle.refbind import IbPqTensor
    names = [f[0] for f in IbPqTensor._fields_]
    assert names[:9] == ["M", "N", "G", "K", "K_l2", "n_levels", "rotate", "n_outlier", "format"]
    assert C.sizeof(IbPqTensor) == 192   # sizeof(ib_pq_tensor) on x86-64
