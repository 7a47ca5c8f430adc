"""libinferbit_amd -- MI355X (gfx950) kernels for libinferbit's decode-time
quantized matvec path, behind a C ABI (include/ibhip.h, libibhip.so).

The Python layer is a thin host-side mirror of the reference's operator
entry points (same names and argument meaning as src/threading.c and
src/kernels/*.c of the reference), used by tests and bench.py.  Device
memory comes from torch tensors on ``cuda`` (plumbing only); every op runs
a hand-written HIP kernel from libibhip.so.  There is no CPU fallback: if
the library is not built, ``lib()`` raises.
"""
from ._lib import IbhError, lib, lib_path, loaded  # noqa: F401
from . import ibf, model, ops  # noqa: F401

__all__ = ["lib", "lib_path", "loaded", "IbhError", "ops", "ibf", "model"]
