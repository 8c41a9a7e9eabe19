"""hi_amd: MI355X (gfx950) batched token sampler for the hi local-inference
stack.  The product is ``libhi_rocm.so`` (C ABI in ``include/hi_rocm.h``);
this package holds its HIP sources (``csrc/``), the build step, a ctypes
binding and the Python front end of the host API.
"""
__version__ = "0.1.0"

from ._lib import HiRocmError, load  # noqa: F401
