"""``import flash_gmm_native as _C`` -- the import the reference's callers use
(``flash_gmm/native_wrapper.py:17-18``, ``benchmark_gpu.py``,
``benchmark_cpu.py``) -- resolves to this package's drop-in module
``flashgmm_amd.flash_gmm_native`` when the repository root is on sys.path.
The name is bound to that module object itself, so both imports share one
set of functions and one workspace cache.
"""
import sys

from flashgmm_amd import flash_gmm_native as _impl

sys.modules[__name__] = _impl
