"""flashgmm_amd -- Flash-GMM's fused diagonal-covariance EM iteration on
MI355X (gfx950): hand-written HIP kernels behind the reference's
``flash_gmm_native`` API.

    from flashgmm_amd import flash_gmm_native as _C     # drop-in module
    from flashgmm_amd.native_wrapper import NativeFlashGMM

The native library is ``flashgmm_amd/libflashgmm.so`` (build with
``python -m flashgmm_amd.build``); its C ABI is ``include/flashgmm.h``.
"""
from . import configs  # noqa: F401

__all__ = ["configs", "flash_gmm_native", "native_wrapper"]


def __getattr__(name):
    # torch-dependent modules load lazily so `import flashgmm_amd.configs`
    # stays cheap for data generation.
    if name in ("flash_gmm_native", "native_wrapper"):
        import importlib
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
