"""Builds the pybind11 module ``flash_gmm_native`` (binding.cpp) against the
two C-ABI libraries that ``python -m flashgmm_amd.build`` produced:

    python -m flashgmm_amd.build
    cd flashgmm_amd/binding && python setup.py build_ext --inplace

A ``CppExtension`` (no CUDAExtension, no hipify): the kernels live in
libflashgmm.so, so this module only needs the HIP runtime headers for the
current-stream query.  The libraries are found through an rpath to
``flashgmm_amd/``.
"""
import os

from setuptools import setup
from torch.utils.cpp_extension import BuildExtension, CppExtension

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def extension(name="flash_gmm_native"):
    return CppExtension(
        name, [os.path.join(HERE, "binding.cpp")],
        include_dirs=[os.path.join(ROOT, "include"), os.path.join(ROCM, "include")],
        define_macros=[("__HIP_PLATFORM_AMD__", "1"), ("USE_ROCM", "1")],
        library_dirs=[PKG, os.path.join(ROCM, "lib")],
        libraries=["flashgmm", "flashgmm_cpu", "amdhip64"],
        extra_link_args=[f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"],
        extra_compile_args=["-O2", "-std=c++17"],
    )


if __name__ == "__main__":
    setup(name="flash_gmm_native", ext_modules=[extension()],
          cmdclass={"build_ext": BuildExtension})
