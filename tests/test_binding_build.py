"""The compiled binding (flashgmm_amd/binding/binding.cpp, built as a
CppExtension with setup.py's settings) on the CPU: it compiles against the
two C-ABI libraries, its TORCH_CHECKs raise the reference's messages
(binding.cpp:38-39,54,65,80), and on CPU tensors it returns exactly what the
ctypes drop-in module returns (the same host library)."""
import importlib.util
import os
import sys
import tempfile

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def ext():
    from torch.utils.cpp_extension import load
    path = os.path.join(ROOT, "flashgmm_amd", "binding", "setup.py")
    spec = importlib.util.spec_from_file_location("fgmm_binding_setup", path)
    setup_mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(setup_mod)
    e = setup_mod.extension("flash_gmm_native_pybind")
    build = tempfile.mkdtemp(prefix="fgmm_binding_")
    ldflags = [f"-L{d}" for d in e.library_dirs] + [f"-l{lib}" for lib in e.libraries]
    ldflags += e.extra_link_args
    cflags = list(e.extra_compile_args) + [f"-D{k}={v}" for k, v in e.define_macros]
    return load(name="flash_gmm_native_pybind", sources=e.sources,
                extra_include_paths=e.include_dirs, extra_cflags=cflags,
                extra_ldflags=ldflags, build_directory=build, with_cuda=False, verbose=False)


def test_binding_checks_raise_reference_messages(ext):
    X = torch.zeros(10, 4)
    mu, var, lp = torch.zeros(2, 4), torch.ones(2, 4), torch.zeros(2)
    for call in (lambda: ext.flash_em_fused(X.double(), mu, var, lp),
                 lambda: ext.standard_e_step(X.double(), mu, var, lp),
                 lambda: ext.flash_e_step(X.double(), mu, var, lp),
                 lambda: ext.standard_m_step(X.double(), torch.zeros(10, 2))):
        with pytest.raises(RuntimeError, match="X must be float32"):
            call()
    with pytest.raises(RuntimeError, match="X must be 2D"):
        ext.standard_e_step(X[0], mu, var, lp)
    with pytest.raises(RuntimeError, match="var must be"):
        ext.flash_em_fused(X, mu, var[:, :2], lp)


def test_binding_matches_drop_in_on_cpu(ext):
    sys.path.insert(0, ROOT)
    from flashgmm_amd import flash_gmm_native as C
    from flashgmm_amd.configs import make_problem
    X, mu, var, lp = (torch.from_numpy(a) for a in make_problem(1))
    for a, b in zip(ext.flash_em_fused(X, mu, var, lp), C.flash_em_fused(X, mu, var, lp)):
        assert torch.equal(a, b)
    for a, b in zip(ext.flash_em_fused(X, mu, var, lp, 128, 32),   # BN/BK as io_env passes
                    C.flash_em_fused(X, mu, var, lp, 128, 32)):
        assert torch.equal(a, b)
    g1, l1 = ext.standard_e_step(X, mu, var, lp)
    g2, l2 = C.standard_e_step(X, mu, var, lp)
    assert torch.equal(g1, g2) and torch.equal(l1, l2)
    g3, _ = ext.flash_e_step(X, mu, var, lp)
    assert torch.equal(g3, g2)
    for a, b in zip(ext.standard_m_step(X, g1), C.standard_m_step(X, g2)):
        assert np.array_equal(a.numpy(), b.numpy(), equal_nan=True)
