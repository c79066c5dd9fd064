"""Drop-in for the reference's ``flash_gmm_native`` extension module on ROCm.

Same function names, argument order, defaults and return order as the
reference's pybind11 module (``flash_gmm/csrc/binding.cpp:94-109``:
``standard_e_step``, ``flash_e_step``, ``flash_em_fused``, ``standard_m_step``),
plus the three stage entry points (``flash_log_normalizer``,
``flash_accumulate_stats``, ``m_step_update``) and the iteration loop
``em_fit``.  Outputs are fresh tensors on the input's device; inputs are
never modified.

Dispatch on the device of X, as the reference's binding does
(``binding.cpp:41-48,55-59,68-75,82-91``):
  * ROCm tensors -> ``libflashgmm.so`` (hand-written HIP kernels for gfx950)
    on torch's current stream;
  * CPU tensors -> ``libflashgmm_cpu.so`` (this package's C++/OpenMP host
    path, fp64 arithmetic, torch.get_num_threads() threads).
Neither path falls back to the other or to Python: a missing library raises.
Every other tensor argument must live on X's device.

Errors are ``RuntimeError`` like the reference's ``TORCH_CHECK``; the dtype
check keeps the reference's message ("X must be float32",
``binding.cpp:38,54,65,80``).  Unlike the reference, shapes, devices,
``d <= 256`` and launch failures are checked too, before any work.  The
reference refuses ``flash_e_step`` on CUDA tensors (``binding.cpp:55-57``);
here it runs on the device.
"""
from __future__ import annotations

import torch

from . import _lib


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _check_device(X: torch.Tensor, fn: str) -> None:
    if not (X.is_cuda or X.device.type == "cpu"):
        raise RuntimeError(
            f"flashgmm_amd.{fn}: tensors must be on a ROCm device or the CPU (got {X.device})")


def _on_host(X: torch.Tensor) -> bool:
    return X.device.type == "cpu"


def _threads() -> int:
    return max(1, torch.get_num_threads())


def _params(X, mu, var, log_pi, fn):
    """Validates (X, mu, var, log_pi); returns contiguous fp32 views and (N, K, d)."""
    if X.dtype != torch.float32:
        raise RuntimeError("X must be float32")
    if X.dim() != 2:
        raise RuntimeError("X must be 2D")
    _check_device(X, fn)
    N, d = X.shape
    if N < 1 or d < 1:
        raise RuntimeError(f"flashgmm_amd.{fn}: X must be non-empty (got {tuple(X.shape)})")
    if d > 256:
        raise RuntimeError(f"flashgmm_amd.{fn}: d must be <= 256 (got {d})")
    if mu.dim() != 2 or mu.shape[1] != d:
        raise RuntimeError(f"flashgmm_amd.{fn}: mu must be [K, {d}] (got {tuple(mu.shape)})")
    K = mu.shape[0]
    if K < 1:
        raise RuntimeError(f"flashgmm_amd.{fn}: K must be >= 1")
    if tuple(var.shape) != (K, d):
        raise RuntimeError(f"flashgmm_amd.{fn}: var must be [{K}, {d}] (got {tuple(var.shape)})")
    if tuple(log_pi.shape) != (K,):
        raise RuntimeError(f"flashgmm_amd.{fn}: log_pi must be [{K}] (got {tuple(log_pi.shape)})")
    out = []
    for name, t in (("mu", mu), ("var", var), ("log_pi", log_pi)):
        if t.dtype != torch.float32:
            raise RuntimeError(f"flashgmm_amd.{fn}: {name} must be float32 (got {t.dtype})")
        if t.device != X.device:
            raise RuntimeError(f"flashgmm_amd.{fn}: {name} is on {t.device}, X on {X.device}")
        out.append(t.contiguous())
    return (X.contiguous(), *out, N, K, d)


def _ws(X, N, K, d, variant, fused=False):
    """The cached device workspace, grown to what the call needs: the fused
    iteration and the device loop need less than the other entry points."""
    lib = _lib.load()
    nbytes = (lib.fgmm_em_fused_workspace_bytes if fused else lib.fgmm_workspace_bytes)(
        N, K, d, variant)
    if nbytes == 0:   # the library rejected the shape; report its reason
        raise RuntimeError("flashgmm_amd: " + lib.fgmm_last_error().decode(errors="replace"))
    return _lib.workspace(X.device, nbytes), nbytes


def flash_em_fused(X, mu, var, log_pi, BN: int = 64, BK: int = 8, *, variant=None):
    """One fused EM iteration; returns ``[new_mu, new_var, new_log_pi,
    log_normalizer]`` (``binding.cpp:62-76,102-105``,
    ``flash_gmm_cuda.cu:402-504``).  ``BN``/``BK`` are accepted for signature
    compatibility; the gfx950 kernels pick their own tiles per (K, d)."""
    if int(BN) < 1 or int(BK) < 1:
        raise RuntimeError(f"flashgmm_amd.flash_em_fused: BN and BK must be >= 1 (got {BN}, {BK})")
    X, mu, var, log_pi, N, K, d = _params(X, mu, var, log_pi, "flash_em_fused")
    new_mu = torch.empty((K, d), dtype=torch.float32, device=X.device)
    new_var = torch.empty((K, d), dtype=torch.float32, device=X.device)
    new_log_pi = torch.empty((K,), dtype=torch.float32, device=X.device)
    ln = torch.empty((N,), dtype=torch.float32, device=X.device)
    if _on_host(X):
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_em_fused(
            _ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K, d, _threads(), _ptr(new_mu),
            _ptr(new_var), _ptr(new_log_pi), _ptr(ln)))
        return [new_mu, new_var, new_log_pi, ln]
    v = _lib.variant_code(variant)
    lib = _lib.load()
    ws, nbytes = _ws(X, N, K, d, v, fused=True)
    _lib.check(lib.fgmm_em_fused(_ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K, d, v,
                                 _ptr(new_mu), _ptr(new_var), _ptr(new_log_pi), _ptr(ln),
                                 _ptr(ws), nbytes, _lib.stream_handle(X.device)))
    return [new_mu, new_var, new_log_pi, ln]


def flash_log_normalizer(X, mu, var, log_pi, *, variant=None):
    """Pass 1: ``log_normalizer[n] = logsumexp_k(log pi_k + log N(x_n | mu_k, var_k))``
    (``flash_gmm_cuda.cu:72-170``; ``flash_e_step.py:144-177``)."""
    X, mu, var, log_pi, N, K, d = _params(X, mu, var, log_pi, "flash_log_normalizer")
    ln = torch.empty((N,), dtype=torch.float32, device=X.device)
    if _on_host(X):
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_log_normalizer(
            _ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K, d, _threads(), _ptr(ln)))
        return ln
    v = _lib.variant_code(variant)
    lib = _lib.load()
    ws, nbytes = _ws(X, N, K, d, v)
    _lib.check(lib.fgmm_log_normalizer(_ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K, d, v,
                                       _ptr(ln), _ptr(ws), nbytes,
                                       _lib.stream_handle(X.device)))
    return ln


def flash_accumulate_stats(X, mu, var, log_pi, log_normalizer, *, variant=None):
    """Pass 2: returns ``[n_k, s_k, sq_k]`` with gamma recomputed on chip
    (``flash_gmm_cuda.cu:179-292``; ``flash_e_step.py:179-219``)."""
    X, mu, var, log_pi, N, K, d = _params(X, mu, var, log_pi, "flash_accumulate_stats")
    if tuple(log_normalizer.shape) != (N,) or log_normalizer.dtype != torch.float32:
        raise RuntimeError(f"flashgmm_amd.flash_accumulate_stats: log_normalizer must be "
                           f"float32 [{N}] (got {log_normalizer.dtype} "
                           f"{tuple(log_normalizer.shape)})")
    if log_normalizer.device != X.device:
        raise RuntimeError("flashgmm_amd.flash_accumulate_stats: log_normalizer is on "
                           f"{log_normalizer.device}, X on {X.device}")
    ln = log_normalizer.contiguous()
    n_k = torch.empty((K,), dtype=torch.float32, device=X.device)
    s_k = torch.empty((K, d), dtype=torch.float32, device=X.device)
    sq_k = torch.empty((K, d), dtype=torch.float32, device=X.device)
    if _on_host(X):
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_accumulate_stats(
            _ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), _ptr(ln), N, K, d, _threads(),
            _ptr(n_k), _ptr(s_k), _ptr(sq_k)))
        return [n_k, s_k, sq_k]
    v = _lib.variant_code(variant)
    lib = _lib.load()
    ws, nbytes = _ws(X, N, K, d, v)
    _lib.check(lib.fgmm_accumulate_stats(_ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), _ptr(ln),
                                         N, K, d, v, _ptr(n_k), _ptr(s_k), _ptr(sq_k),
                                         _ptr(ws), nbytes, _lib.stream_handle(X.device)))
    return [n_k, s_k, sq_k]


def _gamma_estep(X, mu, var, log_pi, variant, fn, standard):
    X, mu, var, log_pi, N, K, d = _params(X, mu, var, log_pi, fn)
    gamma = torch.empty((N, K), dtype=torch.float32, device=X.device)
    ln = torch.empty((N,), dtype=torch.float32, device=X.device)
    if _on_host(X):
        # standard and flash E-steps return the same quantities on the host
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_e_step(
            _ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K, d, _threads(), _ptr(gamma),
            _ptr(ln)))
        return [gamma, ln]
    v = _lib.variant_code(variant)
    lib = _lib.load()
    stream = _lib.stream_handle(X.device)
    if standard:
        # the N x K fp64 matrix lives only for this call, like the reference's L
        nbytes = lib.fgmm_standard_e_step_workspace_bytes(N, K, d, v)
        if nbytes == 0:
            raise RuntimeError("flashgmm_amd: " + lib.fgmm_last_error().decode(errors="replace"))
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=X.device)
        _lib.check(lib.fgmm_standard_e_step(_ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K,
                                            d, v, _ptr(gamma), _ptr(ln), _ptr(ws), nbytes,
                                            stream))
    else:
        ws, nbytes = _ws(X, N, K, d, v)
        _lib.check(lib.fgmm_flash_e_step(_ptr(X), _ptr(mu), _ptr(var), _ptr(log_pi), N, K, d,
                                         v, _ptr(gamma), _ptr(ln), _ptr(ws), nbytes, stream))
    return [gamma, ln]


def standard_e_step(X, mu, var, log_pi, *, variant=None):
    """Materialising E-step; returns ``[gamma, log_normalizer]``
    (``binding.cpp:35-49``, ``flash_gmm_cuda.cu:328-400``).  The N x K
    log-density matrix is formed in fp64 on the device and normalised row by
    row."""
    return _gamma_estep(X, mu, var, log_pi, variant, "standard_e_step", standard=True)


def flash_e_step(X, mu, var, log_pi, BK: int = 4, *, variant=None):
    """Flash E-step returning gamma; returns ``[gamma, log_normalizer]``
    (``binding.cpp:51-60``; CPU-only in the reference,
    ``flash_gmm_cpu.cpp:108-168``).  Pass 1 gives the log-normalizer, a second
    sweep writes gamma.  ``BK`` is accepted for signature compatibility."""
    if int(BK) < 1:
        raise RuntimeError(f"flashgmm_amd.flash_e_step: BK must be >= 1 (got {BK})")
    return _gamma_estep(X, mu, var, log_pi, variant, "flash_e_step", standard=False)


def standard_m_step(X, gamma):
    """M-step from responsibilities; returns ``[mu, var, log_pi]`` with the
    reference's standard arithmetic: no clamp on ``n_k``, ``var`` floored at
    1e-6, ``log_pi = log(n_k / N)`` (``binding.cpp:78-92``,
    ``flash_gmm_cpu.cpp:292-311``)."""
    if X.dtype != torch.float32:
        raise RuntimeError("X must be float32")
    if X.dim() != 2:
        raise RuntimeError("X must be 2D")
    _check_device(X, "standard_m_step")
    N, d = X.shape
    if N < 1 or d < 1:
        raise RuntimeError(f"flashgmm_amd.standard_m_step: X must be non-empty "
                           f"(got {tuple(X.shape)})")
    if gamma.dim() != 2 or gamma.shape[0] != N or gamma.shape[1] < 1:
        raise RuntimeError(f"flashgmm_amd.standard_m_step: gamma must be [{N}, K] "
                           f"(got {tuple(gamma.shape)})")
    if gamma.dtype != torch.float32:
        raise RuntimeError(f"flashgmm_amd.standard_m_step: gamma must be float32 "
                           f"(got {gamma.dtype})")
    if gamma.device != X.device:
        raise RuntimeError(f"flashgmm_amd.standard_m_step: gamma is on {gamma.device}, "
                           f"X on {X.device}")
    K = gamma.shape[1]
    X, gamma = X.contiguous(), gamma.contiguous()
    mu = torch.empty((K, d), dtype=torch.float32, device=X.device)
    var = torch.empty((K, d), dtype=torch.float32, device=X.device)
    log_pi = torch.empty((K,), dtype=torch.float32, device=X.device)
    if _on_host(X):
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_standard_m_step(
            _ptr(X), _ptr(gamma), N, K, d, _threads(), _ptr(mu), _ptr(var), _ptr(log_pi)))
        return [mu, var, log_pi]
    lib = _lib.load()
    nbytes = lib.fgmm_standard_m_step_workspace_bytes(N, K, d)
    if nbytes == 0:
        raise RuntimeError("flashgmm_amd: " + lib.fgmm_last_error().decode(errors="replace"))
    ws = _lib.workspace(X.device, nbytes)
    _lib.check(lib.fgmm_standard_m_step(_ptr(X), _ptr(gamma), N, K, d, _ptr(mu), _ptr(var),
                                        _ptr(log_pi), _ptr(ws), nbytes,
                                        _lib.stream_handle(X.device)))
    return [mu, var, log_pi]


def m_step_update(n_k, s_k, sq_k, N: int):
    """M-step from sufficient statistics with the native clamps; returns
    ``[mu, var, log_pi]`` (``flash_gmm_cuda.cu:298-322``)."""
    for name, t in (("n_k", n_k), ("s_k", s_k), ("sq_k", sq_k)):
        if t.dtype != torch.float32:
            raise RuntimeError(f"flashgmm_amd.m_step_update: {name} must be float32")
    _check_device(s_k, "m_step_update")
    if s_k.dim() != 2:
        raise RuntimeError("flashgmm_amd.m_step_update: s_k must be [K, d]")
    K, d = s_k.shape
    if tuple(n_k.shape) != (K,) or tuple(sq_k.shape) != (K, d):
        raise RuntimeError("flashgmm_amd.m_step_update: expected n_k [K], s_k/sq_k [K, d]")
    if n_k.device != s_k.device or sq_k.device != s_k.device:
        raise RuntimeError("flashgmm_amd.m_step_update: statistics on different devices")
    N = int(N)
    if N < 1:
        raise RuntimeError("flashgmm_amd.m_step_update: N must be >= 1")
    # the contiguous copies stay bound until the call has been queued: a
    # temporary freed earlier could hand its block to the next copy
    n_c, s_c, sq_c = n_k.contiguous(), s_k.contiguous(), sq_k.contiguous()
    mu = torch.empty((K, d), dtype=torch.float32, device=s_k.device)
    var = torch.empty((K, d), dtype=torch.float32, device=s_k.device)
    log_pi = torch.empty((K,), dtype=torch.float32, device=s_k.device)
    if _on_host(s_k):
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_m_step_update(
            _ptr(n_c), _ptr(s_c), _ptr(sq_c), N, K, d, _ptr(mu), _ptr(var), _ptr(log_pi)))
        return [mu, var, log_pi]
    lib = _lib.load()
    _lib.check(lib.fgmm_m_step_update(_ptr(n_c), _ptr(s_c), _ptr(sq_c), N, K, d, _ptr(mu),
                                      _ptr(var), _ptr(log_pi), _lib.stream_handle(s_k.device)))
    return [mu, var, log_pi]


def em_fit(X, mu0, var0, log_pi0, iters: int, *, variant=None):
    """``iters`` fused EM iterations on the device with no host round trip.

    Returns ``(mu, var, log_pi, ll_traj)``; ``ll_traj[it]`` (float64, on the
    device) is the mean log-normalizer under the parameters entering
    iteration ``it`` -- ``NativeFlashGMM.fit``'s per-iteration
    ``log_likelihood`` (``native_wrapper.py:128-137``)."""
    X, mu0, var0, log_pi0, N, K, d = _params(X, mu0, var0, log_pi0, "em_fit")
    iters = int(iters)
    if iters < 1:
        raise RuntimeError("flashgmm_amd.em_fit: iters must be >= 1")
    mu = torch.empty((K, d), dtype=torch.float32, device=X.device)
    var = torch.empty((K, d), dtype=torch.float32, device=X.device)
    log_pi = torch.empty((K,), dtype=torch.float32, device=X.device)
    traj = torch.empty((iters,), dtype=torch.float64, device=X.device)
    if _on_host(X):
        _lib.check_cpu(_lib.load_cpu().fgmm_cpu_em_fit(
            _ptr(X), _ptr(mu0), _ptr(var0), _ptr(log_pi0), N, K, d, iters, _threads(),
            _ptr(mu), _ptr(var), _ptr(log_pi), _ptr(traj)))
        return mu, var, log_pi, traj
    v = _lib.variant_code(variant)
    lib = _lib.load()
    ws, nbytes = _ws(X, N, K, d, v, fused=True)
    _lib.check(lib.fgmm_em_fit(_ptr(X), _ptr(mu0), _ptr(var0), _ptr(log_pi0), N, K, d, iters, v,
                               _ptr(mu), _ptr(var), _ptr(log_pi), _ptr(traj), _ptr(ws), nbytes,
                               _lib.stream_handle(X.device)))
    return mu, var, log_pi, traj


def resolve_variant(N: int, K: int, d: int, variant=None) -> str:
    """Name of the kernel family the library runs for this shape."""
    code = _lib.load().fgmm_resolve_variant(int(N), int(K), int(d), _lib.variant_code(variant))
    return {1: "valu", 2: "mfma", 3: "x32", 4: "mixed", 5: "sparse", 6: "small"}[code]
