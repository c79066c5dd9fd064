"""Streaming EM iteration for X larger than device memory.

Mirrors the reference's streaming classes (``flash_gmm/flash_gmm_v9.py``):
``StreamingFlashGMM(chunk_size).em_step(X, mu, var, log_pi)`` ->
``(new_mu, new_var, new_log_pi, log_normalizer)`` with ``X`` on the host (or
on the device), the parameters and the returned log-normalizer on the
device, and ``StreamingFlashGMMAsync`` overlapping the host-to-device copy of
chunk t+1 with the compute of chunk t (``flash_gmm_v9.py:218-326``).

Here each chunk is read once per iteration: Pass 1 and Pass 2 run back to
back while the chunk is resident and its sufficient statistics are added to
fp64 accumulators on the device (``fgmm_stream_*`` in ``include/flashgmm.h``);
the reference reads every chunk once per pass.  Results equal the resident
``flash_em_fused`` to the parity bar; the log-normalizer is bitwise identical
(it depends on the point alone).
"""
from __future__ import annotations

import torch

from . import _lib
from .flash_gmm_native import _ptr


class StreamingFlashGMM:
    """One EM iteration over X in chunks of ``chunk_size`` rows; chunks of a
    host ``X`` are copied synchronously before they are processed."""

    def __init__(self, chunk_size: int = 500_000, variant=None):
        if int(chunk_size) < 1:
            raise RuntimeError("flashgmm_amd: chunk_size must be >= 1")
        self.chunk_size = int(chunk_size)
        self.variant = variant
        self._ws = None

    # -- helpers ----------------------------------------------------------
    def _check(self, X, mu, var, log_pi):
        if X.dtype != torch.float32:
            raise RuntimeError("X must be float32")
        if X.dim() != 2:
            raise RuntimeError("X must be 2D")
        if not mu.is_cuda:   # X may live on the host; the iteration runs on the device
            raise RuntimeError("flashgmm_amd.StreamingFlashGMM.em_step: mu/var/log_pi must be "
                               f"on a ROCm device (got {mu.device})")
        N, d = X.shape
        K = mu.shape[0]
        if N < 1 or d < 1 or d > 256:
            raise RuntimeError(f"flashgmm_amd: bad X shape {tuple(X.shape)} (need N >= 1, 1 <= d <= 256)")
        if mu.dim() != 2 or mu.shape[1] != d or tuple(var.shape) != (K, d) or tuple(log_pi.shape) != (K,):
            raise RuntimeError("flashgmm_amd: mu/var must be [K, d] and log_pi [K] matching X")
        for name, t in (("mu", mu), ("var", var), ("log_pi", log_pi)):
            if t.dtype != torch.float32:
                raise RuntimeError(f"flashgmm_amd: {name} must be float32")
            if t.device != mu.device:
                raise RuntimeError(f"flashgmm_amd: {name} is on {t.device}, mu on {mu.device}")
        if X.is_cuda and X.device != mu.device:
            raise RuntimeError(f"flashgmm_amd: X is on {X.device}, parameters on {mu.device}")
        return N, K, d

    def _begin(self, mu, var, log_pi, N, K, d):
        lib = _lib.load()
        self._v = _lib.variant_code(self.variant)
        self._cs = min(self.chunk_size, N)
        nb = lib.fgmm_stream_workspace_bytes(self._cs, K, d, self._v)
        if nb == 0:
            raise RuntimeError("flashgmm_amd: " + lib.fgmm_last_error().decode(errors="replace"))
        if self._ws is None or self._ws.numel() < nb or self._ws.device != mu.device:
            self._ws = torch.empty((nb,), dtype=torch.uint8, device=mu.device)
        self._nb = nb
        self._mu, self._var, self._lp = mu.contiguous(), var.contiguous(), log_pi.contiguous()
        _lib.check(lib.fgmm_stream_begin(_ptr(self._mu), _ptr(self._var), _ptr(self._lp),
                                         self._cs, K, d, self._v, _ptr(self._ws), nb,
                                         _lib.stream_handle(mu.device)))
        return lib

    def _chunk(self, lib, Xc, rows, K, d, ln_slice, stream):
        _lib.check(lib.fgmm_stream_chunk(_ptr(Xc), rows, self._cs, K, d, self._v,
                                         _ptr(ln_slice), _ptr(self._ws), self._nb, stream))

    def _end(self, lib, N, K, d, device):
        new_mu = torch.empty((K, d), dtype=torch.float32, device=device)
        new_var = torch.empty((K, d), dtype=torch.float32, device=device)
        new_lp = torch.empty((K,), dtype=torch.float32, device=device)
        self.ll_mean = torch.empty((1,), dtype=torch.float64, device=device)
        _lib.check(lib.fgmm_stream_end(N, self._cs, K, d, self._v, _ptr(new_mu), _ptr(new_var),
                                       _ptr(new_lp), _ptr(self.ll_mean), _ptr(self._ws),
                                       self._nb, _lib.stream_handle(device)))
        return new_mu, new_var, new_lp

    # -- API ----------------------------------------------------------------
    def em_step(self, X, mu, var, log_pi):
        N, K, d = self._check(X, mu, var, log_pi)
        device = mu.device
        lib = self._begin(mu, var, log_pi, N, K, d)
        ln = torch.empty((N,), dtype=torch.float32, device=device)
        stream = _lib.stream_handle(device)
        buf = None if X.is_cuda else torch.empty((self._cs, d), dtype=torch.float32, device=device)
        for start in range(0, N, self._cs):
            rows = min(self._cs, N - start)
            if X.is_cuda:
                Xc = X[start:start + rows].contiguous()
            else:
                Xc = buf[:rows]
                Xc.copy_(X[start:start + rows])
            self._chunk(lib, Xc, rows, K, d, ln[start:start + rows], stream)
        return (*self._end(lib, N, K, d, device), ln)


class StreamingFlashGMMAsync(StreamingFlashGMM):
    """Same iteration; a host ``X`` is staged through two pinned buffers and
    copied on a second stream while the previous chunk computes.  A pinned
    ``X`` (``X.is_pinned()``) is copied without staging."""

    def em_step(self, X, mu, var, log_pi):
        if X.is_cuda:
            return super().em_step(X, mu, var, log_pi)
        N, K, d = self._check(X, mu, var, log_pi)
        device = mu.device
        lib = self._begin(mu, var, log_pi, N, K, d)
        ln = torch.empty((N,), dtype=torch.float32, device=device)
        cs = self._cs
        compute = torch.cuda.current_stream(device)
        copier = torch.cuda.Stream(device)          # default priority
        dev = [torch.empty((cs, d), dtype=torch.float32, device=device) for _ in range(2)]
        pinned_src = X.is_pinned()
        stage = None if pinned_src else [torch.empty((cs, d), dtype=torch.float32,
                                                     pin_memory=True) for _ in range(2)]
        copied = [torch.cuda.Event() for _ in range(2)]
        used = [torch.cuda.Event() for _ in range(2)]
        for ci, start in enumerate(range(0, N, cs)):
            b = ci & 1
            rows = min(cs, N - start)
            if ci >= 2 and not pinned_src:
                copied[b].synchronize()                 # staging buffer b is free again
            src = X[start:start + rows] if pinned_src else stage[b][:rows]
            if not pinned_src:
                src.copy_(X[start:start + rows])
            with torch.cuda.stream(copier):
                if ci >= 2:
                    copier.wait_event(used[b])          # device buffer b is free again
                dev[b][:rows].copy_(src, non_blocking=True)
                copied[b].record(copier)
            compute.wait_event(copied[b])
            self._chunk(lib, dev[b][:rows], rows, K, d, ln[start:start + rows],
                        compute.cuda_stream)
            used[b].record(compute)
        out = self._end(lib, N, K, d, device)
        compute.synchronize()                           # staging/device buffers outlive the copies
        return (*out, ln)


StreamingGMM = StreamingFlashGMMAsync
