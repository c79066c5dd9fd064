"""ctypes binding of ``libflashgmm.so`` (the C ABI in ``include/flashgmm.h``).

The library is loaded after torch, so both share the single HIP runtime
torch already mapped (the library's ``libamdhip64.so.7`` dependency resolves
to it by soname).  There is no fallback: if the library is missing the first
call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libflashgmm.so")

FGMM_OK, FGMM_EINVAL, FGMM_EWORKSPACE, FGMM_EHIP = 0, 1, 2, 3
VARIANTS = {"auto": 0, "valu": 1, "mfma": 2, "x32": 3, "mixed": 4, "sparse": 5, "small": 6}

# name -> (argtypes, restype); mirrors include/flashgmm.h
_P, _L, _I, _Z = ctypes.c_void_p, ctypes.c_long, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "fgmm_version": ([], _I),
    "fgmm_last_error": ([], ctypes.c_char_p),
    "fgmm_resolve_variant": ([_L, _I, _I, _I], _I),
    "fgmm_error_model": ([_I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
                         _I),
    "fgmm_workspace_region": ([_L, _I, _I, _I, ctypes.c_char_p, ctypes.POINTER(_Z),
                               ctypes.POINTER(_Z)], _I),
    "fgmm_workspace_bytes": ([_L, _I, _I, _I], _Z),
    "fgmm_em_fused_workspace_bytes": ([_L, _I, _I, _I], _Z),
    "fgmm_em_fit_switch_iteration": ([], _I),
    "fgmm_em_fused": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P, _P, _P, _Z, _P], _I),
    "fgmm_em_fused_noalloc_max_bytes": ([], _Z),
    "fgmm_em_fused_noalloc": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P, _P, _P], _I),
    "fgmm_log_normalizer": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _Z, _P], _I),
    "fgmm_accumulate_stats": ([_P, _P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P, _P, _Z, _P], _I),
    "fgmm_m_step_update": ([_P, _P, _P, _L, _I, _I, _P, _P, _P, _P], _I),
    "fgmm_em_fit": ([_P, _P, _P, _P, _L, _I, _I, _I, _I, _P, _P, _P, _P, _P, _Z, _P], _I),
    "fgmm_flash_e_step": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P, _Z, _P], _I),
    "fgmm_standard_e_step_workspace_bytes": ([_L, _I, _I, _I], _Z),
    "fgmm_standard_e_step": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P, _Z, _P], _I),
    "fgmm_standard_m_step_workspace_bytes": ([_L, _I, _I], _Z),
    "fgmm_standard_m_step": ([_P, _P, _L, _I, _I, _P, _P, _P, _P, _Z, _P], _I),
    "fgmm_stream_workspace_bytes": ([_L, _I, _I, _I], _Z),
    "fgmm_stream_begin": ([_P, _P, _P, _L, _I, _I, _I, _P, _Z, _P], _I),
    "fgmm_stream_chunk": ([_P, _L, _L, _I, _I, _I, _P, _P, _Z, _P], _I),
    "fgmm_stream_end": ([_L, _L, _I, _I, _I, _P, _P, _P, _P, _P, _Z, _P], _I),
    "fgmm_profile_enable": ([_I], _I),
    "fgmm_profile_read": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_long)], _I),
}

# host path (include/flashgmm_cpu.h): host pointers, synchronous, OpenMP
CPU_LIB_PATH = os.path.join(PKG, "libflashgmm_cpu.so")
CPU_SIGNATURES = {
    "fgmm_cpu_last_error": ([], ctypes.c_char_p),
    "fgmm_cpu_em_fused": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P, _P], _I),
    "fgmm_cpu_log_normalizer": ([_P, _P, _P, _P, _L, _I, _I, _I, _P], _I),
    "fgmm_cpu_accumulate_stats": ([_P, _P, _P, _P, _P, _L, _I, _I, _I, _P, _P, _P], _I),
    "fgmm_cpu_m_step_update": ([_P, _P, _P, _L, _I, _I, _P, _P, _P], _I),
    "fgmm_cpu_e_step": ([_P, _P, _P, _P, _L, _I, _I, _I, _P, _P], _I),
    "fgmm_cpu_standard_m_step": ([_P, _P, _L, _I, _I, _I, _P, _P, _P], _I),
    "fgmm_cpu_em_fit": ([_P, _P, _P, _P, _L, _I, _I, _I, _I, _P, _P, _P, _P], _I),
}

_lib = None
_cpu = None
_lock = threading.Lock()


def load(path: str | None = None):
    """Load and type the library once; raises RuntimeError if it is absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"flashgmm_amd: native library not found at {p}; build it with "
            "`python -m flashgmm_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(p)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _lib = lib
    return lib


def load_cpu(path: str | None = None):
    """Load and type the host-path library once; raises RuntimeError if it is
    absent (there is no Python fallback)."""
    global _cpu
    if _cpu is not None and path is None:
        return _cpu
    p = path or CPU_LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"flashgmm_amd: host library not found at {p}; build it with "
            "`python -m flashgmm_amd.build`")
    lib = ctypes.CDLL(p)
    for name, (args, res) in CPU_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _cpu = lib
    return lib


def check_cpu(rc: int) -> None:
    if rc != FGMM_OK:
        msg = load_cpu().fgmm_cpu_last_error().decode(errors="replace")
        raise RuntimeError(f"flashgmm_amd (host): {msg} (code {rc})")


def check(rc: int) -> None:
    if rc != FGMM_OK:
        msg = load().fgmm_last_error().decode(errors="replace")
        raise RuntimeError(f"flashgmm_amd: {msg} (code {rc})")


def variant_code(variant) -> int:
    if variant is None:
        variant = os.environ.get("FLASH_GMM_VARIANT", "auto")
    if isinstance(variant, int):
        return variant
    try:
        return VARIANTS[str(variant).lower()]
    except KeyError:
        raise RuntimeError(f"flashgmm_amd: unknown variant {variant!r} "
                           f"(expected one of {sorted(VARIANTS)})") from None


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# One workspace per (device, stream), grown on demand.  Calls queued on one
# stream reuse it in stream order; the caching allocator frees a replaced
# buffer in stream order too.
_ws: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    key = (device.index, stream_handle(device))
    with _lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            _ws[key] = buf
        return buf
