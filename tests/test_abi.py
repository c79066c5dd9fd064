"""The C ABI without a GPU: the library loads, exports every symbol
include/flashgmm.h declares, and rejects bad arguments before queuing any
device work (these calls never reach the HIP runtime)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashgmm.h")
LIB = os.path.join(ROOT, "flashgmm_amd", "libflashgmm.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fgmm_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run python -m flashgmm_amd.build")
    from flashgmm_amd import _lib
    return _lib.load()


def test_header_declares_entry_points():
    names = declared()
    for must in ("fgmm_em_fused", "fgmm_log_normalizer", "fgmm_accumulate_stats",
                 "fgmm_m_step_update", "fgmm_em_fit", "fgmm_workspace_bytes",
                 "fgmm_flash_e_step", "fgmm_standard_e_step", "fgmm_standard_m_step"):
        assert must in names


def test_every_declared_symbol_exported(lib):
    raw = ctypes.CDLL(LIB)
    for name in declared():
        assert hasattr(raw, name), f"{name} declared in flashgmm.h but not exported"


def test_python_signatures_cover_header():
    from flashgmm_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared()


def test_version_and_variant_table(lib):
    assert lib.fgmm_version() >= 100
    # matrix cores from K >= 8 and d <= 128 (with the x32 log-normalizer
    # pass from K >= 256), vector ALU otherwise
    assert lib.fgmm_resolve_variant(65536, 256, 128, 0) == 5
    assert lib.fgmm_resolve_variant(262144, 128, 64, 0) == 5
    assert lib.fgmm_resolve_variant(4096, 64, 32, 0) == 2
    assert lib.fgmm_resolve_variant(65536, 9000, 64, 0) == 4        # K > 8192: mixed
    assert lib.fgmm_resolve_variant(1 << 27, 256, 64, 0) == 4       # N * 16 >= 2^31
    assert lib.fgmm_resolve_variant(4096, 8, 32, 0) == 6          # small: one launch
    assert lib.fgmm_resolve_variant(4096, 7, 32, 0) == 6
    assert lib.fgmm_resolve_variant(65536, 8, 32, 0) == 2         # too many workgroups
    assert lib.fgmm_resolve_variant(65536, 7, 32, 0) == 1
    assert lib.fgmm_resolve_variant(4096, 33, 32, 0) == 2         # K > 32
    assert lib.fgmm_resolve_variant(4096, 8, 65, 0) == 2          # d > 64
    assert lib.fgmm_resolve_variant(4096, 64, 200, 0) == 1
    assert lib.fgmm_resolve_variant(4096, 8, 32, 1) == 1          # forced vector ALU


def test_workspace_bytes(lib):
    for N, K, d in ((4096, 8, 32), (65536, 256, 128), (1048576, 512, 128), (1, 1, 1), (5, 3, 256)):
        for v in (0, 1, 2, 4, 5):
            if v in (2, 4, 5) and d > 128:
                assert lib.fgmm_workspace_bytes(N, K, d, v) == 0
                continue
            b = lib.fgmm_workspace_bytes(N, K, d, v)
            assert b > 0 and b % 256 == 0
            assert b >= 8 * N      # holds the fp64 log-normalizer at least
    assert lib.fgmm_workspace_bytes(0, 8, 32, 0) == 0
    assert lib.fgmm_workspace_bytes(10, 8, 257, 0) == 0


def test_fused_workspace_bytes(lib):
    """The fused iteration's workspace is what it validates against, never
    more than the all-entry-point figure, and within 2 x |X| for the sparse
    default at C2, C4 and C5 (lists, sorted runs sharing the lists' values,
    piece rows, dense-fallback rows sized from device counts)."""
    for N, K, d in ((4096, 8, 32), (65536, 256, 128), (262144, 128, 64), (65536, 1024, 64),
                    (1048576, 512, 128), (1, 1, 1), (5, 3, 256)):
        for v in (0, 1, 2, 4, 5):
            full = lib.fgmm_workspace_bytes(N, K, d, v)
            b = lib.fgmm_em_fused_workspace_bytes(N, K, d, v)
            assert (b == 0) == (full == 0)
            assert b <= full and b % 256 == 0
    for N, K, d in ((65536, 256, 128), (65536, 1024, 64), (1048576, 512, 128)):
        assert lib.fgmm_em_fused_workspace_bytes(N, K, d, 0) <= 2 * 4 * N * d
    assert lib.fgmm_em_fused_workspace_bytes(0, 8, 32, 0) == 0


def test_estep_workspace_bytes(lib):
    for N, K, d in ((4096, 8, 32), (65536, 256, 128), (5, 3, 256), (1, 1, 1)):
        # the E-steps run the fp64 matrix-core (or vector) layout
        base = lib.fgmm_workspace_bytes(N, K, d, 2 if (d <= 128 and K >= 8) else 1)
        std = lib.fgmm_standard_e_step_workspace_bytes(N, K, d, 0)
        assert std % 256 == 0 and std >= base + 8 * N * K   # + the fp64 N x K matrix
        # x32 has no gamma-returning form: it runs as the MFMA path
        if d <= 128:
            assert (lib.fgmm_standard_e_step_workspace_bytes(N, K, d, 3)
                    == lib.fgmm_standard_e_step_workspace_bytes(N, K, d, 2))
        m = lib.fgmm_standard_m_step_workspace_bytes(N, K, d)
        assert m > 0 and m % 256 == 0
    assert lib.fgmm_standard_e_step_workspace_bytes(10, 3, 200, 2) == 0
    assert lib.fgmm_standard_m_step_workspace_bytes(10, 0, 8) == 0
    assert lib.fgmm_standard_m_step_workspace_bytes(10, 3, 257) == 0


def test_estep_argument_errors(lib):
    ws = 1 << 30
    for fn in (lib.fgmm_flash_e_step, lib.fgmm_standard_e_step):
        assert fn(0x1000, 0x1000, 0x1000, 0x1000, 0, 4, 8, 0, 0x1000, 0x1000, 0x1000, ws,
                  None) == 1 and b"N must be" in lib.fgmm_last_error()
        assert fn(0x1000, 0x1000, 0x1000, 0x1000, 10, 4, 8, 0, None, 0x1000, 0x1000, ws,
                  None) == 1 and b"gamma must not be NULL" in lib.fgmm_last_error()
        assert fn(0x1000, 0x1000, 0x1000, 0x1000, 10, 4, 8, 0, 0x1000, 0x1000, 0x1000, 64,
                  None) == 2 and b"too small" in lib.fgmm_last_error()
    f = lib.fgmm_standard_m_step
    assert f(0x1000, None, 10, 4, 8, 0x1000, 0x1000, 0x1000, 0x1000, ws, None) == 1
    assert b"gamma must not be NULL" in lib.fgmm_last_error()
    assert f(0x1000, 0x1000, 10, 4, 300, 0x1000, 0x1000, 0x1000, 0x1000, ws, None) == 1
    assert f(0x1000, 0x1000, 10, 4, 8, 0x1000, 0x1000, 0x1000, 0x1001, ws, None) == 2


def _em(lib, N=100, K=4, d=8, variant=0, ws=0x1000, wsb=1 << 30, null=None):
    p = [0x1000] * 8
    if null is not None:
        p[null] = None
    return lib.fgmm_em_fused(p[0], p[1], p[2], p[3], N, K, d, variant, p[4], p[5], p[6], p[7],
                             ws, wsb, None)


def test_argument_errors_before_device_work(lib):
    assert _em(lib, N=0) == 1 and b"N must be" in lib.fgmm_last_error()
    assert _em(lib, K=0) == 1 and b"K must be" in lib.fgmm_last_error()
    assert _em(lib, d=0) == 1 and b"d must be" in lib.fgmm_last_error()
    assert _em(lib, d=257) == 1 and b"d must be" in lib.fgmm_last_error()
    assert _em(lib, d=200, variant=2) == 1 and b"MFMA" in lib.fgmm_last_error()
    assert _em(lib, variant=9) == 1 and b"variant" in lib.fgmm_last_error()
    assert _em(lib, d=200, variant=4) == 1 and b"mixed" in lib.fgmm_last_error()
    assert _em(lib, d=200, variant=5) == 1 and b"sparse" in lib.fgmm_last_error()
    assert _em(lib, K=8193, variant=5) == 1 and b"sparse" in lib.fgmm_last_error()
    assert _em(lib, K=33, variant=6) == 1 and b"small" in lib.fgmm_last_error()
    assert _em(lib, d=65, variant=6) == 1 and b"small" in lib.fgmm_last_error()
    assert _em(lib, N=32257, variant=6) == 1 and b"small" in lib.fgmm_last_error()
    for i in range(8):
        assert _em(lib, null=i) == 1 and b"must not be NULL" in lib.fgmm_last_error()
    assert _em(lib, ws=None) == 2 and b"NULL" in lib.fgmm_last_error()
    assert _em(lib, ws=0x1001) == 2 and b"aligned" in lib.fgmm_last_error()
    assert _em(lib, wsb=16) == 2 and b"too small" in lib.fgmm_last_error()
    assert lib.fgmm_em_fit(1, 1, 1, 1, 100, 4, 8, 0, 0, 1, 1, 1, 1, 0x1000, 1 << 30, None) == 1
    assert b"iters" in lib.fgmm_last_error()
    assert lib.fgmm_m_step_update(None, 1, 1, 10, 4, 8, 1, 1, 1, None) == 1


def test_python_errors_mirror_reference():
    """The reference's TORCH_CHECKs (binding.cpp:38-39,54,65,80) and this
    module's extra checks raise RuntimeError before any work; CPU tensors are
    served by the host path (tests/test_cpu_path.py), other devices refused."""
    import torch
    from flashgmm_amd import flash_gmm_native as C
    X = torch.zeros(10, 4)
    mu, var, lp = torch.zeros(2, 4), torch.ones(2, 4), torch.zeros(2)
    with pytest.raises(RuntimeError, match="X must be float32"):
        C.flash_em_fused(X.double(), mu, var, lp)
    with pytest.raises(RuntimeError, match="X must be 2D"):
        C.flash_log_normalizer(X[0], mu, var, lp)
    with pytest.raises(RuntimeError, match="ROCm device or the CPU"):
        C.flash_em_fused(X.to("meta"), mu.to("meta"), var.to("meta"), lp.to("meta"))
    with pytest.raises(RuntimeError, match="BN and BK"):
        C.flash_em_fused(X, mu, var, lp, 0, 8)
    for fn in (C.standard_e_step, C.flash_e_step):
        with pytest.raises(RuntimeError, match="X must be float32"):
            fn(X.double(), mu, var, lp)
        with pytest.raises(RuntimeError, match="log_pi must be"):
            fn(X, mu, var, lp[:1])
    with pytest.raises(RuntimeError, match="X must be float32"):
        C.standard_m_step(X.double(), torch.zeros(10, 2))
    with pytest.raises(RuntimeError, match="gamma must be"):
        C.standard_m_step(X, torch.zeros(9, 2))
    with pytest.raises(RuntimeError, match="BK must be"):
        C.flash_e_step(X, mu, var, lp, BK=0)
    with pytest.raises(RuntimeError, match="unknown variant"):
        from flashgmm_amd import _lib
        _lib.variant_code("fast")


def test_stream_argument_errors(lib):
    ws = 1 << 30
    b = lib.fgmm_stream_workspace_bytes(1000, 8, 16, 0)
    assert b > 0 and b % 256 == 0
    assert lib.fgmm_stream_workspace_bytes(1000, 8, 16, 3) == lib.fgmm_stream_workspace_bytes(1000, 8, 16, 2)
    assert lib.fgmm_stream_workspace_bytes(0, 8, 16, 0) == 0
    # a chunk larger than the chunk size the workspace was made for
    assert lib.fgmm_stream_chunk(0x1000, 1001, 1000, 8, 16, 0, None, 0x1000, ws, None) == 1
    assert b"chunk rows" in lib.fgmm_last_error()
    assert lib.fgmm_stream_chunk(None, 10, 1000, 8, 16, 0, None, 0x1000, ws, None) == 1
    assert lib.fgmm_stream_chunk(0x1000, 10, 1000, 8, 16, 0, None, 0x1000, 64, None) == 2
    assert lib.fgmm_stream_end(0, 1000, 8, 16, 0, 0x1000, 0x1000, 0x1000, None, 0x1000, ws, None) == 1
    assert lib.fgmm_stream_begin(None, 0x1000, 0x1000, 1000, 8, 16, 0, 0x1000, ws, None) == 1


def test_streaming_python_errors():
    import torch
    from flashgmm_amd import streaming
    X = torch.zeros(10, 4)
    mu, var, lp = torch.zeros(2, 4), torch.ones(2, 4), torch.zeros(2)
    with pytest.raises(RuntimeError, match="X must be float32"):
        streaming.StreamingFlashGMM(4).em_step(X.double(), mu, var, lp)
    with pytest.raises(RuntimeError, match="ROCm device"):
        streaming.StreamingFlashGMMAsync(4).em_step(X, mu, var, lp)
    with pytest.raises(RuntimeError, match="chunk_size"):
        streaming.StreamingFlashGMM(0)
