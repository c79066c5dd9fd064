"""fgmm_em_fused_noalloc: the fused iteration on the library's static scratch.

The entry point is called directly through the C ABI (ctypes), twice in a
row on one GPU, the second time with a smaller problem, so the second call
runs on scratch that still holds the first call's contents.  Each result
must equal fgmm_em_fused's on a caller workspace bit for bit: the same
kernels run on the same inputs, and nothing in them depends on where the
workspace lives.  A problem too large for the scratch is refused before any
device work.
"""
import ctypes

import numpy as np
import pytest

from parity_util import check_params, oracle_iter, problem, to_dev

pytestmark = pytest.mark.gpu


def _call_noalloc(lib, t, N, K, d, variant, outs, stream):
    return lib.fgmm_em_fused_noalloc(t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(),
                                     t[3].data_ptr(), N, K, d, variant,
                                     *(o.data_ptr() for o in outs), stream)


def _outputs(torch, cuda, N, K, d):
    return [torch.empty((K, d), dtype=torch.float32, device=cuda),
            torch.empty((K, d), dtype=torch.float32, device=cuda),
            torch.empty((K,), dtype=torch.float32, device=cuda),
            torch.empty((N,), dtype=torch.float32, device=cuda)]


# (config, N, variant): the larger problem first, then a smaller one on the
# same scratch; the sparse variant at a size whose workspace fits 64 MiB
CALLS = [((3, 131072), "mixed"), ((1, None), "auto"), ((2, 4096), "sparse"),
         ((1, 1000), "sparse")]


def test_noalloc_matches_workspace_entry_point(cuda):
    import torch
    from flashgmm_amd import _lib
    from flashgmm_amd import flash_gmm_native as C
    lib = _lib.load()
    cap = lib.fgmm_em_fused_noalloc_max_bytes()
    assert cap == 64 << 20
    stream = _lib.stream_handle(cuda)
    for (cid, n), vname in CALLS:
        X, mu, var, lp = problem(cid, n)
        N, d = X.shape
        K = mu.shape[0]
        v = _lib.variant_code(vname)
        need = lib.fgmm_workspace_bytes(N, K, d, v)
        assert 0 < need <= cap, (cid, n, vname, need)
        print(f"[case] noalloc C{cid} N={N} K={K} d={d} variant={vname} "
              f"scratch {need >> 20} MiB", flush=True)
        t = to_dev(cuda, X, mu, var, lp)
        outs = _outputs(torch, cuda, N, K, d)
        _lib.check(_call_noalloc(lib, t, N, K, d, v, outs, stream))
        ref = C.flash_em_fused(*t, variant=vname)
        torch.cuda.synchronize(cuda)
        for a, b in zip(outs, ref):
            assert torch.equal(a, b), f"C{cid} N={N} {vname}: differs from fgmm_em_fused"
        if n is None or cid == 1:
            m64, v64, l64, *_ = oracle_iter(cid, n)
            check_params([o.cpu().numpy() for o in outs[:3]], (m64, v64, l64),
                         f"noalloc C{cid} {vname}")


def test_noalloc_refuses_problems_beyond_the_scratch(cuda):
    import torch
    from flashgmm_amd import _lib
    lib = _lib.load()
    N, K, d = 1 << 20, 512, 128   # the sparse workspace is far above 64 MiB
    v = _lib.variant_code("sparse")
    assert lib.fgmm_workspace_bytes(N, K, d, v) > lib.fgmm_em_fused_noalloc_max_bytes()
    x = torch.zeros(16, dtype=torch.float32, device=cuda)   # never read: refused first
    p = x.data_ptr()
    rc = lib.fgmm_em_fused_noalloc(p, p, p, p, N, K, d, v, p, p, p, p,
                                   _lib.stream_handle(cuda))
    assert rc == _lib.FGMM_EWORKSPACE
    assert b"allocation-free" in lib.fgmm_last_error()
