"""The allocation-free LUT forward (``slg_fc_lut_soft_fwd_noalloc``) against
the workspace entry point (``slg_fc_lut_soft_fwd``), through the C ABI.

Both run the same kernels on the same records, so the outputs must be the
same bits. Two calls in a row, the second on a smaller layer and batch,
check that the static scratch keeps no state that leaks into the next call.
"""
import ctypes

import pytest
import torch

from silogic_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH_FLOATS = 4 << 20


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _layer(B, IN, OUT, n, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand((B, IN), generator=g)
    cand = torch.randint(0, IN, (OUT, n, K), generator=g, dtype=torch.int32)
    w = torch.softmax(torch.randn((OUT, n, K), generator=g), dim=2)
    s = torch.sigmoid(torch.randn((OUT, 2 ** n), generator=g))
    return [t.to(DEV).contiguous() for t in (x, cand, w, s)]


def _with_workspace(x, cand, w, s, hybrid):
    B, IN = x.shape
    OUT, n, K = cand.shape
    lib = _lib.lib()
    ws = lib.slg_fc_lut_soft_workspace(OUT, n, K)
    work = torch.empty(ws, device=DEV, dtype=torch.float32)
    y = torch.empty((B, OUT), device=DEV, dtype=torch.float32)
    _lib.check(lib.slg_fc_lut_soft_fwd(_p(x), B, IN, OUT, n, K, _p(cand), _p(w), _p(s),
                                       int(hybrid), _p(y), _p(work), ws, _stream()),
               "slg_fc_lut_soft_fwd")
    return y


def _no_alloc(x, cand, w, s, hybrid):
    B, IN = x.shape
    OUT, n, K = cand.shape
    y = torch.full((B, OUT), float("nan"), device=DEV, dtype=torch.float32)
    _lib.check(_lib.lib().slg_fc_lut_soft_fwd_noalloc(_p(x), B, IN, OUT, n, K, _p(cand), _p(w),
                                                      _p(s), int(hybrid), _p(y), _stream()),
               "slg_fc_lut_soft_fwd_noalloc")
    return y


@pytest.mark.parametrize("hybrid", [False, True])
@pytest.mark.parametrize("n,K", [(6, 8), (4, 4), (2, 1)])
def test_no_alloc_matches_workspace_entry_point(n, K, hybrid):
    # first call: a large layer (most of the scratch at arity 6); second: a
    # smaller layer and batch, which reads only what the second call wrote
    big_out = 20000 if n == 6 else 9000
    for B, IN, OUT, seed in ((300, 1500, big_out, 1), (37, 700, 333, 2)):
        x, cand, w, s = _layer(B, IN, OUT, n, K, seed)
        print(f"no_alloc n={n} K={K} hybrid={hybrid} B={B} IN={IN} OUT={OUT}", flush=True)
        got = _no_alloc(x, cand, w, s, hybrid)
        ref = _with_workspace(x, cand, w, s, hybrid)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref.cpu()), (n, K, hybrid, B, OUT)


def test_no_alloc_rejects_layers_beyond_the_scratch():
    lib = _lib.lib()
    n, K = 6, 8
    OUT = (SCRATCH_FLOATS // lib.slg_fc_lut_soft_workspace(64, n, K) + 1) * 64
    assert lib.slg_fc_lut_soft_workspace(OUT, n, K) > SCRATCH_FLOATS
    x, cand, w, s = _layer(4, 64, 64, n, K, 3)   # valid pointers; the size check comes first
    rc = lib.slg_fc_lut_soft_fwd_noalloc(_p(x), 4, 64, OUT, n, K, _p(cand), _p(w), _p(s), 0,
                                         _p(x), _stream())
    assert rc == -2, rc
    assert b"static scratch" in lib.slg_last_error()
    # a layer that fits still runs after the rejection
    y = _no_alloc(x, cand, w, s, False)
    assert torch.equal(y.cpu(), _with_workspace(x, cand, w, s, False).cpu())
