"""The training forward's conv path, slg_conv_soft_records_arrays +
slg_conv_soft_fwd_records, against slg_conv_soft_fwd on the same separate
arrays (taps, leaf weights, node parameters): the same bits on every LDS
layout the records take (quad with and without its register staging and
padded lane walk, pair with one channel per chunk and with flat lanes,
phase-split, row-major with and without the swapped window read and with
split scalar/vector records), pooled and not, gate16 / multilinear /
hybrid trees, 4 and 8 taps per leaf."""
import ctypes

import pytest
import torch

import silogic_amd as sl
from silogic_amd import _lib, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("node,arity,depth,K,C,H,N,B,pool", [
    ("gate16", 2, 2, 4, 7, 28, 64, 3, True),        # quad, persistent, padded lane walk
    ("gate16", 2, 2, 4, 13, 24, 8, 3, True),        # quad staged without registers
    ("gate16", 2, 2, 4, 64, 14, 128, 2, True),      # pair, flat lanes
    ("gate16", 2, 2, 4, 40, 16, 24, 2, True),       # pair, one channel per chunk
    ("gate16", 2, 2, 4, 48, 22, 8, 2, True),        # phase-split
    ("gate16", 2, 3, 4, 16, 16, 16, 2, True),       # row-major, 8 leaves
    ("gate16", 2, 2, 4, 6, 12, 10, 3, False),       # unpooled
    ("gate16", 2, 1, 8, 64, 14, 12, 2, True),       # eight taps per leaf
    ("multilinear", 6, 1, 4, 9, 32, 16, 2, True),   # LUT6, split records, 512 threads
    ("multilinear", 6, 1, 4, 128, 16, 24, 2, True),  # swapped window read, 1024 threads
    ("multilinear", 4, 1, 4, 64, 14, 10, 2, True),
    ("hybrid", 2, 1, 4, 64, 14, 10, 2, True),
])
def test_records_from_arrays_give_the_array_kernels_bits(node, arity, depth, K, C, H, N, B,
                                                         pool):
    conv = sl.ConvLogicTree(C, N, kernel=3, tree_depth=depth, connect="topk", k=K, n_chan=2,
                            residual_init=False, seed=C + N + K, node=node, arity=arity,
                            tau=0.7).to(DEV)
    g = torch.Generator().manual_seed(H + N)
    x = torch.rand(B, C, H, H, generator=g).to(DEV)
    with torch.no_grad():
        w, npar = conv.soft_params(True)
        w, npar = w.contiguous().float(), npar.contiguous().float()
        cm, ch, cw = (t.to(torch.int32).contiguous() for t in conv._taps())
        kind = conv._kind()
        Ho = H // 2 if pool else H
        want = torch.empty((B, N, Ho, Ho), device=DEV)
        _lib.call("slg_conv_soft_fwd", ops._p(x), B, C, H, H, N, kind, depth, arity, K,
                  ops._p(npar), ops._p(w), ops._p(cm), ops._p(ch), ops._p(cw), 1, int(pool),
                  ops._p(want), ops._stream(x))
        got = ops._conv_soft_launch(x, npar, w, cm, ch, cw, kind, depth, arity, K, 1, pool)
    assert ops.conv_fits_lds((C, H, H), 1, pool, kind, depth, arity, K)
    assert torch.equal(got, want)
