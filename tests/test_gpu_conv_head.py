"""slg_conv_hard_head_wm: the last pooled conv block evaluated inside a
one-layer head (each (word, class) workgroup computes only the conv outputs
its gates read) against slg_conv_hard_fwd_wm followed by the head on the
block's output (slg_fc_hard_net / slg_fc_hard_net_typed): the logits bit for
bit. Cases: gate16 trees of depth 1-3 and LUTs of arity 2-6 (random tables,
so every 3-input byte of a LUT6 takes some value); kernels 1-3 with their
paddings; compact codes in index order and type-placed codes; batches that
end inside a word; config 5's block 1 and head shape. The same for
slg_conv_hard_net_wm (the last block inside a multi-layer head network:
gate16 depths 1-3, LUT arities 2-4, config 3's block 2 and head) and its
refusals."""
import pytest
import torch

import silogic_amd as sl
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _conv_params(N, C, kernel, leaves, g):
    chans = torch.stack([torch.randperm(C, generator=g)[:min(2, C)] for _ in range(N)])
    cm = torch.gather(chans, 1, torch.randint(0, chans.shape[1], (N, leaves), generator=g))
    ch = torch.randint(0, kernel, (N, leaves), generator=g)
    cw = torch.randint(0, kernel, (N, leaves), generator=g)
    leaf = (cm << 8 | ch << 4 | cw).to(torch.int32)
    tt = torch.randint(-(1 << 62), 1 << 62, (N,), generator=g, dtype=torch.int64)
    return leaf.to(DEV), tt.to(DEV)


def _check(B, C, H, W, N, kind, depth, arity, kernel, pad, width, n_cls, typed, seed):
    g = torch.Generator().manual_seed(seed)
    leaves = 2 ** depth if kind == ops.GATE16 else arity
    leaf, tt = _conv_params(N, C, kernel, leaves, g)
    nw = ops.n_words(B)
    xw = torch.zeros((nw, C, H + 2 * pad, W + 2 * pad), dtype=torch.int64)
    xw[:, :, pad:pad + H, pad:pad + W] = torch.randint(
        -(1 << 62), 1 << 62, (nw, C, H, W), generator=g, dtype=torch.int64)
    xw = xw.to(DEV)
    Ho, Wo = (H + 2 * pad - kernel + 1) // 2, (W + 2 * pad - kernel + 1) // 2
    in_dim = N * Ho * Wo
    torch.manual_seed(0)
    head = sl.LogicLayer(in_dim, width, k=4, seed=seed).to(DEV)
    codes = ops.fc_hard_codes_net([head.hard_spec()], compact=True)
    if typed:
        codes = ops.fc_hard_type_place_net(codes, in_dim)
        assert codes.plan is not None
    print(f"conv head: B {B} C {C} {H}x{W} N {N} kind {kind} depth {depth} arity {arity} "
          f"kernel {kernel} pad {pad} width {width} classes {n_cls} typed {typed}", flush=True)
    got = ops.conv_hard_head_wm(xw, B, (C, H, W), leaf, tt, kind, depth, arity, kernel, pad,
                                codes, n_cls)
    blk = ops.conv_hard_wm(xw, B, (C, H, W), leaf, tt, kind, depth, arity, kernel, pad, 0)
    want = ops.fc_hard_net(blk.reshape(nw, in_dim), ops.PACKED_WORD_MAJOR, B, in_dim, codes,
                           n_cls)
    torch.cuda.synchronize()
    assert torch.equal(got, want), int((got != want).any(1).sum())


@pytest.mark.parametrize("typed", [False, True])
@pytest.mark.parametrize("depth", [1, 2, 3])
def test_gate16_trees(depth, typed):
    _check(B=100, C=9, H=10, W=12, N=20, kind=ops.GATE16, depth=depth, arity=2, kernel=3,
           pad=1, width=240, n_cls=4, typed=typed, seed=depth)


@pytest.mark.parametrize("typed", [False, True])
@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
def test_lut_trees(arity, typed):
    _check(B=64 + 33, C=12, H=8, W=8, N=40, kind=ops.MULTILINEAR2, depth=1, arity=arity,
           kernel=3, pad=1, width=300, n_cls=10, typed=typed, seed=10 + arity)


@pytest.mark.parametrize("kernel,pad", [(1, 0), (2, 0), (3, 0)])
def test_kernels_and_paddings(kernel, pad):
    _check(B=70, C=5, H=9, W=11, N=16, kind=ops.GATE16, depth=2, arity=2, kernel=kernel,
           pad=pad, width=128, n_cls=8, typed=False, seed=20 + kernel)


@pytest.mark.parametrize("B", [1, 512])
def test_config_5_block_1_and_head(B):
    # 128 -> 256 channels at 16x16, LUT6, pooled to 8x8 (16384 features); head 1280 -> 10
    _check(B=B, C=128, H=16, W=16, N=256, kind=ops.MULTILINEAR2, depth=1, arity=6, kernel=3,
           pad=1, width=1280, n_cls=10, typed=True, seed=5)


def _check_net(B, C, H, W, N, kind, depth, arity, kernel, pad, widths, n_cls, typed, seed):
    """slg_conv_hard_net_wm against slg_conv_hard_fwd_wm + the fused head."""
    g = torch.Generator().manual_seed(seed)
    leaves = 2 ** depth if kind == ops.GATE16 else arity
    leaf, tt = _conv_params(N, C, kernel, leaves, g)
    nw = ops.n_words(B)
    xw = torch.zeros((nw, C, H + 2 * pad, W + 2 * pad), dtype=torch.int64)
    xw[:, :, pad:pad + H, pad:pad + W] = torch.randint(
        -(1 << 62), 1 << 62, (nw, C, H, W), generator=g, dtype=torch.int64)
    xw = xw.to(DEV)
    Ho, Wo = (H + 2 * pad - kernel + 1) // 2, (W + 2 * pad - kernel + 1) // 2
    in_dim = N * Ho * Wo
    torch.manual_seed(0)
    layers, d = [], in_dim
    for i, w in enumerate(widths):
        layers.append(sl.LogicLayer(d, w, k=4, seed=seed + i).to(DEV))
        d = w
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in layers], compact=True)
    if typed:
        codes = ops.fc_hard_type_place_net(codes, in_dim)
        assert codes.plan is not None
    print(f"conv net: B {B} C {C} {H}x{W} N {N} kind {kind} depth {depth} arity {arity} "
          f"kernel {kernel} pad {pad} widths {widths} classes {n_cls} typed {typed}", flush=True)
    got = ops.conv_hard_net_wm(xw, B, (C, H, W), leaf, tt, kind, depth, arity, kernel, pad,
                               codes, n_cls)
    blk = ops.conv_hard_wm(xw, B, (C, H, W), leaf, tt, kind, depth, arity, kernel, pad, 0)
    want = ops.fc_hard_net(blk.reshape(nw, in_dim), ops.PACKED_WORD_MAJOR, B, in_dim, codes,
                           n_cls)
    torch.cuda.synchronize()
    assert torch.equal(got, want), int((got != want).any(1).sum())


@pytest.mark.parametrize("typed", [False, True])
@pytest.mark.parametrize("depth", [1, 2, 3])
def test_net_gate16_trees(depth, typed):
    _check_net(B=100, C=9, H=10, W=12, N=20, kind=ops.GATE16, depth=depth, arity=2, kernel=3,
               pad=1, widths=[1500, 1200, 240], n_cls=4, typed=typed, seed=30 + depth)


@pytest.mark.parametrize("typed", [False, True])
@pytest.mark.parametrize("arity", [2, 3, 4])
def test_net_lut_trees(arity, typed):
    _check_net(B=64 + 33, C=12, H=8, W=8, N=40, kind=ops.MULTILINEAR2, depth=1, arity=arity,
               kernel=3, pad=1, widths=[3000, 300], n_cls=10, typed=typed, seed=40 + arity)


@pytest.mark.parametrize("B", [70, 1024])
def test_config_3_block_2_and_head(B):
    # 128 -> 256 channels at 7x7, gate16 depth 2, pooled to 3x3 (2304 features);
    # head 2560 -> 2560 -> 10
    _check_net(B=B, C=128, H=7, W=7, N=256, kind=ops.GATE16, depth=2, arity=2, kernel=3, pad=1,
               widths=[2560, 2560], n_cls=10, typed=True, seed=3)


def test_net_refuses_wide_heads():
    # activation buffers of 8192 words: not one of the fused kernels' sizes
    from silogic_amd._lib import HipError
    g = torch.Generator().manual_seed(1)
    leaf, tt = _conv_params(8, 4, 3, 4, g)
    xw = torch.zeros((1, 4, 10, 10), dtype=torch.int64, device=DEV)
    layers = [sl.LogicLayer(8 * 16, 8000, k=4, seed=1).to(DEV),
              sl.LogicLayer(8000, 100, k=4, seed=2).to(DEV)]
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in layers], compact=True)
    with pytest.raises(HipError):
        ops.conv_hard_net_wm(xw, 64, (4, 8, 8), leaf, tt, ops.GATE16, 2, 2, 3, 1, codes, 10)


@pytest.mark.parametrize("arity", [5, 6])
def test_net_refuses_luts_past_arity_4(arity):
    from silogic_amd._lib import HipError
    g = torch.Generator().manual_seed(2)
    leaf, tt = _conv_params(8, 4, 3, arity, g)
    xw = torch.zeros((1, 4, 10, 10), dtype=torch.int64, device=DEV)
    layers = [sl.LogicLayer(8 * 16, 1000, k=4, seed=1).to(DEV),
              sl.LogicLayer(1000, 100, k=4, seed=2).to(DEV)]
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in layers], compact=True)
    with pytest.raises(HipError):
        ops.conv_hard_net_wm(xw, 64, (4, 8, 8), leaf, tt, ops.MULTILINEAR2, 1, arity, 3, 1,
                             codes, 10)
