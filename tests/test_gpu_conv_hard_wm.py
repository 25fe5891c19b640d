"""slg_conv_hard_fwd_wm (word-major, zero-bordered images; LUTs of arity 3-6
evaluated as 3-input functions) and slg_pack_image_wm against
slg_conv_hard_fwd and pack_bits on the reference layout: bit for bit on
every sample b < B, the output border left zero. Cases: gate16 trees of
depth 1-4 and LUT trees of arity 2-6 (random tables: every byte of a LUT6
table takes its own branch); kernels 1-5 and paddings 0-2; output borders
0-2; odd maps (floor pooling); batches that end inside a word; many input
channels; the config blocks' shapes; a large map."""
import pytest
import torch

from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _params(N, C, kernel, leaves, n_chan, g):
    """Leaf codes cm << 8 | ch << 4 | cw (each tree's leaves on n_chan channels,
    or on any channel when n_chan is None) and random truth-table words."""
    if n_chan is None:
        cm = torch.randint(0, C, (N, leaves), generator=g)
    else:
        chans = torch.stack([torch.randperm(C, generator=g)[:n_chan] for _ in range(N)])
        cm = torch.gather(chans, 1, torch.randint(0, n_chan, (N, leaves), generator=g))
    ch = torch.randint(0, kernel, (N, leaves), generator=g)
    cw = torch.randint(0, kernel, (N, leaves), generator=g)
    leaf = (cm << 8 | ch << 4 | cw).to(torch.int32)
    tt = torch.randint(-(1 << 62), 1 << 62, (N,), generator=g, dtype=torch.int64)
    return leaf.to(DEV), tt.to(DEV)


def _check(B, C, H, W, N, kind, depth, arity, kernel, pad, n_chan=2, out_pad=0, seed=0):
    g = torch.Generator().manual_seed(seed)
    nw = ops.n_words(B)
    leaves = 2 ** depth if kind == ops.GATE16 else arity
    leaf, tt = _params(N, C, kernel, leaves, n_chan, g)
    words = torch.randint(-(1 << 62), 1 << 62, (C * H * W, nw), generator=g, dtype=torch.int64)
    xp = words.to(DEV)
    ref = ops.conv_hard(xp.reshape(C, H, W, nw), (C, H, W), leaf, tt, kind, depth, arity,
                        kernel, pad, True)                       # [N, Ho, Wo, nw]
    Ho, Wo = ref.shape[1], ref.shape[2]
    xw = torch.zeros((nw, C, H + 2 * pad, W + 2 * pad), device=DEV, dtype=torch.int64)
    xw[:, :, pad:pad + H, pad:pad + W] = xp.t().reshape(nw, C, H, W)
    got = ops.conv_hard_wm(xw, B, (C, H, W), leaf, tt, kind, depth, arity, kernel, pad,
                           out_pad).cpu()                        # [nw, N, Ho+2op, Wo+2op]
    inner = got[:, :, out_pad:out_pad + Ho, out_pad:out_pad + Wo].reshape(nw, -1)
    border = got.clone()
    border[:, :, out_pad:out_pad + Ho, out_pad:out_pad + Wo] = 0
    assert not border.any(), "the output border was written"
    ref = ref.reshape(-1, nw).t().cpu()
    tail = B - 64 * (nw - 1)                    # valid samples in the last word
    mask = torch.full((nw, 1), -1, dtype=torch.int64)
    if tail < 64:
        mask[-1] = (1 << tail) - 1
    bad = (inner ^ ref) & mask
    assert not bad.any(), f"{int((bad != 0).sum())} words differ"


@pytest.mark.parametrize("depth", [1, 2, 3, 4])
@pytest.mark.parametrize("kernel,pad", [(3, 1), (1, 0), (5, 2), (2, 0)])
def test_gate16_trees(depth, kernel, pad):
    _check(B=200, C=6, H=13, W=11, N=12, kind=ops.GATE16, depth=depth, arity=2,
           kernel=kernel, pad=pad, out_pad=depth % 3, seed=depth * 10 + kernel)


@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
@pytest.mark.parametrize("B", [64, 33, 96 + 7])
def test_lut_trees(arity, B):
    _check(B=B, C=9, H=12, W=12, N=20, kind=ops.MULTILINEAR2, depth=1, arity=arity,
           kernel=3, pad=1, out_pad=1, seed=arity * 100 + B)


def test_every_byte_of_a_lut6_table():
    # 300 channels of random tables: each of the 256 byte values is a table
    # byte of some channel with near certainty (2400 draws)
    _check(B=64, C=5, H=6, W=6, N=300, kind=ops.MULTILINEAR2, depth=1, arity=6, kernel=3,
           pad=1, n_chan=None, seed=5)


@pytest.mark.parametrize("n_chan", [2, None])
def test_many_input_channels(n_chan):
    _check(B=130, C=300, H=8, W=8, N=70, kind=ops.MULTILINEAR2, depth=1, arity=6,
           kernel=3, pad=1, n_chan=n_chan, seed=7)
    _check(B=64, C=1100, H=4, W=6, N=33, kind=ops.GATE16, depth=2, arity=2,
           kernel=3, pad=1, n_chan=n_chan, seed=8)


@pytest.mark.parametrize("shape", [
    (1024 // 8, 7, 28, 28, 64, ops.GATE16, 2, 2),      # config 3 block 0 (a batch slice)
    (1024 // 8, 64, 14, 14, 128, ops.GATE16, 2, 2),    # config 3 block 1
    (1024 // 8, 128, 7, 7, 256, ops.GATE16, 2, 2),     # config 3 block 2
    (512 // 4, 9, 32, 32, 128, ops.MULTILINEAR2, 1, 6),  # config 5 block 0
    (512 // 4, 128, 16, 16, 256, ops.MULTILINEAR2, 1, 6),  # config 5 block 1
])
def test_config_block_shapes(shape):
    B, C, H, W, N, kind, depth, arity = shape
    _check(B=B, C=C, H=H, W=W, N=N, kind=kind, depth=depth, arity=arity, kernel=3, pad=1,
           out_pad=1, seed=B + C)


def test_large_map():
    _check(B=70, C=3, H=200, W=130, N=3, kind=ops.GATE16, depth=1, arity=2, kernel=3, pad=1,
           n_chan=None, seed=12)


@pytest.mark.parametrize("B,pad", [(1, 0), (64, 1), (200, 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.uint8])
def test_pack_image(B, pad, dtype):
    g = torch.Generator().manual_seed(B + pad)
    for (C, H, W) in ((3, 8, 8), (7, 5, 6)):            # vector rows and scalar rows
        x = (torch.rand(B, C, H, W, generator=g) < 0.5).to(dtype).to(DEV)
        got = ops.pack_image_wm(x, pad)
        ref = ops.pack_bits(x.reshape(B, -1), word_major=True).reshape(-1, C, H, W)
        assert torch.equal(got[:, :, pad:pad + H, pad:pad + W], ref)
        border = got.clone()
        border[:, :, pad:pad + H, pad:pad + W] = 0
        assert not border.any()


def test_empty_batch():
    leaf, tt = _params(4, 3, 3, 4, 2, torch.Generator().manual_seed(0))
    xp = torch.zeros((0, 3, 10, 10), device=DEV, dtype=torch.int64)
    out = ops.conv_hard_wm(xp, 0, (3, 8, 8), leaf, tt, ops.GATE16, 2, 2, 3, 1)
    assert out.shape == (0, 4, 4, 4)
