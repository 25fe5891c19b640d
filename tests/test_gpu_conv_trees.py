"""Node trees beyond the benchmark configurations, against the oracle (GPU):
walsh trees, multilinear / hybrid LUT trees deeper than one level (the
reference's own test shapes, tests/test_conv.py:58-75 with arity 4 and depth
2), gate16 trees of depth 5, images whose planes exceed LDS, OrPool windows
other than 2, and n-input walsh FC layers.

Bars: soft values within 1e-5 relative (hybrid: equal up to the fp32
rounding of the reference's straight-through sum, and features within
rounding of the 0.5 threshold may take the other LUT entry); hard outputs
bit for bit; gradients within 1e-4 of the largest reference gradient.
"""
import pytest
import torch
import torch.nn.functional as F

import silogic_amd as sl
from oracle import packed_ref, torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-6


def _close(got, ref, what):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = (got - ref).abs()
    bad = err > RTOL * ref.abs() + ATOL
    assert not bad.any(), f"{what}: {int(bad.sum())} values outside tolerance, max {err.max():.3e}"


def _blk(conv, H):
    binary = conv.node_name in ("gate16", "walsh")
    return dict(prefix="", cin=conv.cin, n=conv.n, kernel=conv.kh, depth=conv.d, stride=1,
                padding=conv.padding, connect=conv.connect,
                k=conv.k if conv.connect != "fixed" else 1, node=conv.node_name,
                node_arity=2 if binary else conv.node_arity, leaves=conv.leaves, tau=conv.tau,
                hw=H)


@pytest.mark.parametrize("node,arity,depth,connect,C,H,N,B", [
    ("walsh", 2, 1, "topk", 5, 10, 12, 4),
    ("walsh", 2, 2, "topk", 6, 11, 16, 3),       # odd map (floor pooling)
    ("walsh", 2, 4, "fixed", 4, 8, 8, 3),
    ("multilinear", 4, 2, "topk", 6, 10, 8, 3),  # the reference's test shape
    ("multilinear", 2, 3, "fixed", 3, 8, 8, 5),
    ("multilinear", 3, 3, "topk", 4, 9, 6, 2),   # 27 leaves
    ("multilinear", 6, 2, "topk", 9, 8, 4, 2),   # 36 leaves
    ("hybrid", 4, 2, "topk", 6, 10, 8, 3),
    ("hybrid", 2, 5, "fixed", 3, 8, 6, 2),       # 32 leaves
    ("gate16", 2, 5, "topk", 4, 8, 6, 2),
    ("gate16", 2, 2, "topk", 48, 32, 8, 2),      # 196 KB image: past LDS
    ("gate16", 2, 2, "topk", 13, 24, 8, 3),      # quad layout, staged without registers
    ("gate16", 2, 2, "topk", 7, 16, 10, 300),    # quad layout, persistent: 300 samples
    ("gate16", 2, 2, "topk", 7, 28, 16, 3),      # quad, lanes walking padded rows (14x14 maps)
    # pooled row-major layout with the window's columns swapped on odd pooled
    # columns (the read pattern of config 5's block 1: 128 channels, 16x16)
    ("multilinear", 6, 1, "topk", 128, 16, 24, 2),
    ("multilinear", 6, 1, "fixed", 128, 16, 12, 3),
    ("gate16", 2, 3, "topk", 128, 16, 16, 2),
])
def test_conv_tree_forward_and_hard(node, arity, depth, connect, C, H, N, B):
    conv = sl.ConvLogicTree(C, N, kernel=3, tree_depth=depth, connect=connect, k=4, n_chan=2,
                            residual_init=False, seed=depth + 7, node=node, arity=arity, tau=0.7)
    sd = {k: v.clone() for k, v in conv.state_dict().items()}
    blk = _blk(conv, H)
    g = torch.Generator().manual_seed(C)
    x = torch.rand(B, C, H, H, generator=g)
    xb = (x > 0.5).float()
    ref = torch_ref.conv_soft(blk, sd, x)
    conv = conv.to(DEV).eval()
    with torch.no_grad():
        y = conv(x.to(DEV))
        yp = conv.forward_pooled(x.to(DEV))
        yh = conv.forward_hard(xb.to(DEV)).cpu()
    if node == "hybrid":
        # the LUT value exactly (the reference rounds within an ulp of it)
        assert (y.cpu() - ref).abs().max() <= 1.2e-7
        assert (yp.cpu() - torch_ref.orpool_soft(ref)).abs().max() <= 1.2e-7
    else:
        _close(y, ref, f"{node} a{arity} d{depth}")
        _close(yp, torch_ref.orpool_soft(ref), f"{node} a{arity} d{depth} pooled")
    assert torch.equal(yh, torch_ref.conv_hard(blk, sd, xb))
    # packed network path: conv + OR pool on words, against the packed oracle
    x3 = packed_ref.pack_conv_input(xb.numpy().astype("uint8"))
    want = packed_ref.packed_or_pool(packed_ref.conv_block(blk, sd, x3, H, H), H, H)
    with torch.no_grad():
        got = conv.packed_forward(torch.from_numpy(x3).to(DEV).view(C, H, H, -1), (C, H, H),
                                  pool=True)
    assert torch.equal(got.cpu().view(N, -1, got.shape[-1]), torch.from_numpy(want))


@pytest.mark.parametrize("node", ["walsh", "multilinear", "hybrid"])
def test_conv_net_with_node_trees(node):
    """LogicConvNet with depth-2 node trees (tests/test_conv.py:89-97):
    soft logits, hard counts, and one training step's gradients."""
    spec = ("LogicConvNet", dict(in_channels=6, in_hw=16, channels=[8, 16], head_widths=[40],
                                 tree_depth=2, node=node, arity=4, node_tau=0.5, k=4, head_k=4,
                                 n_chan=2, seed=0, residual_init=False))
    torch.manual_seed(0)
    net = sl.LogicConvNet(**spec[1])
    sd = {k: v.clone() for k, v in net.state_dict().items()}
    g = torch.Generator().manual_seed(2)
    x = (torch.rand(4, 6, 16, 16, generator=g) > 0.5).float()
    net = net.to(DEV).eval()
    with torch.no_grad():
        hard = net.forward_hard(x.to(DEV)).cpu()
        soft = net(x.to(DEV)).cpu()
    assert torch.equal(hard, torch_ref.forward_hard(spec, sd, x))
    assert soft.shape == (4, 10)
    net.head.feature_ste = False
    with torch.no_grad():
        noste = net(x.to(DEV)).cpu()
    ref = torch_ref.forward(spec, sd, x, ste=False)
    tol = 1.2e-7 if node == "hybrid" else 1e-5
    assert (noste - ref).abs().max() <= tol * max(1.0, ref.abs().max().item())
    # gradients reach every parameter (the reference's test_convlayer_node_types)
    net.train()
    net(x.to(DEV)).sum().backward()
    grads = [p.grad for p in net.parameters() if p.requires_grad]
    assert grads and all(gr is not None for gr in grads)
    assert any(gr.abs().sum() > 0 for gr in grads)


@pytest.mark.parametrize("node,arity,depth,K,C,H,N,B", [
    ("gate16", 2, 2, 4, 64, 14, 128, 3),      # config 3 block 1: one 56-lane chunk per channel
    ("gate16", 2, 2, 4, 40, 16, 24, 2),       # 72 lanes per channel: two chunks
    ("gate16", 2, 2, 4, 64, 13, 20, 2),       # odd map (floor pooling)
    ("gate16", 2, 1, 8, 64, 14, 12, 2),       # eight taps per leaf; parameters kept per wave
    ("multilinear", 4, 1, 4, 64, 14, 10, 2),  # LUT4 trees
    ("hybrid", 2, 1, 4, 64, 14, 10, 2),
    ("gate16", 2, 2, 4, 64, 14, 8, 300),      # more samples than workgroups (persistent)
    ("gate16", 2, 2, 4, 128, 7, 256, 3),      # config 3 block 2: 3x3 maps, flat lanes over quad
    ("gate16", 2, 2, 4, 7, 14, 10, 300),      # 7x7 maps of a small image, 300 samples
])
def test_pair_layout(node, arity, depth, K, C, H, N, B):
    """Pooled blocks on the pair layout (two column-shifted copies: images
    whose quad copies exceed LDS, or whose pooled maps fill few lanes of the
    quad kernel's 16-lane groups), one channel per chunk or flat lanes over
    channels: eval (records) and gradient-mode (separate arrays) forwards
    against the oracle."""
    conv = sl.ConvLogicTree(C, N, kernel=3, tree_depth=depth, connect="topk", k=K, n_chan=2,
                            residual_init=False, seed=C + N, node=node, arity=arity, tau=0.7)
    sd = {k: v.clone() for k, v in conv.state_dict().items()}
    g = torch.Generator().manual_seed(C + H)
    x = torch.rand(B, C, H, H, generator=g)
    ref = torch_ref.orpool_soft(torch_ref.conv_soft(_blk(conv, H), sd, x))
    conv = conv.to(DEV).eval()
    with torch.no_grad():
        y = conv.forward_pooled(x.to(DEV))
    yg = conv.forward_pooled(x.to(DEV).requires_grad_(True)).detach()
    for got, what in ((y, "records"), (yg, "arrays")):
        if node == "hybrid":
            assert (got.cpu() - ref).abs().max() <= 1.2e-7, what
        else:
            _close(got, ref, f"{node} a{arity} d{depth} K{K} {what}")


@pytest.mark.parametrize("H,W", [(4, 16), (2, 32), (32, 16), (16, 32)])
def test_lut6_constant_row_stride(H, W):
    """LUT6 trees on 16- and 32-wide maps run with the row stride as a
    compile-time constant, with and without the swapped window read (tiny
    maps, whose chunks span samples, keep the plain order): records and
    gradient-mode forwards against the oracle, non-square maps."""
    C, N, B = 5, 12, 9
    conv = sl.ConvLogicTree(C, N, kernel=3, tree_depth=1, connect="topk", k=4, n_chan=2,
                            residual_init=False, seed=H + W, node="multilinear", arity=6)
    sd = {k: v.clone() for k, v in conv.state_dict().items()}
    x = torch.rand(B, C, H, W, generator=torch.Generator().manual_seed(W))
    ref = torch_ref.orpool_soft(torch_ref.conv_soft(_blk(conv, H), sd, x))
    conv = conv.to(DEV).eval()
    with torch.no_grad():
        y = conv.forward_pooled(x.to(DEV))
    yg = conv.forward_pooled(x.to(DEV).requires_grad_(True)).detach()
    _close(y, ref, f"LUT6 {H}x{W} records")
    _close(yg, ref, f"LUT6 {H}x{W} arrays")


@pytest.mark.parametrize("size", [1, 2, 3, 4])
def test_orpool_any_size(size):
    x = torch.rand(3, 5, 11, 13, generator=torch.Generator().manual_seed(size))
    pool = sl.OrPool(size)
    xd = x.to(DEV).requires_grad_(True)
    y = pool(xd)
    ref = F.max_pool2d(x, size, size)
    assert torch.equal(y.detach().cpu(), ref)
    xb = (x > 0.5).to(torch.uint8)
    assert torch.equal(pool.forward_hard(xb.to(DEV)).cpu(),
                       F.max_pool2d(xb.float(), size, size).to(torch.uint8))
    gy = torch.randn(ref.shape)
    y.backward(gy.to(DEV))
    xr = x.clone().requires_grad_(True)
    F.max_pool2d(xr, size, size).backward(gy)
    assert torch.equal(xd.grad.cpu(), xr.grad)


@pytest.mark.parametrize("arity", [3, 4, 6])
def test_walsh_n_layer_soft_backward_hard(arity):
    """n-input walsh FC nodes (nodes.py:130-156) as the LUT layer of z's corner
    values plus sigmoid(z / tau): soft values, gradients and hard outputs."""
    layer = sl.WARPLayerN(300, 200, arity=arity, k=8, tau=0.8, seed=arity)
    L = dict(prefix="", node="walsh", arity=arity, conn="topk", node_tau=0.8)
    params = {kk: v.clone().requires_grad_(v.is_floating_point())
              for kk, v in layer.state_dict().items()}
    gen = torch.Generator().manual_seed(arity)
    x = torch.rand(37, 300, generator=gen)
    gy = torch.randn(37, 200, generator=gen)
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.fc_layer_soft(L, params, xr)
    (ref * gy).sum().backward()
    layer = layer.to(DEV).train()
    xg = x.to(DEV).requires_grad_(True)
    out = layer(xg)
    _close(out, ref, f"walsh-{arity} soft")
    (out * gy.to(DEV)).sum().backward()
    for got, want, what in ((xg.grad, xr.grad, "x"),
                            (layer.node.theta.grad, params["node.theta"].grad, "theta"),
                            (layer._conn.conn.grad, params["_conn.conn"].grad, "conn")):
        scale = want.abs().max().item()
        assert (got.cpu() - want).abs().max().item() <= 1e-4 * scale + 1e-6, what
    xb = (x > 0.5).float()
    with torch.no_grad():
        hard = layer.forward_hard(xb.to(DEV)).cpu()
    assert torch.equal(hard, torch_ref.fc_layer_hard(L, params, xb))
