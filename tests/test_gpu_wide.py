"""FC soft layers whose input rows exceed LDS (IN > 40704 fp32 per sample):
the slab-staged kernel, on the records path (IN <= 65536, 16-bit indices)
and on the separate-array path (wider), against the oracle; one training
step's gradients through the slab-staged backward kernels."""
import pytest
import torch

import silogic_amd as sl
from conftest import build_product
from oracle import torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-6


def assert_soft_close(got, ref, what):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = (got - ref).abs()
    bad = err > RTOL * ref.abs() + ATOL
    assert not bad.any(), f"{what}: {int(bad.sum())} values outside tolerance, max {err.max():.3e}"


@pytest.mark.parametrize("in_dim,node,K", [(65536, "gate16", 8), (70001, "walsh", 8),
                                           (50000, "gate16", 4), (41000, "gate16", 5)])
def test_wide_fc_soft_forward(in_dim, node, K):
    spec = ("LogicNet", dict(in_dim=in_dim, width=1100, depth=1, k=K, node=node, tau=2.0))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    L = torch_ref.structure(spec)["layers"][0]
    g = torch.Generator().manual_seed(in_dim)
    x = torch.rand(13, in_dim, generator=g)      # a partial 4-sample tile
    layer = model.layers[0]
    with torch.no_grad():
        y = layer(x.to(DEV))
        assert not ops.fc_soft_groupsum_supported(13, in_dim, 1100, 10)
        logits = model(x.to(DEV))
    ref = torch_ref.fc_layer_soft(L, sd, x)
    assert_soft_close(y, ref, f"IN={in_dim}")
    assert logits.shape == (13, 10)
    if in_dim <= 65536:   # the separate-array path (natural candidate order) as well
        cand, w, npar = layer.soft_params(False)
        y2 = ops.fc_soft(x.to(DEV), cand, w, npar, layer.node.kind, layer._inv_tau())
        assert_soft_close(y2, ref, f"IN={in_dim} arrays")


@pytest.mark.parametrize("in_dim,node", [(45000, "gate16"), (70001, "walsh")])
def test_wide_fc_soft_training_step(in_dim, node):
    """Gradients of the slab-staged backward (records are not used there)."""
    spec = ("LogicNet", dict(in_dim=in_dim, width=300, depth=1, k=8, node=node, tau=2.0))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).train()
    L = torch_ref.structure(spec)["layers"][0]
    g = torch.Generator().manual_seed(3)
    x = torch.rand(6, in_dim, generator=g)
    gy = torch.randn(6, 300, generator=g)
    layer = model.layers[0]
    xd = x.to(DEV).requires_grad_(True)
    assert ops.fc_soft_bwd_supported(xd, layer.soft_params(False)[0])
    out = layer(xd)
    (out * gy.to(DEV)).sum().backward()
    params = {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in sd.items()}
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.fc_layer_soft(L, params, xr)
    (ref * gy).sum().backward()
    assert_soft_close(out, ref, "wide soft")
    scale = xr.grad.abs().max().item()
    assert (xd.grad.cpu() - xr.grad).abs().max().item() <= 1e-4 * scale + 1e-7
    checked = 0
    for name, p in model.named_parameters():
        rg = params[name].grad
        if rg is None or p.grad is None:
            continue
        scale = rg.abs().max().item()
        err = (p.grad.cpu() - rg).abs().max().item()
        assert err <= 1e-4 * scale + 1e-7, (name, err, scale)
        checked += 1
    assert checked > 0
