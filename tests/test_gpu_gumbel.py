"""Walsh layers in training with Gumbel-sigmoid smoothing (nodes.py:145-149):
the kernels give z, the noise is two Gumbel draws per (sample, output) from
torch's generator in the reference's order, so re-seeding reproduces them.
Values and gradients against the oracle fed the same draws."""
import pytest
import torch

from conftest import build_product
from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, ref, rtol, atol, what):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = (got - ref).abs()
    bad = err > rtol * ref.abs() + atol
    assert not bad.any(), f"{what}: {int(bad.sum())} outside tolerance, max {err.max():.3e}"


@pytest.mark.parametrize("ctor,arity", [("WARPNet", 2), ("WARPNetN", 4)])
def test_walsh_gumbel_training_forward_and_gradients(ctor, arity):
    args = dict(in_dim=300, width=200, depth=1, k=4, tau=2.0, gate_select="gumbel")
    if ctor == "WARPNetN":
        args["arity"] = arity
    spec = (ctor, args)
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).train()
    layer = model.layers[0]
    assert not layer.node.plain_softmax()
    L = torch_ref.structure(spec)["layers"][0]
    g = torch.Generator().manual_seed(5)
    B = 37
    x = torch.rand(B, 300, generator=g)
    gy = torch.randn(B, 200, generator=g)

    xd = x.to(DEV).requires_grad_(True)
    torch.cuda.manual_seed(1234)
    out = layer(xd)
    (out * gy.to(DEV)).sum().backward()

    torch.cuda.manual_seed(1234)
    g1 = torch_ref.gumbel((B, 200), DEV).cpu()
    g2 = torch_ref.gumbel((B, 200), DEV).cpu()
    params = {k: v.clone().requires_grad_(v.is_floating_point()) for k, v in sd.items()}
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.fc_layer_soft_gumbel(L, params, xr, g1, g2)
    (ref * gy).sum().backward()

    _close(out, ref, 1e-5, 1e-6, "gumbel-smoothed output")
    # the draws moved the output: a layer without them differs
    with torch.no_grad():
        plain = torch_ref.fc_layer_soft(L, sd, x)
    assert (plain - ref.detach()).abs().max() > 1e-2
    scale = xr.grad.abs().max().item()
    assert (xd.grad.cpu() - xr.grad).abs().max().item() <= 1e-4 * scale + 1e-7
    checked = 0
    for name, p in model.named_parameters():
        rg = params[name].grad
        if rg is None or p.grad is None:
            continue
        s = rg.abs().max().item()
        assert (p.grad.cpu() - rg).abs().max().item() <= 1e-4 * s + 1e-7, name
        checked += 1
    assert checked >= 2       # connection logits and theta
