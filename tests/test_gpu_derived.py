"""Cached derived tables (records, hard codes) on the GPU: a forward after an
in-place weight update or a state-dict load computes with the new weights,
exactly as a fresh model with those weights does."""
import pytest
import torch

import silogic_amd as sl
from conftest import build_product
from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bump(model, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            p.add_(torch.randn(p.shape, generator=g).to(p.device))


@pytest.mark.parametrize("spec", [
    ("LogicNet", dict(in_dim=96, width=300, depth=3, k=8, tau=5.0)),
    ("LogicTreeNet", dict(in_channels=7, in_hw=12, channels=[8, 16], kernel=3, tree_depth=2,
                          connect="topk", k=4, n_chan=2, num_classes=10, head_widths=[40],
                          residual_init=False)),
])
def test_cached_tables_follow_weight_updates(spec):
    model = build_product(spec).to(DEV).eval()
    g = torch.Generator().manual_seed(1)
    if spec[0] == "LogicNet":
        x = torch.bernoulli(torch.full((40, 96), 0.5), generator=g)
    else:
        x = (torch.rand(6, 7, 12, 12, generator=g) > 0.5).float()
    xd = x.to(DEV)
    with torch.no_grad():
        s0, h0 = model(xd).cpu(), model.forward_hard(xd).cpu()
        assert torch.equal(model(xd).cpu(), s0)              # cached tables reused
        _bump(model, 2)
        s1, h1 = model(xd).cpu(), model.forward_hard(xd).cpu()
    sd = {k: v.detach().cpu().clone() for k, v in model.state_dict().items()}
    other = build_product(spec).to(DEV).eval()      # a model that never ran the old weights
    other.load_state_dict(sd)
    with torch.no_grad():
        assert torch.equal(s1, other(xd).cpu())
    assert torch.equal(h1, torch_ref.forward_hard(spec, sd, x))
    assert not torch.equal(s1, s0) and not torch.equal(h1, h0)
    # a state-dict load restores the first weights
    fresh = build_product(spec).to(DEV).eval()
    model.load_state_dict(fresh.state_dict())
    with torch.no_grad():
        assert torch.equal(model(xd).cpu(), fresh(xd).cpu())
        assert torch.equal(model.forward_hard(xd).cpu(), fresh.forward_hard(xd).cpu())
