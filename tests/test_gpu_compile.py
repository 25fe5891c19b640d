"""``torch.compile`` of the networks (the reference's training loop compiles
its model by default, silogic/train.py:134), on the GPU.

With gradients every HIP launch of the module path runs as a
``torch.ops.silogic_hip`` custom operator, so dynamo traces a training step
as one graph (``fullgraph=True``: no break at a ctypes call). With the
``aot_eager`` backend the compiled step runs the same kernels on the same
arguments as eager mode, so the loss and every gradient are the same bits.
"""
import pytest
import torch

from conftest import build_product
from silogic_amd.synthetic import cfg3_images

pytestmark = pytest.mark.gpu
DEV = "cuda"

SPECS = {
    "logicnet": ("LogicNet", dict(in_dim=96, width=300, depth=3, k=8, tau=5.0)),
    "warpnet": ("WARPNet", dict(in_dim=96, width=300, depth=2, k=8)),
    "logictreenet": ("LogicTreeNet", dict(in_channels=7, in_hw=12, channels=[8, 16], kernel=3,
                                          tree_depth=2, connect="topk", k=4, n_chan=2,
                                          num_classes=10, head_widths=[40, 40],
                                          residual_init=False)),
}


def _inputs(name):
    g = torch.Generator().manual_seed(3)
    if name == "logictreenet":
        return cfg3_images(6, 12, g)
    return torch.bernoulli(torch.full((40, 96), 0.5), generator=g)


def _grads(model, fwd, x, y):
    for p in model.parameters():
        p.grad = None
    loss = torch.nn.functional.cross_entropy(fwd(x), y)
    loss.backward()
    return loss.detach(), [p.grad.clone() for p in model.parameters() if p.requires_grad]


@pytest.mark.parametrize("name", sorted(SPECS))
def test_compiled_training_step_matches_eager(name):
    model = build_product(SPECS[name]).to(DEV).train()
    x = _inputs(name).to(DEV)
    y = torch.arange(x.shape[0], device=DEV) % 10
    loss_e, grads_e = _grads(model, model, x, y)
    compiled = torch.compile(model, backend="aot_eager", fullgraph=True)
    loss_c, grads_c = _grads(model, compiled, x, y)
    assert torch.equal(loss_c, loss_e)
    assert len(grads_c) == len(grads_e) > 0
    for i, (gc, ge) in enumerate(zip(grads_c, grads_e)):
        assert torch.equal(gc, ge), i
