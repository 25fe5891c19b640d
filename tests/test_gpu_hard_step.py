"""forward_hard as a cached launch sequence (models._HardStep): the logits are
the general path's bit for bit (conv networks: packing, then
forward_hard_packed; FC networks: the fused network on rows or packed
words), on fp32 and uint8 inputs, over successive calls with new inputs (the
intermediate buffers are reused), and on another stream (a sequence of its
own)."""
import pytest
import torch

import silogic_amd as sl
from silogic_amd import ops
from silogic_amd.synthetic import build_config, config_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _general(model, x):
    if x.dim() == 2:                 # FC: the packed-input path of the same network
        return model.forward_hard_packed(ops.pack_bits(x), x.shape[0])
    B, C, H, W = x.shape
    return model.forward_hard_packed(ops.pack_bits(x.reshape(B, -1)), B, (C, H, W))


@pytest.mark.parametrize("cfg,B", [(3, 70), (5, 33), (1, 130), (4, 100)])
def test_hard_step_matches_the_general_path(cfg, B):
    model = build_config(cfg, sl).eval().to(DEV)
    with torch.no_grad():
        for seed in (3, 4, 5):
            x = config_inputs(cfg, B, seed=seed).to(DEV)
            got = model.forward_hard(x)
            assert model.__dict__["_derived_hard_step"][1] is not None
            assert torch.equal(got, _general(model, x))
            x8 = x.to(torch.uint8)
            assert torch.equal(model.forward_hard(x8), got)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            got_side = model.forward_hard(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert torch.equal(got_side, _general(model, x))


def test_fc_hard_step_with_a_wire_residual():
    model = sl.LogicNet(in_dim=200, width=640, depth=3, num_classes=10, k=8,
                        wire_residual=0.25, seed=3).eval().to(DEV)
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        for B in (64, 77):
            x = (torch.rand(B, 200, generator=g) < 0.5).float().to(DEV)
            assert torch.equal(model.forward_hard(x), _general(model, x))
            assert model.__dict__["_derived_hard_step"][1] is not None
