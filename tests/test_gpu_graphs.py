"""forward_hard replayed from a captured HIP graph (silogic_amd.graphs):
every replay, with new input contents and eager work and synchronisations
between replays, gives the eager result bit for bit (the path records no
memset node, allocation or host read)."""
import pytest
import torch

import silogic_amd as sl
from silogic_amd.graphs import CapturedForward
from silogic_amd.synthetic import build_config, config_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("cfg,B", [(1, 256), (2, 64 * 5 + 3), (3, 64), (5, 32)])
def test_captured_forward_hard_replays_match_eager(cfg, B):
    model = build_config(cfg, sl).eval().to(DEV)
    xs = [config_inputs(cfg, B, seed=s).to(DEV) for s in (11, 12, 13)]
    static = xs[0].clone()
    cap = CapturedForward(model.forward_hard, static)
    for x in xs + xs[:1]:
        with torch.no_grad():
            ref = model.forward_hard(x).clone()          # eager work between replays
        torch.cuda.synchronize()
        got = cap(x)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
