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
            step = model.__dict__["_derived_hard_step"][1]
            assert step is not None
            # the heads evaluate the last conv block themselves: config 5's one
            # layer per (word, class), config 3's two-layer network per word
            assert step.fuses_head == {3: 2, 5: 1}.get(cfg, 0)
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


@pytest.mark.parametrize("cfg,B", [(3, 70), (1, 130)])
def test_hard_step_calls_from_two_threads(cfg, B):
    """Two host threads call forward_hard on one model and one stream with
    different inputs, interleaved: each call returns its own logits (a
    call's launches go out as one run and carry its own pointers)."""
    import threading
    model = build_config(cfg, sl).eval().to(DEV)
    xs = [config_inputs(cfg, B, seed=s).to(DEV) for s in (21, 22)]
    with torch.no_grad():
        refs = [_general(model, x) for x in xs]
        model.forward_hard(xs[0])                      # build the launch sequence once
    torch.cuda.synchronize()
    results = {0: [], 1: []}
    errors = []
    start = threading.Barrier(2)

    def worker(i):
        try:
            start.wait()
            with torch.no_grad():
                for _ in range(40):
                    results[i].append(model.forward_hard(xs[i]))
        except Exception as e:                         # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in (0, 1)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in (0, 1):
        assert len(results[i]) == 40
        for got in results[i]:
            assert torch.equal(got, refs[i])
