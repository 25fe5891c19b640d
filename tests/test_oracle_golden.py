"""Pin the oracle to the reference: every golden vector written by
``tests/golden/make_golden.py`` from the real reference must be reproduced
exactly by the oracle's three independent paths (torch restatement, numpy
bit-packed restatement, per-node LUT simulation)."""
import numpy as np
import pytest
import torch

from oracle import lut_sim, packed_ref, torch_ref


def _hybrid(fixture):
    return fixture.spec[1].get("node") == "hybrid"


def _same(got, ref, fixture, what):
    """Bit-identical, except that a hybrid node's value is the LUT entry
    exactly in the oracle (the reference's fused kernels,
    kernels/multilinear.py:40-61, conv_hybrid.py:34-120) where the reference's
    PyTorch path computes f_disc + f_soft - f_soft.detach() (nodes.py:202-206),
    which rounds to within an ulp of it: there the bar is 1.2e-7 absolute
    (values lie in [0, 1])."""
    if _hybrid(fixture):
        err = (got - ref).abs().max().item() if got.numel() else 0.0
        assert got.shape == ref.shape and err <= 1.2e-7, (what, err)
    else:
        assert torch.equal(got, ref), what


def test_soft_logits_bit_exact(fixture):
    """Soft logits (feature STE on, the reference default) are bit-identical."""
    out = torch_ref.forward(fixture.spec, fixture.sd, fixture.x)
    assert torch.equal(out, fixture.arrays["logits_soft"])


def test_soft_logits_without_ste(fixture):
    out = torch_ref.forward(fixture.spec, fixture.sd, fixture.x, ste=False)
    _same(out, fixture.arrays["logits_soft_noste"], fixture, "logits_soft_noste")


def test_every_soft_activation_bit_exact(fixture):
    tr = {}
    torch_ref.forward(fixture.spec, fixture.sd, fixture.x, trace=tr)
    keys = [k for k in fixture.arrays if k.startswith(("act/", "conv/", "pool/"))]
    assert keys
    for k in keys:
        _same(tr[k], fixture.arrays[k], fixture, k)


def test_hard_logits_and_activations_exact(fixture):
    tr = {}
    out = torch_ref.forward_hard(fixture.spec, fixture.sd, fixture.x, trace=tr)
    assert torch.equal(out, fixture.arrays["logits_hard"])
    for k in [k for k in fixture.arrays if k.startswith(("hact/", "hconv/"))]:
        assert torch.equal(tr[k], fixture.arrays[k]), k


def test_packed_oracle_matches_reference_hard_logits(fixture):
    out = packed_ref.forward_hard(fixture.spec, fixture.sd, fixture.x.numpy())
    np.testing.assert_array_equal(out, fixture.arrays["logits_hard"].numpy())


def test_lut_simulation_matches_reference_hard_logits(fixture):
    if fixture.kind != "fc":
        pytest.skip("the per-node LUT simulator covers FC networks (fpga/circuit.py)")
    layers, C = lut_sim.extract(fixture.spec, fixture.sd)
    scores = lut_sim.simulate(layers, C, fixture.x.numpy())
    np.testing.assert_array_equal(scores, fixture.arrays["logits_hard"].numpy())


def test_gate_count_matches_reference_definition():
    """num_gates = width*depth (models.py:103-104); conv gate_count sums trees at
    every pre-pool position plus head widths (models.py:277-288)."""
    assert torch_ref.num_gates(("LogicNet", dict(in_dim=784, width=10000, depth=6))) == 60000
    spec3 = ("LogicTreeNet", dict(in_channels=7, in_hw=28, channels=[64, 128, 256], kernel=3,
                                  tree_depth=2, k=4, n_chan=2, head_widths=[2560, 2560]))
    assert torch_ref.num_gates(spec3) == 64 * 28 * 28 * 3 + 128 * 14 * 14 * 3 + 256 * 7 * 7 * 3 + 5120
