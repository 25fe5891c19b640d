"""A whole narrow soft FC network in one launch (slg_fc_soft_net_records):
the same bits as a launch per layer on the same records (activations, and
the STE GroupSum logits), and the oracle within 1e-5 through the module."""
import pytest
import torch

import silogic_amd as sl
from conftest import build_product
from oracle import torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _per_layer(model, x, recs, K, head):
    h = x
    for layer, rec in zip(model.layers, recs):
        h = ops.fc_soft_rec(h, rec, layer.in_dim, layer.out_dim, K, layer.node.kind,
                            layer._inv_tau())
    if head:   # on the host: torch's GPU division by a scalar multiplies by its reciprocal
        C = model.head.num_classes
        h = h.cpu()
        per = h.shape[1] // C
        counts = (h > 0.5).float().view(h.shape[0], C, per).sum(2)
        return counts / model.head.tau
    return h


@pytest.mark.parametrize("node,K,widths,C,B", [
    ("gate16", 8, [2000, 2000, 2000], 10, 256),
    ("walsh", 8, [1000, 300], 10, 37),
    ("gate16", 4, [600, 640, 1280], 5, 130),
    ("multilinear", 8, [500, 500], 10, 64),
])
@pytest.mark.parametrize("head", [True, False])
def test_fused_soft_network_matches_per_layer_launches(node, K, widths, C, B, head):
    in_dim = 784
    model = sl.LogicNet(in_dim, widths[0], len(widths), num_classes=C, k=K, node=node,
                        tau=3.0, seed=0)
    # other widths per layer
    if len(set(widths)) > 1:
        layers, d = [], in_dim
        for i, w in enumerate(widths):
            layers.append(sl.LogicLayer(d, w, node=node, k=K, seed=100 + i))
            d = w
        model.layers = torch.nn.ModuleList(layers)
    model = model.to(DEV).eval()
    g = torch.Generator().manual_seed(B)
    x = torch.rand(B, in_dim, generator=g).to(DEV)
    recs = ops.fc_soft_records([l.record_spec() for l in model.layers], K)
    spec = [(rec, l.in_dim, l.out_dim, K, l.node.kind, l._inv_tau())
            for l, rec in zip(model.layers, recs)]
    plan = ops.SoftStackPlan(spec, B, in_dim,
                             (C, float(model.head.tau)) if head else None, 0)
    assert plan.net is not None                 # the one-launch path is taken
    with torch.no_grad():
        got = plan(x)
        ref = _per_layer(model, x, recs, K, head)
    assert torch.equal(got.cpu(), ref.cpu())


def test_config_1_soft_forward_runs_one_launch_and_matches_the_oracle():
    from silogic_amd.synthetic import CONFIGS, build_config, config_inputs
    model = build_config(1, sl).eval()
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    x = config_inputs(1, 256)
    with torch.no_grad():
        got = model(x.to(DEV)).cpu()
    plan = model.layers[0].__dict__["_derived_soft_plan"][1]
    assert plan is not None and plan.net is not None
    ref = torch_ref.forward(CONFIGS[1], sd, x)
    # logits are counts / tau: a feature within fp32 rounding of 0.5 may flip
    diff = (got - ref).abs() * model.head.tau
    assert diff.max().item() <= 2.0 and (diff > 0).float().mean().item() < 0.01


@pytest.mark.parametrize("node,widths,C,B", [
    ("gate16", [6000, 6000, 4000], 10, 4 * 256 + 3),      # 4-sample tiles, 12 chunks per wave
    ("multilinear", [10000, 8000], 10, 4 * 256 + 7),      # 4-sample tiles, 20 chunks per wave
    ("walsh", [12000, 9000, 12000], 6, 2 * 256 + 1),      # 2-sample tiles, 32 chunks per wave
    ("gate16", [16000, 7000], 5, 2 * 300),                # 2-sample tiles, 16 chunks per wave
])
@pytest.mark.parametrize("head", [True, False])
def test_tiled_soft_network_matches_per_layer_launches(node, widths, C, B, head):
    """Layers too wide for two LDS buffers and a batch that gives every CU a
    tile: the network runs one tile per workgroup through every layer with
    one LDS buffer (slg_fc_soft_net_records' second kernel), the same bits as
    a launch per layer."""
    in_dim, K = 784, 8
    layers, d = [], in_dim
    for i, w in enumerate(widths):
        layers.append(sl.LogicLayer(d, w, node=node, k=K, seed=200 + i))
        d = w
    model = sl.LogicNet(in_dim, widths[0], len(widths), num_classes=C, k=K, node=node,
                        tau=3.0, seed=0)
    model.layers = torch.nn.ModuleList(layers)
    model = model.to(DEV).eval()
    g = torch.Generator().manual_seed(B)
    x = torch.rand(B, in_dim, generator=g).to(DEV)
    recs = ops.fc_soft_records([l.record_spec() for l in model.layers], K)
    spec = [(rec, l.in_dim, l.out_dim, K, l.node.kind, l._inv_tau())
            for l, rec in zip(model.layers, recs)]
    plan = ops.SoftStackPlan(spec, B, in_dim,
                             (C, float(model.head.tau)) if head else None, 0)
    assert plan.net is not None                 # the one-launch path is taken
    with torch.no_grad():
        got = plan(x)
        ref = _per_layer(model, x, recs, K, head)
    assert torch.equal(got.cpu(), ref.cpu())


@pytest.mark.parametrize("cfg", [2, 4])
def test_wide_config_soft_forward_runs_one_launch(cfg):
    """Configs 2 and 4 at their soft batch take the tiled network kernel."""
    from silogic_amd.synthetic import BATCHES, build_config, config_inputs
    model = build_config(cfg, sl).eval().to(DEV)
    x = config_inputs(cfg, BATCHES[cfg][0]).to(DEV)
    with torch.no_grad():
        model(x)
    plan = model.layers[0].__dict__["_derived_soft_plan"][1]
    assert plan is not None and plan.net is not None
