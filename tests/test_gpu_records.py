"""The record path of the FC soft layer (``slg_fc_soft_records`` +
``slg_fc_soft_fwd_records`` / ``slg_fc_soft_fwd_groupsum``) at every sample
tile the kernels instantiate, against the oracle (GPU).

The automatic tile follows the input width: IN <= 1280 -> 4 samples,
1281..5088 -> 8, 5089..10176 -> 4, 10177..20352 -> 2, 20353..40704 -> 1
(rows of S samples must fit 159 KB of LDS). Each width band below selects
one of them, with and without the fused GroupSum head; a forced tile covers
the others at a narrow width. IN > 32767 puts index pairs with idx_b >= 32640
in the records, whose 32-bit words are NaN bit patterns: the decoded pairs
are compared bit for bit.
"""
import pytest
import torch

from conftest import build_product
from oracle import torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-6


def _close(got, ref, what):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    bad = (got - ref).abs() > RTOL * ref.abs() + ATOL
    assert not bad.any(), f"{what}: {int(bad.sum())} values outside tolerance"


def _ste_logits_ok(logits, feats, feats_ref, C, tau):
    B, W = feats.shape
    own = (feats.cpu() > 0.5).float().view(B, C, W // C).sum(2) / tau
    assert torch.equal(logits.cpu(), own)
    flips = (feats.cpu() > 0.5) != (feats_ref > 0.5)
    if flips.any():
        assert ((feats_ref[flips] - 0.5).abs() <= RTOL * 0.5 + ATOL).all()


def _layer(in_dim, width, node, seed=0):
    spec = ("LogicNet", dict(in_dim=in_dim, width=width, depth=1, k=8, node=node, tau=7.0,
                             seed_mult=1000 + seed))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    L = torch_ref.structure(spec)["layers"][0]
    return model.to(DEV).eval(), sd, L


@pytest.mark.parametrize("node", ["gate16", "walsh", "multilinear"])
@pytest.mark.parametrize("tile", [1, 2, 4, 8])
def test_records_every_forced_tile(node, tile):
    model, sd, L = _layer(300, 200, node)
    layer = model.layers[0]
    x = torch.rand(8 * 5 + 3, 300, generator=torch.Generator().manual_seed(tile))
    with torch.no_grad():
        rec = ops.fc_soft_records([layer.record_spec()], 8)[0]
        y = ops.fc_soft_rec(x.to(DEV), rec, 300, 200, 8, layer.node.kind, layer._inv_tau(),
                            tile=tile)
    _close(y, torch_ref.fc_layer_soft(L, sd, x), f"{node} tile {tile}")


# (IN, expected automatic tile): config 1's hidden layers (2000 -> 8), config
# 4's first layer (4096 -> 8), config 2's hidden layers (10000 -> 4), config
# 4's hidden layers (16380 -> 2), the widest 2-sample width
@pytest.mark.parametrize("node", ["gate16", "walsh"])
@pytest.mark.parametrize("in_dim,tile", [(2000, 8), (4096, 8), (10000, 4), (16380, 2),
                                         (20352, 2)])
def test_records_automatic_tile_with_and_without_head(node, in_dim, tile):
    width = 640
    model, sd, L = _layer(in_dim, width, node, seed=in_dim)
    layer = model.layers[0]
    # the fused head needs one workgroup per sample tile over all outputs,
    # i.e. enough tiles to fill the GPU: the smallest such batch, plus a
    # partial last tile
    B = tile
    while not ops.fc_soft_groupsum_supported(B, in_dim, width, 10):
        B *= 2
    B += 1
    n = min(B, 129)           # oracle slice
    g = torch.Generator().manual_seed(in_dim)
    x = torch.rand(B, in_dim, generator=g)
    assert ops.fc_soft_groupsum_supported(B, in_dim, width, 10)
    with torch.no_grad():
        rec = ops.fc_soft_records([layer.record_spec()], 8)[0]
        xd = x.to(DEV)
        y_auto = ops.fc_soft_rec(xd, rec, in_dim, width, 8, layer.node.kind, layer._inv_tau())
        y_forced = ops.fc_soft_rec(xd, rec, in_dim, width, 8, layer.node.kind, layer._inv_tau(),
                                   tile=tile)
        logits = ops.fc_soft_rec_groupsum(xd, rec, in_dim, width, 8, layer.node.kind,
                                          layer._inv_tau(), 10, 7.0)
    ref = torch_ref.fc_layer_soft(L, sd, x[:n])
    _close(y_auto[:n], ref, f"{node} IN={in_dim}")
    assert torch.equal(y_auto.cpu(), y_forced.cpu())     # the automatic tile is `tile`
    own = (y_auto.cpu() > 0.5).float().view(B, 10, -1).sum(2) / 7.0
    assert torch.equal(logits.cpu(), own)                # every row, the last tile's too
    _ste_logits_ok(logits[:n], y_auto[:n], ref, 10, 7.0)


@pytest.mark.parametrize("node", ["gate16", "walsh"])
def test_records_wide_input_index_pairs_are_exact(node):
    """IN = 40000 (1-sample tiles): index pairs whose high half is >= 32640
    make NaN bit patterns; the words must hold them unchanged."""
    in_dim, width = 40000, 320
    model, sd, L = _layer(in_dim, width, node, seed=7)
    layer = model.layers[0]
    x = torch.rand(5, in_dim, generator=torch.Generator().manual_seed(7))
    with torch.no_grad():
        spec = layer.record_spec()
        rec = ops.fc_soft_records([spec], 8)[0]
        y = ops.fc_soft_rec(x.to(DEV), rec, in_dim, width, 8, layer.node.kind, layer._inv_tau())
    _close(y, torch_ref.fc_layer_soft(L, sd, x), f"{node} IN=40000")
    # reinterpret on the device, then copy integers (no float op touches the words)
    words = ops.record_words(rec.view(torch.int32).cpu(), width).long() & 0xFFFFFFFF
    pair = words[:, :8]
    idx = torch.stack([pair & 0xFFFF, pair >> 16], dim=1)                # [OUT, 2, 8]
    order = spec[5].long().cpu()
    cand = torch.gather(sd[L["prefix"] + "_conn.cand"].long(), 2, order)
    assert torch.equal(idx, cand)
    assert (idx[:, 1] >= 32640).any()       # the NaN-pattern words are exercised


def test_narrow_input_is_refused():
    model, _, _ = _layer(300, 200, "gate16")
    x = torch.rand(4, 299, device=DEV)
    with pytest.raises(ValueError, match="in_dim"):
        model(x)
    with pytest.raises(ValueError, match="in_dim"):
        model.layers[0](x)
    with pytest.raises(ValueError, match="in_dim"):
        model.forward_hard(x)
    # a wider input reads the first in_dim features, as x[:, cand] does
    xw = torch.rand(4, 310, device=DEV)
    with torch.no_grad():
        assert torch.equal(model.layers[0](xw).cpu(), model.layers[0](xw[:, :300]).cpu())
