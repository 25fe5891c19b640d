"""HIP path vs the oracle / the reference's golden vectors (GPU).

Bars: hard outputs and every integer / packed value bit-exact; soft fp32
values within |got - ref| <= RTOL*|ref| + ATOL with RTOL = 1e-5 (the north
star's 1e-5 relative; ATOL = 1e-6 only covers values near 0, soft values live
in [0, 1]). Soft logits with the feature STE count (x > 0.5): they must equal
the count of the kernel's own features, and any feature whose side of 0.5
differs from the oracle must lie within the soft tolerance of 0.5.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import silogic_amd as sl
from conftest import build_product, load_fixture, random_bits
from oracle import packed_ref, torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-5, 1e-6
DEV = "cuda"


def assert_soft_close(got, ref, what):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    err = (got - ref).abs()
    bound = RTOL * ref.abs() + ATOL
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} values outside tolerance, "
                           f"max err {err.max().item():.3e}")


def assert_ste_logits(logits, feats, feats_ref, C, tau):
    logits, feats, feats_ref = logits.cpu(), feats.cpu(), feats_ref.cpu()
    B, W = feats.shape
    own = (feats > 0.5).float().view(B, C, W // C).sum(2) / tau
    assert torch.equal(logits, own)
    flips = (feats > 0.5) != (feats_ref > 0.5)
    if flips.any():
        assert ((feats_ref[flips] - 0.5).abs() <= RTOL * 0.5 + ATOL).all()


def _gpu_model(fx):
    model = build_product(fx.spec)
    model.load_state_dict(fx.sd, strict=True)   # the reference's own parameters
    return model.to(DEV).eval()


# --------------------------------------------------------------------------
# golden fixtures (tiny versions of the five configs)
# --------------------------------------------------------------------------
def test_fixture_soft_layers(fixture):
    """Each layer on the reference's own previous activation (isolates every
    kernel launch), then the chained forward."""
    model = _gpu_model(fixture)
    A = fixture.arrays
    with torch.no_grad():
        if fixture.kind == "fc":
            h = fixture.x
            for i, layer in enumerate(model.layers):
                y = layer(h.to(DEV))
                assert_soft_close(y, A[f"act/{i}"], f"act/{i}")
                h = A[f"act/{i}"]
        else:
            h = fixture.x
            convs = model._convs()
            for i, conv in enumerate(convs):
                assert_soft_close(conv(h.to(DEV)), A[f"conv/{i}"], f"conv/{i}")
                assert_soft_close(conv.forward_pooled(h.to(DEV)), A[f"pool/{i}"], f"pool/{i}")
                assert_soft_close(model.blocks[2 * i + 1](A[f"conv/{i}"].to(DEV)), A[f"pool/{i}"],
                                  f"orpool/{i}")
                h = A[f"pool/{i}"]
            h = h.flatten(1)
            for j, layer in enumerate(model.head_layers):
                assert_soft_close(layer(h.to(DEV)), A[f"act/{j}"], f"act/{j}")
                h = A[f"act/{j}"]
        last = h
        head = model.head
        assert_ste_logits(head(last.to(DEV)), last, last, head.num_classes, head.tau)
        model.head.feature_ste = False
        assert_soft_close(model(fixture.x.to(DEV)), A["logits_soft_noste"], "logits (no STE)")
        model.head.feature_ste = True
        out = model(fixture.x.to(DEV))
    assert out.shape == A["logits_soft"].shape
    # STE logits of the chained run: recompute the kernel's own final features
    feats = _soft_features(model, fixture.x.to(DEV))
    assert_soft_close(feats, last, "chained final features")
    assert_ste_logits(out, feats, last, model.head.num_classes, model.head.tau)


def _soft_features(model, x):
    with torch.no_grad():
        if hasattr(model, "layers"):
            return model._run(x)
        h = model._apply_blocks(x).flatten(1)
        for layer in model.head_layers:
            h = layer(h)
        return h


def test_fixture_hard_bit_exact(fixture):
    model = _gpu_model(fixture)
    A = fixture.arrays
    out = model.forward_hard(fixture.x.to(DEV)).cpu()
    assert torch.equal(out, A["logits_hard"])
    # uint8 input path gives the same circuit (tests/test_warp.py:55-63)
    out8 = model.forward_hard(fixture.x.to(torch.uint8).to(DEV)).cpu()
    assert torch.equal(out8, A["logits_hard"])
    # per-layer forward_hard on the reference's previous hard activation
    if fixture.kind == "fc":
        h = fixture.x
        for i, layer in enumerate(model.layers):
            assert torch.equal(layer.forward_hard(h.to(DEV)).cpu(), A[f"hact/{i}"]), i
            h = A[f"hact/{i}"]
    else:
        h = fixture.x
        for i, conv in enumerate(model._convs()):
            y = conv.forward_hard(h.to(DEV)).cpu()
            assert torch.equal(y, A[f"hconv/{i}"]), i
            h = model.blocks[2 * i + 1].forward_hard(A[f"hconv/{i}"].to(DEV)).cpu()
            assert torch.equal(h, torch_ref.orpool_hard(A[f"hconv/{i}"]))
        h = h.flatten(1)
        for j, layer in enumerate(model.head_layers):
            assert torch.equal(layer.forward_hard(h.to(DEV)).cpu(), A[f"hact/{j}"]), j
            h = A[f"hact/{j}"]
    assert torch.equal(model.head.forward_hard(h.to(DEV)).cpu(), A["logits_hard"])


# --------------------------------------------------------------------------
# kernels against the oracle on crafted / edge inputs
# --------------------------------------------------------------------------
@pytest.mark.parametrize("B,D", [(1, 1), (63, 8), (64, 64), (65, 257), (200, 784), (1000, 33)])
def test_pack_matches_reference_layout(B, D):
    x = random_bits(B, D)
    xp = ops.pack_bits(x.to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(xp, packed_ref.pack_bits(x.numpy().astype(np.uint8)))
    np.testing.assert_array_equal(ops.unpack_bits(torch.from_numpy(xp).to(DEV), B).cpu().numpy(),
                                  x.numpy().astype(np.uint8))
    xp8 = ops.pack_bits(x.to(torch.uint8).to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(xp8, xp)


def test_all_sixteen_gates_packed():
    """Each gate g as a one-hot gate16 layer: packed kernel == truth table."""
    B, IN = 130, 2
    x = torch.tensor([[i & 1, (i >> 1) & 1] for i in range(B)], dtype=torch.float32)
    layer = sl.LogicLayer(IN, 16, connectome="fixed", seed=0)
    with torch.no_grad():
        layer._conn.idx.copy_(torch.tensor([[1, 0]] * 16))   # a = x[:,1], b = x[:,0]
        layer._conn.cand_i32.copy_(layer._conn.idx.unsqueeze(-1).int())
        layer.node.gate_logits.copy_(torch.eye(16) * 5.0)
    layer = layer.to(DEV)
    y = layer.forward_hard(x.to(DEV)).cpu()
    a, b = x[:, 1].long(), x[:, 0].long()
    for g in range(16):
        ref = torch_ref.TRUTH[g][(a << 1) | b]
        assert torch.equal(y[:, g], ref), g
    # soft path of the same hardened layer agrees on {0,1} inputs
    with torch.no_grad():
        layer.node.gate_logits.copy_(torch.eye(16, device=DEV) * 40.0)
        assert (layer(x.to(DEV)).cpu() - y.float()).abs().max() < 1e-6


def test_walsh_hard_truth_table_near_ties():
    """Corner sums that cancel to (near) zero take the sign of the fp32
    left-to-right sum, as torch's CPU reduction does."""
    L = dict(prefix="", node="walsh", arity=2, node_tau=1.0, conn="fixed", d_in=2, d_out=0)
    g = torch.Generator().manual_seed(3)
    th = torch.randn(4000, 4, generator=g)
    th[:1000, 3] = -(th[:1000, 0] - th[:1000, 1] - th[:1000, 2])   # corner (0,0) cancels
    th[1000:2000] = torch.tensor([0.1, 0.2, 0.3, 0.0])
    th[1000:2000, 3] = -(th[1000:2000, 0] + th[1000:2000, 1] + th[1000:2000, 2])
    th[2000:2100] = torch.tensor([1e-8, 1.0, -1.0, 0.5])
    layer = sl.LogicLayer(2, 4000, node="walsh", connectome="fixed", seed=0)
    with torch.no_grad():
        layer.node.theta.copy_(th)
        layer._conn.idx.copy_(torch.tensor([[1, 0]] * 4000))
        layer._conn.cand_i32.copy_(layer._conn.idx.unsqueeze(-1).int())
    layer = layer.to(DEV)
    x = torch.tensor([[0., 0], [1, 0], [0, 1], [1, 1]])            # (b, a) columns
    y = layer.forward_hard(x.to(DEV)).cpu()
    ops_ = torch.stack([x[:, 1], x[:, 0]], dim=1).unsqueeze(1).expand(4, 4000, 2)
    ref = torch_ref.node_hard(dict(L, d_out=4000), {"node.theta": th}, ops_)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("node", ["gate16", "walsh", "multilinear"])
@pytest.mark.parametrize("conn", ["topk", "fixed"])
@pytest.mark.parametrize("B", [1, 37, 130])
def test_fc_layer_soft_and_hard(node, conn, B):
    spec = ("LogicNet", dict(in_dim=300, width=70, depth=1, num_classes=10, node=node,
                             connectome=conn, k=8, tau=3.0))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    x = random_bits(B, 300)
    L = torch_ref.structure(spec)["layers"][0]
    with torch.no_grad():
        assert_soft_close(model.layers[0](x.to(DEV)), torch_ref.fc_layer_soft(L, sd, x), "soft")
    assert torch.equal(model.layers[0].forward_hard(x.to(DEV)).cpu(),
                       torch_ref.fc_layer_hard(L, sd, x))
    assert torch.equal(model.forward_hard(x.to(DEV)).cpu(), torch_ref.forward_hard(spec, sd, x))


@pytest.mark.parametrize("tile", [1, 2, 4, 8])
def test_fc_soft_every_tile_size(tile):
    spec = ("LogicNet", dict(in_dim=500, width=130, depth=1, k=8))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    x = torch.rand(45, 500)
    layer = model.layers[0]
    with torch.no_grad():
        cand, w, npar = layer.soft_params(False)
        y = ops._fc_soft_launch(x.to(DEV), cand, w, npar, ops.GATE16, 1.0, tile=tile)
    L = torch_ref.structure(spec)["layers"][0]
    assert_soft_close(y, torch_ref.fc_layer_soft(L, sd, x), f"tile {tile}")


def test_records_of_mixed_layers_in_one_launch():
    """One records launch for layers of different node kinds and widths; each
    layer on its records matches the oracle, and the index words equal the
    reference's candidates exactly."""
    specs = [("LogicNet", dict(in_dim=300, width=120, depth=1, k=8, node=n))
             for n in ["gate16", "walsh", "multilinear"]]
    specs.append(("LogicNet", dict(in_dim=77, width=60, depth=1, k=8)))
    models, sds = [], []
    for spec in specs:
        m = build_product(spec)
        sds.append({k: v.clone() for k, v in m.state_dict().items()})
        models.append(m.to(DEV))
    with torch.no_grad():
        recs = ops.fc_soft_records([m.layers[0].record_spec() for m in models], 8)
        for spec, sd, m, rec in zip(specs, sds, models, recs):
            L = torch_ref.structure(spec)["layers"][0]
            x = torch.rand(37, spec[1]["in_dim"])
            layer = m.layers[0]
            OUT = layer.out_dim
            y = ops.fc_soft_rec(x.to(DEV), rec, layer.in_dim, OUT, 8, layer.node.kind,
                                layer._inv_tau())
            assert_soft_close(y, torch_ref.fc_layer_soft(L, sd, x), f"{spec[1]} records")
            # record words: candidates and weights in the scheduled gather order
            words = ops.record_words(rec, OUT).cpu()
            order = layer.gather_order().long().cpu()                     # [OUT, 2, 8]
            assert torch.equal(order.sort(dim=2).values,
                               torch.arange(8).expand(OUT, 2, 8))        # a permutation
            assert words.shape == (OUT, 4 * ops.record_quads(8)) == (OUT, 28)
            pair = words[:, :8].contiguous().view(torch.int32).long() & 0xFFFFFFFF
            idx = torch.stack([pair & 0xFFFF, pair >> 16], dim=1).to(torch.int32)  # [OUT,2,8]
            cand = sd[L["prefix"] + "_conn.cand"].to(torch.int32)
            assert torch.equal(idx, torch.gather(cand, 2, order))
            ref_w = torch.gather(torch.softmax(sd[L["prefix"] + "_conn.conn"], dim=2), 2, order)
            assert_soft_close(words[:, 8:24].reshape(OUT, 2, 8), ref_w, "softmax weights")
            assert not words[:, 24:28].isnan().any()   # node parameters in the last quad
            # natural order records give the same layer output within tolerance
            spec_nat = layer.record_spec()[:5] + (None,)
            rec_nat = ops.fc_soft_records([spec_nat], 8)[0]
            y_nat = ops.fc_soft_rec(x.to(DEV), rec_nat, layer.in_dim, OUT, 8, layer.node.kind,
                                    layer._inv_tau())
            assert_soft_close(y_nat, torch_ref.fc_layer_soft(L, sd, x), "natural order")


def _lane_groups(lanes):
    """gfx950 LDS lane groups of one wave's read (one cycle per group per
    distinct slot of a bank class): b128 (16 bank classes) splits each
    32-lane half by the parity of lane bits 2-4; b64 (32 classes) takes the
    two halves; b32 (64 classes) the whole wave."""
    lane = torch.arange(64)
    if lanes == 16:
        par = ((lane >> 2) & 1) ^ ((lane >> 3) & 1) ^ ((lane >> 4) & 1)
        key = 2 * (lane >> 5) + par
    else:
        key = lane // lanes
    return [torch.nonzero(key == k).flatten() for k in range(64 // lanes)]


def _bank_cycles(idx, lanes):
    """Modelled LDS cycles of the gathers of one slot: over 64-output chunks,
    steps and lane groups, the most distinct indices of one bank class
    (index mod ``lanes``)."""
    OUT, K = idx.shape
    n = OUT - OUT % 64
    chunks = idx[:n].reshape(-1, 64, K)
    total = 0
    for grp in _lane_groups(lanes):
        v = chunks[:, grp].sort(dim=1).values                 # [chunks, lanes, K]
        fresh = torch.ones_like(v, dtype=torch.bool)
        fresh[:, 1:] = v[:, 1:] != v[:, :-1]                  # same index = one read
        one = torch.nn.functional.one_hot(v % lanes, lanes) * fresh.unsqueeze(-1)
        total += int(one.sum(1).max(-1).values.sum())
    return total


@pytest.mark.parametrize("in_dim,lanes", [(10000, 16), (16380, 32)])
def test_gather_schedule_lowers_bank_conflicts(in_dim, lanes):
    """The scheduled order is a per-(output, slot) permutation and cuts the
    modelled LDS bank-conflict cycles well below index order (random
    candidates: ~12.3 -> ~7.9 cycles per b128 wave read, 4 without
    conflicts)."""
    layer = sl.LogicLayer(in_dim, 4096, k=8, seed=3).to(DEV)
    cand = layer._conn.candidates_i32()
    order = layer.gather_order().long()
    assert torch.equal(order.sort(dim=2).values.cpu(), torch.arange(8).expand(4096, 2, 8))
    sched = torch.gather(cand.long(), 2, order).cpu()
    nat = cand.long().cpu()
    for s in range(2):
        before = _bank_cycles(nat[:, s], lanes)
        after = _bank_cycles(sched[:, s], lanes)
        assert after < 0.8 * before, (s, before, after)
    assert layer.gather_order() is layer.gather_order()       # cached per candidate table


@pytest.mark.parametrize("node", ["gate16", "walsh"])
@pytest.mark.parametrize("width", [200, 1000])
def test_fused_groupsum_head(node, width):
    """Last layer + STE GroupSum in one kernel: the logits are exactly the
    class counts of the kernel's own features / tau, and those features match
    the oracle (per = width / 10 outputs per class: 20 puts several classes in
    one wave, 100 makes classes straddle waves; B leaves a partial tile)."""
    spec = ("LogicNet", dict(in_dim=6000, width=width, depth=1, k=8, tau=3.0, node=node))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    B = 2048 + 3
    x = torch.bernoulli(torch.full((B, 6000), 0.3), generator=torch.Generator().manual_seed(4))
    assert ops.fc_soft_groupsum_supported(B, 6000, width, 10)
    L = torch_ref.structure(spec)["layers"][0]
    layer = model.layers[0]
    with torch.no_grad():
        xd = x.to(DEV)
        rec = ops.fc_soft_records([layer.record_spec()], 8)[0]
        logits = ops.fc_soft_rec_groupsum(xd, rec, layer.in_dim, width, 8, layer.node.kind,
                                          layer._inv_tau(),
                                          10, 3.0)
        feats = ops.fc_soft_rec(xd, rec, layer.in_dim, width, 8, layer.node.kind, layer._inv_tau())
        out = model(xd)
    feats_ref = torch_ref.fc_layer_soft(L, sd, x)
    assert_soft_close(feats, feats_ref, "features")
    assert_ste_logits(logits, feats, feats_ref, 10, 3.0)
    assert torch.equal(out.cpu(), logits.cpu())


def test_hard_codes_of_all_layers_in_one_launch():
    spec = ("LogicNet", dict(in_dim=300, width=120, depth=4, k=8))
    model = build_product(spec).to(DEV)
    with torch.no_grad():
        one = ops.fc_hard_codes_net([l.hard_spec() for l in model.layers])
        each = [l.hard_codes() for l in model.layers]
    for a, b in zip(one, each):
        assert torch.equal(a.cpu(), b.cpu())


def test_empty_batch():
    net = sl.LogicNet(32, 40, 2, k=4).to(DEV).eval()
    x = torch.zeros(0, 32, device=DEV)
    with torch.no_grad():
        assert net(x).shape == (0, 10)
        assert net.forward_hard(x).shape == (0, 10)


def test_fused_net_equals_layerwise_path_and_wide_32bit_tiles():
    """Two independent hard pipelines agree: the depth-fused LDS kernel
    (64- and 32-sample tiles) and the layer-by-layer packed kernels."""
    for width in (1000, 12000):   # 12000 words x 8B x 2 exceeds LDS -> 32-sample tiles
        spec = ("LogicNet", dict(in_dim=200, width=width, depth=3, k=8))
        model = build_product(spec)
        sd = {k: v.clone() for k, v in model.state_dict().items()}
        model = model.to(DEV).eval()
        x = random_bits(333, 200)
        xd = x.to(DEV)
        codes = [l.hard_codes() for l in model.layers]
        ccodes = ops.fc_hard_codes_net([l.hard_spec() for l in model.layers], compact=True)
        for c, cc in zip(codes, ccodes):   # compact code = b | a << 14 | tt << 28
            c, cc = c.cpu().long() & 0xFFFFFFFF, cc.cpu().long() & 0xFFFFFFFF
            assert torch.equal(cc & 0x3FFF, c[:, 1] & 0x3FFF)
            assert torch.equal((cc >> 14) & 0x3FFF, c[:, 0])
            assert torch.equal(cc >> 28, c[:, 1] >> 28)
        outs = []
        codes_l, codes = codes, ccodes
        if width == 1000:   # unpacked rows, packing fused (fp32 and uint8)
            outs.append(ops.fc_hard_net(xd, ops.ROWS_F32, 333, 200, codes, 10))
            outs.append(ops.fc_hard_net(xd.to(torch.uint8), ops.ROWS_U8, 333, 200, codes, 10))
        outs.append(ops.fc_hard_net(ops.pack_bits(xd), ops.PACKED, 333, 200, codes, 10))
        outs.append(ops.fc_hard_net(ops.pack_bits(xd, word_major=True), ops.PACKED_WORD_MAJOR,
                                    333, 200, codes, 10))
        xp = ops.pack_bits(xd)
        for c in codes_l:
            xp = ops.fc_hard_layer(xp, c)
        layerwise = ops.groupsum_packed(xp, 333, 10)
        ref = torch_ref.forward_hard(spec, sd, x)
        assert torch.equal(layerwise.cpu(), ref)
        for o in outs:
            assert torch.equal(o.cpu(), ref)


@pytest.mark.parametrize("width,C", [(2050, 2), (6300, 7), (640, 64), (10240, 5), (96, 3)])
def test_fused_net_groupsum_class_shapes(width, C):
    """The fused kernels' GroupSum (bit-sliced counts, one wave per class)
    over classes of 1025, 900, 10, 2048 and 32 words: several 1024-word
    passes per class, classes that are not whole 32-word rows, 64 classes,
    and a layer that fills both 80 KiB activation buffers."""
    spec = ("LogicNet", dict(in_dim=200, width=width, depth=2, num_classes=C, k=8))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    x = random_bits(333, 200)
    xd = x.to(DEV)
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in model.layers], compact=True)
    ref = torch_ref.forward_hard(spec, sd, x)
    assert torch.equal(ops.fc_hard_net(xd, ops.ROWS_F32, 333, 200, codes, C).cpu(), ref)
    assert torch.equal(ops.fc_hard_net(ops.pack_bits(xd, word_major=True), ops.PACKED_WORD_MAJOR,
                                       333, 200, codes, C).cpu(), ref)
    assert torch.equal(model.forward_hard(xd).cpu(), ref)


@pytest.mark.parametrize("depth", [1, 2, 3, 6])
def test_fused_rows_kernel_many_tiles(depth):
    """More 64-sample tiles than CUs (persistent loop, streamed next-tile input)
    and a ragged last tile; depths below 4 load the chunks no layer streamed
    after the last layer."""
    spec = ("LogicNet", dict(in_dim=100, width=60, depth=depth, k=8))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    B = 64 * 600 + 37
    x = random_bits(B, 100)
    out = model.forward_hard(x.to(DEV)).cpu()
    ref = torch_ref.forward_hard(spec, sd, x)
    assert torch.equal(out, ref)
    assert torch.equal(model.forward_hard(x.to(torch.uint8).to(DEV)).cpu(), ref)


def test_wire_residual_hard_and_soft():
    spec = ("LogicNet", dict(in_dim=40, width=40, depth=3, k=8, wire_residual=0.25))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV).eval()
    x = random_bits(70, 40)
    assert torch.equal(model.forward_hard(x.to(DEV)).cpu(), torch_ref.forward_hard(spec, sd, x))
    with torch.no_grad():
        model.head.feature_ste = False
        assert_soft_close(model(x.to(DEV)), torch_ref.forward(spec, sd, x, ste=False), "logits")


@pytest.mark.parametrize("depth", [1, 2, 3, 4])
@pytest.mark.parametrize("connect", ["topk", "fixed"])
def test_conv_gate16_depths(depth, connect):
    conv = sl.ConvLogicTree(6, 12, kernel=3, tree_depth=depth, connect=connect, k=4, n_chan=2,
                            residual_init=False, seed=1)
    sd = {k: v.clone() for k, v in conv.state_dict().items()}
    blk = dict(prefix="", cin=6, n=12, kernel=3, depth=depth, stride=1, padding=1,
               connect=connect, k=conv.k, node="gate16", node_arity=2, leaves=2 ** depth)
    conv = conv.to(DEV).eval()
    x = torch.rand(5, 6, 9, 11)
    with torch.no_grad():
        assert_soft_close(conv(x.to(DEV)), torch_ref.conv_soft(blk, sd, x), "conv")
        assert_soft_close(conv.forward_pooled(x.to(DEV)),
                          torch_ref.orpool_soft(torch_ref.conv_soft(blk, sd, x)), "pooled")
    xb = random_bits(70, 6, 9, 11)
    assert torch.equal(conv.forward_hard(xb.to(DEV)).cpu(), torch_ref.conv_hard(blk, sd, xb))


def test_conv_hard_prep_net_blocks():
    """One launch for the hard parameters of blocks of every node kind,
    gate16 logits read per level in place, against the single-block entry
    point on the concatenated levels; more than 8 blocks split launches."""
    blocks = []
    for i, (node, depth, arity, connect) in enumerate(
            [("gate16", 1, 2, "topk"), ("gate16", 2, 2, "fixed"), ("gate16", 3, 2, "topk"),
             ("gate16", 4, 2, "topk"), ("multilinear", 1, 3, "topk"), ("hybrid", 1, 4, "topk"),
             ("gate16", 2, 2, "topk"), ("multilinear", 1, 2, "fixed"), ("gate16", 3, 2, "fixed")]):
        conv = sl.ConvLogicTree(4, 130 + 70 * i, kernel=3, tree_depth=depth, connect=connect, k=5,
                                n_chan=2, node=node, arity=arity, residual_init=False, seed=i)
        blocks.append(conv.to(DEV).eval())
    got = ops.conv_hard_prep_net([b.hard_spec() for b in blocks])
    assert len(got) == len(blocks)
    for b, (leaf, tt) in zip(blocks, got):
        cm, ch, cw = b._taps()
        want = ops.conv_hard_prep(cm, ch, cw, None if b.connect == "fixed" else b.conn, b._raw(),
                                  b._kind(), b.d, b.node_arity)
        assert torch.equal(leaf, want[0]) and torch.equal(tt, want[1])
        assert torch.equal(b.hard_params()[1], tt)
    bad = list(blocks[2].hard_spec())
    bad[4] = bad[4][::-1]   # levels out of order
    with pytest.raises(ValueError):
        ops.conv_hard_prep_net([bad])


@pytest.mark.parametrize("node", ["multilinear", "hybrid"])
@pytest.mark.parametrize("arity", [2, 3, 4, 5, 6])
def test_conv_multilinear_lut(arity, node):
    """LUT conv trees (multilinear; hybrid, kernels/conv_hybrid.py at depth 1):
    soft values against the oracle (hybrid: within 1e-6 where no leaf is
    within rounding of 0.5), both the records and the separate-array entry points,
    pooled; hard outputs bit for bit."""
    conv = sl.ConvLogicTree(5, 10, kernel=3, tree_depth=1, connect="topk", k=4, n_chan=2,
                            node=node, arity=arity, residual_init=False, seed=2)
    sd = {k: v.clone() for k, v in conv.state_dict().items()}
    blk = dict(prefix="", cin=5, n=10, kernel=3, depth=1, stride=1, padding=1, connect="topk",
               k=conv.k, node=node, node_arity=arity, leaves=arity)
    conv = conv.to(DEV).eval()
    x = torch.rand(3, 5, 8, 7)
    with torch.no_grad():
        ref = torch_ref.conv_soft(blk, sd, x)
        outs = [conv(x.to(DEV)), conv.forward_pooled(x.to(DEV))]
        with torch.enable_grad():   # the separate-array entry point (autograd path)
            outs.append(conv(x.to(DEV).requires_grad_(True)).detach())
    if node == "multilinear":
        assert_soft_close(outs[0], ref, "conv")
        assert_soft_close(outs[1], F.max_pool2d(ref, 2, 2), "conv pooled")
        assert_soft_close(outs[2], ref, "conv (arrays)")
    else:
        patches = F.unfold(x, (3, 3), padding=1)
        leaves = torch_ref.conv_leaves_soft(blk, sd, patches)           # [B, n, L, HW]
        near = ((leaves - 0.5).abs() <= 1e-5).any(2).view(ref.shape)
        for got in (outs[0], outs[2]):   # LUT values: sigmoid on the GPU vs torch's, ~1 ulp
            bad = (got.cpu() - ref).abs() > 1e-6
            assert not (bad & ~near).any(), int((bad & ~near).sum())
    xb = random_bits(66, 5, 8, 7)
    assert torch.equal(conv.forward_hard(xb.to(DEV)).cpu(), torch_ref.conv_hard(blk, sd, xb))


@pytest.mark.parametrize("kernel,hw,cin,B,k,node", [
    (1, (5, 6), 3, 9, 1, "gate16"),          # no padding
    (3, (7, 7), 40, 300, 4, "gate16"),       # many narrow planes
    (5, (12, 9), 4, 17, 8, "gate16"),        # pad 2, 8 taps per leaf
    (3, (4, 4), 3, 2101, 4, "gate16"),       # several samples per workgroup, ragged last
    (3, (9, 10), 6, 33, 8, "multilinear"),   # LUT with 8 taps per leaf
])
def test_conv_staging_and_records(kernel, hw, cin, B, k, node):
    """The records path (no grad) against the oracle and, bit for bit, against
    the separate-array entry point on the same parameters."""
    depth, arity = (2, 2) if node == "gate16" else (1, 4)
    conv = sl.ConvLogicTree(cin, 24, kernel=kernel, padding=kernel // 2, tree_depth=depth,
                            connect="topk", k=k, n_chan=2, node=node, arity=arity,
                            residual_init=False, seed=3)
    sd = {kk: v.clone() for kk, v in conv.state_dict().items()}
    leaves = 2 ** depth if node == "gate16" else arity
    blk = dict(prefix="", cin=cin, n=24, kernel=kernel, depth=depth, stride=1,
               padding=kernel // 2, connect="topk", k=conv.k, node=node,
               node_arity=conv.node_arity, leaves=leaves)
    conv = conv.to(DEV).eval()
    x = torch.rand(B, cin, *hw)
    xd = x.to(DEV)
    with torch.no_grad():
        y, yp = conv(xd), conv.forward_pooled(xd)
        ref = torch_ref.conv_soft(blk, sd, x)
        assert_soft_close(y, ref, "conv")
        assert_soft_close(yp, torch_ref.orpool_soft(ref), "pooled")
        w, npar = conv.soft_params(False)
        cm, ch, cw = conv._taps()
        for pool, got in ((False, y), (True, yp)):
            arr = ops.conv_soft(xd, npar, w, cm, ch, cw, conv._kind(), conv.d, conv.node_arity,
                                cm.shape[-1], conv.padding, pool)
            assert torch.equal(got, arr)
            rec = conv.soft_records(x.shape[1:], pool)
            r = ops.conv_soft_rec(xd, rec, 24, conv._kind(), conv.d, conv.node_arity,
                                  cm.shape[-1], conv.padding, pool)
            assert torch.equal(got, r)


def test_kernels_module_drop_ins():
    """silogic.kernels-compatible entry points (tests/test_triton.py analogues)."""
    layer = sl.LogicLayer(256, 512, connectome="TopK", k=8, seed=0)
    sd = {k: v.clone() for k, v in layer.state_dict().items()}
    layer = layer.to(DEV).eval()
    x = random_bits(64, 256)
    with torch.no_grad():
        w = layer._conn.weights()
        ca = layer._conn.cand_i32
        coef = layer.node.coef()
        y = sl.kernels.dense_logic(x.to(DEV), ca[:, 0].contiguous(), ca[:, 1].contiguous(),
                                   w[:, 0].contiguous(), w[:, 1].contiguous(), coef)
    L = dict(prefix="", node="gate16", arity=2, conn="topk")
    assert_soft_close(y, torch_ref.fc_layer_soft(L, sd, x), "dense_logic")

    wl = sl.WARPLayer(256, 512, k=8, tau=0.5, seed=1)
    sdw = {k: v.clone() for k, v in wl.state_dict().items()}
    wl = wl.to(DEV)
    with torch.no_grad():
        w = wl._conn.weights()
        ca = wl._conn.cand_i32
        y = sl.kernels.warp_logic(x.to(DEV), ca[:, 0].contiguous(), ca[:, 1].contiguous(),
                                  w[:, 0].contiguous(), w[:, 1].contiguous(), wl._coef(),
                                  wl.node.inv_tau)
    Lw = dict(prefix="", node="walsh", arity=2, conn="topk", node_tau=0.5)
    assert_soft_close(y, torch_ref.fc_layer_soft(Lw, sdw, x), "warp_logic")

    conv = sl.ConvLogicTree(6, 16, kernel=3, tree_depth=3, connect="topk", k=4, n_chan=2,
                            seed=1, residual_init=False)
    sdc = {k: v.clone() for k, v in conv.state_dict().items()}
    conv = conv.to(DEV)
    xi = random_bits(4, 6, 16, 16)
    blk = dict(prefix="", n=16, kernel=3, depth=3, stride=1, padding=1, connect="topk",
               k=conv.k, node="gate16", node_arity=2, leaves=8)
    with torch.no_grad():
        yk = sl.kernels.tree_conv_topk(xi.to(DEV), conv._basis_coef().contiguous(),
                                       conv._topk_w(), conv.lc_cm, conv.lc_ch, conv.lc_cw, 3,
                                       conv.k, 1, 1, 16, 16)
    assert_soft_close(yk, torch_ref.conv_soft(blk, sdc, xi), "tree_conv_topk")
    convf = sl.ConvLogicTree(6, 16, kernel=3, tree_depth=2, connect="fixed", n_chan=2, seed=0)
    sdf = {k: v.clone() for k, v in convf.state_dict().items()}
    convf = convf.to(DEV)
    blkf = dict(blk, depth=2, connect="fixed", k=1, leaves=4)
    with torch.no_grad():
        yf = sl.kernels.tree_conv(xi.to(DEV), convf._basis_coef().contiguous(), convf.cm_idx,
                                  convf.ch_idx, convf.cw_idx, 2, 1, 1, 16, 16)
    assert_soft_close(yf, torch_ref.conv_soft(blkf, sdf, xi), "tree_conv")


def test_groupsum_and_orpool_modules():
    x = torch.rand(9, 60)
    gs = sl.GroupSum(10, tau=4.0, feature_ste=False).to(DEV)
    head = dict(C=10, tau=4.0, ste=False)
    assert_soft_close(gs(x.to(DEV)), torch_ref.groupsum_soft(head, x), "groupsum")
    xb = random_bits(9, 60)
    assert torch.equal(gs.forward_hard(xb.to(DEV)).cpu(), torch_ref.groupsum_hard(head, xb))
    assert torch.equal(gs.forward_hard(xb.to(torch.uint8).to(DEV)).cpu(),
                       torch_ref.groupsum_hard(head, xb.to(torch.uint8)))
    xi = torch.rand(2, 3, 7, 9)
    pool = sl.OrPool(2)
    assert torch.equal(pool(xi.to(DEV)).cpu(), F.max_pool2d(xi, 2, 2))
    xu = random_bits(2, 3, 7, 9)
    assert torch.equal(pool.forward_hard(xu.to(DEV)).cpu(), torch_ref.orpool_hard(xu))


def test_gradients_match_the_oracle():
    """Composite backward through the HIP forward: gradients w.r.t. input,
    connections and gate logits match autograd through the oracle (the
    reference's fused-kernel gradient bar is 1e-3, tests/test_triton.py)."""
    spec = ("LogicNet", dict(in_dim=64, width=40, depth=2, k=8, tau=4.0, decoder_ste=False))
    model = build_product(spec)
    params = {k: v.clone().requires_grad_(v.is_floating_point())
              for k, v in model.state_dict().items()}
    x = torch.rand(16, 64)
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.groupsum_soft(dict(C=10, tau=4.0, ste=False),
                                  torch_ref.forward_features(torch_ref.structure(spec), params, xr,
                                                             hard=False))
    ref.pow(2).sum().backward()
    model = model.to(DEV).train()
    xg = x.to(DEV).requires_grad_(True)
    model(xg).pow(2).sum().backward()
    assert (xg.grad.cpu() - xr.grad).abs().max() < 1e-4
    for name, p in model.named_parameters():
        assert (p.grad.cpu() - params[name].grad).abs().max() < 1e-4, name


@pytest.mark.parametrize("node,conn,k,IN,OUT,B", [
    ("gate16", "topk", 8, 100, 300, 37),       # 2-sample weight-gradient tiles
    ("gate16", "topk", 8, 7000, 2000, 70),
    ("gate16", "topk", 8, 25000, 600, 33),     # 1-sample tiles (x tile > 160 KB at 2)
    ("walsh", "topk", 8, 500, 400, 200),       # two gather sample chunks
    ("multilinear", "topk", 4, 300, 200, 50),  # 4-sample tiles
    ("gate16", "fixed", 1, 200, 150, 40),
    ("gate16", "topk", 3, 120, 90, 21),        # candidate count known only at run time
])
def test_fc_soft_backward_kernels(node, conn, k, IN, OUT, B):
    """The HIP backward (input, connection and node gradients) against fp32
    autograd through the oracle's layer (silogic layers.py / connectomes.py /
    nodes.py semantics) with a random upstream gradient."""
    if node == "walsh":
        layer = sl.WARPLayer(IN, OUT, k=k, tau=0.5, seed=4)
        L = dict(prefix="", node="walsh", arity=2, conn=conn, node_tau=0.5)
    else:
        layer = sl.LogicLayer(IN, OUT, node=node, connectome=conn, k=k, seed=4)
        L = dict(prefix="", node=node, arity=2, conn=conn)
    params = {kk: v.clone().requires_grad_(v.is_floating_point())
              for kk, v in layer.state_dict().items()}
    gen = torch.Generator().manual_seed(5)
    x = torch.rand(B, IN, generator=gen)
    gy = torch.randn(B, OUT, generator=gen)
    xr = x.clone().requires_grad_(True)
    (torch_ref.fc_layer_soft(L, params, xr) * gy).sum().backward()
    layer = layer.to(DEV).train()
    xg = x.to(DEV).requires_grad_(True)
    (layer(xg) * gy.to(DEV)).sum().backward()

    def close(got, ref, what):
        got = got.cpu()
        scale = ref.abs().max().item()
        err = (got - ref).abs().max().item()
        assert err <= 1e-4 * scale + 1e-6, f"{what}: max err {err:.3e} (scale {scale:.3e})"

    close(xg.grad, xr.grad, "dL/dx")
    for name, p in layer.named_parameters():
        close(p.grad, params[name].grad, name)
    assert sl.ops.fc_soft_bwd(xg.detach(), *layer.soft_params(True), layer.node.kind,
                              layer._inv_tau(), gy.to(DEV)) is not None   # the HIP kernels ran


@pytest.mark.parametrize("node,depth,arity,connect,k,C,H,N,B,pool,binary", [
    ("gate16", 2, 2, "topk", 4, 7, 12, 24, 5, True, True),      # exact pooling ties
    ("gate16", 2, 2, "topk", 4, 7, 12, 24, 5, False, False),
    ("gate16", 2, 2, "topk", 4, 3, 28, 40, 4, True, True),      # 3 tree groups, last partial
    ("gate16", 3, 2, "topk", 8, 4, 9, 12, 3, True, False),      # odd map: floor pooling
    ("gate16", 1, 2, "fixed", 1, 5, 8, 16, 6, True, True),
    ("multilinear", 1, 6, "topk", 4, 9, 10, 16, 3, True, False),
    ("multilinear", 1, 3, "fixed", 1, 4, 7, 10, 4, False, True),
    ("multilinear", 1, 6, "topk", 4, 9, 32, 20, 2, True, True),  # the 32x32 LUT block
    ("gate16", 2, 2, "topk", 4, 2, 6, 8, 600, True, True),      # several samples per range
    ("hybrid", 1, 6, "topk", 8, 9, 10, 16, 3, True, True),      # the CIFAR recipe's trees
    ("hybrid", 1, 4, "fixed", 1, 4, 8, 10, 4, False, False),
    # trees on the generic kernels: walsh, deeper LUT trees, gate16 depth 5,
    # and an image too large for LDS (48 x 32 x 32 floats)
    ("walsh", 2, 2, "topk", 4, 5, 10, 12, 3, True, False),
    ("walsh", 3, 2, "fixed", 1, 4, 9, 10, 3, False, False),
    ("multilinear", 2, 4, "topk", 4, 6, 10, 8, 3, True, False),
    ("multilinear", 3, 2, "fixed", 1, 4, 8, 8, 3, True, True),
    ("hybrid", 2, 3, "topk", 4, 6, 10, 8, 3, True, False),
    ("gate16", 5, 2, "topk", 4, 4, 8, 6, 2, True, False),
    ("gate16", 2, 2, "topk", 4, 48, 32, 8, 2, True, False),
])
def test_conv_soft_backward_kernel(node, depth, arity, connect, k, C, H, N, B, pool, binary):
    """The HIP conv backward (fused pooling or not) against fp32 autograd
    through the oracle's ConvLogicTree (+ F.max_pool2d) on the CPU: input,
    connection and node-logit gradients."""
    layer = sl.ConvLogicTree(C, N, kernel=3, tree_depth=depth, connect=connect, k=k, seed=3,
                             node=node, arity=arity)
    binary_node = node in ("gate16", "walsh")
    blk = dict(prefix="", cin=C, n=N, kernel=3, depth=depth, stride=1, padding=1,
               connect=connect, k=layer.k if connect != "fixed" else 1, node=node,
               node_arity=2 if binary_node else arity,
               leaves=(2 if binary_node else arity) ** depth, tau=1.0, hw=H)
    params = {kk: v.clone().requires_grad_(v.is_floating_point())
              for kk, v in layer.state_dict().items()}
    gen = torch.Generator().manual_seed(11)
    x = torch.rand(B, C, H, H, generator=gen)
    if binary:
        x = (x > 0.5).float()
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.conv_soft(blk, params, xr)
    if pool:
        ref = torch_ref.orpool_soft(ref)
    gy = torch.randn(ref.shape, generator=gen)
    (ref * gy).sum().backward()
    layer = layer.to(DEV).train()
    xg = x.to(DEV).requires_grad_(True)
    out = layer.forward_pooled(xg) if pool else layer(xg)
    (out * gy.to(DEV)).sum().backward()

    def close(got, ref_, what):
        got = got.cpu()
        scale = ref_.abs().max().item()
        err = (got - ref_).abs().max().item()
        assert err <= 1e-4 * scale + 1e-6, f"{what}: max err {err:.3e} (scale {scale:.3e})"

    close(xg.grad, xr.grad, "dL/dx")
    for name, prm in layer.named_parameters():
        close(prm.grad, params[name].grad, name)
    # the HIP kernel takes this shape (the gradients above came from it)
    cm, ch, cw = layer._taps()
    w, npar = layer.soft_params(True)
    got = ops.conv_soft_bwd(xg.detach(), npar, w, cm, ch, cw, layer._kind(), layer.d,
                            layer.node_arity, cm.shape[-1], layer.padding, pool, gy.to(DEV))
    assert got is not None
    # only the parameter gradients (gx not wanted): same values
    got2 = ops.conv_soft_bwd(xg.detach(), npar, w, cm, ch, cw, layer._kind(), layer.d,
                             layer.node_arity, cm.shape[-1], layer.padding, pool, gy.to(DEV),
                             need_x=False)
    assert got2[0] is None
    assert torch.equal(got2[1], got[1]) and torch.equal(got2[2], got[2])


def test_fc_soft_backward_skewed_references_and_determinism():
    """Input gradient when references pile onto a few inputs (half of all
    candidates name input 3, some twice on one side): against fp32 autograd
    of the gate16 layer written out in torch; two calls agree bit for bit;
    asking only for the input gradient gives the same values."""
    gen = torch.Generator().manual_seed(9)
    IN, OUT, K, B = 500, 700, 8, 300
    cand = torch.randint(0, IN, (OUT, 2, K), generator=gen, dtype=torch.int32)
    cand[torch.rand(OUT, 2, K, generator=gen) < 0.5] = 3
    cand[:, 0, 1] = cand[:, 0, 0]
    w = torch.softmax(torch.randn(OUT, 2, K, generator=gen), -1)
    npar = torch.randn(OUT, 4, generator=gen)
    x = torch.rand(B, IN, generator=gen)
    gy = torch.randn(B, OUT, generator=gen)
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    nr = npar.clone().requires_grad_(True)
    c = cand.long()
    a = (xr[:, c[:, 0]] * wr[:, 0]).sum(-1)
    b = (xr[:, c[:, 1]] * wr[:, 1]).sum(-1)
    y = nr[:, 0] + nr[:, 1] * a + nr[:, 2] * b + nr[:, 3] * a * b
    (y * gy).sum().backward()
    args = (x.to(DEV), cand.to(DEV), w.to(DEV), npar.to(DEV), 0, 1.0, gy.to(DEV))
    gx, gw, gn = ops.fc_soft_bwd(*args)
    gx2, gw2, gn2 = ops.fc_soft_bwd(*args)
    gx3, none_w, none_n = ops.fc_soft_bwd(*args, need_w=False, need_np=False)
    assert none_w is None and none_n is None
    for got, ref, what in ((gx, xr.grad, "gx"), (gw, wr.grad, "gw"), (gn, nr.grad, "gnp")):
        scale = ref.abs().max().item()
        err = (got.cpu() - ref).abs().max().item()
        assert err <= 1e-4 * scale + 1e-6, f"{what}: max err {err:.3e} (scale {scale:.3e})"
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2) and torch.equal(gn, gn2)
    assert torch.equal(gx, gx3)


# --------------------------------------------------------------------------
# FC layers of n-input LUT nodes (multilinear of any arity, hybrid)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("node,arity,conn,k,IN,OUT,B", [
    ("multilinear", 3, "topk", 8, 300, 200, 37),
    ("hybrid", 4, "topk", 8, 500, 300, 70),
    ("hybrid", 6, "topk", 8, 2000, 1100, 300),     # two output groups, several tiles
    ("multilinear", 6, "topk", 4, 100, 64, 9),
    ("hybrid", 2, "fixed", 1, 64, 50, 20),
    ("multilinear", 5, "fixed", 1, 40, 30, 5),
    ("hybrid", 6, "topk", 8, 20000, 300, 16),       # 2-sample tiles
    ("hybrid", 4, "topk", 3, 90, 70, 11),           # K padded to 4
])
def test_fc_lut_layer_forward_backward_hard(node, arity, conn, k, IN, OUT, B):
    """LUT layers (nodes.py:165-206, the fused op kernels/multilinear.py)
    against the oracle: soft values (hybrid: equal except where an operand is
    within rounding of the 0.5 threshold), gradients of x, the connection and
    node logits against fp32 autograd on the CPU, hard outputs bit for bit."""
    layer = sl.LogicLayer(IN, OUT, node=node, connectome=conn, arity=arity, k=k, seed=7)
    L = dict(prefix="", node=node, arity=arity, conn=conn)
    params = {kk: v.clone().requires_grad_(v.is_floating_point())
              for kk, v in layer.state_dict().items()}
    gen = torch.Generator().manual_seed(13)
    x = torch.rand(B, IN, generator=gen)
    gy = torch.randn(B, OUT, generator=gen)
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.fc_layer_soft(L, params, xr)
    (ref * gy).sum().backward()
    layer = layer.to(DEV).train()
    xg = x.to(DEV).requires_grad_(True)
    out = layer(xg)
    (out * gy.to(DEV)).sum().backward()
    got, want = out.detach().cpu(), ref.detach()
    if node == "hybrid":
        with torch.no_grad():
            a = torch_ref.select_soft(L, params, x)
        near = ((a - 0.5).abs() <= 1e-5).any(2)            # operands at the threshold
        bad = (got - want).abs() > 1e-6
        assert not (bad & ~near).any(), int((bad & ~near).sum())
    else:
        assert_soft_close(got, want, "lut soft")

    def close(g, r, what):
        g = g.cpu()
        scale = r.abs().max().item()
        err = (g - r).abs().max().item()
        assert err <= 1e-4 * scale + 1e-6, f"{what}: max err {err:.3e} (scale {scale:.3e})"

    close(xg.grad, xr.grad, "dL/dx")
    for name, p in layer.named_parameters():
        close(p.grad, params[name].grad, name)
    xb = random_bits(B, IN)
    hard = layer.forward_hard(xb.to(DEV)).cpu()
    assert torch.equal(hard, torch_ref.fc_layer_hard(L, {k2: v.detach() for k2, v in
                                                         params.items()}, xb))


def test_hybrid_logicnet_soft_hard_and_packed():
    """A hybrid LogicNet (the MNIST recipe's node, examples/train_mnist.py:51-52,
    at small size): soft logits and gradients against the oracle, hard counts
    bit for bit, and the bit-packed conversion's logits equal counts / tau."""
    from silogic_amd import bitpacking as bp
    spec = ("LogicNet", dict(in_dim=100, width=200, depth=2, node="hybrid", arity=4, k=8,
                             tau=4.0, decoder_ste=False))
    model = build_product(spec)
    st = torch_ref.structure(spec)
    params = {k: v.clone().requires_grad_(v.is_floating_point())
              for k, v in model.state_dict().items()}
    gen = torch.Generator().manual_seed(21)
    x = (torch.rand(50, 100, generator=gen) > 0.5).float()
    xr = x.clone().requires_grad_(True)
    ref = torch_ref.groupsum_soft(st["head"], torch_ref.forward_features(st, params, xr, hard=False))
    ref.pow(2).sum().backward()
    model = model.to(DEV).train()
    xg = x.to(DEV).requires_grad_(True)
    out = model(xg)
    out.pow(2).sum().backward()
    assert (out.detach().cpu() - ref.detach()).abs().max() < 1e-4
    assert (xg.grad.cpu() - xr.grad).abs().max() < 1e-4
    for name, p in model.named_parameters():
        assert (p.grad.cpu() - params[name].grad).abs().max() < 1e-4, name
    model.eval()
    counts = torch_ref.forward_hard(spec, {k: v.detach() for k, v in params.items()}, x)
    assert torch.equal(model.forward_hard(x.to(DEV)).cpu(), counts)
    packed = bp.convert_logic_net(model)
    logits = packed(x.to(torch.uint8).to(DEV))
    assert torch.equal(logits.cpu(), counts / torch.tensor(4.0))


def test_kernels_dropin_hybrid_ops():
    """silogic.kernels' hybrid ops through the drop-in module, with the
    reference's argument layout (kernels/multilinear.py:160-174,
    kernels/conv_hybrid.py:196), against the oracle."""
    from silogic_amd import kernels
    assert kernels.HAS_MULTILINEAR and kernels.HAS_CONV_HYBRID
    layer = sl.LogicLayer(60, 40, node="hybrid", arity=3, k=4, seed=5)
    L = dict(prefix="", node="hybrid", arity=3, conn="topk")
    sd = layer.state_dict()
    x = torch.rand(9, 60)
    ref = torch_ref.fc_layer_soft(L, sd, x)
    cand = layer._conn.candidates_i32()
    w = torch.softmax(sd["_conn.conn"], dim=2)
    s = torch.sigmoid(sd["node.logits"])
    got = kernels.multilinear_logic(x.to(DEV), cand.to(DEV), w.to(DEV), s.to(DEV), 3).cpu()
    with torch.no_grad():
        a = torch_ref.select_soft(L, sd, x)
    near = ((a - 0.5).abs() <= 1e-5).any(2)
    assert not (((got - ref).abs() > 1e-6) & ~near).any()
    conv = sl.ConvLogicTree(4, 6, kernel=3, tree_depth=1, k=4, node="hybrid", arity=4, seed=4)
    blk = dict(prefix="", cin=4, n=6, kernel=3, depth=1, stride=1, padding=1, connect="topk",
               k=conv.k, node="hybrid", node_arity=4, leaves=4)
    csd = conv.state_dict()
    xc = torch.rand(2, 4, 7, 7)
    cref = torch_ref.conv_soft(blk, csd, xc)
    sc = torch.sigmoid(csd["tree_nodes.0.logits"]).view(6, 1, 16)       # [N, nodes, 2^arity]
    wc = torch.softmax(csd["conn"], dim=2)
    cgot = kernels.conv_hybrid(xc.to(DEV), sc.to(DEV), wc.to(DEV), conv.lc_cm.to(DEV),
                               conv.lc_ch.to(DEV), conv.lc_cw.to(DEV), 1, 4, conv.k, 1, 1, 7,
                               7).cpu()
    leaves = torch_ref.conv_leaves_soft(blk, csd, F.unfold(xc, (3, 3), padding=1))
    cnear = ((leaves - 0.5).abs() <= 1e-5).any(2).view(cref.shape)
    assert not (((cgot - cref).abs() > 1e-6) & ~cnear).any()
