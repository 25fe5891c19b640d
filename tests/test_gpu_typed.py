"""Type-uniform placement of the fused hard network
(slg_fc_hard_type_place_net + slg_fc_hard_net_typed) on unpacked rows and
packed words: a relabelling of the circuit in which each wave's first rows
hold one gate type, so the logits must be the same bits as the unplaced
network's, whatever the mix of gate types (uniform draws, or one type
dominating so that it takes several waves and the plan shrinks U)."""
import pytest
import torch

import silogic_amd as sl
from oracle import torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _net(in_dim, widths, skew=None, seed=11):
    torch.manual_seed(0)
    layers, d = [], in_dim
    for i, w in enumerate(widths):
        layer = sl.LogicLayer(d, w, k=4, seed=seed + i)
        if skew is not None:
            gate, frac = skew
            g = torch.Generator().manual_seed(seed + 100 + i)
            pick = torch.rand(w, generator=g) < frac
            with torch.no_grad():
                layer.node.gate_logits[pick, gate] += 10.0
        layers.append(layer)
        d = w
    net = torch.nn.Module()
    net.layers = torch.nn.ModuleList(layers).to(DEV)
    return net


def _codes(net):
    return ops.fc_hard_codes_net([l.hard_spec() for l in net.layers], compact=True)


def _check_plan(typed, widths, in_dim):
    S = ops.fc_hard_type_slots(in_dim, widths)
    maxo = S // 1024
    plan = typed.plan.cpu()
    for l, w in enumerate(widths):
        U, rows = int(plan[l, 0]), int(plan[l, 1])
        assert 0 <= U <= rows <= maxo, (l, U, rows)
        assert rows * 1024 >= (w if U == 0 else 0)
        assert all(0 <= int(t) < 16 for t in plan[l, 2:18])
        # each row records the layout it belongs to: slots per thread, input width
        assert int(plan[l, 18]) == maxo and int(plan[l, 19]) == in_dim
    assert int(plan[-1, 0]) == 0
    return plan


@pytest.mark.parametrize("in_dim,widths,C,skew", [
    (784, [2000, 2000, 2000], 10, None),
    (200, [300, 250, 90], 10, None),
    (64, [1000, 1000, 1000], 10, (6, 0.7)),     # xor dominates: several waves of one type
    (100, [4000, 4000, 40], 4, (3, 0.5)),       # pass-through a
    (100, [3000, 3000, 30], 5, (0, 0.6)),       # constant 0
    (50, [40], 4, None),                        # one layer: nothing to place
    (1024, [9000, 7000, 5000, 100], 10, (12, 0.4)),
])
def test_typed_network_is_bit_exact(in_dim, widths, C, skew):
    net = _net(in_dim, widths, skew)
    codes = _codes(net)
    typed = ops.fc_hard_type_place_net(codes, in_dim)
    again = ops.fc_hard_type_place_net(codes, in_dim)
    assert all(torch.equal(a, b) for a, b in zip(typed, again))      # deterministic
    assert torch.equal(typed.plan, again.plan)
    plan = _check_plan(typed, widths, in_dim)
    if len(widths) > 1 and widths[0] >= 1000:
        assert int(plan[0, 0]) >= 1                                   # uniform rows in use
    g = torch.Generator().manual_seed(1)
    B = 64 * 9 + 17
    x = (torch.rand(B, in_dim, generator=g) < 0.4).float()
    ref = ops.fc_hard_net(x.to(DEV), ops.ROWS_F32, B, in_dim, codes, C)
    got = ops.fc_hard_net(x.to(DEV), ops.ROWS_F32, B, in_dim, typed, C)
    assert torch.equal(got, ref)
    got8 = ops.fc_hard_net(x.to(torch.uint8).to(DEV), ops.ROWS_U8, B, in_dim, typed, C)
    assert torch.equal(got8, ref)


@pytest.mark.parametrize("in_dim,widths,C,skew", [
    (784, [2000, 2000, 2000], 10, None),        # 64-sample words, MAXO 2
    (1500, [1500, 1500, 30], 5, (6, 0.6)),      # inputs wider than a workgroup
    (4096, [8000, 8000, 50], 10, None),         # MAXO 8
    (2000, [16380, 16380, 100], 10, (3, 0.3)),  # MAXO 16: 32-sample words
])
def test_typed_network_on_packed_input_is_bit_exact(in_dim, widths, C, skew):
    """Packed input ([in0][nw] and [nw][in0]) through the type-placed codes:
    the logits of the unplaced network, bit for bit, for 64- and 32-sample
    words."""
    net = _net(in_dim, widths, skew, seed=41)
    codes = _codes(net)
    typed = ops.fc_hard_type_place_net(codes, in_dim)
    _check_plan(typed, widths, in_dim)
    g = torch.Generator().manual_seed(7)
    B = 64 * 5 + 29
    x = (torch.rand(B, in_dim, generator=g) < 0.45).float().to(DEV)
    ref = ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, C)
    assert torch.equal(ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, typed, C), ref)
    for word_major, kind in ((False, ops.PACKED), (True, ops.PACKED_WORD_MAJOR)):
        xp = ops.pack_bits(x, word_major=word_major)
        plain = ops.fc_hard_net(xp, kind, B, in_dim, codes, C)
        assert torch.equal(plain, ref)
        assert torch.equal(ops.fc_hard_net(xp, kind, B, in_dim, typed, C), plain)


def test_typed_codes_take_rows_wider_than_a_workgroup():
    """Rows wider than 1024 features are packed per tile inside the network
    kernel: the logits of the packed input's, bit for bit; a wire residual
    with type-placed codes is refused."""
    net = _net(1500, [1500, 30])
    codes = _codes(net)
    typed = ops.fc_hard_type_place_net(codes, 1500)
    g = torch.Generator().manual_seed(3)
    x = (torch.rand(64 + 7, 1500, generator=g) < 0.5).float().to(DEV)
    want = ops.fc_hard_net(ops.pack_bits(x), ops.PACKED, 71, 1500, codes, 10)
    assert torch.equal(ops.fc_hard_net(x, ops.ROWS_F32, 71, 1500, typed, 10), want)
    with pytest.raises(ValueError):
        ops.fc_hard_net(ops.pack_bits(x), ops.PACKED, 71, 1500, typed, 10, wire_r=8)


def test_config_2_typed_forward_hard_matches_the_oracle():
    """Config 2 (784 -> 6 x 10000): forward_hard on fp32 rows takes the
    type-uniform layout (at least eight uniform rows of ten per hidden layer) and
    matches the oracle bit for bit on a batch slice."""
    from silogic_amd.synthetic import CONFIGS, build_config, config_inputs
    model = build_config(2, sl).eval()
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    x = config_inputs(2, 64 * 3 + 9)
    with torch.no_grad():
        got = model.forward_hard(x.to(DEV)).cpu()
    codes = model.layers[0].__dict__["_derived_net_codes"][1]
    assert codes.plan is not None
    plan = codes.plan.cpu()
    assert all(int(plan[l, 0]) >= 8 and int(plan[l, 1]) <= 10 for l in range(5)), plan[:, :2]
    assert torch.equal(got, torch_ref.forward_hard(CONFIGS[2], sd, x))


@pytest.mark.parametrize("in_dim,widths,C,B", [
    (784, [2000, 2000], 10, 1),                       # 16-sample chunks, one sample
    (784, [2000, 2000, 2000, 2000], 10, 63),          # four layers, a partial tile
    (300, [1500] * 5, 10, 64),                        # 11-sample chunks, one chunk after the loop
    (1024, [3000] * 8, 10, 65),                       # deeper than the chunks
    (128, [700, 900, 300], 3, 130),
])
def test_typed_network_edge_batches_and_depths(in_dim, widths, C, B):
    net = _net(in_dim, widths, seed=31)
    codes = _codes(net)
    typed = ops.fc_hard_type_place_net(codes, in_dim)
    _check_plan(typed, widths, in_dim)
    g = torch.Generator().manual_seed(B)
    x = (torch.rand(B, in_dim, generator=g) < 0.5).float()
    ref = ops.fc_hard_net(x.to(DEV), ops.ROWS_F32, B, in_dim, codes, C)
    assert torch.equal(ops.fc_hard_net(x.to(DEV), ops.ROWS_F32, B, in_dim, typed, C), ref)
    x8 = x.to(torch.uint8).to(DEV)
    assert torch.equal(ops.fc_hard_net(x8, ops.ROWS_U8, B, in_dim, typed, C), ref)


@pytest.mark.parametrize("in_dim", [784, 786, 200, 1024])
@pytest.mark.parametrize("B", [1, 63, 64 * 3 + 5, 64 * 300 + 7])
def test_row_streams_match_the_packed_path(in_dim, B):
    """The rows kernel's fused packing (one feature a thread, chunks of
    samples streamed during the layers) must give the bits pack_bits gives
    (v >= 1, NaN and negatives 0) on non-binary fp32 rows, on partial tiles
    and on more tiles than workgroups, through plain and type-placed codes."""
    net = _net(in_dim, [1200, 1100, 900], seed=57)
    codes = _codes(net)
    typed = ops.fc_hard_type_place_net(codes, in_dim)
    g = torch.Generator().manual_seed(B + in_dim)
    x = torch.rand(B, in_dim, generator=g) * 3.0 - 1.0
    x[torch.rand(B, in_dim, generator=g) < 0.1] = 1.0
    x[torch.rand(B, in_dim, generator=g) < 0.01] = float("nan")
    x = x.to(DEV)
    ref = ops.fc_hard_net(ops.pack_bits(x), ops.PACKED, B, in_dim, codes, 10)
    assert torch.equal(ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, 10), ref)
    assert torch.equal(ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, typed, 10), ref)


def test_typed_plan_for_another_width_gives_nan_logits():
    """Codes placed for one input width, run through the C ABI for another:
    a different slot count (1500 -> 2 slots per thread, 2500 -> 4) and the
    same slot count with another width both give NaN logits (the kernel
    checks the plan's own record before it reads a code)."""
    import ctypes
    from silogic_amd import _lib
    net = _net(100, [1500, 1500, 40])
    widths = [1500, 1500, 40]
    typed = ops.fc_hard_type_place_net(_codes(net), 100)
    _check_plan(typed, widths, 100)
    B = 70
    for in_dim in (2500, 1000):
        assert ops.fc_hard_type_slots(in_dim, widths) > 0
        x = (torch.rand(B, in_dim, generator=torch.Generator().manual_seed(5)) < 0.5).float()
        xp = ops.pack_bits(x.to(DEV), word_major=True)
        out = torch.zeros((B, 4), device=DEV)
        _lib.call("slg_fc_hard_net_typed", ops._p(xp), ops.PACKED_WORD_MAJOR, B, in_dim,
                  len(typed), typed.widths, typed.ptrs, ops._p(typed.plan), 4, ops._p(out),
                  ops._stream(xp))
        torch.cuda.synchronize()
        assert torch.isnan(out).all(), in_dim
        with pytest.raises(ValueError):
            ops.fc_hard_net(xp, ops.PACKED_WORD_MAJOR, B, in_dim, typed, 4)


def test_forward_hard_on_inputs_of_two_widths():
    """One model, forward_hard on inputs 100 wide and then 2500 wide (the
    layer reads indices below 100, so the extra columns change nothing):
    the type-placed codes are kept per input width (the slot count differs:
    2 and 4 per thread), and both calls give the oracle's logits."""
    torch.manual_seed(0)
    model = sl.LogicNet(in_dim=100, width=1500, depth=2, num_classes=10, k=4, seed=5).eval()
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    g = torch.Generator().manual_seed(6)
    x = (torch.rand(130, 100, generator=g) < 0.5).float()
    wide = torch.cat([x, (torch.rand(130, 2400, generator=g) < 0.5).float()], dim=1)
    ref = torch_ref.forward_hard(("LogicNet", dict(in_dim=100, width=1500, depth=2,
                                                   num_classes=10, k=4)), sd, x)
    with torch.no_grad():
        for inp in (x, wide, x, wide):
            got = model.forward_hard(inp.to(DEV)).cpu()
            assert torch.equal(got, ref)
            codes = model.layers[0].__dict__["_derived_net_codes"][1]
            assert codes.plan is not None and codes.in_dim == inp.shape[1]
