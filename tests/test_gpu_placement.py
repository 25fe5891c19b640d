"""Bank-aware placement of the fused hard network's outputs
(slg_fc_hard_place_net): a relabelling of the circuit, so the logits stay
bit-exact, that cuts the modelled LDS conflict cost of the operand reads."""
import pytest
import torch

import silogic_amd as sl
from oracle import torch_ref
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _codes(model):
    return ops.fc_hard_codes_net([l.hard_spec() for l in model.layers], compact=True)


def _half_wave_cost(codes):
    """Mean over 32-slot groups and both operands of the most distinct words
    of one bank class (word index mod 32) the group reads."""
    tot, n = 0, 0
    for c in codes[:-1]:                      # the layers whose outputs are placed
        c = c.long().cpu() & 0xFFFFFFFF
        S = c.shape[0] - c.shape[0] % 32
        for op in ((c >> 14) & 0x3FFF, c & 0x3FFF):
            g = op[:S].view(-1, 32)
            for row in g:
                u = torch.unique(row)
                tot += int(torch.bincount(u % 32, minlength=32).max())
                n += 1
    return tot / n


@pytest.mark.parametrize("in_dim,widths,C", [(200, [300, 250, 90], 10), (64, [1000, 1000, 1000], 10),
                                             (784, [2000, 2000, 2000, 2000], 10), (50, [40], 4),
                                             (100, [33, 65, 20], 5)])
def test_placed_network_is_bit_exact(in_dim, widths, C):
    torch.manual_seed(0)
    layers = []
    d = in_dim
    for i, w in enumerate(widths):
        layers.append(sl.LogicLayer(d, w, k=4, seed=11 + i))
        d = w
    net = torch.nn.Module()
    net.layers = torch.nn.ModuleList(layers).to(DEV)
    codes = _codes(net)
    placed = ops.fc_hard_place_net(codes)
    again = ops.fc_hard_place_net(codes)
    assert all(torch.equal(a, b) for a, b in zip(placed, again))          # deterministic
    for l, (c, p) in enumerate(zip(codes, placed)):
        expect = c.shape[0] if l == len(codes) - 1 else (c.shape[0] + 31) // 32 * 32
        assert p.shape[0] == expect
    g = torch.Generator().manual_seed(1)
    B = 64 * 7 + 5
    x = (torch.rand(B, in_dim, generator=g) < 0.4).float().to(DEV)
    ref = ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, C)
    got = ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, placed, C)
    assert torch.equal(got, ref)
    xp = ops.pack_bits(x, word_major=True)
    assert torch.equal(ops.fc_hard_net(xp, ops.PACKED_WORD_MAJOR, B, in_dim, placed, C), ref)


def test_placement_cuts_modelled_conflicts_at_config_2():
    """Config 2's network (784 -> 6 x 10000): the placed reads cost about 1.7
    modelled cycles per 32-lane half instead of about 3.5 (1 = conflict-free),
    and forward_hard (which places the codes) matches the oracle bit for
    bit on a batch slice."""
    from silogic_amd.synthetic import CONFIGS, build_config, config_inputs
    model = build_config(2, sl).eval()
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    model = model.to(DEV)
    codes = _codes(model)
    placed = ops.fc_hard_place_net(codes)
    before, after = _half_wave_cost(codes), _half_wave_cost(placed)
    assert after < 0.6 * before and after < 2.0, (before, after)
    x = config_inputs(2, 64 * 3 + 9)
    with torch.no_grad():
        got = model.forward_hard(x.to(DEV)).cpu()
    assert torch.equal(got, torch_ref.forward_hard(CONFIGS[2], sd, x))
