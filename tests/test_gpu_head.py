"""Small networks on packed words at small batches (a conv network's head).
One-layer networks take a workgroup per (sample word, class), which reads
its gates' operand words from memory; deeper ones the fused kernel. The
class counts must equal the per-layer packed kernels plus
slg_groupsum_packed, for both packed layouts; plain, bank-placed and
type-placed codes; classes of one gate to several thousand (GroupSum passes
of 1024 words); partial words; and batches on either side of the switch to
the fused kernel (one workgroup per word from half the CUs on)."""
import pytest
import torch

import silogic_amd as sl
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layers(in_dim, widths, seed):
    torch.manual_seed(0)
    out, d = [], in_dim
    for i, w in enumerate(widths):
        out.append(sl.LogicLayer(d, w, k=4, seed=seed + i).to(DEV))
        d = w
    return out


@pytest.mark.parametrize("in_dim,widths,C", [
    (16384, [1280], 10),        # config 5's head
    (2304, [2560, 2560], 10),   # config 3's head
    (100, [40], 4),
    (300, [3000], 3),
    (200, [2100], 1),           # one class of 2100 gates: three GroupSum passes
    (64, [7], 7),               # one gate per class
    (500, [700, 90], 9),
    (40, [5000, 2048], 2),      # a class of 1024 gates over a wide layer 0
])
@pytest.mark.parametrize("B", [1, 64 * 3 + 5, 64 * 100, 64 * 200 + 1])
def test_small_head_counts(in_dim, widths, C, B):
    layers = _layers(in_dim, widths, seed=in_dim + widths[0])
    g = torch.Generator().manual_seed(B)
    x = (torch.rand(B, in_dim, generator=g) < 0.5).float().to(DEV)
    xp = ops.pack_bits(x)
    h = xp
    for layer in layers:
        h = layer.packed_forward(h)
    ref = ops.groupsum_packed(h, B, C)
    codes = ops.fc_hard_codes_net([layer.hard_spec() for layer in layers], compact=True)
    variants = [("plain", codes), ("bank", ops.NetCodes(ops.fc_hard_place_net(codes)))]
    if ops.fc_hard_type_slots(in_dim, widths) > 0:
        variants.append(("typed", ops.fc_hard_type_place_net(codes, in_dim)))
    xw = ops.pack_bits(x, word_major=True)
    for kind, words in ((ops.PACKED, xp), (ops.PACKED_WORD_MAJOR, xw)):
        for name, c in variants:
            got = ops.fc_hard_net(words, kind, B, in_dim, c, C)
            assert torch.equal(got, ref), (kind, name)
