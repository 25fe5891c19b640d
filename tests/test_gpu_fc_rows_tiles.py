"""The fused hard FC network on unpacked rows that the streaming rows kernel
does not take (more than 1024 features, or 32-sample words): each
workgroup packs its own tile's rows in LDS (fp32: bit = x >= 1, bytes:
bit = x != 0) before the layers. Bar: the logits of the same network on
the rows packed by ``pack_bits``, bit for bit. Cases: 64- and 32-sample
words; 4-feature vector reads and the one-feature path (a width that is
not a multiple of 4, or a row pointer off the vector alignment); batches
of one sample, inside one word, across words; fp32 values either side of
the threshold and bytes other than 0 and 1; compact, bank-placed (wire
residual) and type-placed codes."""
import pytest
import torch

import silogic_amd as sl
from silogic_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _codes(in_dim, widths, seed):
    torch.manual_seed(0)
    layers, d = [], in_dim
    for i, w in enumerate(widths):
        layers.append(sl.LogicLayer(d, w, k=4, seed=seed + i).to(DEV))
        d = w
    return ops.fc_hard_codes_net([l.hard_spec() for l in layers], compact=True)


def _rows(B, in_dim, dtype, g, misalign):
    """Rows with values either side of the bit test; ``misalign`` shifts the
    row pointer one element off the 4-feature vector alignment."""
    n = B * in_dim
    if dtype == torch.float32:
        flat = torch.rand(n + 1, generator=g) * 2.0            # [0, 2): x >= 1 half the time
        flat[::7] = 1.0                                         # the threshold itself
        flat[3::11] = 0.9999999
    else:
        pick = torch.randint(0, 4, (n + 1,), generator=g)
        flat = torch.tensor([0, 1, 2, 255], dtype=torch.uint8)[pick]
    flat = flat.to(DEV)
    return flat[1:].view(B, in_dim) if misalign else flat[:n].view(B, in_dim)


def _check(in_dim, widths, C, B, dtype, misalign=False, typed=False, wire_r=0, seed=5):
    spw = ops.fc_hard_net_supported(in_dim, widths, C)
    assert spw in (32, 64)
    assert not (spw == 64 and in_dim <= 1024), "the streaming rows kernel takes this case"
    codes = _codes(in_dim, widths, seed)
    if typed:
        codes = ops.fc_hard_type_place_net(codes, in_dim)
        assert codes.plan is not None
    g = torch.Generator().manual_seed(B * 31 + in_dim)
    x = _rows(B, in_dim, dtype, g, misalign)
    kind = ops.ROWS_F32 if dtype == torch.float32 else ops.ROWS_U8
    print(f"rows tiles: in_dim {in_dim} widths {widths} B {B} {dtype} spw {spw} "
          f"misalign {misalign} typed {typed} wire_r {wire_r}", flush=True)
    got = ops.fc_hard_net(x, kind, B, in_dim, codes, C, wire_r)
    xp = ops.pack_bits(x.contiguous(), word_major=True)
    want = ops.fc_hard_net(xp, ops.PACKED_WORD_MAJOR, B, in_dim, codes, C, wire_r)
    torch.cuda.synchronize()
    assert got.shape == (B, C)
    assert torch.equal(got, want), int((got != want).any(1).sum())


@pytest.mark.parametrize("dtype", [torch.float32, torch.uint8])
@pytest.mark.parametrize("B", [1, 31, 33, 64 * 3 + 5])
def test_wide_rows_64_sample_words(dtype, B):
    _check(2048, [3000, 3000, 100], 10, B, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.uint8])
@pytest.mark.parametrize("B", [1, 32, 64 * 2 + 13])
def test_rows_32_sample_words(dtype, B):
    _check(4096, [16380, 16380, 50], 10, B, dtype, seed=9)


@pytest.mark.parametrize("dtype", [torch.float32, torch.uint8])
@pytest.mark.parametrize("in_dim,widths,C", [
    (1030, [2000, 40], 4),            # width 2 mod 4: one feature at a time, 64-sample words
    (1501, [16380, 30], 5),           # odd width, 32-sample words
])
def test_rows_one_feature_path(dtype, in_dim, widths, C):
    _check(in_dim, widths, C, 64 + 9, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.uint8])
def test_rows_off_the_vector_alignment(dtype):
    _check(2048, [3000, 100], 10, 70, dtype, misalign=True)


@pytest.mark.parametrize("in_dim,widths,C", [
    (2048, [3000, 3000, 100], 10),
    (4096, [16380, 16380, 50], 10),
])
def test_rows_type_placed_codes(in_dim, widths, C):
    _check(in_dim, widths, C, 64 * 2 + 3, torch.float32, typed=True, seed=21)


def test_rows_wire_residual():
    # equal widths: each layer's first wire_r outputs copy its inputs
    _check(2048, [2048, 2048, 100], 10, 64 + 40, torch.float32, wire_r=16, seed=33)


def _stack(in_dim, widths, seed, ones_last=False):
    torch.manual_seed(0)
    layers, d = [], in_dim
    for i, w in enumerate(widths):
        layer = sl.LogicLayer(d, w, k=4, seed=seed + i)
        if ones_last and i == len(widths) - 1:
            with torch.no_grad():
                layer.node.gate_logits[:, 15] += 10.0       # gate 15: constant 1
        layers.append(layer.to(DEV))
        d = w
    return layers


@pytest.mark.parametrize("C,G", [
    (16, 1024),      # 32-sample words, one 1024-word pass
    (15, 1025),      # one 2048-word pass, a partial row
    (10, 1638),      # config 4's classes
    (8, 2047),
    (8, 2048),       # a pass that counts to 2048 (twelve bit slices)
    (5, 3000),       # two passes: 2048 + 952 words
    (2, 4096),       # two full passes
])
def test_groupsum_of_32_sample_words(C, G):
    """The fused network's class counts on 32-sample words: a last layer of
    constant-1 gates counts G for every sample; random last layers match the
    per-layer kernels followed by the separate packed GroupSum kernel."""
    in_dim, widths, B = 1000, [16380, C * G], 64 + 21
    assert ops.fc_hard_net_supported(in_dim, widths, C) == 32
    g = torch.Generator().manual_seed(C * G)
    x = (torch.rand(B, in_dim, generator=g) < 0.5).float().to(DEV)
    print(f"groupsum: C {C} G {G}", flush=True)
    ones = _stack(in_dim, widths, 61, ones_last=True)
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in ones], compact=True)
    got = ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, C)
    assert torch.equal(got, torch.full((B, C), float(G), device=DEV))
    rnd = _stack(in_dim, widths, 71)
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in rnd], compact=True)
    got = ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, C)
    xp = ops.pack_bits(x)
    for c in ops.fc_hard_codes_net([l.hard_spec() for l in rnd]):
        xp = ops.fc_hard_layer(xp, c)
    want = ops.groupsum_packed(xp, B, C)
    assert torch.equal(got, want), int((got != want).any(1).sum())


@pytest.mark.parametrize("C,G", [
    (1, 7),
    (3, 250),
    (10, 1000),      # config 2's classes
    (5, 1024),       # one full pass
    (9, 1025),       # a second pass of one word
    (4, 2047),
    (3, 3000),       # three passes
    (13, 640),
])
def test_groupsum_of_64_sample_words(C, G):
    """The fused network's class counts on 64-sample words: constant-1 last
    layers count G for every sample; random last layers match the per-layer
    kernels followed by the separate packed GroupSum kernel. Rows here
    stream through the rows kernel (1000 features) and, packed, through the
    packed-network kernel; class counts from 1 to 13 and class sizes across
    one to three 1024-word passes."""
    in_dim, widths, B = 1000, [3000, C * G], 64 * 2 + 21
    assert ops.fc_hard_net_supported(in_dim, widths, C) == 64
    g = torch.Generator().manual_seed(C * G + 1)
    x = (torch.rand(B, in_dim, generator=g) < 0.5).float().to(DEV)
    print(f"groupsum 64: C {C} G {G}", flush=True)
    ones = _stack(in_dim, widths, 81, ones_last=True)
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in ones], compact=True)
    full = torch.full((B, C), float(G), device=DEV)
    assert torch.equal(ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, C), full)
    xw = ops.pack_bits(x, word_major=True)
    assert torch.equal(ops.fc_hard_net(xw, ops.PACKED_WORD_MAJOR, B, in_dim, codes, C), full)
    rnd = _stack(in_dim, widths, 91)
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in rnd], compact=True)
    got = ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, codes, C)
    got_p = ops.fc_hard_net(xw, ops.PACKED_WORD_MAJOR, B, in_dim, codes, C)
    xp = ops.pack_bits(x)
    for c in ops.fc_hard_codes_net([l.hard_spec() for l in rnd]):
        xp = ops.fc_hard_layer(xp, c)
    want = ops.groupsum_packed(xp, B, C)
    assert torch.equal(got, want), int((got != want).any(1).sum())
    assert torch.equal(got_p, want)


@pytest.mark.parametrize("B", [1, 64, 200, 64 * 64, 64 * 65])
def test_small_batches_take_32_sample_tiles(B):
    """Rows of a 64-sample-word network at batches of at most one tile per
    four CUs are packed per 32-sample tile (256 CUs: B <= 4096); above, the
    streaming rows kernel. Both match the packed 64-sample words' path."""
    in_dim, widths, C = 784, [2000, 2000, 2000], 10
    assert ops.fc_hard_net_supported(in_dim, widths, C) == 64
    codes = _codes(in_dim, widths, 51)
    typed = ops.fc_hard_type_place_net(codes, in_dim)
    g = torch.Generator().manual_seed(B)
    x = (torch.rand(B, in_dim, generator=g) < 0.4).float().to(DEV)
    print(f"small batch rows: B {B}", flush=True)
    want = ops.fc_hard_net(ops.pack_bits(x, word_major=True), ops.PACKED_WORD_MAJOR, B, in_dim,
                           codes, C)
    for c in (codes, typed):
        assert torch.equal(ops.fc_hard_net(x, ops.ROWS_F32, B, in_dim, c, C), want)
        assert torch.equal(ops.fc_hard_net(x.to(torch.uint8), ops.ROWS_U8, B, in_dim, c, C), want)
