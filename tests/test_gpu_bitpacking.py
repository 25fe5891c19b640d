"""silogic_amd.bitpacking (the reference's silogic.bitpacking API) against the
numpy restatement in oracle/packed_ref.py: packed layouts bit for bit, logits
exactly (the reference's tests/test_bitpacking.py compares argmax only)."""
import numpy as np
import pytest
import torch

import silogic_amd as sl
from silogic_amd import bitpacking as bp
from silogic_amd.bitpacking.packed_layer import (BitpackedConvLUTLayer, BitpackedConvTreeLayer,
                                                 BitpackedFCLayer, BitpackedLUTLayer)
from conftest import build_product
from oracle import packed_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _bits(shape, seed=0):
    return np.random.default_rng(seed).integers(0, 2, shape, dtype=np.uint8)


def _words(shape, seed=0):
    return np.random.default_rng(seed).integers(-2 ** 63, 2 ** 63 - 1, shape, dtype=np.int64,
                                                endpoint=True)


@pytest.mark.parametrize("B,dim", [(1, 1), (63, 8), (64, 64), (65, 256), (200, 784)])
def test_pack_roundtrip_and_layout(B, dim):
    x = _bits((B, dim), seed=B + dim)
    packed = bp.pack_bits(x)
    assert isinstance(packed, np.ndarray) and packed.dtype == np.int64
    assert np.array_equal(packed, packed_ref.pack_bits(x))
    assert np.array_equal(bp.unpack_bits(packed, B), x)
    t = bp.pack_bits(torch.from_numpy(x).to(DEV))            # tensors stay on the GPU
    assert t.is_cuda and np.array_equal(t.cpu().numpy(), packed)


def test_n_words():
    assert [bp.n_words(b) for b in (1, 64, 65, 128, 129)] == [1, 1, 2, 2, 3]


def test_group_sum_and_mask():
    B, width, nc = 137, 100, 10
    x = _bits((B, width), seed=3)
    packed = bp.pack_bits(x)
    ref = x.reshape(B, nc, width // nc).sum(2).astype(np.float32)
    np.testing.assert_array_equal(bp.group_sum_packed(packed, B, nc, tau=1.0), ref)
    np.testing.assert_array_equal(bp.group_sum_packed(packed, B, nc, tau=4.0), ref / 4.0)
    # rows past C * (dim // C) do not count (ops.py:88-97)
    extra = np.concatenate([packed, packed[:3]])
    np.testing.assert_array_equal(bp.group_sum_packed(extra, B, nc), ref)
    w = _words((5, 3), seed=4)
    assert np.array_equal(bp.mask_last_word(w.copy(), 150), packed_ref.mask_last_word(w.copy(), 150))
    t = torch.from_numpy(w).to(DEV)
    assert np.array_equal(bp.mask_last_word(t, 150).cpu().numpy(),
                          packed_ref.mask_last_word(w.copy(), 150))


def test_apply_gate_all_16():
    a, b = _words((7, 5), seed=5), _words((7, 5), seed=6)
    for g in range(16):
        assert np.array_equal(bp.apply_gate(a, b, g), packed_ref.GATE_OPS[g](a, b)), g
    assert np.array_equal(bp.code_to_gate16(), packed_ref.code_to_gate16())


def test_fc_layer_matches_oracle_and_checks_bounds():
    rng = np.random.default_rng(7)
    IN, OUT, nw = 90, 300, 5
    gates = rng.integers(0, 16, OUT)
    a, b = rng.integers(0, IN, OUT), rng.integers(0, IN, OUT)
    x = _words((IN, nw), seed=8)
    layer = BitpackedFCLayer(gates, a, b)
    ref = np.empty((OUT, nw), dtype=np.int64)
    for o in range(OUT):
        ref[o] = packed_ref.GATE_OPS[gates[o]](x[a[o]], x[b[o]])
    assert np.array_equal(layer.forward(x), ref)
    assert sum(layer.gate_histogram.values()) == OUT
    with pytest.raises(ValueError):
        layer.forward(x[: a.max()])                           # operand rows past the input


@pytest.mark.parametrize("arity", [1, 2, 3, 4, 5, 6])
def test_lut_layer(arity):
    rng = np.random.default_rng(arity)
    IN, OUT, nw = 40, 70, 3
    tt = rng.integers(0, 2, (OUT, 2 ** arity)).astype(bool)
    idx = rng.integers(0, IN, (OUT, arity))
    x = _words((IN, nw), seed=10 + arity)
    ref = packed_ref.lut_eval(tt, [x[idx[:, j]] for j in range(arity)])
    assert np.array_equal(BitpackedLUTLayer(tt, idx).forward(x), ref)


@pytest.mark.parametrize("k,stride,pad,H,W", [(3, 1, 1, 7, 9), (3, 2, 1, 8, 8), (1, 1, 0, 5, 4),
                                               (5, 1, 2, 6, 5), (3, 1, 0, 6, 6)])
def test_packed_unfold(k, stride, pad, H, W):
    x3 = _words((3, H * W, 2), seed=H * W + k)
    ref = packed_ref.packed_unfold(x3, k, stride, pad, H, W)
    assert np.array_equal(bp.packed_unfold(x3, k, k, stride, pad, H, W), ref)
    t = bp.packed_unfold_gpu(torch.from_numpy(x3).to(DEV), k, k, stride, pad, H, W)
    assert np.array_equal(t.cpu().numpy(), ref)


@pytest.mark.parametrize("H,W", [(8, 8), (7, 9), (2, 3)])
def test_packed_or_pool(H, W):
    x3 = _words((4, H * W, 3), seed=H + W)
    assert np.array_equal(bp.packed_or_pool(x3, H, W, 2), packed_ref.packed_or_pool(x3, H, W))
    # a 3x3 window is the OR of the 2x2-pool's definition over 9 positions
    p3 = bp.packed_or_pool(x3, H, W, 3)
    Ho, Wo = H // 3, W // 3
    ref = np.zeros((4, Ho * Wo, 3), dtype=np.int64)
    for dy in range(3):
        for dx in range(3):
            l = (np.arange(Ho * Wo) // max(Wo, 1) * 3 + dy) * W + (np.arange(Ho * Wo) % max(Wo, 1)) * 3 + dx
            ref |= x3[:, l, :]
    assert np.array_equal(p3, ref)


def _fc_case(spec, B, D, seed=0):
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    x = _bits((B, D), seed=seed)
    return model.to(DEV).eval(), sd, x


@pytest.mark.parametrize("spec,B,D", [
    (("LogicNet", dict(in_dim=128, width=200, depth=4, k=8)), 200, 128),
    (("LogicNet", dict(in_dim=128, width=200, depth=4, connectome="fixed")), 200, 128),
    (("WARPNet", dict(in_dim=128, width=200, depth=4, k=8)), 200, 128),
    (("LogicNet", dict(in_dim=64, width=100, depth=2, node="multilinear", arity=2, k=4)), 100, 64),
    (("LogicNet", dict(in_dim=128, width=200, depth=4, k=8, wire_residual=0.1)), 100, 128),
    (("LogicNet", dict(in_dim=256, width=500, depth=4, k=8)), 1024, 256),
])
def test_convert_logic_net(spec, B, D):
    model, sd, x = _fc_case(spec, B, D)
    net = bp.convert_logic_net(model)
    ref = packed_ref.forward_hard(spec, sd, x)                  # raw counts
    tau = model.head.tau
    logits = net(x)
    assert isinstance(logits, np.ndarray) and logits.shape == ref.shape
    np.testing.assert_array_equal(logits, ref / np.float32(tau))     # counts / tau in fp32
    t = net(torch.from_numpy(x).to(DEV))
    assert t.is_cuda and np.array_equal(t.cpu().numpy(), logits)
    # the per-layer kernels (the path for layers the fused kernel cannot take)
    packed = bp.pack_bits(torch.from_numpy(x).to(DEV))
    for layer in net.packed_layers:
        prev = packed
        packed = layer.forward(packed)
        if net.wire_r and prev.shape[0] == packed.shape[0]:
            packed[:net.wire_r] = prev[:net.wire_r]
    per_layer = bp.group_sum_packed(packed, B, model.head.num_classes, tau)
    assert np.array_equal(per_layer.cpu().numpy(), logits)
    hard = model.forward_hard(torch.from_numpy(x).to(DEV)).cpu().numpy()
    assert np.array_equal(logits, hard / np.float32(tau))


CONV_CASES = [
    dict(in_channels=3, in_hw=8, channels=[8, 16], head_widths=[80], connect="fixed",
         kernel=3, tree_depth=2, n_chan=2),
    dict(in_channels=3, in_hw=8, channels=[8, 16], head_widths=[80], connect="topk", k=4,
         kernel=3, tree_depth=2, n_chan=2),
    dict(in_channels=3, in_hw=16, channels=[4, 8], head_widths=[80], connect="fixed",
         kernel=3, tree_depth=2, n_chan=2),
    dict(in_channels=3, in_hw=8, channels=[8, 16], head_widths=[80], node="multilinear",
         arity=4, tree_depth=1, connect="topk", k=4, kernel=3, n_chan=2),
    dict(in_channels=2, in_hw=9, channels=[6], head_widths=[40], connect="topk", k=4,
         kernel=3, tree_depth=3, n_chan=2),
    dict(in_channels=4, in_hw=6, channels=[4, 4], head_widths=[20], connect="topk", k=4,
         kernel=3, tree_depth=2, n_chan=2, wire_residual=0.5),
]


@pytest.mark.parametrize("args", CONV_CASES)
def test_convert_logic_conv_net(args):
    spec = ("LogicConvNet", dict(args, num_classes=10))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    B = 64 if args["in_hw"] == 16 else 20
    x = _bits((B, args["in_channels"], args["in_hw"], args["in_hw"]), seed=B)
    model = model.to(DEV).eval()
    net = bp.convert_logic_conv_net(model)
    ref = packed_ref.forward_hard(spec, sd, x)
    tau = model.head.tau
    logits = net(x)
    np.testing.assert_array_equal(logits, ref / np.float32(tau))
    gpu_net = bp.BitpackedConvGPUNet.from_conv_net(net, args["in_hw"], args["in_hw"], device="cuda")
    assert np.array_equal(gpu_net(x), logits)
    hard = model.forward_hard(torch.from_numpy(x).to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(hard, ref)
    if args.get("wire_residual"):
        return                      # the per-block walk below has no residual copy
    # the unfold -> tree -> pool kernels on every block (the non-fused path)
    H = args["in_hw"]
    x3 = bp.pack_conv_input(torch.from_numpy(x).to(DEV))
    for layer in net.bp_conv_layers:
        y = layer.forward_packed(bp.packed_unfold(x3, layer.kh, layer.kw, 1, layer.padding, H, H))
        x3 = bp.packed_or_pool(y, H, H, 2)
        H //= 2
    packed = x3.reshape(-1, x3.shape[-1])
    for layer in net.packed_head_layers:
        packed = layer.forward(packed)
    alt = bp.group_sum_packed(packed, B, 10, tau)
    assert np.array_equal(alt.cpu().numpy(), logits)


@pytest.mark.parametrize("arity,depth", [(2, 2), (3, 2), (2, 4), (4, 1)])
def test_conv_lut_tree_layer(arity, depth):
    """k-ary LUT trees (deeper than the fused kernel takes) on unfolded input."""
    rng = np.random.default_rng(arity * 10 + depth)
    n, L, nw, P = 9, 12, 2, 27
    leaves = arity ** depth
    leaf = rng.integers(0, P, (n, leaves))
    tts = [rng.integers(0, 2, (n * arity ** (depth - 1 - i), 2 ** arity)).astype(bool)
           for i in range(depth)]
    xu = _words((P, L, nw), seed=3)
    layer = BitpackedConvLUTLayer(leaf, tts, arity, kh=3, kw=3, stride=1, padding=1, cin=3)
    cur = xu[leaf.reshape(-1)].reshape(n, leaves, L, nw)
    for i in range(depth):
        m = cur.shape[1] // arity
        tt = tts[i].reshape(n, m, -1)
        res = np.empty((n, m, L, nw), dtype=np.int64)
        for mi in range(m):
            res[:, mi] = packed_ref.lut_eval(tt[:, mi], [cur[:, mi * arity + j] for j in range(arity)])
        cur = res
    assert np.array_equal(layer.forward_packed(xu), cur[:, 0])


def test_conv_gate_tree_layer_depth5():
    """A gate16 tree deeper than the fused kernel's 4 levels."""
    rng = np.random.default_rng(11)
    n, L, nw, P, depth = 5, 6, 2, 18, 5
    leaf = rng.integers(0, P, (n, 2 ** depth))
    gates = [rng.integers(0, 16, (n, 2 ** (depth - 1 - i))) for i in range(depth)]
    xu = _words((P, L, nw), seed=12)
    layer = BitpackedConvTreeLayer(leaf, gates, kh=3, kw=3, stride=1, padding=1, cin=2)
    assert not layer.fused_ok()
    cur = xu[leaf.reshape(-1)].reshape(n, 2 ** depth, L, nw)
    for g in gates:
        a, b = cur[:, 0::2], cur[:, 1::2]
        res = np.empty_like(a)
        for oi in range(n):
            for mi in range(g.shape[1]):
                res[oi, mi] = packed_ref.GATE_OPS[g[oi, mi]](a[oi, mi], b[oi, mi])
        cur = res
    assert np.array_equal(layer.forward_packed(xu), cur[:, 0])
