"""GPU input encoders (silogic/data.py:23-131, encoders.py:12-49) against
the CPU oracle, and packed encoder output fed straight into the hard
networks."""
import numpy as np
import pytest
import torch

import silogic_amd as sl
from conftest import build_product
from oracle import encode_ref, packed_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("shape,thr", [((5, 1, 28, 28), sl.MNIST_THRESH),
                                       ((70, 3, 32, 32), sl.CIFAR3_THRESH),
                                       ((129, 784), sl.SEVEN_THRESH),
                                       ((3, 2, 5, 7), sl.FIVE_THRESH)])
def test_thermometer_layouts(shape, thr):
    g = torch.Generator().manual_seed(3)
    x = torch.rand(shape, generator=g)
    x.view(-1)[:4] = torch.tensor(thr[:1] * 4)                      # values at a level
    ref = encode_ref.binarize(x, thr)
    assert torch.equal(sl.binarize(x.to(DEV), thr).cpu(), ref)
    if len(shape) == 4:
        assert torch.equal(sl.binarize_spatial(x.to(DEV), thr).cpu(),
                           encode_ref.binarize_spatial(x, thr))
    want = packed_ref.pack_bits(ref.numpy())                         # [T*D, nw]
    rows = sl.binarize_packed(x.to(DEV), thr).cpu().numpy()
    words = sl.binarize_packed(x.to(DEV), thr, word_major=True).cpu().numpy()
    np.testing.assert_array_equal(rows, want)
    np.testing.assert_array_equal(words, want.T)


@pytest.mark.parametrize("shape,thr", [((4, 3, 32, 32), None), ((2, 1, 9, 13), [0.05, 0.3, 1.0])])
def test_edge_bits(shape, thr):
    g = torch.Generator().manual_seed(4)
    x = torch.rand(shape, generator=g)
    got = sl.edge_bits(x.to(DEV), thr).cpu()
    levels = sl.EDGE_THRESH if thr is None else thr
    ref = encode_ref.edge_bits(x, levels)
    assert got.shape == ref.shape and got.dtype == torch.uint8
    resp = encode_ref.edge_responses(x)                              # [N, 3C, H, W]
    near = torch.cat([torch.cat([((resp - t).abs() <= 1e-6), ((resp + t).abs() <= 1e-6)], 1)
                      for t in levels], 1)
    assert not ((got != ref) & ~near).any()


def test_learned_thermometer_encoder():
    torch.manual_seed(0)
    enc = sl.LearnedThermometerEncoder(40, bits=5, scale=8.0)
    enc.thresholds.data += 0.05 * torch.randn(40, 5)
    x = torch.rand(300, 40)
    t = enc.thresholds.detach().clone().requires_grad_(True)
    xr = x.clone().requires_grad_(True)
    ref = encode_ref.learned_thermo(xr, t, 8.0)
    g = torch.randn(300, 200)
    (ref * g).sum().backward()
    enc = enc.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    out = enc(xg)
    (out * g.to(DEV)).sum().backward()
    assert torch.equal(out.detach().cpu(), ref.detach().round())     # the bits exactly
    for got, want in ((xg.grad, xr.grad), (enc.thresholds.grad, t.grad)):
        err = (got.cpu() - want).abs().max().item()
        assert err <= 1e-5 * want.abs().max().item() + 1e-6, err
    hard = enc.forward_hard(x.to(DEV)).cpu()
    assert torch.equal(hard, encode_ref.learned_thermo_hard(x, t.detach()))
    np.testing.assert_array_equal(enc.forward_packed(x.to(DEV)).cpu().numpy(),
                                  packed_ref.pack_bits(hard.numpy()))


def test_packed_encoding_feeds_the_hard_networks():
    """Pixels -> packed bits in one kernel -> the hard circuit: same class
    counts as the uint8 path (FC word-major, fused; conv rows)."""
    g = torch.Generator().manual_seed(5)
    net = build_product(("LogicNet", dict(in_dim=784, width=500, depth=3, k=8, tau=10.0)))
    net = net.to(DEV).eval()
    img = torch.rand(200, 1, 28, 28, generator=g).to(DEV)
    want = net.forward_hard(sl.binarize(img, sl.MNIST_THRESH))
    words = sl.binarize_packed(img, sl.MNIST_THRESH, word_major=True)
    assert torch.equal(net.forward_hard_packed(words, 200, word_major=True), want)
    rows = sl.binarize_packed(img, sl.MNIST_THRESH)
    assert torch.equal(net.forward_hard_packed(rows, 200), want)
    conv = build_product(("LogicConvNet", dict(in_channels=9, in_hw=16, channels=[16, 32],
                                               head_widths=[320], node="multilinear", arity=6,
                                               tree_depth=1, residual_init=False,
                                               tau=10.0))).to(DEV).eval()
    pix = torch.rand(70, 3, 16, 16, generator=g).to(DEV)
    want_c = conv.forward_hard(sl.binarize_spatial(pix, sl.CIFAR3_THRESH))
    got_c = conv.forward_hard_packed(sl.binarize_packed(pix, sl.CIFAR3_THRESH), 70, (9, 16, 16))
    assert torch.equal(got_c, want_c)


def test_pixel_bytes_encode_as_the_reference_loaders_scale_them():
    """uint8 pixel input is taken as x / 255 in fp32 (data.py:49-57) and
    packed directly: same words as encoding the scaled floats."""
    g = torch.Generator().manual_seed(6)
    pix = torch.randint(0, 256, (130, 784), generator=g, dtype=torch.uint8)
    pix[0, :256] = torch.arange(256, dtype=torch.uint8)            # every byte value
    thr = sl.SEVEN_THRESH
    ref = encode_ref.binarize(pix.float() / 255.0, thr)
    want = packed_ref.pack_bits(ref.numpy())
    np.testing.assert_array_equal(sl.binarize_packed(pix.to(DEV), thr).cpu().numpy(), want)
    np.testing.assert_array_equal(
        sl.binarize_packed(pix.to(DEV), thr, word_major=True).cpu().numpy(), want.T)


def test_pixel_bytes_at_threshold_edges_and_unaligned_input():
    """Thresholds at a byte's exact value (51 / 255 == 0.2 in fp32), at 0
    and 1 and above 1; input whose address is not 4-byte aligned takes the
    one-feature-per-lane path and gives the same words."""
    g = torch.Generator().manual_seed(8)
    pix = torch.randint(0, 256, (67, 784), generator=g, dtype=torch.uint8)
    pix[0, :256] = torch.arange(256, dtype=torch.uint8)
    thr = [0.0, 51 / 255, 1.0, 1.5]
    want = packed_ref.pack_bits(encode_ref.binarize(pix.float() / 255.0, thr).numpy())
    buf = torch.empty(pix.numel() + 1, dtype=torch.uint8, device=DEV)
    buf[1:] = pix.reshape(-1).to(DEV)
    shifted = buf[1:].view(67, 784)
    assert shifted.data_ptr() % 4 != 0
    for x in (pix.to(DEV), shifted):
        np.testing.assert_array_equal(sl.binarize_packed(x, thr).cpu().numpy(), want)
        np.testing.assert_array_equal(sl.binarize_packed(x, thr, word_major=True).cpu().numpy(),
                                      want.T)
    # the equality case: byte 51 passes 51 / 255, byte 50 does not
    bits = encode_ref.binarize(pix[:1].float() / 255.0, thr)[0]
    assert bits[784 + 51] == 1 and bits[784 + 50] == 0 and bits[2 * 784 + 255] == 1
    assert bits[3 * 784:].sum() == 0 and bits[:784].sum() == 784
