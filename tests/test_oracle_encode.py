"""Pin the encoder oracle (oracle/encode_ref.py) on the CPU."""
import torch

from oracle import encode_ref


def test_binarize_known_answer_of_the_reference():
    """tests/test_data.py:12-19 of the reference: block per threshold,
    row-major flatten, >=."""
    x = torch.tensor([[[[0.1, 0.3], [0.5, 0.9]]]])
    bits = encode_ref.binarize(x, [0.2, 0.6])
    assert bits.dtype == torch.uint8
    assert torch.equal(bits, torch.tensor([[0, 1, 1, 1, 0, 0, 0, 1]], dtype=torch.uint8))
    assert torch.equal(encode_ref.binarize(torch.tensor([[0.5]]), [0.5]),
                       torch.tensor([[1]], dtype=torch.uint8))          # >= at the level


def test_binarize_spatial_channel_order_and_memory_order():
    """Channel t*C + c holds threshold t of colour c; the memory order is
    binarize's (data.py:75-89 vs 23-40)."""
    x = torch.rand(2, 3, 5, 4)
    thr = [0.2, 0.5, 0.8]
    sp = encode_ref.binarize_spatial(x, thr)
    assert sp.shape == (2, 9, 5, 4)
    for t, level in enumerate(thr):
        for c in range(3):
            assert torch.equal(sp[:, t * 3 + c], (x[:, c] >= level).to(torch.uint8))
    assert torch.equal(sp.reshape(2, -1), encode_ref.binarize(x, thr))


def test_edge_detectors_impulse_and_constant_image():
    """An impulse's responses are the detector kernels mirrored around it; a
    constant image has zero Laplacian inside and the zero-padding border
    responses at the edges; shapes as test_data.py:28-33."""
    x = torch.zeros(1, 1, 7, 7)
    x[0, 0, 3, 3] = 1.0
    r = encode_ref.edge_responses(x)[0]                                  # [3, 7, 7]
    for det, k in enumerate([encode_ref.SOBEL_X, encode_ref.SOBEL_Y, encode_ref.LAPLACE]):
        assert torch.equal(r[det, 2:5, 2:5], k.flip(0).flip(1))
        assert r[det].abs().sum() == k.abs().sum()
    bits = encode_ref.edge_bits(x, [0.5])                                 # [1, 6, 7, 7]
    assert bits.shape == (1, 6, 7, 7)
    assert bits[0, 5, 3, 3] == 1 and bits[0, 2, 3, 3] == 0               # Laplacian -4 < -0.5
    assert bits[0, 2, 2, 3] == 1                                         # Laplacian +1 above
    c = torch.full((1, 2, 6, 6), 0.5)
    rc = encode_ref.edge_responses(c)[0]
    assert torch.equal(rc[2, 1:-1, 1:-1], torch.zeros(4, 4))            # colour 0 Laplacian
    assert rc[2, 0, 0] == -1.0 and rc[2, 0, 2] == -0.5                   # corner, edge
    assert encode_ref.edge_bits(torch.rand(2, 3, 8, 8)).shape == (2, 3 * 3 * 2 * 2, 8, 8)


def test_learned_thermometer_values_gradient_and_hard():
    """encoders.py:36-49 (the reference's test_lut_nodes.py:67-75): values
    are the bits up to rounding, the gradient is that of
    sigmoid((x - t) * scale) (finite differences of the soft pass), hard is
    uint8 [B, F*bits] with feature-major order f*bits + i."""
    torch.manual_seed(0)
    x = torch.rand(8, 16, dtype=torch.float64, requires_grad=True)
    t = torch.rand(16, 4, dtype=torch.float64, requires_grad=True)
    e = encode_ref.learned_thermo(x, t, 10.0)
    assert e.shape == (8, 64)
    assert (e.detach() - e.detach().round()).abs().max() < 1e-12
    hard = encode_ref.learned_thermo_hard(x.detach(), t.detach())
    assert torch.equal(hard.double(), e.detach().round())
    assert hard[2, 5 * 4 + 3] == int(x[2, 5] > t[5, 3])
    g = torch.randn(8, 64, dtype=torch.float64)
    (e * g).sum().backward()
    eps = 1e-6
    soft = lambda xx, tt: torch.sigmoid((xx.unsqueeze(-1) - tt[None]) * 10.0).reshape(8, -1)
    for (i, j) in [(0, 0), (3, 7), (7, 15)]:
        xp, xm = x.detach().clone(), x.detach().clone()
        xp[i, j] += eps
        xm[i, j] -= eps
        fd = ((soft(xp, t.detach()) - soft(xm, t.detach())) * g).sum() / (2 * eps)
        assert abs(fd.item() - x.grad[i, j].item()) < 1e-6
    tp, tm = t.detach().clone(), t.detach().clone()
    tp[5, 2] += eps
    tm[5, 2] -= eps
    fd = ((soft(x.detach(), tp) - soft(x.detach(), tm)) * g).sum() / (2 * eps)
    assert abs(fd.item() - t.grad[5, 2].item()) < 1e-6
