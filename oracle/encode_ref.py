"""CPU restatement of the reference's input encoders (test infrastructure:
imported only by tests/, never by the product).

* binarize          -- silogic/data.py:23-40
* binarize_spatial  -- silogic/data.py:75-89
* edge_bits         -- silogic/data.py:95-131 (same kernels, F.conv2d)
* learned_thermo    -- silogic/encoders.py:36-49 (soft STE and hard)

Pinned in tests/test_oracle_encode.py by the reference's own known-answer
test (tests/test_data.py:12-19), shape checks (test_data.py:22-33,
test_lut_nodes.py:67-75), impulse / constant-image closed forms of the edge
detectors, and a finite-difference check of the learned encoder's gradient.
"""
import torch
import torch.nn.functional as F

SOBEL_X = torch.tensor([[-1., 0, 1], [-2, 0, 2], [-1, 0, 1]])        # data.py:95
SOBEL_Y = SOBEL_X.t().contiguous()
LAPLACE = torch.tensor([[0., 1, 0], [1, -4, 1], [0, 1, 0]])


def binarize(x, thresholds):
    flat = x.reshape(x.shape[0], -1)
    return torch.cat([(flat >= t).to(torch.uint8) for t in thresholds], dim=1)


def binarize_spatial(x, thresholds):
    return torch.cat([(x >= t).to(torch.uint8) for t in thresholds], dim=1)


def edge_responses(x):
    C = x.shape[1]
    ker = torch.stack([SOBEL_X, SOBEL_Y, LAPLACE]).to(x.dtype)
    w = ker.unsqueeze(1).repeat(C, 1, 1, 1)                          # [C*3, 1, 3, 3]
    return F.conv2d(x, w, padding=1, groups=C)                       # [N, C*3, H, W]


def edge_bits(x, edge_thr=(0.12, 0.25)):
    resp = edge_responses(x)
    bits = []
    for t in edge_thr:
        bits.append((resp > t).to(torch.uint8))
        bits.append((resp < -t).to(torch.uint8))
    return torch.cat(bits, dim=1)


def learned_thermo(x, thresholds, scale):
    """Soft pass: hard bits carrying the sigmoid gradient (encoders.py:40-44)."""
    d = x.unsqueeze(-1) - thresholds[None]
    hard = (d > 0).float()
    soft = torch.sigmoid(d * scale)
    return (hard + soft - soft.detach()).reshape(x.shape[0], -1)


def learned_thermo_hard(x, thresholds):
    d = x.unsqueeze(-1) - thresholds[None]
    return (d > 0).to(torch.uint8).reshape(x.shape[0], -1)
