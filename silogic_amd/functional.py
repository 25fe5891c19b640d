"""Gate algebra constants and parameter-side helpers (mirror of
silogic/functional.py's public names).

The 16-gate coefficient table, the truth tables derived from it and the
corner ordering are interface facts shared with the reference (checkpoints
and kernels index them), so they are identical; everything that computes on
activations lives in the HIP kernels.
"""
import math

import torch
import torch.nn.functional as F

# The 16 two-input Boolean functions in the basis {1, A, B, A*B}; row i gives
# [c0, c1, c2, c3] with gate_i(a, b) = c0 + c1 a + c2 b + c3 ab, in the
# standard DiffLogic order (silogic/functional.py:24-44).
BASIS_COEFFS = torch.tensor([
    [0, 0, 0, 0],    # 0  False
    [0, 0, 0, 1],    # 1  A and B
    [0, 1, 0, -1],   # 2  A and not B
    [0, 1, 0, 0],    # 3  A
    [0, 0, 1, -1],   # 4  not A and B
    [0, 0, 1, 0],    # 5  B
    [0, 1, 1, -2],   # 6  A xor B
    [0, 1, 1, -1],   # 7  A or B
    [1, -1, -1, 1],  # 8  nor
    [1, -1, -1, 2],  # 9  xnor
    [1, 0, -1, 0],   # 10 not B
    [1, 0, -1, 1],   # 11 A or not B
    [1, -1, 0, 0],   # 12 not A
    [1, -1, 0, 1],   # 13 not A or B
    [1, 0, 0, -1],   # 14 nand
    [1, 0, 0, 0],    # 15 True
], dtype=torch.float32)

GATE_A = 3  # pass-through of the first input


def _truth_from_basis(c):
    # column g is the gate output at address g = (a << 1) | b
    corners = [(0, 0), (0, 1), (1, 0), (1, 1)]
    cols = [c[:, 0] + c[:, 1] * a + c[:, 2] * b + c[:, 3] * (a * b) for a, b in corners]
    return torch.stack(cols, dim=1).round().to(torch.uint8)


TRUTH_TABLES = _truth_from_basis(BASIS_COEFFS)  # [16, 4]

# 4-bit truth-table code per gate: bit g = output at address g (the encoding
# the hard kernels use, see include/silogic_hip.h)
TT_CODES = [int(sum(int(TRUTH_TABLES[i, g]) << g for g in range(4))) for i in range(16)]


def ste_threshold(s):
    """Forward ``(s > 0)``, gradient of ``sigmoid(s)``."""
    hard = (s > 0).float()
    soft = torch.sigmoid(s)
    return hard + soft - soft.detach()


def sign_ste(w):
    """Forward ``{-1,+1}`` (``w >= 0`` -> +1), clipped identity gradient."""
    hard = torch.where(w >= 0, 1.0, -1.0)
    clip = torch.clamp(w, -1, 1)
    return clip + (hard - clip).detach()


def ternary_ste(w, delta=0.5):
    """Forward ``{-1,0,+1}`` with dead zone ``delta``, clipped identity gradient."""
    hard = torch.where(w > delta, 1.0, torch.where(w < -delta, -1.0, 0.0))
    clip = torch.clamp(w, -1, 1)
    return clip + (hard - clip).detach()


def binarize_ste(x, thresh=0.5):
    """Forward ``(x > thresh)``, identity gradient."""
    return (x > thresh).float() + (x - x.detach())


def residual_logit(p, tau=1.0):
    """Logit ``z`` with ``sigmoid(z / tau) == p`` (p clamped to [1e-4, 1-1e-4])."""
    p = min(max(float(p), 1e-4), 1 - 1e-4)
    return tau * math.log(p / (1 - p))


def gate_probs(logits, training, dim=-1, gate_select="softmax", gumbel_tau=1.0):
    """Gate selection weights: softmax, or in training Gumbel-ST / hard-ST."""
    if training and gate_select == "gumbel":
        return F.gumbel_softmax(logits, tau=gumbel_tau, hard=True, dim=dim)
    soft = F.softmax(logits, dim=dim)
    if training and gate_select == "hard":
        idx = soft.argmax(dim=dim, keepdim=True)
        hard = torch.zeros_like(soft).scatter_(dim, idx, 1.0)
        return soft + (hard - soft).detach()
    return soft


def corner_bits(n, dtype=torch.float32):
    """``[2^n, n]`` corner patterns; row p holds bit j of p in column j."""
    return torch.tensor([[(p >> j) & 1 for j in range(n)] for p in range(2 ** n)], dtype=dtype)


def walsh_monomials(u):
    """``[B, out, n] -> [B, out, 2^n]``; column i = prod of u_j over bits j of i."""
    phi = torch.ones(u.shape[0], u.shape[1], 1, device=u.device, dtype=u.dtype)
    for j in range(u.shape[2]):
        phi = torch.cat([phi, phi * u[:, :, j:j + 1]], dim=2)
    return phi
