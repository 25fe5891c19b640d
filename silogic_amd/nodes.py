"""Node parameterizations (mirror of silogic/nodes.py): they hold the
parameters and provide the per-node quantities the HIP kernels consume.

* ``gate16`` — softmax mixture over the 16 gates; kernel parameter is the
  BasisProj coefficient vector ``softmax(gate_logits) @ BASIS`` [out, 4].
* ``walsh`` — Walsh coefficients ``theta``; arity 2 uses the change of
  variables to ``(a, b)`` coefficients and ``sigmoid(z / tau)``.
* ``multilinear`` — one logit per truth-table entry; kernel parameter is
  ``sigmoid(logits)``; hard truth table ``logits > 0``.

Parameter shapes, names, initial draws (global RNG, silogic/nodes.py:74, 123,
172) and ``residual_init`` follow the reference so checkpoints load. The
DWN/perceptron/polynomial relaxations (``hybrid``, ``linear``,
``polynomial``) are not part of the gate-layer hot path and are rejected.
"""
import torch
import torch.nn as nn

from . import ops
from .functional import (BASIS_COEFFS, TRUTH_TABLES, GATE_A, gate_probs, residual_logit,
                         corner_bits, walsh_monomials)

NODES = ("gate16", "walsh", "multilinear", "hybrid", "linear", "polynomial")
RELAXATIONS = ("probabilistic", "hybrid", "linear", "polynomial")
SUPPORTED = ("gate16", "walsh", "multilinear", "hybrid")
_NODE_ALIASES = {
    "gate16": "gate16", "gate": "gate16",
    "walsh": "walsh",
    "multilinear": "multilinear", "probabilistic": "multilinear",
    "hybrid": "hybrid", "linear": "linear", "polynomial": "polynomial",
}


class Node(nn.Module):
    """Base class; ``kind`` is the kernel node id, ``raw()`` the parameter the
    HIP prep kernels read."""

    kind = None

    def __init__(self, out_dim, arity):
        super().__init__()
        self.out_dim = out_dim
        self.arity = arity

    def forward(self, operands):
        raise NotImplementedError(
            "silogic_amd evaluates nodes inside the fused layer kernels; call the layer")

    def residual_init(self, p):
        raise NotImplementedError


class Gate16Node(Node):
    """Softmax mixture over the 16 two-input functions (arity 2)."""

    kind = ops.GATE16

    def __init__(self, out_dim, arity=2, gate_eval="basis", gate_select="softmax",
                 gumbel_tau=1.0):
        super().__init__(out_dim, 2)
        assert arity == 2, "gate16 nodes are two-input"
        self.gate_eval = gate_eval
        self.gate_select = gate_select
        self.gumbel_tau = gumbel_tau
        self.gate_logits = nn.Parameter(torch.randn(out_dim, 16) * 0.1)
        self.register_buffer("basis", BASIS_COEFFS.clone())
        self.register_buffer("truth", TRUTH_TABLES.clone())

    def _probs(self):
        return gate_probs(self.gate_logits, self.training, dim=1,
                          gate_select=self.gate_select, gumbel_tau=self.gumbel_tau)

    def coef(self):
        """BasisProj coefficients ``[out, 4]`` (differentiable torch)."""
        return self._probs() @ self.basis

    kernel_param = coef

    def plain_softmax(self):
        """True when the kernel prep (plain softmax) equals ``_probs``."""
        return not (self.training and self.gate_select in ("gumbel", "hard"))

    def raw(self):
        return self.gate_logits

    @torch.no_grad()
    def residual_init(self, p):
        self.gate_logits.normal_(0, 0.1)
        self.gate_logits[:, GATE_A] = residual_logit(p)


def gumbel_noise(shape, device):
    """Standard Gumbel samples ``-log(-log u)``, ``u`` uniform from torch's
    generator clamped to ``[1e-6, 1 - 1e-6]`` (nodes.py:46-48): the same
    draws as the reference for the same generator state."""
    u = torch.rand(shape, device=device).clamp_(1e-6, 1 - 1e-6)
    return -torch.log(-torch.log(u))


class WalshNode(Node):
    """Walsh-Hadamard node ``z = sum_i theta_i phi_i(2a-1)``, ``sigmoid(z/tau)``."""

    kind = ops.WALSH

    def __init__(self, out_dim, arity=2, tau=1.0, gate_select="softmax"):
        super().__init__(out_dim, arity)
        self.tau = tau
        self.gate_select = gate_select
        self.theta = nn.Parameter(torch.randn(out_dim, 2 ** arity) * 0.1)

    @property
    def inv_tau(self):
        return 1.0 / self.tau

    def _z(self, *operands_ab):
        u = [2 * v - 1 for v in operands_ab]
        if self.arity == 2:
            t = self.theta
            return t[:, 0] + t[:, 1] * u[0] + t[:, 2] * u[1] + t[:, 3] * (u[0] * u[1])
        um = torch.stack(u, dim=2)
        return (walsh_monomials(um) * self.theta[None]).sum(2)

    def coef(self):
        """``(a, b)``-space coefficients of z (arity 2)."""
        t = self.theta
        return torch.stack([t[:, 0] - t[:, 1] - t[:, 2] + t[:, 3],
                            2 * (t[:, 1] - t[:, 3]), 2 * (t[:, 2] - t[:, 3]),
                            4 * t[:, 3]], dim=1)

    kernel_param = coef

    def _corner_monomials(self, device):
        """``[2^n, 2^n]`` monomial values at the corners: row p is
        walsh_monomials(2c - 1) for corner c = bits of p (entry q = product
        of u_j over the bits j of q, functional.py:176-185)."""
        u = 2 * corner_bits(self.arity).to(device) - 1                 # [P, n]
        return walsh_monomials(u.unsqueeze(0))[0]                       # [P, P]

    def corner_z(self):
        """z at the ``2^n`` corners ``[out, 2^n]`` (differentiable): z is
        multilinear in the operands, so the interpolation of these values is
        z itself."""
        return self.theta @ self._corner_monomials(self.theta.device).t()

    @torch.no_grad()
    def corner_z_hard(self):
        """z at the corners with the fp32 expression of forward_hard
        (``(walsh_monomials(u) * theta).sum(2)``, nodes.py:152-156), evaluated
        on the CPU as the reference computes it, on the parameter's device."""
        t = self.theta.detach().float().cpu()
        P = 2 ** self.arity
        cols = []
        for p in range(P):
            u = (2 * corner_bits(self.arity)[p] - 1).view(1, 1, -1).expand(1, t.shape[0], -1)
            cols.append((walsh_monomials(u) * t[None]).sum(2)[0])
        return torch.stack(cols, dim=1).to(self.theta.device)

    def plain_softmax(self):
        return not (self.training and self.gate_select == "gumbel")

    def gumbel_sigmoid(self, z):
        """Training output with Gumbel-sigmoid smoothing (nodes.py:147-149):
        ``sigmoid((z + g1 - g2) / tau)`` with two fresh Gumbel draws per
        element, in the reference's order."""
        g1 = gumbel_noise(z.shape, z.device)
        g2 = gumbel_noise(z.shape, z.device)
        return torch.sigmoid((z + g1 - g2) * self.inv_tau)

    def raw(self):
        return self.theta

    @torch.no_grad()
    def residual_init(self, p):
        self.theta.zero_()
        self.theta[:, 2 ** (self.arity - 1)] = residual_logit(p, self.tau)


class MultilinearNode(Node):
    """One logit per truth-table entry, multilinear interpolation (arity n)."""

    kind = ops.MULTILINEAR2

    def __init__(self, out_dim, arity=2):
        super().__init__(out_dim, arity)
        self.register_buffer("corners", corner_bits(arity))
        self.logits = nn.Parameter(torch.randn(out_dim, 2 ** arity) * 0.1)

    def kernel_param(self):
        return torch.sigmoid(self.logits)

    def plain_softmax(self):
        return True

    def raw(self):
        return self.logits

    @torch.no_grad()
    def residual_init(self, p):
        c = residual_logit(p)
        bit0 = self.corners[:, 0]
        self.logits.copy_((2 * bit0 - 1) * c + 0.1 * torch.randn_like(self.logits))


class HybridNode(MultilinearNode):
    """DWN-style: the forward reads the LUT at the address of the operands
    thresholded at 0.5; the gradient is the multilinear node's (straight
    through), silogic/nodes.py:198-206. Same parameters as the multilinear
    node (``logits`` [out, 2^arity])."""

    hybrid = True


MultilinearNode.hybrid = False

_BUILDERS = {"gate16": Gate16Node, "walsh": WalshNode, "multilinear": MultilinearNode,
             "hybrid": HybridNode}


def build_node(name, out_dim, arity=2, **kw):
    """Construct a node parameterization by name."""
    key = _NODE_ALIASES.get(str(name).lower())
    if key is None:
        raise ValueError(f"unknown node {name!r}; choose from {NODES}")
    if key not in SUPPORTED:
        raise NotImplementedError(
            f"node {name!r} is not on the MI355X gate-layer path (supported: {SUPPORTED})")
    if key == "gate16":
        return Gate16Node(out_dim, arity, gate_eval=kw.get("gate_eval", "basis"),
                          gate_select=kw.get("gate_select", "softmax"),
                          gumbel_tau=kw.get("gumbel_tau", 1.0))
    if key == "walsh":
        return WalshNode(out_dim, arity, tau=kw.get("tau", 1.0),
                         gate_select=kw.get("gate_select", "softmax"))
    if key == "hybrid":
        return HybridNode(out_dim, arity)
    return MultilinearNode(out_dim, arity)
