"""Classification head (mirror of silogic/heads.py): ``GroupSum``.

``forward`` = per-class block sum of the features (of ``x > 0.5`` when
``feature_ste``) divided by ``tau`` (silogic/heads.py:34-39); ``forward_hard``
= raw integer block counts as float, no ``tau`` (heads.py:41-45). Both run on
the HIP kernels. The learned decoders are not part of the gate-layer hot path.
"""
import torch
import torch.nn as nn

from . import ops


class GroupSum(nn.Module):
    """Aggregate logic outputs into class logits by group counting."""

    def __init__(self, num_classes=10, tau=1.0, feature_ste=False):
        super().__init__()
        self.num_classes = num_classes
        self.tau = tau
        self.feature_ste = feature_ste

    def forward(self, x):
        return ops.groupsum_soft(x, self.num_classes, self.tau, self.feature_ste)

    @torch.no_grad()
    def forward_hard(self, x):
        return ops.groupsum_hard(x, self.num_classes)


def build_decoder(kind, width, num_classes=10, tau=1.0, feature_ste=True):
    """``"groupsum"`` only; learned decoders are outside this build's scope."""
    if kind == "groupsum":
        assert width % num_classes == 0, "width must be divisible by classes"
        return GroupSum(num_classes=num_classes, tau=tau, feature_ste=feature_ste)
    raise NotImplementedError(
        f"decoder {kind!r} is not on the MI355X gate-layer path (use 'groupsum')")
