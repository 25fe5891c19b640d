"""silogic_amd — the silogic gate-layer hot path, native to MI355X (gfx950).

A drop-in for the reference's Python API on the path it covers: the same
class names, constructor arguments, parameter initialisation (per seed) and
``state_dict`` keys as ``silogic``, with every forward computed by
hand-written HIP kernels in ``libsilogic_hip.so`` behind a C ABI
(``include/silogic_hip.h``):

>>> import torch, silogic_amd as sl
>>> torch.manual_seed(0)
>>> net = sl.LogicNet(784, 2000, 4, k=8, tau=10.0).cuda().eval()
>>> x = (torch.rand(256, 784) > 0.5).float().cuda()
>>> net(x).shape, net.forward_hard(x).shape
(torch.Size([256, 10]), torch.Size([256, 10]))

Compute is GPU-only; CPU tensors raise. Covered: nodes ``gate16``,
``walsh`` (any arity), ``multilinear`` and ``hybrid`` (arity 2-6) in FC
layers and conv trees (binary trees of depth 1-5, LUT trees of at most 36
leaves); wiring ``topk``, ``blocktopk``, ``fixed``; ``GroupSum`` heads;
``ConvLogicTree`` + ``OrPool``; the layer and network presets.
"""

__version__ = "0.1.0"

from .functional import (BASIS_COEFFS, TRUTH_TABLES, GATE_A, ste_threshold, sign_ste,
                         ternary_ste, binarize_ste, gate_probs, residual_logit, corner_bits,
                         walsh_monomials)
from .connectomes import build_connectome
from .nodes import build_node, NODES, RELAXATIONS
from .heads import GroupSum, build_decoder
from .layers import (LogicLayer, WARPLayer, WARPLayerN, LUTkLayer, LUTNodeLayer, ConvLogicTree,
                     ConvLogicLayer, OrPool)
from .models import LogicNet, WARPNet, WARPNetN, LUTkNet, LUTNodeNet, LogicConvNet, LogicTreeNet
from .encoders import LearnedThermometerEncoder
from .data import (binarize, binarize_spatial, binarize_packed, edge_bits, MNIST_THRESH,
                   SEVEN_THRESH, FOUR_THRESH, FIVE_THRESH, CIFAR3_THRESH, EDGE_THRESH)
from . import derived, kernels, library, ops

__all__ = [
    "BASIS_COEFFS", "TRUTH_TABLES", "GATE_A", "ste_threshold", "sign_ste", "ternary_ste",
    "binarize_ste", "gate_probs", "residual_logit", "corner_bits", "walsh_monomials",
    "build_connectome", "build_node", "NODES", "RELAXATIONS", "GroupSum", "build_decoder",
    "LogicLayer", "WARPLayer", "WARPLayerN", "LUTkLayer", "LUTNodeLayer", "ConvLogicTree",
    "ConvLogicLayer", "OrPool", "LogicNet", "WARPNet", "WARPNetN", "LUTkNet", "LUTNodeNet",
    "LogicConvNet", "LogicTreeNet", "kernels", "ops",
    "LearnedThermometerEncoder", "binarize", "binarize_spatial", "binarize_packed", "edge_bits",
    "MNIST_THRESH", "SEVEN_THRESH", "FOUR_THRESH", "FIVE_THRESH", "CIFAR3_THRESH", "EDGE_THRESH",
]
