"""Synthetic inputs and the five benchmark configurations.

There is no dataset access on the benchmark machines, so every input is drawn
from a seeded ``torch.Generator`` on the CPU:

* FC configs: ``torch.bernoulli(full((B, D), p), generator=g)`` as fp32 {0,1}.
* Config 3 images: ``rand((B,1,H,W))`` pixels, five thermometer planes at
  thresholds 1/6..5/6 (``pixel >= t``, the rule of the reference's
  ``binarize_spatial``, silogic/data.py:75-89) plus two edge planes
  ``pixel[:, x+1] - pixel[:, x] > 0`` (horizontal) and
  ``pixel[y+1, :] - pixel[y, :] > 0`` (vertical), zero in the last column/row.
* Config 5 images: ``rand((B,3,H,W))`` thermometer-encoded at 0.25/0.5/0.75,
  threshold-major channel order (``channel = t*3 + c``), as
  ``binarize_spatial(x, CIFAR3_THRESH)`` does (silogic/data.py:71,75-89).

``build_config(i)`` constructs BASELINE config ``i`` with the pinned choices:
``torch.manual_seed(0)`` right before construction and ``seed=0``; config 3
uses ``head_widths=[2560, 2560]`` and ``residual_init=False``; config 4 uses
width 16380 (16384 is not divisible by 10 classes, silogic/heads.py:126);
config 5 uses ``residual_init=False``.
"""
import torch

FIVE_THRESH = [1 / 6, 2 / 6, 3 / 6, 4 / 6, 5 / 6]
CIFAR3_THRESH = [0.25, 0.5, 0.75]


def bernoulli_inputs(B, D, p, gen):
    """``[B, D]`` fp32 {0,1} with P(1) = p, drawn from ``gen``."""
    return torch.bernoulli(torch.full((B, D), float(p)), generator=gen)


def thermometer(x, thresholds):
    """``[N,C,H,W]`` in [0,1] -> ``[N, C*len(t), H, W]`` fp32 planes ``x >= t``."""
    return torch.cat([(x >= t).float() for t in thresholds], dim=1)


def cfg3_images(B, hw, gen):
    """Config-3 input: 5 thermometer planes + 2 edge planes -> ``[B,7,hw,hw]``."""
    pix = torch.rand((B, 1, hw, hw), generator=gen)
    planes = thermometer(pix, FIVE_THRESH)
    eh = torch.zeros_like(pix)
    eh[..., :, :-1] = (pix[..., :, 1:] - pix[..., :, :-1] > 0).float()
    ev = torch.zeros_like(pix)
    ev[..., :-1, :] = (pix[..., 1:, :] - pix[..., :-1, :] > 0).float()
    return torch.cat([planes, eh, ev], dim=1)


def cfg5_images(B, hw, gen):
    """Config-5 input: 3 uniform channels x 3 thresholds -> ``[B,9,hw,hw]``."""
    x = torch.rand((B, 3, hw, hw), generator=gen)
    return thermometer(x, CIFAR3_THRESH)


CONFIGS = {
    1: ("LogicNet", dict(in_dim=784, width=2000, depth=4, num_classes=10,
                         node="gate16", connectome="topk", k=8, tau=10.0)),
    2: ("LogicNet", dict(in_dim=784, width=10000, depth=6, num_classes=10,
                         node="gate16", connectome="topk", k=8, tau=10.0)),
    3: ("LogicTreeNet", dict(in_channels=7, in_hw=28, channels=[64, 128, 256],
                             kernel=3, tree_depth=2, node="gate16", connect="topk",
                             k=4, n_chan=2, num_classes=10, head_widths=[2560, 2560],
                             residual_init=False)),
    4: ("WARPNet", dict(in_dim=4096, width=16380, depth=4, num_classes=10, k=8)),
    5: ("LogicConvNet", dict(in_channels=9, in_hw=32, channels=[128, 256],
                             head_widths=[1280], num_classes=10, node="multilinear",
                             arity=6, tree_depth=1, connect="topk", k=4, n_chan=2,
                             residual_init=False)),
}

# (soft batch, hard batch, input kind, Bernoulli p)
BATCHES = {
    1: (256, 256, "fc", 0.5),
    2: (4096, 65536, "fc", 0.2),
    3: (1024, 1024, "cfg3", None),
    4: (4096, 4096, "fc", 0.5),
    5: (512, 512, "cfg5", None),
}


def build_config(i, module=None):
    """Construct config ``i`` from ``module`` (default: :mod:`silogic_amd`)."""
    if module is None:
        import silogic_amd as module
    ctor, args = CONFIGS[i]
    torch.manual_seed(0)
    return getattr(module, ctor)(seed=0, **args)


def config_inputs(i, B=None, seed=1):
    """Inputs of config ``i`` (``B`` defaults to the hard batch)."""
    soft_b, hard_b, kind, p = BATCHES[i]
    B = hard_b if B is None else B
    g = torch.Generator().manual_seed(seed)
    ctor, args = CONFIGS[i]
    if kind == "fc":
        return bernoulli_inputs(B, args["in_dim"], p, g)
    if kind == "cfg3":
        return cfg3_images(B, args["in_hw"], g)
    return cfg5_images(B, args["in_hw"], g)
