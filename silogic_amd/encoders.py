"""Learnable thermometer encoder (silogic/encoders.py:12-49) on the GPU."""
import torch
import torch.nn as nn

from . import _lib, ops
from .data import _encode


class _LearnedThermoFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, thresholds, scale):
        ctx.save_for_backward(x, thresholds)
        ctx.scale = scale
        F, T = thresholds.shape
        return _encode(x, thresholds, True, 2, T).to(torch.float32)

    @staticmethod
    def backward(ctx, g):
        x, thr = ctx.saved_tensors
        B, F = x.shape
        T = thr.shape[1]
        need_x, need_t = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gx = torch.empty_like(x) if need_x else None
        gt = torch.empty_like(thr) if need_t else None
        ws = _lib.lib().slg_learned_thermo_bwd_workspace(B, F, T)
        work = torch.empty(max(ws, 1), device=x.device, dtype=torch.float32)
        _lib.call("slg_learned_thermo_bwd", ops._p(x), B, F, T, ops._p(thr), float(ctx.scale),
                  ops._p(ops._c(g, torch.float32)), ops._p(gx), ops._p(gt), ops._p(work), ws,
                  ops._stream(x))
        return gx, gt, None


class LearnedThermometerEncoder(nn.Module):
    """Thermometer encoder with learnable per-feature thresholds (arguments
    as silogic.encoders.LearnedThermometerEncoder): input ``[B, F]`` ->
    ``[B, F*bits]``, bit ``f*bits + i`` = ``x_f > t_{f,i}``. The soft forward
    returns the hard bits with the gradient of ``sigmoid((x - t) * scale)``
    (straight-through; the value is exact where the reference's
    ``hard + soft - soft.detach()`` carries fp32 rounding)."""

    def __init__(self, num_features, bits, init_lo=0.0, init_hi=1.0, scale=10.0):
        super().__init__()
        self.num_features = num_features
        self.bits = bits
        self.scale = scale
        t = torch.linspace(init_lo, init_hi, bits + 2)[1:-1]
        self.thresholds = nn.Parameter(t.repeat(num_features, 1))

    def forward(self, x):
        ops.require_gpu(x)
        return _LearnedThermoFn.apply(ops._as_f32(x), ops._c(self.thresholds, torch.float32),
                                      self.scale)

    @torch.no_grad()
    def forward_hard(self, x):
        ops.require_gpu(x)
        return _encode(ops._as_f32(x), ops._c(self.thresholds.detach(), torch.float32), True, 2,
                       self.bits)

    @torch.no_grad()
    def forward_packed(self, x, word_major=False):
        """The bits of :meth:`forward_hard` packed 64 samples per word:
        ``[F*bits, nw]`` (``word_major``: ``[nw, F*bits]``)."""
        ops.require_gpu(x)
        return _encode(ops._as_f32(x), ops._c(self.thresholds.detach(), torch.float32), True,
                       1 if word_major else 0, self.bits)
