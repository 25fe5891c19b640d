"""The HIP entry points as PyTorch custom operators (namespace ``silogic_hip``).

Each op is registered with ``torch.library.custom_op``, a fake (meta)
implementation that gives output shapes and dtypes without running a
kernel, and, for the differentiable ops, ``register_autograd`` with a
backward that is itself a custom op (the HIP backward kernels; for shapes
they do not take, the autograd backward differentiates the op's torch
expression instead). So
``torch.compile`` / FX tracing see opaque operators instead of a graph
break at the ctypes call. The drop-ins of ``silogic_amd.kernels`` (the
reference's ``silogic.kernels``, kernels/__init__.py:21-55) call these ops.

Gradients an op does not need come back from the backward ops as empty
``[0]`` tensors (a custom op returns tensors, not None) and are turned into
None before autograd sees them.
"""
from typing import List, Tuple

import torch
from torch import Tensor

from . import ops

_NS = "silogic_hip"


def _none(t, need):
    return t if need else None


def _empty(ref):
    return ref.new_empty((0,))


def _composite(fn, tensors, needs, gy):
    """Gradients of ``fn(*tensors)`` by autograd on its torch expression: the
    backward of shapes the HIP kernels do not take. Runs in the autograd
    backward itself (an op's implementation cannot record a graph)."""
    with torch.enable_grad():
        leaves = [t.detach().float().requires_grad_(n) for t, n in zip(tensors, needs)]
        y = fn(*leaves)
        inputs = [t for t, n in zip(leaves, needs) if n]
        grads = list(torch.autograd.grad(y, inputs, gy)) if inputs else []
    return tuple(grads.pop(0) if n else None for n in needs)


# ---------------------------------------------------------------------------
# FC soft layer (dense_logic / warp_logic)
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::fc_soft", mutates_args=())
def fc_soft(x: Tensor, cand: Tensor, w: Tensor, npar: Tensor, node_kind: int,
            inv_tau: float) -> Tensor:
    """``x [B,IN]``, ``cand/w [OUT,2,K]``, ``npar [OUT,4]`` -> ``[B,OUT]``."""
    ops.require_gpu(x, cand, w, npar)
    return ops._fc_soft_launch(ops._as_f32(x), ops._c(cand, torch.int32),
                               ops._c(w, torch.float32), ops._c(npar, torch.float32),
                               node_kind, inv_tau)


@fc_soft.register_fake
def _(x, cand, w, npar, node_kind, inv_tau):
    return x.new_empty((x.shape[0], cand.shape[0]), dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::fc_soft_bwd", mutates_args=())
def fc_soft_bwd(x: Tensor, cand: Tensor, w: Tensor, npar: Tensor, node_kind: int, inv_tau: float,
                gy: Tensor, need_x: bool, need_w: bool,
                need_np: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """``(gx, gw, gnp)`` of fc_soft; unneeded ones are empty."""
    got = ops.fc_soft_bwd(x, cand, w, npar, node_kind, inv_tau, gy, need_x, need_w, need_np)
    if got is None:
        raise NotImplementedError("fc_soft backward: shape outside the HIP kernels "
                                  "(K > 16 or 2*OUT*K >= 2^31)")
    gx, gw, gn = got
    return (gx if gx is not None else _empty(x), gw if gw is not None else _empty(x),
            gn if gn is not None else _empty(x))


@fc_soft_bwd.register_fake
def _(x, cand, w, npar, node_kind, inv_tau, gy, need_x, need_w, need_np):
    f32 = torch.float32
    return (x.new_empty(x.shape, dtype=f32) if need_x else x.new_empty((0,), dtype=f32),
            x.new_empty(w.shape, dtype=f32) if need_w else x.new_empty((0,), dtype=f32),
            x.new_empty(npar.shape, dtype=f32) if need_np else x.new_empty((0,), dtype=f32))


def _fc_soft_setup(ctx, inputs, output):
    x, cand, w, npar, node_kind, inv_tau = inputs
    ctx.save_for_backward(x, cand, w, npar)
    ctx.meta = (node_kind, inv_tau)


def _fc_soft_backward(ctx, gy):
    x, cand, w, npar = ctx.saved_tensors
    need = ctx.needs_input_grad
    if not ops.fc_soft_bwd_supported(x, cand):
        gx, gw, gn = _composite(lambda a, b, c: ops.fc_soft_torch(a, cand, b, c, *ctx.meta),
                                (x, w, npar), (need[0], need[2], need[3]), gy)
        return gx, None, gw, gn, None, None
    gx, gw, gn = fc_soft_bwd(x, cand, w, npar, *ctx.meta, gy, need[0], need[2], need[3])
    return _none(gx, need[0]), None, _none(gw, need[2]), _none(gn, need[3]), None, None


fc_soft.register_autograd(_fc_soft_backward, setup_context=_fc_soft_setup)


# The reference's own signatures (kernels/dense.py:123-125, warp.py:104-105):
# separate candidate and weight arrays per operand, through the C ABI's
# slg_dense_logic_fwd / slg_warp_logic_fwd. The backward stacks them into the
# [OUT,2,K] layout of fc_soft_bwd.
@torch.library.custom_op(f"{_NS}::dense_logic", mutates_args=())
def dense_logic(x: Tensor, ca: Tensor, cb: Tensor, wa: Tensor, wb: Tensor, coef: Tensor,
                node_kind: int, inv_tau: float) -> Tensor:
    """``x [B,IN]``, ``ca/cb [OUT,K]`` int32, ``wa/wb [OUT,K]``, ``coef [OUT,4]``
    -> ``[B,OUT]`` (gate16: the BasisProj node; walsh: its sigmoid)."""
    return ops.dense_logic_launch(x, ca, cb, wa, wb, coef, node_kind, inv_tau)


@dense_logic.register_fake
def _(x, ca, cb, wa, wb, coef, node_kind, inv_tau):
    return x.new_empty((x.shape[0], ca.shape[0]), dtype=torch.float32)


def _dense_setup(ctx, inputs, output):
    x, ca, cb, wa, wb, coef, node_kind, inv_tau = inputs
    ctx.save_for_backward(x, ca, cb, wa, wb, coef)
    ctx.meta = (node_kind, inv_tau)


def _dense_backward(ctx, gy):
    x, ca, cb, wa, wb, coef = ctx.saved_tensors
    need = ctx.needs_input_grad
    need_w = need[3] or need[4]
    cand = torch.stack([ca, cb], dim=1).to(torch.int32)
    w = torch.stack([wa, wb], dim=1)
    if not ops.fc_soft_bwd_supported(x, cand):
        gx, gw, gn = _composite(lambda a, b, c: ops.fc_soft_torch(a, cand, b, c, *ctx.meta),
                                (x, w, coef), (need[0], need_w, need[5]), gy)
    else:
        gx, gw, gn = fc_soft_bwd(x, cand, w, coef, *ctx.meta, gy, need[0], need_w, need[5])
    gwa = gw[:, 0] if need[3] else None
    gwb = gw[:, 1] if need[4] else None
    return _none(gx, need[0]), None, None, gwa, gwb, _none(gn, need[5]), None, None


dense_logic.register_autograd(_dense_backward, setup_context=_dense_setup)


# GroupSum.forward (heads.py:34-39): block sums of x (or of x > 0.5 with the
# feature STE) / tau; both forms have d logit / d x = 1/tau on the block.
@torch.library.custom_op(f"{_NS}::groupsum_soft", mutates_args=())
def groupsum_soft(x: Tensor, C: int, tau: float, ste: bool) -> Tensor:
    return ops.groupsum_soft_launch(x, C, tau, ste)


@groupsum_soft.register_fake
def _(x, C, tau, ste):
    return x.new_empty((x.shape[0], C), dtype=torch.float32)


def _groupsum_setup(ctx, inputs, output):
    x, C, tau, ste = inputs
    ctx.meta = (x.shape[1], C, tau)


def _groupsum_backward(ctx, g):
    W, C, tau = ctx.meta
    gx = (g / tau).unsqueeze(2).expand(g.shape[0], C, W // C).reshape(g.shape[0], W)
    return gx, None, None, None


groupsum_soft.register_autograd(_groupsum_backward, setup_context=_groupsum_setup)


# OrPool.forward (layers.py:558-559): 2x2 max pool; the gradient of
# F.max_pool2d (to the first maximum of each window).
@torch.library.custom_op(f"{_NS}::orpool", mutates_args=())
def orpool(x: Tensor, size: int) -> Tensor:
    return ops.orpool_launch(x, size)


@orpool.register_fake
def _(x, size):
    B, C, H, W = x.shape
    return x.new_empty((B, C, H // size, W // size))


def _orpool_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.size = inputs[1]


def _orpool_backward(ctx, g):
    (x,) = ctx.saved_tensors
    s = ctx.size
    xf = x.float()
    _, idx = torch.ops.aten.max_pool2d_with_indices(xf, [s, s], [s, s])
    gx = torch.ops.aten.max_pool2d_with_indices_backward(g, xf, [s, s], [s, s], [0, 0], [1, 1],
                                                         False, idx)
    return gx, None


orpool.register_autograd(_orpool_backward, setup_context=_orpool_setup)


# ---------------------------------------------------------------------------
# LUT FC layer (multilinear_logic)
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::fc_lut_soft", mutates_args=())
def fc_lut_soft(x: Tensor, cand: Tensor, w: Tensor, s: Tensor, hybrid: bool) -> Tensor:
    """``x [B,IN]``, ``cand/w [OUT,n,K]``, ``s [OUT,2^n]`` -> ``[B,OUT]``."""
    ops.require_gpu(x, cand, w, s)
    return ops._fc_lut_launch(ops._as_f32(x), ops._c(cand, torch.int32), ops._c(w, torch.float32),
                              ops._c(s, torch.float32), hybrid)


@fc_lut_soft.register_fake
def _(x, cand, w, s, hybrid):
    return x.new_empty((x.shape[0], cand.shape[0]), dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::fc_lut_soft_bwd", mutates_args=())
def fc_lut_soft_bwd(x: Tensor, cand: Tensor, w: Tensor, s: Tensor, gy: Tensor, need_x: bool,
                    need_w: bool, need_s: bool) -> Tuple[Tensor, Tensor, Tensor]:
    got = ops.fc_lut_soft_bwd(x, cand, w, s, gy, need_x, need_w, need_s)
    if got is None:
        raise NotImplementedError("fc_lut_soft backward: the input width exceeds what the "
                                  "kernels stage in LDS")
    gx, gw, gs = got
    return (gx if gx is not None else _empty(x), gw if gw is not None else _empty(x),
            gs if gs is not None else _empty(x))


@fc_lut_soft_bwd.register_fake
def _(x, cand, w, s, gy, need_x, need_w, need_s):
    f32 = torch.float32
    return (x.new_empty(x.shape, dtype=f32) if need_x else x.new_empty((0,), dtype=f32),
            x.new_empty(w.shape, dtype=f32) if need_w else x.new_empty((0,), dtype=f32),
            x.new_empty(s.shape, dtype=f32) if need_s else x.new_empty((0,), dtype=f32))


def _fc_lut_setup(ctx, inputs, output):
    x, cand, w, s, hybrid = inputs
    ctx.save_for_backward(x, cand, w, s)


def _fc_lut_backward(ctx, gy):
    x, cand, w, s = ctx.saved_tensors
    need = ctx.needs_input_grad
    gx, gw, gs = fc_lut_soft_bwd(x, cand, w, s, gy, need[0], need[2], need[3])
    return _none(gx, need[0]), None, _none(gw, need[2]), _none(gs, need[3]), None


fc_lut_soft.register_autograd(_fc_lut_backward, setup_context=_fc_lut_setup)


# ---------------------------------------------------------------------------
# Conv tree layer with the fused 2x2 OrPool (tree_conv, tree_conv_topk,
# conv_hybrid)
# ---------------------------------------------------------------------------
def _conv_out_shape(x, cm, pad, pool):
    B, _, H, W = x.shape
    kern = 2 * pad + 1
    Hf, Wf = H + 2 * pad - kern + 1, W + 2 * pad - kern + 1
    Ho, Wo = (Hf // 2, Wf // 2) if pool else (Hf, Wf)
    return (B, cm.shape[0], Ho, Wo)


@torch.library.custom_op(f"{_NS}::conv_soft", mutates_args=())
def conv_soft(x: Tensor, npar: Tensor, w: Tensor, cm: Tensor, ch: Tensor, cw: Tensor,
              node_kind: int, depth: int, arity: int, K: int, pad: int, pool: bool) -> Tensor:
    """``x [B,C,H,W]`` -> ``[B,N,Ho,Wo]`` (pooled when ``pool``)."""
    ops.require_gpu(x, npar, w, cm)
    return ops._conv_soft_launch(ops._as_f32(x), ops._c(npar, torch.float32),
                                 ops._c(w, torch.float32), ops._c(cm, torch.int32),
                                 ops._c(ch, torch.int32), ops._c(cw, torch.int32), node_kind,
                                 depth, arity, K, pad, pool)


@conv_soft.register_fake
def _(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
    return x.new_empty(_conv_out_shape(x, cm, pad, pool), dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::conv_soft_bwd", mutates_args=())
def conv_soft_bwd(x: Tensor, npar: Tensor, w: Tensor, cm: Tensor, ch: Tensor, cw: Tensor,
                  node_kind: int, depth: int, arity: int, K: int, pad: int, pool: bool, gy: Tensor,
                  need_x: bool, need_np: bool, need_w: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """``(gx, gnp, gw)`` of conv_soft; unneeded ones are empty."""
    meta = (node_kind, depth, arity, K, pad, pool)
    got = ops.conv_soft_bwd(x, npar, w, cm, ch, cw, *meta, gy, need_x, need_np, need_w)
    if got is None:
        raise NotImplementedError("conv_soft backward: shape outside the HIP kernels")
    gx, gn, gw = got
    return (gx if gx is not None else _empty(x), gn if gn is not None else _empty(x),
            gw if gw is not None else _empty(x))


@conv_soft_bwd.register_fake
def _(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool, gy, need_x, need_np,
      need_w):
    f32 = torch.float32
    return (x.new_empty(x.shape, dtype=f32) if need_x else x.new_empty((0,), dtype=f32),
            x.new_empty(npar.shape, dtype=f32) if need_np else x.new_empty((0,), dtype=f32),
            x.new_empty(w.shape, dtype=f32) if need_w else x.new_empty((0,), dtype=f32))


def _conv_setup(ctx, inputs, output):
    x, npar, w, cm, ch, cw = inputs[:6]
    ctx.save_for_backward(x, npar, w, cm, ch, cw)
    ctx.meta = tuple(inputs[6:])


def _conv_backward(ctx, gy):
    x, npar, w, cm, ch, cw = ctx.saved_tensors
    need = ctx.needs_input_grad
    if not ops.conv_soft_bwd_supported(x, cm, *ctx.meta):
        gx, gn, gw = _composite(
            lambda a, b, c: ops.conv_soft_torch(a, b, c, cm, ch, cw, *ctx.meta), (x, npar, w),
            need[:3], gy)
        return (gx, gn, gw) + (None,) * 9
    gx, gn, gw = conv_soft_bwd(x, npar, w, cm, ch, cw, *ctx.meta, gy, need[0], need[1], need[2])
    return (_none(gx, need[0]), _none(gn, need[1]), _none(gw, need[2])) + (None,) * 9


conv_soft.register_autograd(_conv_backward, setup_context=_conv_setup)


# The reference's tree_conv / tree_conv_topk signature (kernels/conv.py:399-400,
# conv_topk.py:175-189) through slg_tree_conv_fwd: gate16 trees, Top-K leaves
# (w [N,2^d,K]) or fixed ones (K = 1, w all ones), stride 1, 'same' padding.
@torch.library.custom_op(f"{_NS}::tree_conv", mutates_args=())
def tree_conv(x: Tensor, coef: Tensor, w: Tensor, cm: Tensor, ch: Tensor, cw: Tensor, depth: int,
              K: int, pad: int) -> Tensor:
    return ops.tree_conv_launch(x, coef, w, cm, ch, cw, depth, K, pad)


@tree_conv.register_fake
def _(x, coef, w, cm, ch, cw, depth, K, pad):
    return x.new_empty(_conv_out_shape(x, cm, pad, False), dtype=torch.float32)


def _tree_conv_setup(ctx, inputs, output):
    x, coef, w, cm, ch, cw, depth, K, pad = inputs
    ctx.save_for_backward(x, coef, w, cm, ch, cw)
    ctx.meta = (ops.GATE16, depth, 2, K, pad, False)


def _tree_conv_backward(ctx, gy):
    x, coef, w, cm, ch, cw = ctx.saved_tensors
    need = ctx.needs_input_grad
    gx, gn, gw = conv_soft_bwd(x, coef, w, cm, ch, cw, *ctx.meta, gy, need[0], need[1], need[2])
    return (_none(gx, need[0]), _none(gn, need[1]), _none(gw, need[2])) + (None,) * 6


tree_conv.register_autograd(_tree_conv_backward, setup_context=_tree_conv_setup)


# ---------------------------------------------------------------------------
# Hard path: packing, the depth-fused network, the packed GroupSum
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::pack_bits", mutates_args=())
def pack_bits(x: Tensor, word_major: bool) -> Tensor:
    """``[B, D]`` {0,1} -> ``[D, nw]`` int64 (``[nw, D]`` with word_major)."""
    return ops.pack_bits(x, word_major)


@pack_bits.register_fake
def _(x, word_major):
    B = x.shape[0]
    D = x.numel() // B if B else x[0].numel()
    nw = ops.n_words(B)
    return x.new_empty((nw, D) if word_major else (D, nw), dtype=torch.int64)


@torch.library.custom_op(f"{_NS}::fc_hard_net", mutates_args=())
def fc_hard_net(x: Tensor, in_kind: int, B: int, in_dim: int, codes: List[Tensor], C: int,
                wire_r: int) -> Tensor:
    """Depth-fused packed FC network + GroupSum -> logits ``[B, C]`` (counts)."""
    return ops.fc_hard_net(x, in_kind, B, in_dim, codes, C, wire_r)


@fc_hard_net.register_fake
def _(x, in_kind, B, in_dim, codes, C, wire_r):
    return x.new_empty((B, C), dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::groupsum_packed", mutates_args=())
def groupsum_packed(xp: Tensor, B: int, C: int) -> Tensor:
    """Packed ``[W, nw]`` -> per-class counts ``[B, C]`` (no tau)."""
    return ops.groupsum_packed(xp, B, C)


@groupsum_packed.register_fake
def _(xp, B, C):
    return xp.new_empty((B, C), dtype=torch.float32)
