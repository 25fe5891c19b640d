"""Drop-in for the reference's ``silogic.kernels`` dispatch module
(silogic/kernels/__init__.py:21-55): the same function names, argument
meaning and ``HAS_*`` capability flags, implemented by the HIP library.

* :func:`dense_logic` — silogic/kernels/dense.py:123-125
* :func:`warp_logic`  — silogic/kernels/warp.py:104-105
* :func:`tree_conv`   — silogic/kernels/conv.py:399-400 (stride 1, 'same')
* :func:`tree_conv_af`, :func:`build_inverse_map` — kernels/conv.py:247-345
* :func:`tree_conv_topk` — silogic/kernels/conv_topk.py:175-189
* :func:`multilinear_logic` — silogic/kernels/multilinear.py:160-174 (hybrid LUT layer)
* :func:`conv_hybrid` — silogic/kernels/conv_hybrid.py:196 (hybrid LUT trees, any depth)

The flags are True when ``libsilogic_hip.so`` loads. Each function calls the
``torch.ops.silogic_hip`` custom operator of its kernel (``library.py``:
fake shapes for tracing, autograd through the HIP backward kernels).
"""
import torch

from . import _lib, ops
from . import library as _ops_lib  # noqa: F401  (registers torch.ops.silogic_hip)

_op = torch.ops.silogic_hip

_OK = _lib.available()
HAS_DENSE = HAS_WARP = HAS_CONV = HAS_CONV_TOPK = _OK
HAS_MULTILINEAR = HAS_CONV_HYBRID = _OK


def dense_logic(x, ca, cb, wa, wb, coef):
    """x[B,IN], ca/cb[OUT,K] int32, wa/wb[OUT,K], coef[OUT,4] -> [B,OUT]
    (``slg_dense_logic_fwd``)."""
    return _op.dense_logic(x, ca.to(torch.int32), cb.to(torch.int32), wa, wb, coef,
                           ops.GATE16, 1.0)


def warp_logic(x, ca, cb, wa, wb, coef, inv_tau):
    """As :func:`dense_logic`, then ``sigmoid(z * inv_tau)``
    (``slg_warp_logic_fwd``)."""
    return _op.dense_logic(x, ca.to(torch.int32), cb.to(torch.int32), wa, wb, coef,
                           ops.WALSH, float(inv_tau))


def _i32(t):
    return t.to(torch.int32).contiguous()


def _check_same(stride, pad, H, W, Ho, Wo):
    if stride != 1 or Ho != H or Wo != W:
        raise NotImplementedError("tree_conv on MI355X: stride 1, 'same' padding only")


def tree_conv(x, coef, cm, ch, cw, depth, stride, pad, Ho, Wo):
    """Fixed-wiring gate tree conv: coef [N,2^d-1,4], cm/ch/cw [N,2^d]
    (``slg_tree_conv_fwd`` with K = 1)."""
    _check_same(stride, pad, x.shape[2], x.shape[3], Ho, Wo)
    N, leaves = cm.shape
    w = torch.ones(N, leaves, 1, device=x.device)
    return _op.tree_conv(x, coef, w, _i32(cm.unsqueeze(-1)), _i32(ch.unsqueeze(-1)),
                         _i32(cw.unsqueeze(-1)), depth, 1, pad)


def build_inverse_map(cm, ch, cw, C):
    """CSR inverse map of fixed leaf taps (silogic/kernels/conv.py:247-265):
    for each input channel c, the (out channel n, leaf l, dy, dx) that read
    it, in ascending (n, l) order. cm/ch/cw [N, leaves] int -> (off [C+1],
    en, el, edy, edx) int32 on the CPU, the reference's output."""
    N, leaves = cm.shape
    c = cm.reshape(-1).long().cpu()
    order = torch.argsort(c, stable=True)
    off = torch.zeros(C + 1, dtype=torch.int32)
    off[1:] = torch.cumsum(torch.bincount(c, minlength=C)[:C], 0).to(torch.int32)
    i32 = lambda t: t.to(torch.int32)  # noqa: E731
    return (off, i32(order // leaves), i32(order % leaves), i32(ch.reshape(-1).cpu()[order]),
            i32(cw.reshape(-1).cpu()[order]))


def tree_conv_af(x, coef, cm, ch, cw, inv, depth, stride, pad, Ho, Wo):
    """Fixed-wiring gate tree conv with an atomic-free backward
    (silogic/kernels/conv.py:336-345). The HIP backward is atomic-free for
    every tree (a reference table it builds itself on the device), so the
    inverse map ``inv`` of :func:`build_inverse_map` is checked for shape and
    otherwise not needed; the result is :func:`tree_conv`'s."""
    off = inv[0]
    if off.shape[0] != x.shape[1] + 1 or len(inv) != 5:
        raise ValueError("tree_conv_af: inv must be build_inverse_map(cm, ch, cw, C) for "
                         "the input's channels")
    return tree_conv(x, coef, cm, ch, cw, depth, stride, pad, Ho, Wo)


def tree_conv_topk(x, coef, w, cm, ch, cw, depth, K, stride, pad, Ho, Wo):
    """Top-K gate tree conv: w/cm/ch/cw [N,2^d,K] (``slg_tree_conv_fwd``)."""
    _check_same(stride, pad, x.shape[2], x.shape[3], Ho, Wo)
    return _op.tree_conv(x, coef, w, _i32(cm), _i32(ch), _i32(cw), depth, K, pad)


def multilinear_logic(x, cand, w, s, arity):
    """Hybrid (DWN-STE) LUT layer: x [B,IN], cand/w [OUT,arity,K], s
    [OUT,2^arity] = sigmoid(logits) -> [B,OUT] = s at the address of the
    operands thresholded at 0.5, with the multilinear gradient."""
    if cand.shape[1] != arity:
        raise ValueError("multilinear_logic: cand must be [OUT, arity, K]")
    return _op.fc_lut_soft(x, cand.to(torch.int32), w, s, True)


def conv_hybrid(x, s, w, cm, ch, cw, depth, node_arity, K, stride, pad, Ho, Wo):
    """Hybrid LUT tree conv of any depth (kernels/conv_hybrid.py:190-213):
    s [N, nodes, 2^arity] level-major, w/cm/ch/cw [N, leaves, K]; stride 1,
    'same' padding."""
    _check_same(stride, pad, x.shape[2], x.shape[3], Ho, Wo)
    N = cm.shape[0]
    npar = s.reshape(N, 2 ** node_arity) if depth == 1 else s.reshape(N, -1, 2 ** node_arity)
    return _op.conv_soft(x, npar, w, _i32(cm), _i32(ch), _i32(cw), ops.HYBRID, depth,
                         node_arity, K, pad, False)
