"""Torch-level wrappers of the HIP entry points.

Every function here takes CUDA (HIP) tensors, allocates its outputs with
torch, and launches the kernels of ``libsilogic_hip.so`` on torch's current
stream. Nothing here computes on the CPU: a CPU tensor or a missing library
raises.

Autograd: the soft ops are ``torch.autograd.Function`` s whose forward is
the HIP kernel. Their backward recomputes the op with differentiable torch
GPU ops and backpropagates through that (a composite backward, the analogue
of the reference's backward kernels in silogic/kernels/*.py, which are not
part of this build's hot path).
"""
import ctypes

import torch
import torch.nn.functional as F

from . import _lib

GATE16, WALSH, MULTILINEAR2, HYBRID = 0, 1, 2, 3
NODE_KINDS = {"gate16": GATE16, "walsh": WALSH, "multilinear": MULTILINEAR2}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "silogic_amd computes on the GPU only (HIP kernels, no CPU fallback): "
                "move the module and its inputs to a ROCm device with .cuda()")
    _lib.lib()


def _c(t, dtype=None):
    if t is None:
        return None
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _as_f32(x):
    if x.dtype != torch.float32:
        x = x.float()
    return x.contiguous()


# ---------------------------------------------------------------------------
# FC soft
# ---------------------------------------------------------------------------
def fc_soft_prep(conn, raw, node_kind, out_dim, K):
    """HIP prep: softmax(conn) -> w [OUT,2,K]; node param [OUT,4]."""
    require_gpu(raw)
    w = torch.empty((out_dim, 2, K), device=raw.device, dtype=torch.float32)
    npar = torch.empty((out_dim, 4), device=raw.device, dtype=torch.float32)
    conn = _c(conn, torch.float32)
    raw = _c(raw, torch.float32)
    _lib.call("slg_fc_soft_prep", _p(conn), out_dim, K, node_kind, _p(raw), _p(w), _p(npar),
              _stream(raw))
    return w, npar


def _fc_soft_launch(x, cand, w, npar, node_kind, inv_tau, tile=0, threads=0):
    B, IN = x.shape
    OUT, two, K = cand.shape
    if two != 2 or w.shape != cand.shape or npar.shape != (OUT, 4):
        raise ValueError(f"fc_soft: cand {tuple(cand.shape)}, w {tuple(w.shape)}, "
                         f"node_param {tuple(npar.shape)} are inconsistent")
    y = torch.empty((B, OUT), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_soft_fwd", _p(x), B, IN, OUT, K, _p(cand), _p(w), node_kind, _p(npar),
              float(inv_tau), _p(y), int(tile), int(threads), _stream(x))
    return y


def fc_soft_torch(x, cand, w, npar, node_kind, inv_tau):
    """Differentiable torch expression of the FC soft op (backward only)."""
    g = x[:, cand.long()]                        # [B, OUT, 2, K]
    ops = (g * w.unsqueeze(0)).sum(-1)           # [B, OUT, 2]
    a, b = ops[..., 0], ops[..., 1]
    c = npar
    if node_kind == MULTILINEAR2:
        ua, ub = 1 - a, 1 - b
        return (ua * ub) * c[:, 0] + (a * ub) * c[:, 1] + (ua * b) * c[:, 2] + (a * b) * c[:, 3]
    z = c[:, 0] + c[:, 1] * a + c[:, 2] * b + c[:, 3] * (a * b)
    return torch.sigmoid(z * inv_tau) if node_kind == WALSH else z


def fc_soft_bwd(x, cand, w, npar, node_kind, inv_tau, gy, need_x=True, need_w=True,
                need_np=True):
    """HIP backward of the FC soft op: ``(gx, gw, gnp)`` (None where not
    needed), or None when the kernels do not take the shape."""
    require_gpu(x, cand, w, npar, gy)
    x, cand = _as_f32(x.detach()), _c(cand, torch.int32)
    w, npar = _c(w.detach(), torch.float32), _c(npar.detach(), torch.float32)
    B, IN = x.shape
    OUT, _, K = cand.shape
    ws = _lib.lib().slg_fc_soft_bwd_workspace(B, IN, OUT, K)
    if ws < 0:
        return None
    gy = _c(gy, torch.float32)
    gx = torch.empty_like(x) if need_x else None
    gw = torch.empty((OUT, 2, K), device=x.device, dtype=torch.float32) if need_w else None
    gn = torch.empty((OUT, 4), device=x.device, dtype=torch.float32) if need_np else None
    work = torch.empty(max(ws, 1), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_soft_bwd", _p(x), B, IN, OUT, K, _p(cand), _p(w), node_kind, _p(npar),
              float(inv_tau), _p(gy), _p(gx), _p(gw), _p(gn), _p(work), ws, _stream(x))
    return gx, gw, gn


class FCSoftFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cand, w, npar, node_kind, inv_tau):
        x = _as_f32(x)
        cand, w, npar = _c(cand, torch.int32), _c(w, torch.float32), _c(npar, torch.float32)
        ctx.save_for_backward(x, cand, w, npar)
        ctx.meta = (node_kind, inv_tau)
        return _fc_soft_launch(x, cand, w, npar, node_kind, inv_tau)

    @staticmethod
    def backward(ctx, gy):
        x, cand, w, npar = ctx.saved_tensors
        node_kind, inv_tau = ctx.meta
        need = ctx.needs_input_grad
        got = fc_soft_bwd(x, cand, w, npar, node_kind, inv_tau, gy, need[0], need[2], need[3])
        if got is not None:
            gx, gw, gn = got
            return gx, None, gw, gn, None, None
        # shapes the HIP backward does not take: the composite torch backward
        with torch.enable_grad():
            xs = x.detach().requires_grad_(need[0])
            ws = w.detach().requires_grad_(need[2])
            ns = npar.detach().requires_grad_(need[3])
            y = fc_soft_torch(xs, cand, ws, ns, node_kind, inv_tau)
            inputs = [t for t, n in ((xs, need[0]), (ws, need[2]), (ns, need[3])) if n]
            grads = list(torch.autograd.grad(y, inputs, gy)) if inputs else []
        gx = grads.pop(0) if need[0] else None
        gw = grads.pop(0) if need[2] else None
        gn = grads.pop(0) if need[3] else None
        return gx, None, gw, gn, None, None


def fc_soft(x, cand, w, npar, node_kind, inv_tau=1.0):
    """``[B,IN] -> [B,OUT]`` soft FC layer (autograd-aware)."""
    require_gpu(x, cand, w, npar)
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad or npar.requires_grad):
        return FCSoftFn.apply(x, cand, w, npar, node_kind, inv_tau)
    return _fc_soft_launch(_as_f32(x), _c(cand, torch.int32), _c(w, torch.float32),
                           _c(npar, torch.float32), node_kind, inv_tau)


# ---------------------------------------------------------------------------
# FC layers of n-input LUT nodes (multilinear of any arity, hybrid)
# ---------------------------------------------------------------------------
def _fc_lut_launch(x, cand, w, s, hybrid):
    B, IN = x.shape
    OUT, n, K = cand.shape
    if w.shape != cand.shape or tuple(s.shape) != (OUT, 2 ** n):
        raise ValueError("fc_lut_soft: cand/w [OUT,n,K] and s [OUT,2^n] expected")
    ws = _lib.lib().slg_fc_lut_soft_workspace(OUT, n, K)
    if ws < 0:
        raise NotImplementedError(f"fc_lut_soft: arity {n} / K {K} (arity 2..6, K 1..8)")
    work = torch.empty(ws, device=x.device, dtype=torch.float32)
    y = torch.empty((B, OUT), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_lut_soft_fwd", _p(x), B, IN, OUT, n, K, _p(cand), _p(w), _p(s),
              int(bool(hybrid)), _p(y), _p(work), ws, _stream(x))
    return y


def fc_lut_soft_bwd(x, cand, w, s, gy, need_x=True, need_w=True, need_s=True):
    """HIP backward of the LUT layer: ``(gx, gw, gs)`` (None where not
    needed), or None when the kernels do not take the shape."""
    require_gpu(x, cand, w, s, gy)
    x, cand = _as_f32(x.detach()), _c(cand, torch.int32)
    w, s = _c(w.detach(), torch.float32), _c(s.detach(), torch.float32)
    B, IN = x.shape
    OUT, n, K = cand.shape
    ws = _lib.lib().slg_fc_lut_soft_bwd_workspace(B, IN, OUT, n, K)
    if ws < 0:
        return None
    gy = _c(gy, torch.float32)
    gx = torch.empty_like(x) if need_x else None
    gw = torch.empty_like(w) if need_w else None
    gs = torch.empty_like(s) if need_s else None
    work = torch.empty(max(ws, 1), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_lut_soft_bwd", _p(x), B, IN, OUT, n, K, _p(cand), _p(w), _p(s), _p(gy),
              _p(gx), _p(gw), _p(gs), _p(work), ws, _stream(x))
    return gx, gw, gs


class FCLutFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cand, w, s, hybrid):
        x = _as_f32(x)
        cand, w, s = _c(cand, torch.int32), _c(w, torch.float32), _c(s, torch.float32)
        ctx.save_for_backward(x, cand, w, s)
        return _fc_lut_launch(x, cand, w, s, hybrid)

    @staticmethod
    def backward(ctx, gy):
        x, cand, w, s = ctx.saved_tensors
        need = ctx.needs_input_grad
        got = fc_lut_soft_bwd(x, cand, w, s, gy, need[0], need[2], need[3])
        if got is None:
            raise NotImplementedError("fc_lut_soft backward: the input width exceeds what the "
                                      "kernels stage in LDS")
        gx, gw, gs = got
        return gx, None, gw, gs, None


def fc_lut_soft(x, cand, w, s, hybrid):
    """``[B,IN] -> [B,OUT]`` LUT layer (multilinear interpolation of ``s``, or
    the hybrid lookup), autograd-aware (the multilinear gradient)."""
    require_gpu(x, cand, w, s)
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad or s.requires_grad):
        return FCLutFn.apply(x, cand, w, s, hybrid)
    return _fc_lut_launch(_as_f32(x), _c(cand, torch.int32), _c(w, torch.float32),
                          _c(s, torch.float32), hybrid)


def fc_lut_hard_codes(cand, conn, logits, in_dim):
    """``(idx [OUT,n] int32, tt [OUT] int64)`` for ``fc_lut_hard``."""
    require_gpu(cand, logits)
    cand = _c(cand, torch.int32)
    OUT, n, K = cand.shape
    idx = torch.empty((OUT, n), device=cand.device, dtype=torch.int32)
    tt = torch.empty((OUT,), device=cand.device, dtype=torch.int64)
    _lib.call("slg_fc_lut_hard_prep", _p(cand), _p(None if conn is None else
                                                   _c(conn.detach(), torch.float32)),
              OUT, n, K, in_dim, _p(_c(logits.detach(), torch.float32)), _p(idx), _p(tt),
              _stream(cand))
    return idx, tt


MAX_RECORD_LAYERS = 16


def _ptrs(ts):
    return (ctypes.c_void_p * len(ts))(*[None if t is None else t.data_ptr() for t in ts])


def fc_soft_schedule(cand, in_dim):
    """Bank-aware gather order ``[OUT,2,K]`` uint8 for ``cand [OUT,2,K]``."""
    require_gpu(cand)
    cand = _c(cand, torch.int32)
    OUT, two, K = cand.shape
    order = torch.empty((OUT, 2, K), device=cand.device, dtype=torch.uint8)
    _lib.call("slg_fc_soft_schedule", _p(cand), OUT, K, int(in_dim), _p(order), _stream(cand))
    return order


def fc_soft_records(specs, K):
    """Per-output parameter records of several FC soft layers, one launch per
    16 layers. ``specs``: ``(cand [OUT,2,K], conn [OUT,2,K] or None, raw,
    in_dim, node_kind, order or None)`` per layer (``raw``: gate logits
    [OUT,16], walsh theta or multilinear logits [OUT,4]; ``order`` from
    :func:`fc_soft_schedule`). Returns ``[ceil(OUT/64), record_quads(K), 64, 4]`` float32
    tensors (the chunk-major record layout; index words reinterpreted)."""
    recs = []
    for g in range(0, len(specs), MAX_RECORD_LAYERS):
        part = specs[g:g + MAX_RECORD_LAYERS]
        cands, conns, raws, ins, outs, kinds, orders = [], [], [], [], [], [], []
        for cand, conn, raw, in_dim, kind, order in part:
            require_gpu(cand, conn, raw, order)
            OUT = cand.shape[0]
            if tuple(cand.shape) != (OUT, 2, K) or (conn is not None and conn.shape != cand.shape):
                raise ValueError(f"fc_soft_records: cand {tuple(cand.shape)} / conn "
                                 f"{None if conn is None else tuple(conn.shape)} for K={K}")
            if raw.shape != (OUT, 16 if kind == GATE16 else 4):
                raise ValueError(f"fc_soft_records: raw {tuple(raw.shape)} for node kind {kind}")
            if order is not None and (order.shape != cand.shape or order.dtype != torch.uint8):
                raise ValueError("fc_soft_records: order must be uint8 shaped like cand")
            cands.append(_c(cand, torch.int32))
            conns.append(_c(conn, torch.float32))
            raws.append(_c(raw, torch.float32))
            orders.append(_c(order))
            ins.append(int(in_dim))
            outs.append(OUT)
            kinds.append(int(kind))
        dev = raws[0].device
        out = [torch.empty(((o + 63) // 64, record_quads(K), 64, 4), device=dev,
                           dtype=torch.float32)
               for o in outs]
        n = len(part)
        _lib.call("slg_fc_soft_records", n, _ptrs(cands), _ptrs(conns), _ptrs(raws),
                  (ctypes.c_int64 * n)(*ins), (ctypes.c_int64 * n)(*outs), K,
                  (ctypes.c_int32 * n)(*kinds), _ptrs(orders), _ptrs(out), _stream(raws[0]))
        recs.extend(out)
    return recs


def record_quads(K):
    """Quads per soft FC record: K index words (idx_a | idx_b << 16), K words
    w_a, K words w_b, zero padding to a whole quad, one quad of node
    parameters."""
    return (3 * K + 3) // 4 + 1


def record_words(rec, out_dim):
    """``[OUT, 4 * record_quads(K)]`` view of chunk-major records (for
    inspection)."""
    n64, K1 = rec.shape[0], rec.shape[1]
    return rec.permute(0, 2, 1, 3).reshape(n64 * 64, 4 * K1)[:out_dim]


def _check_rec(x, rec, out_dim, K):
    if rec.dim() != 4 or tuple(rec.shape) != ((out_dim + 63) // 64, record_quads(K), 64, 4) or \
            rec.dtype != torch.float32 or not rec.is_contiguous():
        raise ValueError(f"fc_soft: records {tuple(rec.shape)} {rec.dtype} for OUT={out_dim}, K={K}")
    if x.dim() != 2:
        raise ValueError(f"fc_soft: x must be [B, IN], got {tuple(x.shape)}")


def fc_soft_rec(x, rec, out_dim, K, node_kind, inv_tau=1.0, tile=0, threads=0):
    """Soft FC layer on records (no autograd): ``[B,IN] -> [B,OUT]``."""
    require_gpu(x, rec)
    x = _as_f32(x)
    _check_rec(x, rec, out_dim, K)
    B, IN = x.shape
    y = torch.empty((B, out_dim), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_soft_fwd_records", _p(x), B, IN, out_dim, K, _p(rec), node_kind,
              float(inv_tau), _p(y), int(tile), int(threads), _stream(x))
    return y


def fc_soft_groupsum_supported(B, IN, OUT, C):
    return bool(_lib.lib().slg_fc_soft_groupsum_supported(B, IN, OUT, C))


def fc_soft_rec_groupsum(x, rec, out_dim, K, node_kind, inv_tau, C, tau):
    """Last soft layer fused with the STE GroupSum head: ``[B,IN] -> [B,C]``."""
    require_gpu(x, rec)
    x = _as_f32(x)
    _check_rec(x, rec, out_dim, K)
    B, IN = x.shape
    logits = torch.empty((B, C), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_soft_fwd_groupsum", _p(x), B, IN, out_dim, K, _p(rec), node_kind,
              float(inv_tau), int(C), float(tau), _p(logits), _stream(x))
    return logits


# ---------------------------------------------------------------------------
# GroupSum / OrPool
# ---------------------------------------------------------------------------
class GroupSumSoftFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, C, tau, ste):
        x = _as_f32(x)
        B, W = x.shape
        out = torch.empty((B, C), device=x.device, dtype=torch.float32)
        _lib.call("slg_groupsum_soft", _p(x), B, W, C, float(tau), int(bool(ste)), _p(out),
                  _stream(x))
        ctx.meta = (W, C, tau)
        return out

    @staticmethod
    def backward(ctx, g):
        # both the plain sum and the straight-through (x>0.5) + x - x.detach()
        # have d logit / d x = 1/tau on the class block (silogic/heads.py:34-39)
        W, C, tau = ctx.meta
        gx = (g / tau).unsqueeze(2).expand(g.shape[0], C, W // C).reshape(g.shape[0], W)
        return gx, None, None, None


def groupsum_soft(x, C, tau, ste):
    require_gpu(x)
    return GroupSumSoftFn.apply(x, C, tau, ste)


def groupsum_hard(x, C):
    require_gpu(x)
    if x.dtype == torch.bool:
        x = x.to(torch.uint8)
    dtype = 1 if x.dtype == torch.uint8 else 0
    x = x.contiguous() if dtype == 1 else _as_f32(x)
    B, W = x.shape
    out = torch.empty((B, C), device=x.device, dtype=torch.float32)
    _lib.call("slg_groupsum_hard", _p(x), dtype, B, W, C, _p(out), _stream(x))
    return out


class OrPoolFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        out = _orpool_launch(x)
        ctx.save_for_backward(x)
        return out

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        with torch.enable_grad():
            xs = x.detach().requires_grad_(True)
            y = F.max_pool2d(xs, 2, 2)
            (gx,) = torch.autograd.grad(y, [xs], g)
        return gx


def _orpool_launch(x):
    dtype = 1 if x.dtype == torch.uint8 else 0
    x = x.contiguous() if dtype == 1 else _as_f32(x)
    B, Cc, H, W = x.shape
    out = torch.empty((B, Cc, H // 2, W // 2), device=x.device, dtype=x.dtype)
    _lib.call("slg_orpool", _p(x), dtype, B, Cc, H, W, _p(out), _stream(x))
    return out


def orpool(x):
    require_gpu(x)
    if x.dtype == torch.bool:
        x = x.to(torch.uint8)
    if torch.is_grad_enabled() and x.requires_grad:
        return OrPoolFn.apply(x)
    return _orpool_launch(x)


# ---------------------------------------------------------------------------
# hard (bit-packed)
# ---------------------------------------------------------------------------
def n_words(B):
    return (B + 63) >> 6


def _in_kind(x):
    if x.dtype == torch.bool:
        x = x.to(torch.uint8)
    if x.dtype == torch.uint8:
        return x.contiguous(), 1
    return _as_f32(x), 0


def pack_bits(x, word_major=False):
    """``[B, D]`` {0,1} -> packed ``[D, ceil(B/64)]`` (int64 storage of uint64),
    or ``[ceil(B/64), D]`` with ``word_major``."""
    require_gpu(x)
    x, kind = _in_kind(x.reshape(x.shape[0], -1))
    B, D = x.shape
    shape = (n_words(B), D) if word_major else (D, n_words(B))
    xp = torch.empty(shape, device=x.device, dtype=torch.int64)
    _lib.call("slg_pack_bits", _p(x), kind, B, D, int(word_major), _p(xp), _stream(x))
    return xp


def _words_for(xp, B, what):
    """``xp`` [rows, >= ceil(B/64)] cut to exactly ceil(B/64) words per row
    (the kernels take that as the row stride)."""
    nw = n_words(B)
    if xp.dim() != 2 or xp.shape[1] < nw:
        raise ValueError("%s: packed input must be [rows, >= %d] for B = %d" % (what, nw, B))
    return xp if xp.shape[1] == nw and xp.is_contiguous() else xp[:, :nw].contiguous()


def unpack_bits(xp, B):
    require_gpu(xp)
    xp = _words_for(xp, B, "unpack_bits")
    D = xp.shape[0]
    out = torch.empty((B, D), device=xp.device, dtype=torch.uint8)
    _lib.call("slg_unpack_bits", _p(xp), B, D, _p(out), _stream(xp))
    return out


def fc_hard_codes(cand, conn, raw, node_kind, in_dim):
    """Per-output packed codes ``[OUT, 2]`` int32 (a, b | tt<<28).

    ``cand`` [OUT,2,K] int32 with ``conn`` [OUT,2,K], or ``cand`` = idx
    [OUT,2] int32 with ``conn`` None (fixed wiring)."""
    require_gpu(cand, raw)
    cand = _c(cand, torch.int32)
    OUT = cand.shape[0]
    K = cand.shape[2] if cand.dim() == 3 else 1
    codes = torch.empty((OUT, 2), device=cand.device, dtype=torch.int32)
    _lib.call("slg_fc_hard_prep", _p(cand), _p(_c(conn, torch.float32)), OUT, K, in_dim,
              node_kind, _p(_c(raw, torch.float32)), _p(codes), _stream(cand))
    return codes


MAX_COMPACT_IN = 1 << 14


def fc_hard_codes_net(specs, compact=False):
    """Codes of several layers, one launch per 16 layers. ``specs``:
    ``(cand, conn or None, raw, node_kind, in_dim)`` per layer, as
    :func:`fc_hard_codes`. Returns ``[OUT, 2]`` int32 tensors, or with
    ``compact`` the depth-fused network's ``[OUT]`` int32 codes
    (b | a << 14 | tt << 28; inputs at most 16384 wide)."""
    out = []
    for g in range(0, len(specs), MAX_RECORD_LAYERS):
        part = specs[g:g + MAX_RECORD_LAYERS]
        cands, conns, raws, ins, outs, Ks, kinds = [], [], [], [], [], [], []
        for cand, conn, raw, kind, in_dim in part:
            require_gpu(cand, conn, raw)
            cand = _c(cand, torch.int32)
            OUT = cand.shape[0]
            K = cand.shape[2] if cand.dim() == 3 else 1
            if (conn is None) != (cand.dim() == 2) or (conn is not None and conn.shape != cand.shape):
                raise ValueError("fc_hard_codes_net: cand/conn shapes are inconsistent")
            if raw.shape != (OUT, 16 if kind == GATE16 else 4):
                raise ValueError(f"fc_hard_codes_net: raw {tuple(raw.shape)} for node kind {kind}")
            cands.append(cand)
            conns.append(_c(conn, torch.float32))
            raws.append(_c(raw, torch.float32))
            ins.append(int(in_dim))
            outs.append(OUT)
            Ks.append(K)
            kinds.append(int(kind))
        shape = (lambda o: (o,)) if compact else (lambda o: (o, 2))
        codes = [torch.empty(shape(o), device=raws[0].device, dtype=torch.int32) for o in outs]
        n = len(part)
        _lib.call("slg_fc_hard_prep_net", n, _ptrs(cands), _ptrs(conns), _ptrs(raws),
                  (ctypes.c_int64 * n)(*ins), (ctypes.c_int64 * n)(*outs),
                  (ctypes.c_int32 * n)(*Ks), (ctypes.c_int32 * n)(*kinds), int(bool(compact)),
                  _ptrs(codes), _stream(raws[0]))
        out.extend(codes)
    return out


def fc_hard_layer(xp, codes):
    require_gpu(xp, codes)
    IN, nw = xp.shape
    OUT = codes.shape[0]
    if codes.shape != (OUT, 2) or codes.dtype != torch.int32:
        raise ValueError("fc_hard_layer: codes must be [OUT, 2] int32 from fc_hard_codes")
    out = torch.empty((OUT, nw), device=xp.device, dtype=torch.int64)
    _lib.call("slg_fc_hard_layer", _p(xp), IN, nw, _p(codes), OUT, _p(out), _stream(xp))
    return out


def fc_hard_net_supported(in_dim, widths, C):
    arr = (ctypes.c_int64 * len(widths))(*widths)
    return _lib.lib().slg_fc_hard_net_supported(in_dim, len(widths), arr, C)


ROWS_F32, ROWS_U8, PACKED, PACKED_WORD_MAJOR = 0, 1, 2, 3


def fc_hard_net(x, in_kind, B, in_dim, codes, C, wire_r=0):
    """Depth-fused packed FC network + GroupSum -> logits ``[B, C]``.

    ``in_kind``: ROWS_F32 / ROWS_U8 ([B, in_dim], packed inside the kernel),
    PACKED ([in_dim, nw]) or PACKED_WORD_MAJOR ([nw, in_dim]). ``codes``:
    compact per-layer codes from ``fc_hard_codes_net(..., compact=True)``."""
    require_gpu(x, *codes)
    if any(c.dim() != 1 or c.dtype != torch.int32 for c in codes):
        raise ValueError("fc_hard_net: codes must be compact [OUT] int32 codes")
    widths = [c.shape[0] for c in codes]
    w_arr = (ctypes.c_int64 * len(widths))(*widths)
    c_arr = (ctypes.c_void_p * len(codes))(*[c.data_ptr() for c in codes])
    out = torch.empty((B, C), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_hard_net", _p(x), in_kind, B, in_dim, len(codes), w_arr, c_arr, C,
              int(wire_r), _p(out), _stream(x))
    return out


def groupsum_packed(xp, B, C):
    require_gpu(xp)
    xp = _words_for(xp, B, "groupsum_packed")
    W = xp.shape[0]
    if W % C:
        raise ValueError("groupsum_packed: %d rows not divisible by %d classes" % (W, C))
    out = torch.empty((B, C), device=xp.device, dtype=torch.float32)
    _lib.call("slg_groupsum_packed", _p(xp), W, B, C, _p(out), _stream(xp))
    return out


def fc_lut_hard(xp, idx, tt):
    """Packed LUT layer: ``xp`` [IN, nw], ``idx`` [OUT, arity] int32, ``tt``
    [OUT] int64 truth tables (entry sum_j x_j << j at that bit) -> [OUT, nw]."""
    require_gpu(xp, idx, tt)
    IN, nw = xp.shape
    idx, tt = _c(idx, torch.int32), _c(tt, torch.int64)
    OUT, arity = idx.shape
    if tt.shape != (OUT,):
        raise ValueError("fc_lut_hard: tt must be [OUT] int64")
    out = torch.empty((OUT, nw), device=xp.device, dtype=torch.int64)
    _lib.call("slg_fc_lut_hard", _p(_c(xp)), IN, nw, _p(idx), arity, _p(tt), OUT, _p(out),
              _stream(xp))
    return out


def packed_unfold(x3, kh, kw, stride, padding, H, W):
    """``x3`` [C, H*W, nw] -> [C*kh*kw, Ho*Wo, nw] (zero padding)."""
    require_gpu(x3)
    C, L, nw = x3.shape
    if L != H * W:
        raise ValueError("packed_unfold: L = %d is not H*W = %d" % (L, H * W))
    Ho = (H + 2 * padding - kh) // stride + 1
    Wo = (W + 2 * padding - kw) // stride + 1
    if Ho <= 0 or Wo <= 0:
        raise ValueError("packed_unfold: empty output")
    out = torch.empty((C * kh * kw, Ho * Wo, nw), device=x3.device, dtype=torch.int64)
    _lib.call("slg_packed_unfold", _p(_c(x3)), C, H, W, nw, kh, kw, stride, padding, _p(out),
              _stream(x3))
    return out


def packed_or_pool(x3, H, W, ps=2):
    """``x3`` [C, H*W, nw] -> [C, (H//ps)*(W//ps), nw], OR over windows."""
    require_gpu(x3)
    C, L, nw = x3.shape
    if L != H * W:
        raise ValueError("packed_or_pool: L = %d is not H*W = %d" % (L, H * W))
    out = torch.empty((C, (H // ps) * (W // ps), nw), device=x3.device, dtype=torch.int64)
    if out.numel():
        _lib.call("slg_packed_or_pool", _p(_c(x3)), C, H, W, nw, ps, _p(out), _stream(x3))
    return out


def lut_tree_hard(xu, leaf, arity, depth, tables):
    """LUT tree on unfolded input ``xu`` [P, L, nw]: ``leaf`` [N, arity**depth]
    int32 flat P indices, ``tables`` [N, nodes] int64 level-major -> [N, L, nw]."""
    require_gpu(xu, leaf, tables)
    P, L, nw = xu.shape
    leaf, tables = _c(leaf, torch.int32), _c(tables, torch.int64)
    N = leaf.shape[0]
    nodes = sum(arity ** i for i in range(depth))
    if leaf.shape != (N, arity ** depth) or tables.shape != (N, nodes):
        raise ValueError("lut_tree_hard: leaf / table shapes do not match arity %d depth %d"
                         % (arity, depth))
    out = torch.empty((N, L, nw), device=xu.device, dtype=torch.int64)
    _lib.call("slg_lut_tree_hard", _p(_c(xu)), P, L, nw, N, _p(leaf), arity, depth, _p(tables),
              _p(out), _stream(xu))
    return out


# ---------------------------------------------------------------------------
# conv
# ---------------------------------------------------------------------------
def conv_soft_prep(conn, raw, node_kind, N, leaves, K, depth, arity):
    require_gpu(raw)
    w = torch.empty((N, leaves, K), device=raw.device, dtype=torch.float32)
    if node_kind == GATE16:
        npar = torch.empty((N, leaves - 1, 4), device=raw.device, dtype=torch.float32)
    else:
        npar = torch.empty((N, 2 ** arity), device=raw.device, dtype=torch.float32)
    _lib.call("slg_conv_soft_prep", _p(_c(conn, torch.float32)), N, leaves, K, node_kind, depth,
              arity, _p(_c(raw, torch.float32)), _p(w), _p(npar), _stream(raw))
    return w, npar


def _conv_soft_launch(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
    B, Cc, H, W = x.shape
    N = cm.shape[0]
    leaves = 2 ** depth if node_kind == GATE16 else arity
    nparam = (N, leaves - 1, 4) if node_kind == GATE16 else (N, 2 ** arity)
    if (cm.shape != (N, leaves, K) or ch.shape != cm.shape or cw.shape != cm.shape
            or w.shape != cm.shape or tuple(npar.shape) != nparam):
        raise ValueError("conv_soft: tap / weight / node parameter shapes are inconsistent")
    kern = 2 * pad + 1
    Hf, Wf = H + 2 * pad - kern + 1, W + 2 * pad - kern + 1
    Ho, Wo = (Hf // 2, Wf // 2) if pool else (Hf, Wf)
    out = torch.empty((B, N, Ho, Wo), device=x.device, dtype=torch.float32)
    _lib.call("slg_conv_soft_fwd", _p(x), B, Cc, H, W, N, node_kind, depth, arity, K, _p(npar),
              _p(w), _p(cm), _p(ch), _p(cw), pad, int(bool(pool)), _p(out), _stream(x))
    return out


class _StraightThrough(torch.autograd.Function):
    """Value of ``disc`` exactly, gradient into ``soft`` (the hybrid node)."""

    @staticmethod
    def forward(ctx, disc, soft):
        return disc.clone()

    @staticmethod
    def backward(ctx, g):
        return None, g


def conv_soft_torch(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
    """Differentiable torch expression of the fused conv op (backward only)."""
    B, Cc, H, W = x.shape
    N, leaves = cm.shape[0], cm.shape[1]
    kern = 2 * pad + 1
    patches = F.unfold(x, (kern, kern), padding=pad)                  # [B, C*k*k, L]
    flat = (cm.long() * kern * kern + ch.long() * kern + cw.long()).reshape(-1)
    g = patches[:, flat, :].view(B, N, leaves, K, -1)
    vals = (g * w.view(1, N, leaves, K, 1)).sum(3)                    # [B, N, leaves, L]
    if node_kind == GATE16:
        nb, cnt = 0, leaves
        while cnt > 1:
            c = npar[:, nb:nb + cnt // 2, :].unsqueeze(0).unsqueeze(-1)
            a, b = vals[:, :, 0::2, :], vals[:, :, 1::2, :]
            vals = c[:, :, :, 0] + c[:, :, :, 1] * a + c[:, :, :, 2] * b + c[:, :, :, 3] * (a * b)
            nb += cnt // 2
            cnt //= 2
        out = vals[:, :, 0, :]
    else:
        corners = torch.tensor([[(p >> j) & 1 for j in range(arity)] for p in range(2 ** arity)],
                               dtype=x.dtype, device=x.device)
        c = corners.view(1, 1, 1, -1, arity)

        def lut(v):
            a = v.permute(0, 1, 3, 2).unsqueeze(3)                   # [B, N, L, 1, A]
            prod = (c * a + (1 - c) * (1 - a)).prod(-1)               # [B, N, L, P]
            return (prod * npar.view(1, N, 1, -1)).sum(-1)
        out = lut(vals)
        if node_kind == HYBRID:  # discrete value, multilinear gradient (nodes.py:202-206)
            with torch.no_grad():
                disc = lut((vals >= 0.5).to(vals.dtype))
            out = _StraightThrough.apply(disc, out)
    Hf, Wf = H + 2 * pad - kern + 1, W + 2 * pad - kern + 1
    out = out.view(B, N, Hf, Wf)
    return F.max_pool2d(out, 2, 2) if pool else out


def conv_soft_bwd(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool, gy,
                  need_x=True, need_np=True, need_w=True):
    """HIP backward of the conv soft op: ``(gx, gnp, gw)`` (None where not
    needed), or None when the kernel does not take the shape."""
    require_gpu(x, npar, w, cm, gy)
    x = _as_f32(x.detach())
    npar, w = _c(npar.detach(), torch.float32), _c(w.detach(), torch.float32)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    B, Cc, H, W = x.shape
    N = cm.shape[0]
    ws = _lib.lib().slg_conv_soft_bwd_workspace(B, Cc, H, W, N, node_kind, depth, arity, K, pad,
                                                int(bool(pool)))
    if ws < 0:
        return None
    gy = _c(gy, torch.float32)
    gx = torch.empty_like(x) if need_x else None
    gn = torch.empty_like(npar) if need_np else None
    gw = torch.empty_like(w) if need_w else None
    work = torch.empty(max(ws, 1), device=x.device, dtype=torch.float32)
    _lib.call("slg_conv_soft_bwd", _p(x), B, Cc, H, W, N, node_kind, depth, arity, K, _p(npar),
              _p(w), _p(cm), _p(ch), _p(cw), pad, int(bool(pool)), _p(gy), _p(gx), _p(gw),
              _p(gn), _p(work), ws, _stream(x))
    return gx, gn, gw


class ConvSoftFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
        x = _as_f32(x)
        npar, w = _c(npar, torch.float32), _c(w, torch.float32)
        ctx.save_for_backward(x, npar, w, cm, ch, cw)
        ctx.meta = (node_kind, depth, arity, K, pad, pool)
        return _conv_soft_launch(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool)

    @staticmethod
    def backward(ctx, gy):
        x, npar, w, cm, ch, cw = ctx.saved_tensors
        meta = ctx.meta
        need = ctx.needs_input_grad
        got = conv_soft_bwd(x, npar, w, cm, ch, cw, *meta, gy, need[0], need[1], need[2])
        if got is not None:
            return got + (None,) * 9
        # shapes the HIP backward does not take: the composite torch backward
        with torch.enable_grad():
            xs = x.detach().requires_grad_(need[0])
            ns = npar.detach().requires_grad_(need[1])
            ws = w.detach().requires_grad_(need[2])
            y = conv_soft_torch(xs, ns, ws, cm, ch, cw, *meta)
            inputs = [t for t, n in ((xs, need[0]), (ns, need[1]), (ws, need[2])) if n]
            grads = list(torch.autograd.grad(y, inputs, gy)) if inputs else []
        gx = grads.pop(0) if need[0] else None
        gn = grads.pop(0) if need[1] else None
        gw = grads.pop(0) if need[2] else None
        return (gx, gn, gw) + (None,) * 9


def conv_soft(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
    require_gpu(x, npar, w, cm)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    if torch.is_grad_enabled() and (x.requires_grad or w.requires_grad or npar.requires_grad):
        return ConvSoftFn.apply(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool)
    return _conv_soft_launch(_as_f32(x), _c(npar, torch.float32), _c(w, torch.float32), cm, ch,
                             cw, node_kind, depth, arity, K, pad, pool)


def conv_soft_records(conn, cm, ch, cw, raw, node_kind, depth, arity, K, in_shape, pad, pool):
    """Per-channel records (taps resolved for in_shape = (C, H, W), pad and
    the pooling flag, leaf weights, node parameters) for conv_soft_rec;
    [N, R] float32."""
    require_gpu(raw, cm)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    N = cm.shape[0]
    leaves = 2 ** depth if node_kind == GATE16 else arity
    if cm.shape != (N, leaves, K) or ch.shape != cm.shape or cw.shape != cm.shape:
        raise ValueError("conv_soft_records: tap shapes are inconsistent")
    if conn is not None and tuple(conn.shape) != (N, leaves, K):
        raise ValueError("conv_soft_records: conn shape %s" % (tuple(conn.shape),))
    R = _lib.lib().slg_conv_soft_record_floats(node_kind, depth, arity, K, int(bool(pool)))
    if R <= 0:
        raise ValueError("conv_soft_records: unsupported node %d depth %d arity %d K %d"
                         % (node_kind, depth, arity, K))
    C, H, W = in_shape
    rec = torch.empty((N, R), device=raw.device, dtype=torch.float32)
    _lib.call("slg_conv_soft_records", _p(_c(conn, torch.float32)), _p(cm), _p(ch), _p(cw), N, K,
              node_kind, depth, arity, _p(_c(raw, torch.float32)), C, H, W, pad,
              int(bool(pool)), _p(rec), _stream(raw))
    return rec


def conv_soft_rec(x, rec, N, node_kind, depth, arity, K, pad, pool):
    """Fused soft conv (+ 2x2 max pool) from records built by conv_soft_records
    for x's (C, H, W), the same pad and the same pooling flag; forward only."""
    require_gpu(x, rec)
    x = _as_f32(x)
    B, Cc, H, W = x.shape
    R = _lib.lib().slg_conv_soft_record_floats(node_kind, depth, arity, K, int(bool(pool)))
    if R <= 0 or tuple(rec.shape) != (N, R) or rec.dtype != torch.float32 or not rec.is_contiguous():
        raise ValueError("conv_soft_rec: records do not match node %d depth %d arity %d K %d"
                         % (node_kind, depth, arity, K))
    kern = 2 * pad + 1
    Hf, Wf = H + 2 * pad - kern + 1, W + 2 * pad - kern + 1
    Ho, Wo = (Hf // 2, Wf // 2) if pool else (Hf, Wf)
    out = torch.empty((B, N, Ho, Wo), device=x.device, dtype=torch.float32)
    _lib.call("slg_conv_soft_fwd_records", _p(x), B, Cc, H, W, N, node_kind, depth, arity, K,
              _p(rec), pad, int(bool(pool)), _p(out), _stream(x))
    return out


def conv_hard_prep(cm, ch, cw, conn, raw, node_kind, depth, arity):
    require_gpu(cm, raw)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    N, leaves, K = cm.shape
    leaf = torch.empty((N, leaves), device=cm.device, dtype=torch.int32)
    tt = torch.empty((N,), device=cm.device, dtype=torch.int64)
    _lib.call("slg_conv_hard_prep", _p(cm), _p(ch), _p(cw), _p(_c(conn, torch.float32)), N,
              leaves, K, node_kind, depth, arity, _p(_c(raw, torch.float32)), _p(leaf), _p(tt),
              _stream(cm))
    return leaf, tt


MAX_CONV_PREP_BLOCKS = 8


def conv_hard_prep_net(specs):
    """Hard parameters of several conv blocks, one launch per 8 blocks.
    ``specs``: ``(cm, ch, cw, conn or None, raw_levels, node_kind, depth,
    arity)`` per block, ``raw_levels`` a list of the gate16 per-level logits
    ``[N, 2^(depth-1-l), 16]`` or ``[logits [N, 2^arity]]``. Returns
    ``[(leaf [N, leaves] int32, tt [N] int64)]``."""
    out = []
    for g in range(0, len(specs), MAX_CONV_PREP_BLOCKS):
        part = specs[g:g + MAX_CONV_PREP_BLOCKS]
        cms, chs, cws, conns, raws, Ns, Ks, kinds, depths, ars, leafs, tts = \
            [], [], [], [], [], [], [], [], [], [], [], []
        for cm, ch, cw, conn, levels, kind, depth, arity in part:
            require_gpu(cm, *levels)
            cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
            N, leaves, K = cm.shape
            if ch.shape != cm.shape or cw.shape != cm.shape or (
                    conn is not None and tuple(conn.shape) != (N, leaves, K)):
                raise ValueError("conv_hard_prep_net: tap/conn shapes are inconsistent")
            if kind == GATE16:
                want = [(N, 2 ** (depth - 1 - l), 16) for l in range(depth)]
            else:
                want = [(N, 2 ** arity)]
            if [tuple(t.shape) for t in levels] != want:
                raise ValueError("conv_hard_prep_net: logits %s for node kind %d depth %d arity %d"
                                 % ([tuple(t.shape) for t in levels], kind, depth, arity))
            levels = [_c(t, torch.float32) for t in levels]
            conn = _c(conn, torch.float32)
            cms.append(cm)
            chs.append(ch)
            cws.append(cw)
            conns.append(conn)
            raws += levels + [None] * (4 - len(levels))
            Ns.append(N)
            Ks.append(K)
            kinds.append(int(kind))
            depths.append(int(depth))
            ars.append(int(arity))
            leafs.append(torch.empty((N, leaves), device=cm.device, dtype=torch.int32))
            tts.append(torch.empty((N,), device=cm.device, dtype=torch.int64))
        n = len(part)
        _lib.call("slg_conv_hard_prep_net", n, _ptrs(cms), _ptrs(chs), _ptrs(cws), _ptrs(conns),
                  _ptrs(raws), (ctypes.c_int64 * n)(*Ns), (ctypes.c_int32 * n)(*Ks),
                  (ctypes.c_int32 * n)(*kinds), (ctypes.c_int32 * n)(*depths),
                  (ctypes.c_int32 * n)(*ars), _ptrs(leafs), _ptrs(tts), _stream(cms[0]))
        out.extend(zip(leafs, tts))
    return out


def conv_hard(xp, shape_chw, leaf, tt, node_kind, depth, arity, kernel, pad, pool):
    """Packed conv: ``xp`` [C,H,W,nw] -> [N,Ho,Wo,nw] (pooled if ``pool``)."""
    require_gpu(xp, leaf, tt)
    Cc, H, W = shape_chw
    nw = xp.shape[-1]
    N = leaf.shape[0]
    leaves = 2 ** depth if node_kind == GATE16 else arity
    if xp.numel() != Cc * H * W * nw or leaf.shape != (N, leaves) or tt.shape != (N,):
        raise ValueError("conv_hard: packed input / leaf / truth-table shapes are inconsistent")
    Hf, Wf = H + 2 * pad - kernel + 1, W + 2 * pad - kernel + 1
    Ho, Wo = (Hf // 2, Wf // 2) if pool else (Hf, Wf)
    out = torch.empty((N, Ho, Wo, nw), device=xp.device, dtype=torch.int64)
    _lib.call("slg_conv_hard_fwd", _p(xp), Cc, H, W, nw, N, node_kind, depth, arity, _p(leaf),
              _p(tt), kernel, pad, int(bool(pool)), _p(out), _stream(xp))
    return out
