"""Torch-level wrappers of the HIP entry points.

Every function here takes CUDA (HIP) tensors, allocates its outputs with
torch, and launches the kernels of ``libsilogic_hip.so`` on torch's current
stream. Nothing here computes on the CPU: a CPU tensor or a missing library
raises.

Autograd: with gradients the soft ops run as the ``torch.ops.silogic_hip``
custom operators of ``library.py`` (opaque to ``torch.compile``), whose
backward runs the HIP backward kernels; for shapes those kernels do not take,
the autograd backward differentiates the op's torch expression
(``fc_soft_torch``, ``conv_soft_torch``). Without gradients the wrappers
launch the kernels directly.
"""
import ctypes

import torch
import torch.nn.functional as F

from . import _lib

GATE16, WALSH, MULTILINEAR2, HYBRID = 0, 1, 2, 3
NODE_KINDS = {"gate16": GATE16, "walsh": WALSH, "multilinear": MULTILINEAR2}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t):
    """torch's current stream on ``t``'s device, as a raw handle."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.get_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "silogic_amd computes on the GPU only (HIP kernels, no CPU fallback): "
                "move the module and its inputs to a ROCm device with .cuda()")
    if not torch.compiler.is_compiling():   # traced code reaches the library in the ops
        _lib.lib()


def _grad_path(*ts):
    """True when the op must run as a differentiable custom operator: some
    input needs a gradient, or torch.compile is tracing."""
    if torch.compiler.is_compiling():
        return True
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)



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


def dense_logic_launch(x, ca, cb, wa, wb, coef, node_kind, inv_tau):
    """The reference's separate-array form through ``slg_dense_logic_fwd``
    (gate16) / ``slg_warp_logic_fwd`` (walsh)."""
    require_gpu(x, ca, cb, wa, wb, coef)
    x = _as_f32(x)
    ca, cb = _c(ca, torch.int32), _c(cb, torch.int32)
    wa, wb, coef = _c(wa, torch.float32), _c(wb, torch.float32), _c(coef, torch.float32)
    B, IN = x.shape
    OUT, K = ca.shape
    if cb.shape != ca.shape or wa.shape != ca.shape or wb.shape != ca.shape or \
            coef.shape != (OUT, 4):
        raise ValueError("dense_logic: ca/cb/wa/wb must be [OUT,K] and coef [OUT,4]")
    y = torch.empty((B, OUT), device=x.device, dtype=torch.float32)
    if node_kind == GATE16:
        _lib.call("slg_dense_logic_fwd", _p(x), B, IN, OUT, K, _p(ca), _p(cb), _p(wa), _p(wb),
                  _p(coef), _p(y), _stream(x))
    elif node_kind == WALSH:
        _lib.call("slg_warp_logic_fwd", _p(x), B, IN, OUT, K, _p(ca), _p(cb), _p(wa), _p(wb),
                  _p(coef), float(inv_tau), _p(y), _stream(x))
    else:
        raise ValueError("dense_logic: node kind %d (gate16 or walsh)" % node_kind)
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


def fc_soft_bwd_supported(x, cand):
    """Whether the HIP backward takes ``x [B,IN]`` against ``cand [OUT,2,K]``."""
    B, IN = x.shape
    OUT, _, K = cand.shape
    return _lib.lib().slg_fc_soft_bwd_workspace(B, IN, OUT, K) >= 0


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


def fc_soft(x, cand, w, npar, node_kind, inv_tau=1.0):
    """``[B,IN] -> [B,OUT]`` soft FC layer (autograd-aware)."""
    require_gpu(x, cand, w, npar)
    if _grad_path(x, w, npar):
        return torch.ops.silogic_hip.fc_soft(x, cand, w, npar, node_kind, float(inv_tau))
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


def fc_lut_soft(x, cand, w, s, hybrid):
    """``[B,IN] -> [B,OUT]`` LUT layer (multilinear interpolation of ``s``, or
    the hybrid lookup), autograd-aware (the multilinear gradient)."""
    require_gpu(x, cand, w, s)
    if _grad_path(x, w, s):
        return torch.ops.silogic_hip.fc_lut_soft(x, cand, w, s, bool(hybrid))
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


def _check_rec(x, rec, in_dim, out_dim, K):
    if rec.dim() != 4 or tuple(rec.shape) != ((out_dim + 63) // 64, record_quads(K), 64, 4) or \
            rec.dtype != torch.float32 or not rec.is_contiguous():
        raise ValueError(f"fc_soft: records {tuple(rec.shape)} {rec.dtype} for OUT={out_dim}, K={K}")
    if x.dim() != 2:
        raise ValueError(f"fc_soft: x must be [B, IN], got {tuple(x.shape)}")
    check_width(x, in_dim)


def check_width(x, in_dim):
    """Raise when ``x`` [B, IN] is narrower than the layer's ``in_dim`` (the
    reference's ``x[:, cand]`` raises there; wider inputs are read as the
    reference reads them, by index)."""
    if x.shape[-1] < in_dim:
        raise ValueError(f"LogicLayer: input has {x.shape[-1]} features, the layer reads "
                         f"indices up to in_dim = {in_dim}")


def fc_soft_rec(x, rec, in_dim, out_dim, K, node_kind, inv_tau=1.0, tile=0, threads=0):
    """Soft FC layer on records built for ``in_dim`` inputs (no autograd):
    ``[B,IN] -> [B,OUT]``."""
    require_gpu(x, rec)
    x = _as_f32(x)
    _check_rec(x, rec, in_dim, out_dim, K)
    B, IN = x.shape
    y = torch.empty((B, out_dim), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_soft_fwd_records", _p(x), B, IN, out_dim, K, _p(rec), int(in_dim),
              node_kind, float(inv_tau), _p(y), int(tile), int(threads), _stream(x))
    return y


def fc_soft_groupsum_supported(B, IN, OUT, C):
    return bool(_lib.lib().slg_fc_soft_groupsum_supported(B, IN, OUT, C))


def fc_soft_rec_groupsum(x, rec, in_dim, out_dim, K, node_kind, inv_tau, C, tau):
    """Last soft layer fused with the STE GroupSum head: ``[B,IN] -> [B,C]``."""
    require_gpu(x, rec)
    x = _as_f32(x)
    _check_rec(x, rec, in_dim, out_dim, K)
    B, IN = x.shape
    logits = torch.empty((B, C), device=x.device, dtype=torch.float32)
    _lib.call("slg_fc_soft_fwd_groupsum", _p(x), B, IN, out_dim, K, _p(rec), int(in_dim),
              node_kind, float(inv_tau), int(C), float(tau), _p(logits), _stream(x))
    return logits


class SoftStackPlan:
    """Launches of a soft FC stack on records without gradients (the layers
    of one network, the last one fused with the STE GroupSum head when
    ``head`` is given), prepared once for a batch size and input width:
    a call allocates the activations and launches, nothing else.

    ``layers``: ``(rec, in_dim, out_dim, K, node_kind, inv_tau)`` per layer;
    ``head``: ``(C, tau)`` or None; ``wire_r``: wire residual width."""

    def __init__(self, layers, B, IN, head, wire_r):
        self.B, self.IN, self.wire_r = B, IN, wire_r
        self.layers = []
        width = IN
        for rec, in_dim, out_dim, K, kind, inv_tau in layers:
            require_gpu(rec)
            x_like = torch.empty((0, width), device=rec.device)
            _check_rec(x_like, rec, in_dim, out_dim, K)
            self.layers.append((rec, ctypes.c_void_p(rec.data_ptr()), int(width), int(in_dim),
                                int(out_dim), int(K), int(kind), float(inv_tau)))
            width = out_dim
        self.head = head
        self.fwd = _lib.lib().slg_fc_soft_fwd_records
        self.fwd_head = _lib.lib().slg_fc_soft_fwd_groupsum
        # narrow layers and a small batch: the whole stack in one launch
        # (slg_fc_soft_net_records), activations kept in LDS
        L = len(self.layers)
        kinds = {t[6] for t in self.layers}
        taus = {t[7] for t in self.layers}
        Ks = {t[5] for t in self.layers}
        out_arr = (ctypes.c_int64 * L)(*[t[4] for t in self.layers])
        C = head[0] if head is not None else 0
        self.net = None
        # which one-launch kernel (1: two LDS buffers, 2: one buffer, tiles
        # through every layer); 0: a launch per layer
        self.net_kind = 0
        if not wire_r and len(kinds) == 1 and len(taus) == 1 and len(Ks) == 1:
            self.net_kind = _lib.lib().slg_fc_soft_net_supported(B, IN, L, out_arr, Ks.pop(), C)
        if self.net_kind:
            self.net = ((ctypes.c_void_p * L)(*[t[1].value for t in self.layers]),
                        (ctypes.c_int64 * L)(*[t[3] for t in self.layers]), out_arr)
        self.fwd_net = _lib.lib().slg_fc_soft_net_records

    def __call__(self, x):
        """``x`` [B, IN] float32 -> the last layer's ``[B, OUT]`` activations, or
        the ``[B, C]`` logits when the head is fused."""
        if x.shape != (self.B, self.IN) or x.dtype != torch.float32 or not x.is_cuda:
            raise ValueError(f"soft stack planned for [{self.B}, {self.IN}] float32 input, "
                             f"got {tuple(x.shape)} {x.dtype}")
        h = x.contiguous()
        st = _stream(h)
        B, last = self.B, len(self.layers) - 1
        if self.net is not None:
            recs, ins, outs = self.net
            _, _, _, _, out_dim, K, kind, inv_tau = self.layers[-1]
            if self.head is not None:
                C, tau = self.head
                res = torch.empty((B, C), device=h.device, dtype=torch.float32)
            else:
                C, tau = 0, 1.0
                res = torch.empty((B, out_dim), device=h.device, dtype=torch.float32)
            _lib.check(self.fwd_net(_p(h), B, self.IN, last + 1, recs, ins, outs, K, kind,
                                    inv_tau, C, float(tau), _p(res), st),
                       "slg_fc_soft_net_records")
            return res
        for i, (_, rec_p, width, in_dim, out_dim, K, kind, inv_tau) in enumerate(self.layers):
            if i == last and self.head is not None:
                C, tau = self.head
                logits = torch.empty((B, C), device=h.device, dtype=torch.float32)
                _lib.check(self.fwd_head(_p(h), B, width, out_dim, K, rec_p, in_dim, kind,
                                         inv_tau, C, tau, _p(logits), st),
                           "slg_fc_soft_fwd_groupsum")
                return logits
            y = torch.empty((B, out_dim), device=h.device, dtype=torch.float32)
            _lib.check(self.fwd(_p(h), B, width, out_dim, K, rec_p, in_dim, kind, inv_tau, _p(y),
                                0, 0, st), "slg_fc_soft_fwd_records")
            if self.wire_r and width == out_dim:
                y = torch.cat([h[:, :self.wire_r], y[:, self.wire_r:]], dim=1)
            h = y
        return h


# ---------------------------------------------------------------------------
# GroupSum / OrPool
# ---------------------------------------------------------------------------
def groupsum_soft_launch(x, C, tau, ste):
    require_gpu(x)
    x = _as_f32(x)
    B, W = x.shape
    out = torch.empty((B, C), device=x.device, dtype=torch.float32)
    _lib.call("slg_groupsum_soft", _p(x), B, W, C, float(tau), int(bool(ste)), _p(out),
              _stream(x))
    return out


def groupsum_soft(x, C, tau, ste):
    require_gpu(x)
    if _grad_path(x):
        return torch.ops.silogic_hip.groupsum_soft(x, int(C), float(tau), bool(ste))
    return groupsum_soft_launch(x, C, tau, ste)


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


def orpool_launch(x, size=2):
    dtype = 1 if x.dtype == torch.uint8 else 0
    x = x.contiguous() if dtype == 1 else _as_f32(x)
    B, Cc, H, W = x.shape
    out = torch.empty((B, Cc, H // size, W // size), device=x.device, dtype=x.dtype)
    _lib.call("slg_orpool", _p(x), dtype, B, Cc, H, W, int(size), _p(out), _stream(x))
    return out


def orpool(x, size=2):
    """``size`` x ``size`` OR (max) pool with stride ``size`` and floor."""
    require_gpu(x)
    if x.dtype == torch.bool:
        x = x.to(torch.uint8)
    if x.is_floating_point() and _grad_path(x):
        return torch.ops.silogic_hip.orpool(x, int(size))
    return orpool_launch(x, size)


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


def fc_hard_place_net(codes):
    """Bank-aware placement of a fused network's compact codes
    (``slg_fc_hard_place_net``): every layer but the last becomes
    ``round_up(OUT, 32)`` slots with the next layer's operands renamed; the
    logits of ``fc_hard_net`` are unchanged. Returns the placed codes."""
    require_gpu(*codes)
    if any(c.dim() != 1 or c.dtype != torch.int32 for c in codes):
        raise ValueError("fc_hard_place_net: codes must be compact [OUT] int32 codes")
    codes = [c.contiguous() for c in codes]
    L = len(codes)
    widths = [c.shape[0] for c in codes]
    dev = codes[0].device
    placed = [torch.empty(((w + 31) // 32 * 32 if l + 1 < L else w,), device=dev,
                          dtype=torch.int32) for l, w in enumerate(widths)]
    n_ws = max(1, sum(widths[:-1]))
    ws = torch.empty(n_ws, device=dev, dtype=torch.int32)
    _lib.call("slg_fc_hard_place_net", L, (ctypes.c_int64 * L)(*widths), _ptrs(codes),
              _ptrs(placed), _p(ws), n_ws, _stream(codes[0]))
    return placed


def fc_hard_type_slots(in_dim, widths):
    """Slots per layer of the type-uniform layout (0: it does not apply)."""
    arr = (ctypes.c_int64 * len(widths))(*widths)
    return _lib.lib().slg_fc_hard_type_slots(in_dim, len(widths), arr)


def fc_hard_type_place_net(codes, in_dim):
    """Type-uniform placement of a fused network's compact codes
    (``slg_fc_hard_type_place_net``) for inputs ``in_dim`` wide:
    every layer but the last becomes ``fc_hard_type_slots`` slots whose first
    rows hold one gate type per wave, with the next layer's operands renamed;
    the logits of ``fc_hard_net`` are unchanged. Returns a :class:`NetCodes`
    carrying the plan."""
    require_gpu(*codes)
    if any(c.dim() != 1 or c.dtype != torch.int32 for c in codes):
        raise ValueError("fc_hard_type_place_net: codes must be compact [OUT] int32 codes")
    codes = [c.contiguous() for c in codes]
    L = len(codes)
    widths = [c.shape[0] for c in codes]
    S = fc_hard_type_slots(in_dim, widths)
    if S <= 0:
        raise ValueError("fc_hard_type_place_net: the type-uniform layout does not apply to "
                         "inputs %d wide and widths %s" % (in_dim, widths))
    dev = codes[0].device
    placed = [torch.empty((S,), device=dev, dtype=torch.int32) for _ in widths]
    plan = torch.empty((L, 20), device=dev, dtype=torch.int32)
    w_arr = (ctypes.c_int64 * L)(*widths)
    n_ws = _lib.lib().slg_fc_hard_type_place_workspace(L, w_arr)
    ws = torch.empty(n_ws, device=dev, dtype=torch.int32)
    _lib.call("slg_fc_hard_type_place_net", L, in_dim, w_arr,
              _ptrs(codes), _ptrs(placed), _p(plan), _p(ws), n_ws, _stream(codes[0]))
    return NetCodes(placed, plan=plan, in_dim=in_dim, widths=widths)


class NetCodes(list):
    """Compact per-layer codes of a fused hard network (a list of ``[OUT]``
    int32 tensors) with their width and pointer arrays for the C ABI, built
    once: the tensors must not be replaced or resized afterwards. ``plan``
    (with the ``in_dim`` it was placed for) marks codes laid out by
    :func:`fc_hard_type_place_net`, which the network kernels read without a
    wire residual."""

    def __init__(self, codes, plan=None, in_dim=None, widths=None):
        super().__init__(codes)
        require_gpu(*self)
        if any(c.dim() != 1 or c.dtype != torch.int32 or not c.is_contiguous() for c in self):
            raise ValueError("fc_hard_net: codes must be compact [OUT] int32 codes")
        widths = widths if widths is not None else [c.shape[0] for c in self]
        self.widths = (ctypes.c_int64 * len(self))(*widths)
        self.ptrs = (ctypes.c_void_p * len(self))(*[c.data_ptr() for c in self])
        self.plan, self.in_dim = plan, in_dim


def fc_hard_net(x, in_kind, B, in_dim, codes, C, wire_r=0):
    """Depth-fused packed FC network + GroupSum -> logits ``[B, C]``.

    ``in_kind``: ROWS_F32 / ROWS_U8 ([B, in_dim], packed inside the kernel),
    PACKED ([in_dim, nw]) or PACKED_WORD_MAJOR ([nw, in_dim]). ``codes``:
    compact per-layer codes from ``fc_hard_codes_net(..., compact=True)``
    (a list of tensors, or a :class:`NetCodes`)."""
    if not isinstance(codes, NetCodes):
        codes = NetCodes(codes)
    require_gpu(x)
    w_arr, c_arr = codes.widths, codes.ptrs
    out = torch.empty((B, C), device=x.device, dtype=torch.float32)
    if codes.plan is not None:
        if wire_r or in_dim != codes.in_dim:
            raise ValueError("fc_hard_net: type-placed codes take inputs %s wide and no "
                             "wire residual" % codes.in_dim)
        _lib.call("slg_fc_hard_net_typed", _p(x), in_kind, B, in_dim, len(codes), w_arr, c_arr,
                  _p(codes.plan), C, _p(out), _stream(x))
        return out
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


def tree_shape(node_kind, depth, arity):
    """``(leaves, nodes, params per node)`` of a conv node tree: binary
    gate16 / walsh trees (4 coefficients a node) or arity-n LUT trees (2^n
    values a node)."""
    a = 2 if node_kind in (GATE16, WALSH) else arity
    leaves = a ** depth
    nodes = (leaves - 1) // (a - 1)
    return leaves, nodes, 4 if node_kind in (GATE16, WALSH) else 2 ** a


def conv_param_shapes(node_kind, depth, arity, N):
    """Accepted node-parameter shapes: ``[N, nodes, P]``, and for a depth-1
    LUT also ``[N, 2^arity]``."""
    _, nodes, P = tree_shape(node_kind, depth, arity)
    shapes = [(N, nodes, P)]
    if node_kind not in (GATE16, WALSH) and depth == 1:
        shapes.append((N, P))
    return shapes


def _conv_soft_launch(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
    B, Cc, H, W = x.shape
    N = cm.shape[0]
    leaves, _, _ = tree_shape(node_kind, depth, arity)
    if (cm.shape != (N, leaves, K) or ch.shape != cm.shape or cw.shape != cm.shape
            or w.shape != cm.shape
            or tuple(npar.shape) not in conv_param_shapes(node_kind, depth, arity, N)):
        raise ValueError("conv_soft: tap / weight / node parameter shapes are inconsistent")
    kern = 2 * pad + 1
    Hf, Wf = H + 2 * pad - kern + 1, W + 2 * pad - kern + 1
    Ho, Wo = (Hf // 2, Wf // 2) if pool else (Hf, Wf)
    out = torch.empty((B, N, Ho, Wo), device=x.device, dtype=torch.float32)
    if B > 0 and node_kind in (GATE16, MULTILINEAR2, HYBRID) and \
            conv_fits_lds((Cc, H, W), pad, pool, node_kind, depth, arity, K):
        # records built from these arrays, then the records kernels: the same
        # bits as slg_conv_soft_fwd, with the per-channel parameter work done
        # once per channel instead of once per workgroup and chunk
        R = _lib.lib().slg_conv_soft_record_floats(node_kind, depth, arity, K, int(bool(pool)))
        rec = torch.empty((N, R), device=x.device, dtype=torch.float32)
        st = _stream(x)
        _lib.call("slg_conv_soft_records_arrays", _p(npar), _p(w), _p(cm), _p(ch), _p(cw), N, K,
                  node_kind, depth, arity, Cc, H, W, pad, int(bool(pool)), _p(rec), st)
        _lib.call("slg_conv_soft_fwd_records", _p(x), B, Cc, H, W, N, node_kind, depth, arity, K,
                  _p(rec), pad, int(bool(pool)), _p(out), st)
        return out
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
    """Differentiable torch expression of the fused conv op (backward only),
    for the trees the LDS kernels take (gate16 trees, depth-1 LUTs)."""
    if node_kind == WALSH or (node_kind != GATE16 and depth != 1):
        raise NotImplementedError("conv_soft_torch: gate16 trees and depth-1 LUTs")
    npar = npar.reshape(npar.shape[0], -1, 4) if node_kind == GATE16 else \
        npar.reshape(npar.shape[0], -1)
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


def conv_soft_bwd_supported(x, cm, node_kind, depth, arity, K, pad, pool):
    """Whether the HIP backward takes this conv layer shape."""
    B, Cc, H, W = x.shape
    return _lib.lib().slg_conv_soft_bwd_workspace(B, Cc, H, W, cm.shape[0], node_kind, depth,
                                                  arity, K, pad, int(bool(pool))) >= 0


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


def conv_soft(x, npar, w, cm, ch, cw, node_kind, depth, arity, K, pad, pool):
    require_gpu(x, npar, w, cm)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    if _grad_path(x, w, npar):
        return torch.ops.silogic_hip.conv_soft(x, npar, w, cm, ch, cw, int(node_kind), int(depth),
                                    int(arity), int(K), int(pad), bool(pool))
    return _conv_soft_launch(_as_f32(x), _c(npar, torch.float32), _c(w, torch.float32), cm, ch,
                             cw, node_kind, depth, arity, K, pad, pool)


def tree_conv_launch(x, coef, w, cm, ch, cw, depth, K, pad):
    """The reference's tree_conv / tree_conv_topk form through
    ``slg_tree_conv_fwd`` (gate16 tree, stride 1, 'same' padding)."""
    require_gpu(x, coef, w, cm)
    x = _as_f32(x)
    coef, w = _c(coef, torch.float32), _c(w, torch.float32)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    B, Cc, H, W = x.shape
    N = cm.shape[0]
    leaves = 2 ** depth
    if cm.shape != (N, leaves, K) or ch.shape != cm.shape or cw.shape != cm.shape or \
            w.shape != cm.shape or tuple(coef.shape) != (N, leaves - 1, 4):
        raise ValueError("tree_conv: coef [N,2^d-1,4] and w/cm/ch/cw [N,2^d,K] expected")
    out = torch.empty((B, N, H, W), device=x.device, dtype=torch.float32)
    _lib.call("slg_tree_conv_fwd", _p(x), B, Cc, H, W, N, int(depth), int(K), _p(coef), _p(w),
              _p(cm), _p(ch), _p(cw), 1, int(pad), H, W, _p(out), _stream(x))
    return out


def conv_fits_lds(chw, pad, pool, node_kind, depth, arity, K):
    """True when the LDS-staged conv kernels (and the records forward) take
    images of shape ``chw``; the others run on the generic kernels."""
    C, H, W = chw
    return bool(_lib.lib().slg_conv_soft_lds_fit(C, H, W, node_kind, depth, arity, K, pad,
                                                 int(bool(pool))))


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


def conv_tree_hard_prep(cm, ch, cw, conn, levels, node_kind, depth, arity):
    """Hard parameters of any conv node tree: ``(leaf [N, leaves] int32,
    tables [N, nodes] int64)``; ``levels`` holds each tree level's parameters
    as the module stores them (gate16 logits [N, m, 16], walsh theta
    [N*m, 4], LUT logits [N*m, 2^arity])."""
    require_gpu(cm, *levels)
    cm, ch, cw = _c(cm, torch.int32), _c(ch, torch.int32), _c(cw, torch.int32)
    N, leaves, K = cm.shape
    want_leaves, nodes, _ = tree_shape(node_kind, depth, arity)
    if leaves != want_leaves or len(levels) != depth or ch.shape != cm.shape or \
            cw.shape != cm.shape or (conn is not None and tuple(conn.shape) != (N, leaves, K)):
        raise ValueError("conv_tree_hard_prep: tap / level shapes do not match the tree")
    a = 2 if node_kind in (GATE16, WALSH) else arity
    for i, t in enumerate(levels):
        m = a ** (depth - 1 - i)
        want = {GATE16: (N, m, 16), WALSH: (N * m, 4)}.get(node_kind, (N * m, 2 ** a))
        if tuple(t.shape) != want:
            raise ValueError(f"conv_tree_hard_prep: level {i} parameters {tuple(t.shape)}, "
                             f"expected {want}")
    levels = [_c(t.detach(), torch.float32) for t in levels]
    leaf = torch.empty((N, leaves), device=cm.device, dtype=torch.int32)
    tables = torch.empty((N, nodes), device=cm.device, dtype=torch.int64)
    conn = None if conn is None else _c(conn.detach(), torch.float32)
    _lib.call("slg_conv_tree_hard_prep", _p(cm), _p(ch), _p(cw), _p(conn), N, K, node_kind,
              depth, arity, _ptrs(levels), _p(leaf), _p(tables), _stream(cm))
    return leaf, tables


def conv_tree_hard(xp, shape_chw, leaf, tables, arity, depth, kernel, pad, pool):
    """Packed node tree: ``xp`` [C,H,W,nw] -> [N,Ho,Wo,nw] (OR-pooled if ``pool``)."""
    require_gpu(xp, leaf, tables)
    Cc, H, W = shape_chw
    nw = xp.shape[-1]
    N = leaf.shape[0]
    if xp.numel() != Cc * H * W * nw or leaf.shape != (N, arity ** depth) or \
            tables.shape != (N, (arity ** depth - 1) // (arity - 1)):
        raise ValueError("conv_tree_hard: packed input / leaf / table shapes are inconsistent")
    Hf, Wf = H + 2 * pad - kernel + 1, W + 2 * pad - kernel + 1
    Ho, Wo = (Hf // 2, Wf // 2) if pool else (Hf, Wf)
    out = torch.empty((N, Ho, Wo, nw), device=xp.device, dtype=torch.int64)
    if out.numel():
        _lib.call("slg_conv_tree_hard_fwd", _p(_c(xp)), Cc, H, W, nw, N, arity, depth, _p(leaf),
                  _p(tables), kernel, pad, int(bool(pool)), _p(out), _stream(xp))
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


def pack_image_wm(x, pad):
    """``[B, C, H, W]`` images (fp32 or uint8) -> word-major packed words
    ``[nw, C, H + 2 pad, W + 2 pad]`` with a zero border (``slg_pack_image_wm``
    writes the interior into a zeroed buffer)."""
    require_gpu(x)
    x, kind = _in_kind(x)
    if x.dim() != 4:
        raise ValueError("pack_image_wm: x must be [B, C, H, W], got %s" % (tuple(x.shape),))
    B, C, H, W = x.shape
    xp = torch.zeros((n_words(B), C, H + 2 * pad, W + 2 * pad), device=x.device, dtype=torch.int64)
    _lib.call("slg_pack_image_wm", _p(x), kind, B, C, H, W, pad, _p(xp), _stream(x))
    return xp


def conv_hard_wm(xp, B, shape_chw, leaf, tt, node_kind, depth, arity, kernel, pad, out_pad=0):
    """Pooled packed conv on zero-bordered word-major words: ``xp``
    [nw, C, H + 2 pad, W + 2 pad] -> [nw, N, Ho + 2 out_pad, Wo + 2 out_pad]
    with a zero border (``slg_conv_hard_fwd_wm`` writes the interior of a
    zeroed buffer)."""
    require_gpu(xp, leaf, tt)
    Cc, H, W = shape_chw
    nw = n_words(B)
    N = leaf.shape[0]
    leaves = 2 ** depth if node_kind == GATE16 else arity
    if (tuple(xp.shape) != (nw, Cc, H + 2 * pad, W + 2 * pad) or not xp.is_contiguous()
            or leaf.shape != (N, leaves) or tt.shape != (N,)):
        raise ValueError("conv_hard_wm: packed input / leaf / truth-table shapes are inconsistent")
    Ho, Wo = (H + 2 * pad - kernel + 1) // 2, (W + 2 * pad - kernel + 1) // 2
    out = torch.zeros((nw, N, Ho + 2 * out_pad, Wo + 2 * out_pad), device=xp.device,
                      dtype=torch.int64)
    _lib.call("slg_conv_hard_fwd_wm", _p(xp), B, Cc, H, W, N, node_kind, depth, arity, _p(leaf),
              _p(tt), kernel, pad, _p(out), out_pad, _stream(xp))
    return out


def conv_hard_head_wm(xp, B, shape_chw, leaf, tt, node_kind, depth, arity, kernel, pad, codes,
                      C):
    """The last pooled conv block and a one-layer head + GroupSum in one
    launch (``slg_conv_hard_head_wm``): ``xp`` as for :func:`conv_hard_wm`,
    ``codes`` the head's compact codes on the block's ``N * Ho * Wo``
    outputs (a list of one tensor, or a one-layer :class:`NetCodes`, type-
    placed or not). Returns logits ``[B, C]``, the class counts of
    ``conv_hard_wm`` followed by ``fc_hard_net`` on its output."""
    if not isinstance(codes, NetCodes):
        codes = NetCodes(codes)
    require_gpu(xp, leaf, tt)
    Cc, H, W = shape_chw
    N = leaf.shape[0]
    leaves = 2 ** depth if node_kind == GATE16 else arity
    if (tuple(xp.shape) != (n_words(B), Cc, H + 2 * pad, W + 2 * pad) or not xp.is_contiguous()
            or leaf.shape != (N, leaves) or tt.shape != (N,) or len(codes) != 1):
        raise ValueError("conv_hard_head_wm: packed input / leaf / truth-table / codes shapes "
                         "are inconsistent")
    in_dim = N * ((H + 2 * pad - kernel + 1) // 2) * ((W + 2 * pad - kernel + 1) // 2)
    if codes.plan is not None and codes.in_dim != in_dim:
        raise ValueError("conv_hard_head_wm: type-placed codes take inputs %s wide, the block "
                         "gives %d" % (codes.in_dim, in_dim))
    out = torch.empty((B, C), device=xp.device, dtype=torch.float32)
    plan = _p(codes.plan) if codes.plan is not None else None
    _lib.call("slg_conv_hard_head_wm", _p(xp), B, Cc, H, W, N, node_kind, depth, arity, _p(leaf),
              _p(tt), kernel, pad, int(codes.widths[0]), codes.ptrs[0], plan, C, _p(out),
              _stream(xp))
    return out


def conv_hard_net_wm(xp, B, shape_chw, leaf, tt, node_kind, depth, arity, kernel, pad, codes, C):
    """The last pooled conv block and a whole fused head network + GroupSum
    in one launch (``slg_conv_hard_net_wm``): arguments as
    :func:`conv_hard_head_wm`, ``codes`` the head's compact per-layer codes
    (a list, or a :class:`NetCodes`, type-placed or not; no wire residual).
    Returns logits ``[B, C]``, those of ``conv_hard_wm`` followed by
    ``fc_hard_net`` on its output."""
    if not isinstance(codes, NetCodes):
        codes = NetCodes(codes)
    require_gpu(xp, leaf, tt)
    Cc, H, W = shape_chw
    N = leaf.shape[0]
    leaves = 2 ** depth if node_kind == GATE16 else arity
    if (tuple(xp.shape) != (n_words(B), Cc, H + 2 * pad, W + 2 * pad) or not xp.is_contiguous()
            or leaf.shape != (N, leaves) or tt.shape != (N,)):
        raise ValueError("conv_hard_net_wm: packed input / leaf / truth-table shapes are "
                         "inconsistent")
    in_dim = N * ((H + 2 * pad - kernel + 1) // 2) * ((W + 2 * pad - kernel + 1) // 2)
    if codes.plan is not None and codes.in_dim != in_dim:
        raise ValueError("conv_hard_net_wm: type-placed codes take inputs %s wide, the block "
                         "gives %d" % (codes.in_dim, in_dim))
    out = torch.empty((B, C), device=xp.device, dtype=torch.float32)
    plan = _p(codes.plan) if codes.plan is not None else None
    _lib.call("slg_conv_hard_net_wm", _p(xp), B, Cc, H, W, N, node_kind, depth, arity, _p(leaf),
              _p(tt), kernel, pad, len(codes), codes.widths, codes.ptrs, plan, C, _p(out),
              _stream(xp))
    return out


# the custom operators the autograd paths above dispatch to (library.py uses
# this module's launch helpers, so it is imported once they are defined)
from . import library as _library  # noqa: E402,F401
