"""Numpy restatement of the reference's bit-packed hard inference.

Layout (silogic/bitpacking/ops.py:1-49): activations are ``[dim, nw]`` int64
with ``nw = ceil(B/64)``; sample ``b`` is bit ``b % 64`` of word ``b // 64``
(little-endian, so the same bytes read as ``[dim, 2*nw]`` uint32 put sample b
at bit ``b % 32`` of uint32 word ``b // 32``). Conv activations are
B-packed ``[C, H*W, nw]`` (packed_layer.py:1-16).

Hard parameters are extracted from a reference ``state_dict`` the way
silogic/bitpacking/convert.py does: argmax wiring (61-73), gate16 types by
argmax (78-81), Walsh arity-2 -> gate16 by corner signs (84-97), multilinear
arity-2 -> gate16 with address bits 1 and 2 swapped (126-136), n-input LUT
truth tables (100-123).

Test infrastructure only (see :mod:`oracle`).
"""
import numpy as np
import torch

from . import torch_ref


def n_words(B):
    """64-bit words for B samples (ops.py:27-29)."""
    return (B + 63) >> 6


def pack_bits(x):
    """``[B, dim]`` {0,1} -> ``[dim, nw]`` int64 (ops.py:32-49)."""
    x = np.asarray(x)
    B, dim = x.shape
    nw = n_words(B)
    pad = nw * 64 - B
    if pad:
        x = np.concatenate([x, np.zeros((pad, dim), dtype=x.dtype)], axis=0)
    xt = np.ascontiguousarray(x.T.astype(np.uint8))
    return np.ascontiguousarray(np.packbits(xt, axis=1, bitorder="little")).view(np.int64)


def unpack_bits(packed, B):
    """``[dim, nw]`` int64 -> ``[B, dim]`` uint8 (ops.py:52-63)."""
    bits = np.unpackbits(np.ascontiguousarray(packed).view(np.uint8), axis=1,
                         bitorder="little")
    return np.ascontiguousarray(bits[:, :B].T).astype(np.uint8)


def mask_last_word(packed, B):
    """Zero the padding bits of the last word (ops.py:107-115)."""
    r = B % 64
    if r:
        packed[:, -1] &= np.int64((1 << r) - 1)
    return packed


def group_sum_packed(xp, B, C):
    """Per-class popcounts ``[B, C]`` float32 from packed ``[W, nw]``.

    The reference divides by tau here (ops.py:66-104); this returns the raw
    counts, which is what ``GroupSum.forward_hard`` returns (heads.py:41-45).
    """
    W = xp.shape[0]
    g = W // C
    out = np.empty((B, C), dtype=np.float32)
    for c in range(C):
        bits = np.unpackbits(np.ascontiguousarray(xp[c * g:(c + 1) * g]).view(np.uint8),
                             axis=1, bitorder="little")
        out[:, c] = bits[:, :B].sum(axis=0, dtype=np.int64).astype(np.float32)
    return out


# the 16 gates on packed words, gate order of the basis table (ops.py:123-140)
GATE_OPS = [
    lambda a, b: np.zeros_like(a), lambda a, b: a & b, lambda a, b: a & ~b,
    lambda a, b: a.copy(), lambda a, b: ~a & b, lambda a, b: b.copy(),
    lambda a, b: a ^ b, lambda a, b: a | b, lambda a, b: ~(a | b),
    lambda a, b: ~(a ^ b), lambda a, b: ~b, lambda a, b: a | ~b,
    lambda a, b: ~a, lambda a, b: ~a | b, lambda a, b: ~(a & b),
    lambda a, b: np.full_like(a, np.int64(-1)),
]


def code_to_gate16():
    """4-bit truth-table code -> gate index; code bit k = output at address k
    = (a<<1)|b (ops.py:148-165)."""
    tt = torch_ref.TRUTH.numpy()
    lut = np.zeros(16, dtype=np.int32)
    for g in range(16):
        code = int(tt[g, 0]) | (int(tt[g, 1]) << 1) | (int(tt[g, 2]) << 2) | (int(tt[g, 3]) << 3)
        lut[code] = g
    return lut


def gate_codes(L, sd):
    """``[out]`` gate16 index of an arity-2 FC layer (convert.py:170-217)."""
    p = L["prefix"]
    if L["node"] == "gate16":
        return sd[p + "node.gate_logits"].argmax(dim=1).numpy().astype(np.int32)
    if L["node"] == "walsh":
        return walsh2_gates(sd[p + "node.theta"].numpy())
    tt = (sd[p + "node.logits"].numpy() > 0).astype(np.int32)
    code = tt[:, 0] | (tt[:, 2] << 1) | (tt[:, 1] << 2) | (tt[:, 3] << 3)
    return code_to_gate16()[code]


def walsh2_gates(t):
    """Arity-2 walsh theta ``[rows, 4]`` -> gate16 index: the sign of z at the
    four corners, as the converter evaluates it (convert.py:84-97)."""
    t0, t1, t2, t3 = t[:, 0], t[:, 1], t[:, 2], t[:, 3]
    b0 = (t0 - t1 - t2 + t3) > 0
    b1 = (t0 - t1 + t2 - t3) > 0
    b2 = (t0 + t1 - t2 - t3) > 0
    b3 = (t0 + t1 + t2 + t3) > 0
    code = (b0.astype(np.int32) | (b1.astype(np.int32) << 1)
            | (b2.astype(np.int32) << 2) | (b3.astype(np.int32) << 3))
    return code_to_gate16()[code]


def walsh_truth(theta, n):
    """``[rows, 2^n]`` truth tables of n-input walsh nodes: the node's own hard
    rule evaluated at each corner (``_lut_truth_tables``, convert.py:100-123,
    calling WalshNode.forward_hard, nodes.py:152-156)."""
    theta = torch.as_tensor(theta)
    rows = theta.shape[0]
    cols = []
    for p in range(2 ** n):
        corner = torch.tensor([(p >> j) & 1 for j in range(n)], dtype=torch.float32)
        u = (2 * corner - 1).view(1, 1, n).expand(1, rows, n)
        z = (torch_ref.walsh_monomials(u) * theta[None]).sum(2)
        cols.append((z > 0)[0])
    return torch.stack(cols, dim=1).numpy()


def fc_layer(L, sd, xp):
    """Packed arity-2 FC layer: ``out[o] = gate_o(x[a_o], x[b_o])``
    (packed_layer.py:85-116)."""
    idx = torch_ref.hard_indices(L, sd).numpy().astype(np.int64)
    gates = gate_codes(L, sd)
    out = np.empty((idx.shape[0], xp.shape[1]), dtype=np.int64)
    for g in range(16):
        sel = np.where(gates == g)[0]
        if len(sel):
            out[sel] = GATE_OPS[g](xp[idx[sel, 0]], xp[idx[sel, 1]])
    return out


def lut_truth(logits):
    """``[rows, 2^n]`` bool truth tables ``logits > 0`` (nodes.py:188)."""
    return (np.asarray(logits) > 0)


def lut_eval(tt, inputs):
    """Sum-of-products LUT on packed words (packed_layer.py:121-178).

    ``tt``: ``[rows, 2^n]`` bool; ``inputs``: list of n arrays ``[rows, ...]``
    int64, input j = address bit j.
    """
    n = len(inputs)
    out = np.zeros_like(inputs[0])
    for e in range(2 ** n):
        on = tt[:, e]
        if not on.any():
            continue
        m = np.full_like(inputs[0], np.int64(-1))
        for j in range(n):
            m &= inputs[j] if (e >> j) & 1 else ~inputs[j]
        out[on] |= m[on]
    return out


def pack_conv_input(x):
    """``[B,C,H,W]`` {0,1} -> ``[C, H*W, nw]`` int64 (packed_layer.py:184-214)."""
    x = np.asarray(x)
    B, C, H, W = x.shape
    flat = np.ascontiguousarray(x.reshape(B, C * H * W))
    return pack_bits(flat).reshape(C, H * W, -1)


def packed_unfold(x3, k, stride, pad, H, W):
    """``[C, L_in, nw] -> [C*k*k, L_out, nw]`` with zero padding
    (packed_layer.py:224-283); row order ``c*k*k + dy*k + dx`` as F.unfold."""
    C, L_in, nw = x3.shape
    Ho = (H + 2 * pad - k) // stride + 1
    Wo = (W + 2 * pad - k) // stride + 1
    oy = np.arange(Ho * Wo) // Wo
    ox = np.arange(Ho * Wo) % Wo
    c_arr = np.arange(C).repeat(k * k)
    dy = np.tile(np.arange(k).repeat(k), C)
    dx = np.tile(np.arange(k), C * k)
    iy = oy[None, :] * stride - pad + dy[:, None]
    ix = ox[None, :] * stride - pad + dx[:, None]
    ok = (iy >= 0) & (iy < H) & (ix >= 0) & (ix < W)
    l_in = np.where(ok, iy * W + ix, L_in)
    xpad = np.concatenate([x3, np.zeros((C, 1, nw), dtype=np.int64)], axis=1)
    return xpad[c_arr[:, None], l_in, :]


def packed_or_pool(x3, H, W):
    """2x2 OR pool on ``[C, H*W, nw]`` with floor (packed_layer.py:286-319)."""
    C, _, nw = x3.shape
    Ho, Wo = H // 2, W // 2
    oy = np.arange(Ho * Wo) // Wo
    ox = np.arange(Ho * Wo) % Wo
    out = np.zeros((C, Ho * Wo, nw), dtype=np.int64)
    for dy in range(2):
        for dx in range(2):
            out |= x3[:, (oy * 2 + dy) * W + (ox * 2 + dx), :]
    return out


def conv_block(blk, sd, x3, H, W):
    """Packed ConvLogicTree forward on ``[C, H*W, nw]`` (packed_layer.py:324-540)."""
    p = blk["prefix"]
    un = packed_unfold(x3, blk["kernel"], blk["stride"], blk["padding"], H, W)
    if blk["connect"] == "fixed":
        leaf = sd[p + "leaf_idx"].numpy()
    else:
        sel = sd[p + "conn"].argmax(dim=2)
        leaf = torch.gather(sd[p + "leaf_cand"], 2, sel.unsqueeze(-1)).squeeze(-1).numpy()
    n, leaves = leaf.shape
    cur = un[leaf.reshape(-1)].reshape(n, leaves, un.shape[1], un.shape[2])
    if blk["node"] == "gate16":
        for i in range(blk["depth"]):
            gates = sd[f"{p}gate_logits.{i}"].argmax(dim=2).numpy()   # [n, nodes]
            a, b = cur[:, 0::2], cur[:, 1::2]
            res = np.empty_like(a)
            for g in range(16):
                oi, ni = np.where(gates == g)
                if len(oi):
                    res[oi, ni] = GATE_OPS[g](a[oi, ni], b[oi, ni])
            cur = res
        return cur[:, 0]
    if blk["node"] == "walsh":   # tree nodes as gate16 (convert.py:141-165)
        for i in range(blk["depth"]):
            m = cur.shape[1] // 2
            gates = walsh2_gates(sd[f"{p}tree_nodes.{i}.theta"].numpy()).reshape(n, m)
            a, b = cur[:, 0::2], cur[:, 1::2]
            res = np.empty_like(a)
            for g in range(16):
                oi, ni = np.where(gates == g)
                if len(oi):
                    res[oi, ni] = GATE_OPS[g](a[oi, ni], b[oi, ni])
            cur = res
        return cur[:, 0]
    k = blk["node_arity"]
    for i in range(blk["depth"]):
        m = cur.shape[1] // k
        tt = lut_truth(sd[f"{p}tree_nodes.{i}.logits"].numpy()).reshape(n, m, -1)
        res = np.empty((n, m) + cur.shape[2:], dtype=np.int64)
        for mi in range(m):
            ins = [cur[:, mi * k + j] for j in range(k)]
            res[:, mi] = lut_eval(tt[:, mi], ins)
        cur = res
    return cur[:, 0]


def forward_hard(spec, sd, x):
    """Hard logits (raw popcounts, as ``forward_hard``) via the packed path."""
    st = torch_ref.structure(spec)
    x = np.asarray(x)
    B = x.shape[0]
    xb = (x.astype(np.float32) >= 1.0).astype(np.uint8) if x.dtype != np.uint8 else x
    if st["kind"] == "fc":
        xp = pack_bits(xb)
        wire_r = st.get("wire_r", 0)
        for L in st["layers"]:
            prev = xp
            xp = _fc_any(L, sd, xp)
            if wire_r and prev.shape[0] == xp.shape[0]:   # packed_model.py:104-108
                xp[:wire_r] = prev[:wire_r]
    else:
        _, C, H, W = xb.shape
        x3 = pack_conv_input(xb)
        wr = st.get("wire_residual", 0.0)
        for blk in st["blocks"]:
            y = conv_block(blk, sd, x3, H, W)
            if wr > 0:   # same-size conv: copy input channels before the pool (221-227)
                r = min(int(blk["n"] * wr), x3.shape[0])
                if r > 0:
                    y[:r] = x3[:r, :H * W]
            x3 = packed_or_pool(y, H, W)
            H, W = H // 2, W // 2
        xp = x3.reshape(-1, x3.shape[2])
        for L in st["head_layers"]:
            xp = _fc_any(L, sd, xp)
    mask_last_word(xp, B)
    return group_sum_packed(xp, B, st["head"]["C"])


def _fc_any(L, sd, xp):
    if L["arity"] == 2:
        return fc_layer(L, sd, xp)
    idx = torch_ref.hard_indices(L, sd).numpy()
    if L["node"] == "walsh":
        tt = walsh_truth(sd[L["prefix"] + "node.theta"], L["arity"])
    else:
        tt = lut_truth(sd[L["prefix"] + "node.logits"].numpy())
    return lut_eval(tt, [xp[idx[:, j]] for j in range(idx.shape[1])])
