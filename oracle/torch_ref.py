"""The reference's pure-PyTorch CPU path, restated as functions of
``(spec, state_dict, x)``.

Each function follows the reference op-for-op (same torch calls, same order),
so on the same torch build its fp32 results are the reference's results. It
holds no parameters of its own: the parameters come from a ``state_dict``
whose keys are the reference's keys. A ``spec`` is ``(ctor_name, kwargs)`` as
passed to the reference constructor; :func:`structure` expands the defaults
the reference constructors apply.

Test infrastructure only (see :mod:`oracle`).
"""
import torch
import torch.nn.functional as F

# silogic/functional.py:24-44 — the 16 two-input functions in the {1,A,B,AB}
# basis, rows in the standard DiffLogic order. A table that must be identical.
BASIS = torch.tensor([
    [0, 0, 0, 0], [0, 0, 0, 1], [0, 1, 0, -1], [0, 1, 0, 0],
    [0, 0, 1, -1], [0, 0, 1, 0], [0, 1, 1, -2], [0, 1, 1, -1],
    [1, -1, -1, 1], [1, -1, -1, 2], [1, 0, -1, 0], [1, 0, -1, 1],
    [1, -1, 0, 0], [1, -1, 0, 1], [1, 0, 0, -1], [1, 0, 0, 0],
], dtype=torch.float32)


def truth_tables():
    """``[16,4]`` uint8, column = gate16 address ``(a<<1)|b``
    (silogic/functional.py:50-69)."""
    c = BASIS
    tt = torch.stack([c[:, 0], c[:, 0] + c[:, 2], c[:, 0] + c[:, 1],
                      c[:, 0] + c[:, 1] + c[:, 2] + c[:, 3]], dim=1)
    return tt.round().to(torch.uint8)


TRUTH = truth_tables()


def corner_bits(n):
    """``[2^n, n]`` corner bit patterns, bit j of row p (functional.py:169-173)."""
    return torch.tensor([[(p >> j) & 1 for j in range(n)] for p in range(2 ** n)],
                        dtype=torch.float32)


def walsh_monomials(u):
    """``[B,out,n] -> [B,out,2^n]`` (functional.py:176-185)."""
    phi = torch.ones(u.shape[0], u.shape[1], 1, dtype=u.dtype)
    for j in range(u.shape[2]):
        phi = torch.cat([phi, phi * u[:, :, j:j + 1]], dim=2)
    return phi


# --------------------------------------------------------------------------
# structure: expand constructor defaults (silogic/models.py)
# --------------------------------------------------------------------------
_NODE_ALIAS = {"gate16": "gate16", "gate": "gate16", "walsh": "walsh",
               "multilinear": "multilinear", "probabilistic": "multilinear",
               "hybrid": "hybrid"}
_CONN_ALIAS = {"f": "fixed", "fixed": "fixed", "topk": "topk", "blocktopk": "topk"}


def _fc_layer(prefix, d_in, d_out, node, connectome, arity, k, node_tau):
    node = _NODE_ALIAS[str(node).lower()]
    if node == "gate16":
        arity = 2
    conn = _CONN_ALIAS[str(connectome).lower()]
    return dict(prefix=prefix, d_in=d_in, d_out=d_out, node=node, arity=arity,
                conn=conn, k=min(k, d_in), node_tau=node_tau)


def structure(spec):
    """Layer-by-layer description of a reference model built from ``spec``."""
    ctor, a = spec
    a = dict(a)
    if ctor in ("LogicNet", "WARPNet", "WARPNetN", "LUTkNet", "LUTNodeNet"):
        if ctor in ("WARPNet", "WARPNetN"):   # models.py:107-125
            arity = 2 if ctor == "WARPNet" else a.get("arity", 6)
            node, node_tau, tau = "walsh", a.get("tau", 1.0), 20.0
            connectome, ste = "topk", True
        elif ctor == "LUTkNet":               # models.py:128-138: arity k, cand_k candidates
            node, arity, node_tau, tau = "multilinear", a.get("k", 4), 1.0, a.get("tau", 4.0)
            connectome, ste = "topk", True
            a["k"] = a.get("cand_k", 4)
        elif ctor == "LUTNodeNet":            # models.py:141-147
            node, arity, node_tau = a.get("relaxation", "probabilistic"), a.get("arity", 4), 1.0
            tau, connectome, ste = a.get("tau", 10.0), "topk", True
        else:                   # models.py:59-79
            node, arity = a.get("node", "gate16"), a.get("arity", 2)
            node_tau, tau = a.get("node_tau", 1.0), a.get("tau", 1.0)
            connectome, ste = a.get("connectome", "topk"), a.get("decoder_ste", True)
        layers, d_in = [], a["in_dim"]
        for i in range(a["depth"]):
            layers.append(_fc_layer(f"layers.{i}.", d_in, a["width"], node,
                                    connectome, arity, a.get("k", 8), node_tau))
            d_in = a["width"]
        return dict(kind="fc", layers=layers,
                    wire_r=int(a["width"] * a.get("wire_residual", 0.0)),
                    head=dict(C=a.get("num_classes", 10), tau=tau, ste=ste))
    if ctor in ("LogicConvNet", "LogicTreeNet"):   # models.py:208-246
        node = _NODE_ALIAS[str(a.get("node", "gate16")).lower()]
        node_arity = 2 if node in ("gate16", "walsh") else a.get("arity", 2)
        depth = a.get("tree_depth")
        if depth is None:
            depth = 2 if node_arity == 2 else 1
        kernel = a.get("kernel", 3)
        blocks, c, hw = [], a["in_channels"], a["in_hw"]
        for i, n in enumerate(a["channels"]):
            n_chan = a.get("n_chan", 2)
            pool_sz = n_chan * kernel * kernel
            blocks.append(dict(prefix=f"blocks.{2 * i}.", cin=c, n=n, kernel=kernel,
                               depth=depth, stride=1, padding=kernel // 2,
                               connect=a.get("connect", "topk"),
                               k=min(a.get("k", 4), pool_sz), node=node,
                               node_arity=node_arity, leaves=node_arity ** depth,
                               tau=a.get("node_tau", 1.0), hw=hw))
            c, hw = n, hw // 2
        feat = c * hw * hw
        hws = a.get("head_widths")
        if hws is None:
            hws = [a.get("head_width")] * a.get("head_depth", 2)
        head_layers, d_in = [], feat
        for j, w in enumerate(hws):
            # head LogicLayer: node=node, arity left at its default 2, tau default 1
            head_layers.append(_fc_layer(f"head_layers.{j}.", d_in, w, node,
                                         a.get("head_connect", "topk"), 2,
                                         a.get("head_k", 8), 1.0))
            d_in = w
        return dict(kind="conv", blocks=blocks, head_layers=head_layers, feat=feat,
                    wire_residual=a.get("wire_residual", 0.0),
                    head=dict(C=a.get("num_classes", 10), tau=a.get("tau", 100.0),
                              ste=a.get("decoder_ste", True)))
    raise ValueError(f"unsupported spec {ctor}")


# --------------------------------------------------------------------------
# FC layer (silogic/connectomes.py, nodes.py, layers.py:125-135)
# --------------------------------------------------------------------------
def select_soft(L, sd, x):
    p = L["prefix"]
    if L["conn"] == "fixed":                                   # connectomes.py:58-59
        return x[:, sd[p + "_conn.idx"]]
    w = F.softmax(sd[p + "_conn.conn"], dim=2)                 # connectomes.py:114-127
    g = x[:, sd[p + "_conn.cand"]]
    return torch.einsum("boak,oak->boa", g, w)


def hard_indices(L, sd):
    """``[out, arity]`` hard wire indices (connectomes.py:129-132)."""
    p = L["prefix"]
    if L["conn"] == "fixed":
        return sd[p + "_conn.idx"]
    sel = sd[p + "_conn.conn"].argmax(dim=2)
    return torch.gather(sd[p + "_conn.cand"], 2, sel.unsqueeze(-1)).squeeze(-1)


def node_soft(L, sd, ops):
    p = L["prefix"]
    if L["node"] == "gate16":                                  # nodes.py:86-91
        a, b = ops[..., 0], ops[..., 1]
        c = F.softmax(sd[p + "node.gate_logits"], dim=1) @ BASIS
        return c[:, 0] + c[:, 1] * a + c[:, 2] * b + c[:, 3] * (a * b)
    if L["node"] == "walsh":                                   # nodes.py:145-150
        u = 2 * ops - 1
        z = (walsh_monomials(u) * sd[p + "node.theta"][None]).sum(2)
        return torch.sigmoid(z * (1.0 / L["node_tau"]))
    if L["node"] == "hybrid":                                  # nodes.py:202-206
        return hybrid_f(ops, sd[p + "node.logits"], L["arity"])
    return multilinear_f(ops, sd[p + "node.logits"], L["arity"])


class _Straight(torch.autograd.Function):
    """Value of ``disc``, gradient into ``soft``: the hybrid node's
    ``f_disc + f_soft - f_soft.detach()`` (nodes.py:202-206) without the
    fp32 rounding of that sum, i.e. the LUT value exactly, as the reference's
    fused kernels return it (kernels/multilinear.py:40-61)."""

    @staticmethod
    def forward(ctx, disc, soft):
        return disc.clone()

    @staticmethod
    def backward(ctx, g):
        return None, g


def hybrid_f(ops, logits, n):
    f_soft = multilinear_f(ops, logits, n)
    with torch.no_grad():
        f_disc = multilinear_f((ops >= 0.5).float(), logits, n)
    return _Straight.apply(f_disc, f_soft)


def multilinear_f(ops, logits, n):
    """``sum_P sigmoid(l_P) prod_j (c_Pj a_j + (1-c_Pj)(1-a_j))`` (nodes.py:174-178)."""
    au = ops.unsqueeze(2)
    c = corner_bits(n).view(1, 1, -1, n)
    prod = (c * au + (1 - c) * (1 - au)).prod(3)
    return (prod * torch.sigmoid(logits)[None]).sum(2)


def node_hard(L, sd, ops):
    p = L["prefix"]
    if L["node"] == "gate16":                                  # nodes.py:100-106
        a, b = ops[..., 0], ops[..., 1]
        gate = sd[p + "node.gate_logits"].argmax(dim=1)
        idx = (a.long() << 1) | b.long()
        return torch.gather(TRUTH[gate], 1, idx.t()).t().to(torch.uint8)
    if L["node"] == "walsh":                                   # nodes.py:152-156
        u = 2 * ops.float() - 1
        z = (walsh_monomials(u) * sd[p + "node.theta"][None]).sum(2)
        return (z > 0).to(torch.uint8)
    return multilinear_hard(ops, sd[p + "node.logits"], L["arity"])


def multilinear_hard(ops, logits, n):
    """``(logits > 0)[sum_j a_j 2^j]`` (nodes.py:183-189)."""
    a = ops.long()
    shifts = (2 ** torch.arange(n)).view(1, 1, -1)
    addr = (a * shifts).sum(dim=2)
    tt = (logits > 0).to(torch.uint8)
    return torch.gather(tt, 1, addr.t()).t()


def fc_layer_soft(L, sd, x):
    return node_soft(L, sd, select_soft(L, sd, x))


def gumbel(shape, device):
    """The reference's Gumbel draw (nodes.py:46-48)."""
    u = torch.rand(shape, device=device).clamp_(1e-6, 1 - 1e-6)
    return -torch.log(-torch.log(u))


def fc_layer_soft_gumbel(L, sd, x, g1, g2):
    """Walsh layer in training with Gumbel-sigmoid smoothing (nodes.py:145-149):
    ``sigmoid((z + g1 - g2) / tau)`` for given draws ``g1``, ``g2`` [B, out]."""
    p = L["prefix"]
    u = 2 * select_soft(L, sd, x) - 1
    z = (walsh_monomials(u) * sd[p + "node.theta"][None]).sum(2)
    return torch.sigmoid((z + g1 - g2) * (1.0 / L["node_tau"]))


def fc_layer_hard(L, sd, x):
    x = x.to(torch.uint8)                                      # layers.py:131-135
    ops = x[:, hard_indices(L, sd)]
    return node_hard(L, sd, ops).to(torch.uint8)


# --------------------------------------------------------------------------
# GroupSum (silogic/heads.py:16-45)
# --------------------------------------------------------------------------
def groupsum_soft(head, x, ste=None):
    ste = head["ste"] if ste is None else ste
    b, w = x.shape
    if ste:
        x = (x > 0.5).float() + (x - x.detach())
    return x.view(b, head["C"], w // head["C"]).sum(dim=2) / head["tau"]


def groupsum_hard(head, x):
    b, w = x.shape
    return x.view(b, head["C"], w // head["C"]).sum(dim=2).float()


# --------------------------------------------------------------------------
# ConvLogicTree / OrPool (silogic/layers.py:375-563)
# --------------------------------------------------------------------------
def _hw_out(blk, H, W):
    k, s, p = blk["kernel"], blk["stride"], blk["padding"]
    return (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1


def conv_leaves_soft(blk, sd, patches):
    p = blk["prefix"]
    B, _, L = patches.shape
    if blk["connect"] == "fixed":                              # layers.py:378-381
        g = patches[:, sd[p + "leaf_idx"].reshape(-1), :]
        return g.view(B, blk["n"], blk["leaves"], L)
    w = F.softmax(sd[p + "conn"], dim=2)                       # layers.py:382-386
    g = patches[:, sd[p + "leaf_cand"].reshape(-1), :]
    g = g.view(B, blk["n"], blk["leaves"], blk["k"], L)
    return torch.einsum("bnlkL,nlk->bnlL", g, w)


def conv_soft(blk, sd, x):
    B, C, H, W = x.shape
    Ho, Wo = _hw_out(blk, H, W)
    patches = F.unfold(x, (blk["kernel"], blk["kernel"]), stride=blk["stride"],
                       padding=blk["padding"])
    vals = conv_leaves_soft(blk, sd, patches)
    p = blk["prefix"]
    if blk["node"] == "gate16":                                # layers.py:388-401
        for i in range(blk["depth"]):
            c = F.softmax(sd[f"{p}gate_logits.{i}"], dim=2) @ BASIS
            a, b = vals[:, :, 0::2, :], vals[:, :, 1::2, :]
            c = c.unsqueeze(0).unsqueeze(-1)
            vals = (c[:, :, :, 0] + c[:, :, :, 1] * a + c[:, :, :, 2] * b
                    + c[:, :, :, 3] * (a * b))
        out = vals[:, :, 0, :]
    else:
        out = _node_tree(blk, sd, vals, hard=False)
    return out.view(B, blk["n"], Ho, Wo)


def _node_tree(blk, sd, vals, hard):
    """k-ary tree of node modules, spatial folded into batch (layers.py:432-446)."""
    k = blk["node_arity"]
    B = vals.shape[0]
    for i in range(blk["depth"]):
        n, km, L = vals.shape[1], vals.shape[2], vals.shape[3]
        m = km // k
        ops = vals.view(B, n, m, k, L).permute(0, 4, 1, 2, 3).reshape(B * L, n * m, k)
        logits = sd.get(f"{blk['prefix']}tree_nodes.{i}.logits")
        if blk["node"] == "walsh":                            # nodes.py:145-156
            theta = sd[f"{blk['prefix']}tree_nodes.{i}.theta"]
            u = 2 * ops.float() - 1
            z = (walsh_monomials(u) * theta[None]).sum(2)
            out = (z > 0).to(torch.uint8) if hard else torch.sigmoid(z * (1.0 / blk["tau"]))
            vals = out.view(B, L, n, m).permute(0, 2, 3, 1)
            continue
        if blk["node"] not in ("multilinear", "hybrid"):
            raise NotImplementedError(blk["node"])
        if hard:
            out = multilinear_hard(ops, logits, k)
        elif blk["node"] == "hybrid":                          # nodes.py:202-206
            out = hybrid_f(ops, logits, k)
        else:
            out = multilinear_f(ops, logits, k)
        vals = out.view(B, L, n, m).permute(0, 2, 3, 1)
    return vals[:, :, 0, :]


def conv_hard(blk, sd, x):
    B, C, H, W = x.shape
    x = x.to(torch.uint8)                                      # layers.py:529-541
    Ho, Wo = _hw_out(blk, H, W)
    patches = F.unfold(x.float(), (blk["kernel"], blk["kernel"]), stride=blk["stride"],
                       padding=blk["padding"]).to(torch.uint8)
    p = blk["prefix"]
    if blk["connect"] == "fixed":                              # layers.py:505-513
        idx = sd[p + "leaf_idx"].reshape(-1)
    else:
        sel = sd[p + "conn"].argmax(dim=2)
        idx = torch.gather(sd[p + "leaf_cand"], 2, sel.unsqueeze(-1)).squeeze(-1)
        idx = idx.reshape(-1)
    vals = patches[:, idx, :].view(B, blk["n"], blk["leaves"], -1)
    if blk["node"] == "gate16":                                # layers.py:515-527
        for i in range(blk["depth"]):
            gate = sd[f"{p}gate_logits.{i}"].argmax(dim=2)
            a, b = vals[:, :, 0::2, :], vals[:, :, 1::2, :]
            t_idx = (a.long() << 1) | b.long()
            tt = TRUTH[gate].unsqueeze(0).expand(B, -1, -1, -1)
            vals = torch.gather(tt, 3, t_idx)
        out = vals[:, :, 0, :]
    else:
        out = _node_tree(blk, sd, vals, hard=True)
    return out.view(B, blk["n"], Ho, Wo).to(torch.uint8)


def orpool_soft(x):
    return F.max_pool2d(x, 2, 2)                               # layers.py:558-559


def orpool_hard(x):
    return F.max_pool2d(x.float(), 2, 2).to(torch.uint8)       # layers.py:561-563


# --------------------------------------------------------------------------
# networks (silogic/models.py:88-101, 248-275)
# --------------------------------------------------------------------------
def forward_features(st, sd, x, hard, trace=None):
    """Run all layers; return the final features (before the head)."""
    if st["kind"] == "fc":
        for i, L in enumerate(st["layers"]):
            y = fc_layer_hard(L, sd, x) if hard else fc_layer_soft(L, sd, x)
            if st["wire_r"] and x.shape[1] == y.shape[1]:
                y = torch.cat([x[:, :st["wire_r"]], y[:, st["wire_r"]:]], dim=1)
            x = y
            if trace is not None:
                trace[f"{'h' if hard else ''}act/{i}"] = x
        return x
    for i, blk in enumerate(st["blocks"]):
        x_in = x
        y = conv_hard(blk, sd, x) if hard else conv_soft(blk, sd, x)
        if st["wire_residual"] > 0:
            r = min(int(blk["n"] * st["wire_residual"]), x_in.shape[1])
            if r > 0:
                y = torch.cat([x_in[:, :r], y[:, r:]], dim=1)
        if trace is not None:
            trace[f"{'h' if hard else ''}conv/{i}"] = y
        x = orpool_hard(y) if hard else orpool_soft(y)
        if trace is not None:
            trace[f"{'h' if hard else ''}pool/{i}"] = x
    x = x.flatten(1)
    for j, L in enumerate(st["head_layers"]):
        x = fc_layer_hard(L, sd, x) if hard else fc_layer_soft(L, sd, x)
        if trace is not None:
            trace[f"{'h' if hard else ''}act/{j}"] = x
    return x


@torch.no_grad()
def forward(spec, sd, x, trace=None, ste=None):
    st = structure(spec)
    return groupsum_soft(st["head"], forward_features(st, sd, x, False, trace), ste)


@torch.no_grad()
def forward_hard(spec, sd, x, trace=None):
    st = structure(spec)
    return groupsum_hard(st["head"], forward_features(st, sd, x, True, trace))


def num_gates(spec):
    """``width * depth`` (models.py:103-104) or ``gate_count(in_hw)``
    (models.py:277-288) — the gate-eval count per sample."""
    st = structure(spec)
    if st["kind"] == "fc":
        return sum(L["d_out"] for L in st["layers"])
    total = 0
    for blk in st["blocks"]:
        k = blk["node_arity"]
        total += blk["n"] * blk["hw"] * blk["hw"] * ((k ** blk["depth"] - 1) // (k - 1))
    return total + sum(L["d_out"] for L in st["head_layers"])
