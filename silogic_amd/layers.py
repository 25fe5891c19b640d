"""Logic layers (mirror of silogic/layers.py): ``LogicLayer`` and its presets,
``ConvLogicTree`` (alias ``ConvLogicLayer``) and ``OrPool``.

Construction, parameter names and ``state_dict`` layout follow the reference
(silogic/layers.py:51-75, 271-373) so checkpoints and seeds carry over.
Compute runs on the HIP kernels of ``libsilogic_hip.so``:

* ``LogicLayer.forward`` -> Top-K gather + node. Without gradients the
  parameters (``softmax(conn)``, node coefficients, clamped indices) are
  packed into one record per output by ``slg_fc_soft_records`` and the layer
  runs on ``slg_fc_soft_fwd_records``; with gradients they come from
  differentiable torch ops (the reference's ``_fused`` split,
  layers.py:111-123) and the layer runs on ``slg_fc_soft_fwd``.
* ``LogicLayer.forward_hard`` -> pack, one packed layer, unpack.
* ``ConvLogicTree.forward`` -> ``slg_conv_soft_fwd``; networks call
  ``forward_pooled``, which fuses the following ``OrPool``.

There is no CPU path: CPU inputs raise.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import derived, ops
from .connectomes import build_connectome, FixedConnectome
from .functional import BASIS_COEFFS, TRUTH_TABLES, GATE_A, gate_probs
from .nodes import build_node, _NODE_ALIASES


def _needs_grad(module, *xs):
    if not torch.is_grad_enabled():
        return False
    if any(x is not None and x.requires_grad for x in xs):
        return True
    return any(p.requires_grad for p in module.parameters())


class LogicLayer(nn.Module):
    """A layer of logic nodes: connectome (input wiring) + node (gate
    parameterization). Arguments as silogic.layers.LogicLayer; the HIP path
    covers arity-2 nodes (gate16, walsh, multilinear) with top-k / block-top-k
    / fixed wiring. ``use_triton`` is accepted for API compatibility and
    ignored (the HIP kernels always run)."""

    def __init__(self, in_dim, out_dim, node="gate16", connectome="topk", arity=2,
                 k=8, gate_eval="basis", residual_p=0.0, seed=None,
                 window=0, tau=1.0, degree=None, gate_select="softmax",
                 gumbel_tau=1.0, use_triton=True):
        super().__init__()
        self._node_name = _NODE_ALIASES.get(str(node).lower(), node)
        if self._node_name == "gate16":
            arity = 2
        self.in_dim = in_dim
        self.out_dim = out_dim
        self.arity = arity
        self.k = k
        self.gate_eval = gate_eval
        self.use_triton = use_triton
        self.connectome = connectome
        self._conn = build_connectome(connectome, in_dim, out_dim, arity, k, seed, window)
        if gate_select == "hard" and hasattr(self._conn, "ste"):
            self._conn.ste = True
        self.node = build_node(node, out_dim, arity, gate_eval=gate_eval, tau=tau,
                               degree=degree, gate_select=gate_select, gumbel_tau=gumbel_tau)
        if residual_p > 0:
            self.node.residual_init(residual_p)

    # -- compatibility accessors ---------------------------------------------
    @property
    def gate_logits(self):
        return self.node.gate_logits

    @property
    def theta(self):
        return self.node.theta

    @property
    def conn_a(self):
        return self._conn.conn[:, 0]

    @property
    def conn_b(self):
        return self._conn.conn[:, 1]

    # -- HIP dispatch ----------------------------------------------------------
    @property
    def is_lut(self):
        """An n-input LUT layer (the hybrid node, or a multilinear or walsh
        node of arity other than 2): ``slg_fc_lut_*`` instead of the gate
        kernels."""
        return getattr(self.node, "hybrid", False) or (
            self._node_name in ("multilinear", "walsh") and self.arity != 2)

    @property
    def is_walsh_n(self):
        """An n-input walsh layer (nodes.py:130-156): z is multilinear in the
        operands, so it is the LUT layer's interpolation of z's corner values
        (``WalshNode.corner_z``), followed by sigmoid(z / tau)."""
        return self._node_name == "walsh" and self.arity != 2

    def _check_supported(self):
        if self.arity != 2 or self.is_lut:
            raise NotImplementedError(
                f"LogicLayer arity {self.arity} / node {self._node_name}: the gate kernels "
                "take arity-2 gate16 / walsh / multilinear nodes (LUT layers run slg_fc_lut_*)")

    def lut_hard_codes(self):
        """``(idx [out, n] int32, tt [out] int64)`` of a LUT layer (HIP prep;
        bit p of tt is ``logits[p] > 0``). For an n-input walsh node the
        "logits" are z at the corners, evaluated on the CPU with the node's
        own fp32 expression (nodes.py:152-156), so that its signs are the
        reference's also at near-ties."""
        conn = None if isinstance(self._conn, FixedConnectome) else self._conn.conn
        logits = self.node.corner_z_hard() if self.is_walsh_n else self.node.logits
        return ops.fc_lut_hard_codes(self._conn.candidates_i32(), conn, logits, self.in_dim)

    def _inv_tau(self):
        return self.node.inv_tau if self._node_name == "walsh" else 1.0

    def soft_params(self, grad):
        """``(cand_i32, w, node_param)`` for the soft kernel."""
        conn = self._conn
        cand = conn.candidates_i32()
        plain = self.node.plain_softmax() and not getattr(conn, "ste", False)
        if grad or not plain:
            if self._node_name == "walsh" and not self.node.plain_softmax():
                raise NotImplementedError("walsh Gumbel smoothing adds noise per (sample, "
                                          "output), which no kernel parameter holds: "
                                          "LogicLayer.forward runs it")
            return cand, conn.weights(), self.node.kernel_param()
        raw_conn = None if isinstance(conn, FixedConnectome) else conn.conn
        w, npar = ops.fc_soft_prep(raw_conn, self.node.raw(), self.node.kind, self.out_dim,
                                   conn.k)
        return cand, w, npar

    def records_ok(self):
        """Whether the forward without gradients runs on per-output records:
        a plain softmax selection over inputs below 65536 (records hold 16-bit
        input indices), not a LUT layer."""
        if self.is_lut or self.in_dim > 65536:
            return False
        self._check_supported()
        return self.node.plain_softmax() and not getattr(self._conn, "ste", False)

    def record_spec(self):
        """``(cand, conn, raw, in_dim, node_kind, order)`` for
        ``ops.fc_soft_records`` when :meth:`records_ok`, else ``None``."""
        if not self.records_ok():
            return None
        conn = self._conn
        raw_conn = None if isinstance(conn, FixedConnectome) else conn.conn
        cand = conn.candidates_i32()
        return cand, raw_conn, self.node.raw(), self.in_dim, self.node.kind, self.gather_order(cand)

    @property
    def n_candidates(self):
        return self._conn.k

    def gather_order(self, cand=None):
        """Bank-aware order in which the soft kernel gathers each output's
        candidates (``slg_fc_soft_schedule``). It depends only on the
        candidate table, a buffer that training does not change, so it is
        computed once per table (a new device, a loaded state dict or any
        in-place change of the buffer recomputes it). ``None`` for K = 1."""
        cand = self._conn.candidates_i32() if cand is None else cand
        if cand.shape[-1] < 2:
            return None
        key = (cand.data_ptr(), cand._version, str(cand.device), self.in_dim)
        cached = getattr(self, "_order_cache", None)
        if cached is None or cached[0] != key:
            self._order_cache = (key, ops.fc_soft_schedule(cand, self.in_dim))
        return self._order_cache[1]

    def forward(self, x):
        ops.require_gpu(x)
        ops.check_width(x, self.in_dim)
        if self._node_name == "walsh" and not self.node.plain_softmax():
            # Gumbel-sigmoid smoothing in training (nodes.py:145-149): the
            # kernels return z (arity 2: the gate kernel on z's (a, b)-space
            # coefficients; arity n: the LUT kernel on z's corner values),
            # the noise and the sigmoid are torch ops on [B, out]
            conn = self._conn
            if self.is_walsh_n:
                z = ops.fc_lut_soft(x, conn.candidates_i32(), conn.weights(),
                                    self.node.corner_z(), False)
            else:
                self._check_supported()
                z = ops.fc_soft(x, conn.candidates_i32(), conn.weights(), self.node.coef(),
                                ops.GATE16, 1.0)
            return self.node.gumbel_sigmoid(z)
        if self.is_lut:
            conn = self._conn
            if self.is_walsh_n:
                z = ops.fc_lut_soft(x, conn.candidates_i32(), conn.weights(),
                                    self.node.corner_z(), False)
                return torch.sigmoid(z * self.node.inv_tau)
            return ops.fc_lut_soft(x, conn.candidates_i32(), conn.weights(),
                                   torch.sigmoid(self.node.logits), self.node.hybrid)
        self._check_supported()
        grad = _needs_grad(self, x)
        if not grad and self.records_ok():
            K = self.n_candidates
            rec = derived.cached(self, "_derived_records", (derived.state_key(self), K),
                                 lambda: ops.fc_soft_records([self.record_spec()], K)[0])
            return ops.fc_soft_rec(x, rec, self.in_dim, self.out_dim, K, self.node.kind,
                                   self._inv_tau())
        cand, w, npar = self.soft_params(grad)
        return ops.fc_soft(x, cand, w, npar, self.node.kind, self._inv_tau())

    def hard_spec(self):
        """``(cand, conn, raw, node_kind, in_dim)`` for the hard-code prep."""
        self._check_supported()
        cand, conn = self._conn.hard_inputs()
        return cand, conn, self.node.raw(), self.node.kind, self.in_dim

    def hard_codes(self):
        """Per-output ``(a, b | tt << 28)`` codes [out, 2] int32 (HIP prep)."""
        return ops.fc_hard_codes(*self.hard_spec())

    def packed_forward(self, xp):
        """Packed ``[in, nw]`` -> ``[out, nw]`` words."""
        if self.is_lut:
            return ops.fc_lut_hard(xp, *self.lut_hard_codes())
        return ops.fc_hard_layer(xp, self.hard_codes())

    @torch.no_grad()
    def forward_hard(self, x):
        ops.require_gpu(x)
        ops.check_width(x, self.in_dim)
        B = x.shape[0]
        return ops.unpack_bits(self.packed_forward(ops.pack_bits(x)), B)


class WARPLayer(LogicLayer):
    """2-input Walsh (WARP) node with Top-K connectivity (preset)."""

    def __init__(self, in_dim, out_dim, k=8, tau=1.0, residual_p=0.0, seed=None,
                 gate_select="softmax"):
        super().__init__(in_dim, out_dim, node="walsh", connectome="topk", arity=2,
                         k=k, tau=tau, residual_p=residual_p, seed=seed,
                         gate_select=gate_select)

    def _z(self, a, b):
        return self.node._z(a, b)

    def _coef(self):
        return self.node.coef()


class WARPLayerN(LogicLayer):
    """Arity-``n`` Walsh (WARP) node with Top-K connectivity (preset,
    silogic/layers.py:162-174)."""

    def __init__(self, in_dim, out_dim, arity=6, k=8, tau=1.0, residual_p=0.0,
                 seed=None, gate_select="softmax"):
        super().__init__(in_dim, out_dim, node="walsh", connectome="topk", arity=arity,
                         k=k, tau=tau, residual_p=residual_p, seed=seed,
                         gate_select=gate_select)

    @property
    def theta(self):
        return self.node.theta


class LUTkLayer(LogicLayer):
    """k-input multilinear LUT node (one FPGA LUT_k) with Top-K input
    selection (preset, silogic/layers.py:177-199): ``k`` LUT inputs drawn
    among ``cand_k`` candidates each."""

    def __init__(self, in_dim, out_dim, k=4, learn_conn=True, cand_k=4, seed=None):
        conn = "topk" if learn_conn else "fixed"
        super().__init__(in_dim, out_dim, node="multilinear", connectome=conn,
                         arity=k, k=cand_k, seed=seed)
        self.k = k
        self.learn_conn = learn_conn

    @property
    def lut(self):
        return self.node.logits

    @property
    def conn(self):
        return self._conn.conn

    @property
    def cand(self):
        return self._conn.cand


class LUTNodeLayer(LogicLayer):
    """n-input LUT node with a selectable relaxation (preset,
    silogic/layers.py:202-224): ``probabilistic`` (multilinear) or
    ``hybrid`` on the HIP path."""

    def __init__(self, in_dim, out_dim, arity=4, relaxation="probabilistic", k=8,
                 degree=None, residual_p=0.0, seed=None):
        super().__init__(in_dim, out_dim, node=relaxation, connectome="topk",
                         arity=arity, k=k, degree=degree, residual_p=residual_p,
                         seed=seed)
        self.relaxation = relaxation
        self.n = arity
        self.k = self._conn.k

    @property
    def conn(self):
        return self._conn.conn

    @property
    def cand(self):
        return self._conn.cand


class ConvLogicTree(nn.Module):
    """Logic-gate-tree convolution (arguments as silogic.layers.ConvLogicTree).

    The HIP path covers every tree the reference builds for the gate16,
    walsh, multilinear and hybrid nodes (binary trees of depth 1-5, LUT trees
    of arity 2-6 with at most 36 leaves), stride 1 with ``padding = kernel //
    2``. Gate16 trees of depth 1-4 and depth-1 LUTs run on the LDS-staged
    kernels (records without gradients); the others on the generic tree
    kernels, with parameters from differentiable torch ops."""

    def __init__(self, in_channels, out_channels, kernel=3, tree_depth=None,
                 stride=1, padding=1, connect="topk", k=4, n_chan=2,
                 residual_init=True, seed=0, node="gate16",
                 arity=4, tau=1.0, degree=None, gate_select="softmax",
                 gumbel_tau=1.0, use_triton=True):
        super().__init__()
        self.node_name = _NODE_ALIASES.get(str(node).lower(), node)
        self.gate_select = gate_select
        self.gumbel_tau = gumbel_tau
        self.node_arity = 2 if self.node_name in ("gate16", "walsh") else arity
        if tree_depth is None:
            tree_depth = 2 if self.node_arity == 2 else 1
        self.cin = in_channels
        self.n = out_channels
        self.kh = self.kw = kernel
        self.d = tree_depth
        self.leaves = self.node_arity ** tree_depth
        self.stride = stride
        self.padding = padding
        self.connect = connect
        self.k = k
        self.tau = tau
        self.use_triton = use_triton
        if self.node_name not in ("gate16", "walsh", "multilinear", "hybrid"):
            raise NotImplementedError(f"conv node {node!r} is not on the MI355X path")
        if not 2 <= self.node_arity <= 6 or self.leaves > 36 or tree_depth > 5:
            raise NotImplementedError(
                f"{self.node_name} conv trees: arity 2..6 with at most 36 leaves (depth <= 5), "
                f"got arity {self.node_arity} depth {tree_depth}")
        if stride != 1 or 2 * padding + 1 != kernel:
            raise NotImplementedError("conv trees: stride 1 with padding = kernel // 2")
        gen = torch.Generator().manual_seed(seed)

        # Each tree observes n_chan random input channels; its leaf candidates
        # are those channels' receptive-field positions (flat c*k*k + dy*k + dx).
        pool_sz = n_chan * kernel * kernel
        cand_pool = []
        for _ in range(out_channels):
            chans = torch.randperm(in_channels, generator=gen)[:n_chan]
            idxs = []
            for c in chans:
                base = int(c) * kernel * kernel
                idxs.extend(range(base, base + kernel * kernel))
            cand_pool.append(torch.tensor(idxs))
        cand_pool = torch.stack(cand_pool)
        kk2 = kernel * kernel
        if connect == "fixed":
            sel = torch.stack([
                cand_pool[i][torch.randint(0, pool_sz, (self.leaves,), generator=gen)]
                for i in range(out_channels)])
            self.register_buffer("leaf_idx", sel)
            self.register_buffer("cm_idx", (sel // kk2).to(torch.int32))
            rem = sel % kk2
            self.register_buffer("ch_idx", (rem // kernel).to(torch.int32))
            self.register_buffer("cw_idx", (rem % kernel).to(torch.int32))
        else:
            kk = min(k, pool_sz)
            self.k = kk
            cand = torch.stack([
                torch.stack([cand_pool[i][torch.randperm(pool_sz, generator=gen)[:kk]]
                             for _ in range(self.leaves)])
                for i in range(out_channels)])
            self.register_buffer("leaf_cand", cand)
            self.conn = nn.Parameter(torch.randn(out_channels, self.leaves, kk))
            self.register_buffer("lc_cm", (cand // kk2).to(torch.int32))
            rem = cand % kk2
            self.register_buffer("lc_ch", (rem // kernel).to(torch.int32))
            self.register_buffer("lc_cw", (rem % kernel).to(torch.int32))

        if self.node_name == "gate16":
            self.gate_logits = nn.ParameterList()
            for i in range(tree_depth):
                nodes = 2 ** (tree_depth - 1 - i)
                w = torch.zeros(out_channels, nodes, 16)
                if residual_init:
                    w[:, :, GATE_A] = 5.0
                else:
                    w.normal_(0, 0.1)
                self.gate_logits.append(nn.Parameter(w))
            self.register_buffer("basis", BASIS_COEFFS.clone())
            self.register_buffer("truth", TRUTH_TABLES.clone())
        else:
            self.tree_nodes = nn.ModuleList()
            for i in range(tree_depth):
                m = self.node_arity ** (tree_depth - 1 - i)
                nd = build_node(self.node_name, out_channels * m, arity=self.node_arity,
                                tau=tau, degree=degree, gate_select=gate_select,
                                gumbel_tau=gumbel_tau)
                if residual_init:
                    nd.residual_init(0.9)
                self.tree_nodes.append(nd)

    # -- parameters --------------------------------------------------------------
    @property
    def gates_per_output(self):
        k = self.node_arity
        return (k ** self.d - 1) // (k - 1)

    def _hw_out(self, H, W):
        Ho = (H + 2 * self.padding - self.kh) // self.stride + 1
        Wo = (W + 2 * self.padding - self.kw) // self.stride + 1
        return Ho, Wo

    def _taps(self):
        if self.connect == "fixed":
            return (self.cm_idx.unsqueeze(-1), self.ch_idx.unsqueeze(-1),
                    self.cw_idx.unsqueeze(-1))
        return self.lc_cm, self.lc_ch, self.lc_cw

    def _kind(self):
        return {"gate16": ops.GATE16, "walsh": ops.WALSH, "hybrid": ops.HYBRID}.get(
            self.node_name, ops.MULTILINEAR2)

    @property
    def generic(self):
        """True for trees outside the LDS-staged kernels' set (walsh trees,
        LUT trees deeper than one level, gate16 trees of depth 5): their
        parameters come from torch ops, the hard path from per-node tables."""
        if self.node_name == "gate16":
            return self.d > 4
        return self.node_name == "walsh" or self.d != 1

    def _raw(self):
        if self.node_name == "gate16":
            return torch.cat([g for g in self.gate_logits], dim=1)   # [n, nodes, 16]
        return self.tree_nodes[0].logits                             # [n, 2^arity]

    def _topk_w(self):
        w = F.softmax(self.conn, dim=2)
        if self.gate_select == "hard":
            hard = F.one_hot(self.conn.argmax(dim=2), w.shape[-1]).to(w.dtype)
            w = hard + w - w.detach()
        return w

    def _basis_coef(self):
        gl = torch.cat([g for g in self.gate_logits], dim=1)
        p = gate_probs(gl, self.training, dim=2, gate_select=self.gate_select,
                       gumbel_tau=self.gumbel_tau)
        return p @ self.basis

    def _node_params(self):
        """Differentiable node parameters ``[n, nodes, P]``, level-major (the
        kernels' tree layout): gate16 BasisProj coefficients, walsh (a, b)
        coefficients times 1/tau, LUT values sigmoid(logits) (the reference's
        ``_hybrid_s``, layers.py:499-503)."""
        if self.node_name == "gate16":
            return self._basis_coef()
        if self.node_name == "walsh":
            return torch.cat([nd.coef().view(self.n, -1, 4) for nd in self.tree_nodes],
                             dim=1) * (1.0 / self.tau)
        P = 2 ** self.node_arity
        return torch.cat([torch.sigmoid(nd.logits).view(self.n, -1, P)
                          for nd in self.tree_nodes], dim=1)

    def soft_params(self, grad):
        K = 1 if self.connect == "fixed" else self.k
        if self.generic:
            w = (torch.ones(self.n, self.leaves, 1, device=self.cm_idx.device)
                 if self.connect == "fixed" else self._topk_w())
            return w, self._node_params()
        if grad or not self._plain_soft():
            w = (torch.ones(self.n, self.leaves, 1, device=self.cm_idx.device)
                 if self.connect == "fixed" else self._topk_w())
            npar = (self._basis_coef() if self.node_name == "gate16"
                    else torch.sigmoid(self.tree_nodes[0].logits))
            return w, npar
        conn = None if self.connect == "fixed" else self.conn
        return ops.conv_soft_prep(conn, self._raw(), self._kind(), self.n, self.leaves, K,
                                  self.d, self.node_arity)

    def _plain_soft(self):
        return self.gate_select == "softmax" or (
            not self.training and self.gate_select != "hard")

    def soft_records(self, in_shape, pool):
        """Per-channel records for input (C, H, W) and the pooled or plain
        forward: resolved taps, softmax leaf weights and node parameters
        (forward only, plain softmax)."""
        def build():
            cm, ch, cw = self._taps()
            conn = None if self.connect == "fixed" else self.conn
            return ops.conv_soft_records(conn, cm, ch, cw, self._raw(), self._kind(), self.d,
                                         self.node_arity, cm.shape[-1], tuple(in_shape),
                                         self.padding, pool)
        key = (derived.state_key(self), tuple(in_shape), bool(pool))
        return derived.cached(self, "_derived_records", key, build)

    def _soft(self, x, pool):
        ops.require_gpu(x)
        if x.shape[1] < self.cin:
            raise ValueError(f"ConvLogicTree: input has {x.shape[1]} channels, the trees read "
                             f"channels up to in_channels = {self.cin}")
        cm, ch, cw = self._taps()
        K = cm.shape[-1]
        if not self.generic and not _needs_grad(self, x) and self._plain_soft() and \
                not torch.compiler.is_compiling() and ops.conv_fits_lds(tuple(x.shape[1:]), self.padding,
                                                                        pool, self._kind(), self.d,
                                                                        self.node_arity, K):
            rec = self.soft_records(x.shape[1:], pool)
            return ops.conv_soft_rec(x, rec, self.n, self._kind(), self.d, self.node_arity, K,
                                     self.padding, pool)
        w, npar = self.soft_params(_needs_grad(self, x))
        return ops.conv_soft(x, npar, w, cm, ch, cw, self._kind(), self.d, self.node_arity, K,
                             self.padding, pool)

    def forward(self, x):
        return self._soft(x, pool=False)

    def forward_pooled(self, x):
        """``OrPool(2)(self(x))`` in one kernel (only the pooled map is written)."""
        return self._soft(x, pool=True)

    def hard_spec(self):
        """Arguments of ``ops.conv_hard_prep_net`` (or, for a generic tree,
        ``ops.conv_tree_hard_prep``) for this block: taps, connection logits
        and the node parameters per tree level, read in place."""
        cm, ch, cw = self._taps()
        conn = None if self.connect == "fixed" else self.conn
        if self.node_name == "gate16":
            levels = list(self.gate_logits)
        elif self.node_name == "walsh":
            levels = [nd.theta for nd in self.tree_nodes]
        else:
            levels = [nd.logits for nd in self.tree_nodes]
        return cm, ch, cw, conn, levels, self._kind(), self.d, self.node_arity

    def hard_params(self):
        """``(leaf [n, leaves] int32, tt)`` of the hard forward: ``tt`` [n]
        int64 (one word of tables per channel) for the LDS-kernel trees,
        [n, nodes] int64 per-node tables for a generic tree."""
        if self.generic:
            return ops.conv_tree_hard_prep(*self.hard_spec())
        return ops.conv_hard_prep_net([self.hard_spec()])[0]

    def packed_forward(self, xp, chw, pool, params=None):
        """Packed ``[C,H,W,nw]`` -> ``[n,Ho,Wo,nw]`` (2x2 OR-pooled if ``pool``);
        ``params`` = ``hard_params()`` when the caller computed them already."""
        leaf, tt = self.hard_params() if params is None else params
        if self.generic:
            return ops.conv_tree_hard(xp, chw, leaf, tt, self.node_arity, self.d, self.kh,
                                      self.padding, pool)
        return ops.conv_hard(xp, chw, leaf, tt, self._kind(), self.d, self.node_arity,
                             self.kh, self.padding, pool)

    @torch.no_grad()
    def forward_hard(self, x):
        ops.require_gpu(x)
        B, C, H, W = x.shape
        xp = ops.pack_bits(x.reshape(B, -1))
        yp = self.packed_forward(xp, (C, H, W), pool=False)
        Ho, Wo = self._hw_out(H, W)
        return ops.unpack_bits(yp.view(-1, yp.shape[-1]), B).view(B, self.n, Ho, Wo)


ConvLogicLayer = ConvLogicTree


class OrPool(nn.Module):
    """Logical OR pooling = spatial ``size`` x ``size`` max-pool with stride
    ``size`` (floor), silogic/layers.py:548-563."""

    def __init__(self, size=2):
        super().__init__()
        self.size = size

    def forward(self, x):
        return ops.orpool(x, self.size)

    @torch.no_grad()
    def forward_hard(self, x):
        return ops.orpool(x.to(torch.uint8), self.size)
