"""Networks (mirror of silogic/models.py): ``LogicNet`` (+ the ``WARPNet``,
``WARPNetN``, ``LUTkNet``, ``LUTNodeNet`` presets) and ``LogicConvNet`` /
``LogicTreeNet``.

Construction and ``state_dict`` keys follow the reference (per-layer seeds
``seed*seed_mult+i``, conv block seeds ``seed*17+i``, head seeds ``seed*31+j``;
silogic/models.py:59-86, 208-246).

``forward`` runs layer by layer on the HIP soft kernels (conv blocks with
their OrPool fused). Without gradients, the parameters of every FC layer are
prepared in one launch (per-output records) and the last FC layer is fused
with the GroupSum head when the head thresholds its features (the feature
STE, on by default). ``forward_hard`` runs the network as one bit-packed
circuit: 64 samples per word, the FC stack depth-fused in LDS with the
GroupSum popcount at the end (``slg_fc_hard_net``), conv blocks as packed
tree + OR-pool kernels. It returns the same raw integer counts as the
reference's ``GroupSum.forward_hard`` (heads.py:41-45).
"""
import ctypes
import threading

import torch
import torch.nn as nn

from . import derived, ops
from .heads import GroupSum, build_decoder
from .layers import LogicLayer, ConvLogicTree, OrPool, _needs_grad


def _per_layer(v, i):
    return v[i] if isinstance(v, (list, tuple)) else v


def _soft_fc_stack(layers, head, x, wire_r):
    """Soft forward of arity-2 FC layers + GroupSum head on records (no
    gradients). Returns ``None`` when a layer needs the autograd path (a
    non-softmax selection) so the caller runs layer by layer. The records
    are built once per parameter version and the launches once per batch
    shape (``ops.SoftStackPlan``)."""
    if x.dtype != torch.float32:
        x = x.float()
    pkey = derived.state_key(*layers)
    shape_key = (pkey, tuple(x.shape), tuple(layer.training for layer in layers), id(head),
                 getattr(head, "feature_ste", None), getattr(head, "tau", None), wire_r)

    def build():
        Ks = {layer.n_candidates for layer in layers}
        if not layers or not all(layer.records_ok() for layer in layers) or len(Ks) != 1:
            return None
        K = Ks.pop()
        recs = derived.cached(
            layers[0], "_derived_net_records", (pkey, K),
            lambda: ops.fc_soft_records([layer.record_spec() for layer in layers], K))
        B, IN = x.shape
        last = layers[-1]
        w_last = layers[-2].out_dim if len(layers) > 1 else IN    # the last layer's input width
        ste = (isinstance(head, GroupSum) and head.feature_ste
               and not (wire_r and w_last == last.out_dim))
        spec = [(rec, layer.in_dim, layer.out_dim, K, layer.node.kind, layer._inv_tau())
                for layer, rec in zip(layers, recs)]
        head_args = (head.num_classes, float(head.tau)) if ste else None
        plan = ops.SoftStackPlan(spec, B, IN, head_args, wire_r)
        # a launch per layer fuses the head only where one workgroup holds
        # every output of its tile; the one-launch network always can
        if ste and plan.net is None and not ops.fc_soft_groupsum_supported(
                B, w_last, last.out_dim, head.num_classes):
            plan = ops.SoftStackPlan(spec, B, IN, None, wire_r)
        return plan

    plan = derived.cached(layers[0], "_derived_soft_plan", shape_key, build)
    if plan is None:
        return None
    out = plan(x)
    return out if plan.head is not None else head(out)


def _hard_fc_plan(layers, in_dim, C):
    """``(lut, widths, spw, typable)`` of an FC stack's hard forward: LUT
    layers run one packed kernel each; otherwise ``spw`` (64 or 32) says the
    fused network fits LDS and ``typable`` that the type-uniform layout
    applies."""
    def plan():
        widths = [layer.out_dim for layer in layers]
        lut = any(layer.is_lut for layer in layers)
        spw = 0 if lut else ops.fc_hard_net_supported(in_dim, widths, C)
        return lut, widths, spw, spw and ops.fc_hard_type_slots(in_dim, widths) > 0

    return derived.cached(
        layers[0], "_derived_net_plan", (in_dim, C, tuple(id(layer) for layer in layers)), plan)


def _hard_fc_net_codes(layers, in_dim, wire_r, typed):
    """The fused network's codes (cached per parameter version): type-placed
    when ``typed``, bank-placed without a wire residual, else in index order."""
    def build():
        codes = ops.fc_hard_codes_net([layer.hard_spec() for layer in layers], compact=True)
        if typed:
            return ops.fc_hard_type_place_net(codes, in_dim)
        return ops.NetCodes(codes if wire_r else ops.fc_hard_place_net(codes))

    # the type-uniform layout's slot count follows the input width, so the
    # width is part of the key
    return derived.cached(layers[0], "_derived_net_codes",
                          (derived.state_key(*layers), int(in_dim), bool(wire_r), typed), build)


def _hard_fc_stack(layers, x, in_kind, B, in_dim, C, wire_r):
    """Run arity-2 FC layers as a packed circuit and return class counts.

    ``in_kind`` is ROWS_F32 / ROWS_U8 for ``[B, in_dim]`` inputs or PACKED for
    ``[in_dim, nw]`` words. Depth-fused in LDS when the widths fit, with the
    packing of rows fused into it; otherwise one packed kernel per layer."""
    lut, widths, spw, typable = _hard_fc_plan(layers, in_dim, C)
    if lut:
        # LUT layers: one packed kernel per layer (gate or LUT)
        xp = x if in_kind == ops.PACKED else ops.pack_bits(x)
        for layer in layers:
            yp = layer.packed_forward(xp)
            if wire_r and yp.shape[0] == xp.shape[0]:
                yp[:wire_r] = xp[:wire_r]
            xp = yp
        return ops.groupsum_packed(xp, B, C)
    if spw:
        # one gate type per wave row where the layout fits, else a bank-aware
        # output order; both relabel the circuit (the logits are the same
        # bits). The wire residual copies inputs by position, so it keeps
        # the order.
        typed = bool(not wire_r and typable)
        codes = _hard_fc_net_codes(layers, in_dim, wire_r, typed)
        return ops.fc_hard_net(x, in_kind, B, in_dim, codes, C, wire_r)
    codes = ops.fc_hard_codes_net([layer.hard_spec() for layer in layers])
    xp = x if in_kind == ops.PACKED else ops.pack_bits(x)
    for c in codes:
        yp = ops.fc_hard_layer(xp, c)
        if wire_r and yp.shape[0] == xp.shape[0]:
            yp[:wire_r] = xp[:wire_r]
        xp = yp
    return ops.groupsum_packed(xp, B, C)


class LogicNet(nn.Module):
    """Stack of logic layers followed by a GroupSum head (arguments as
    silogic.models.LogicNet)."""

    def __init__(self, in_dim, width, depth, num_classes=10, node="gate16",
                 connectome="topk", arity=2, k=8, tau=1.0, gate_eval="basis",
                 node_tau=1.0, residual_p=0.0, seed=0,
                 wire_residual=0.0, decoder="groupsum", degree=None, seed_mult=1000,
                 gate_select="softmax", gumbel_tau=1.0, decoder_ste=True,
                 use_triton=True):
        super().__init__()
        layers = []
        d_in = in_dim
        for i in range(depth):
            layers.append(LogicLayer(
                d_in, width, node=_per_layer(node, i), connectome=connectome,
                arity=arity, k=k, gate_eval=gate_eval, residual_p=residual_p,
                degree=degree, tau=node_tau,
                gate_select=_per_layer(gate_select, i), gumbel_tau=gumbel_tau,
                use_triton=use_triton,
                seed=None if seed is None else seed * seed_mult + i))
            d_in = width
        self.layers = nn.ModuleList(layers)
        self.head = build_decoder(decoder, width, num_classes, tau, feature_ste=decoder_ste)
        self.width = width
        self.depth = depth
        self.node = node
        self.connectome = connectome
        self.k = k
        self.decoder_kind = decoder
        self.wire_r = int(width * wire_residual)

    def _run(self, x):
        for layer in self.layers:
            y = layer(x)
            if self.wire_r and x.shape[1] == y.shape[1]:
                y = torch.cat([x[:, :self.wire_r], y[:, self.wire_r:]], dim=1)
            x = y
        return x

    def forward(self, x):
        ops.require_gpu(x)
        ops.check_width(x, self.layers[0].in_dim)
        if not _needs_grad(self, x):
            out = _soft_fc_stack(self.layers, self.head, x, self.wire_r)
            if out is not None:
                return out
        return self.head(self._run(x))

    @torch.no_grad()
    def forward_hard(self, x):
        ops.require_gpu(x)
        ops.check_width(x, self.layers[0].in_dim)
        if (x.dim() == 2 and x.dtype in (torch.float32, torch.uint8) and x.is_contiguous()
                and not torch.compiler.is_compiling()):
            key = (derived.state_key(self), tuple(x.shape), x.dtype, x.get_device(),
                   ops._stream(x).value)
            step = derived.cached(self, "_derived_hard_step", key,
                                  lambda: _HardStep.for_fc(self, x))
            if step is not None:
                return step(x)
        x, kind = ops._in_kind(x)
        return _hard_fc_stack(self.layers, x, kind, x.shape[0], x.shape[1],
                              self.head.num_classes, self.wire_r)

    @torch.no_grad()
    def forward_hard_packed(self, xp, B, word_major=False):
        """``forward_hard`` on packed input for ``B`` samples: ``[in_dim, nw]``
        rows, or ``[nw, in_dim]`` words with ``word_major`` (the layouts of
        ``ops.pack_bits`` and ``data.binarize_packed``): class counts."""
        ops.require_gpu(xp)
        if word_major:
            if xp.dim() != 2 or xp.shape[0] != ops.n_words(B):
                raise ValueError("forward_hard_packed: word-major input must be [nw, in_dim]")
            in_dim = xp.shape[1]
            if any(layer.is_lut for layer in self.layers) or not ops.fc_hard_net_supported(
                    in_dim, [l.out_dim for l in self.layers], self.head.num_classes):
                xp, kind = xp.t().contiguous(), ops.PACKED     # the per-layer kernels take rows
            else:
                xp, kind = xp.contiguous(), ops.PACKED_WORD_MAJOR
        else:
            xp, kind = ops._words_for(xp, B, "forward_hard_packed"), ops.PACKED
            in_dim = xp.shape[0]
        return _hard_fc_stack(self.layers, xp, kind, B, in_dim, self.head.num_classes,
                              self.wire_r)

    def num_gates(self):
        return self.width * self.depth


class WARPNet(LogicNet):
    """Stack of 2-input Walsh (WARP) layers + GroupSum head (tau 20)."""

    def __init__(self, in_dim, width, depth, num_classes=10, k=8, tau=1.0,
                 residual_p=0.0, seed=0, gate_select="softmax"):
        super().__init__(in_dim, width, depth, num_classes=num_classes, node="walsh",
                         arity=2, k=k, node_tau=tau, tau=20.0, residual_p=residual_p,
                         seed=seed, gate_select=gate_select)


class WARPNetN(LogicNet):
    """Stack of arity-``n`` Walsh (WARP) layers + GroupSum head (preset,
    silogic/models.py:117-125)."""

    def __init__(self, in_dim, width, depth, arity=6, num_classes=10, k=8, tau=1.0,
                 residual_p=0.0, seed=0, gate_select="softmax"):
        super().__init__(in_dim, width, depth, num_classes=num_classes, node="walsh",
                         arity=arity, k=k, node_tau=tau, tau=20.0, residual_p=residual_p,
                         seed=seed, gate_select=gate_select)


class LUTkNet(LogicNet):
    """Stack of k-input multilinear LUT layers + GroupSum head (preset,
    silogic/models.py:128-138)."""

    def __init__(self, in_dim, width, depth, k=4, num_classes=10, tau=4.0, cand_k=4, seed=0):
        super().__init__(in_dim, width, depth, num_classes=num_classes, node="multilinear",
                         arity=k, k=cand_k, tau=tau, seed=seed)
        self.lut_inputs = k

    def num_luts(self):
        return self.width * self.depth


class LUTNodeNet(LogicNet):
    """Stack of n-input LUT-node layers (selectable relaxation) + GroupSum
    head (preset, silogic/models.py:141-147)."""

    def __init__(self, in_dim, width, depth, arity=4, relaxation="probabilistic",
                 num_classes=10, k=8, tau=10.0, residual_p=0.0, seed=0):
        super().__init__(in_dim, width, depth, num_classes=num_classes, node=relaxation,
                         arity=arity, k=k, tau=tau, residual_p=residual_p, seed=seed)


class LogicConvNet(nn.Module):
    """Convolutional logic-gate-tree network with a logic head (arguments as
    silogic.models.LogicConvNet)."""

    def __init__(self, in_channels, in_hw, channels, head_width=None,
                 num_classes=10, tree_depth=None, kernel=3, connect="topk",
                 k=4, head_connect="topk", head_k=8, head_depth=2,
                 n_chan=2, residual_init=True, tau=100.0, seed=0,
                 wire_residual=0.0, head_widths=None,
                 decoder="groupsum", node="gate16", arity=2, node_tau=1.0,
                 degree=None, gate_select="softmax", gumbel_tau=1.0,
                 decoder_ste=True, use_triton=True):
        super().__init__()
        self.blocks = nn.ModuleList()
        c = in_channels
        for i, n in enumerate(channels):
            self.blocks.append(ConvLogicTree(
                c, n, kernel=kernel, tree_depth=tree_depth, stride=1,
                padding=kernel // 2, connect=connect, k=k, n_chan=n_chan,
                residual_init=residual_init, seed=seed * 17 + i,
                node=node, arity=arity, tau=node_tau, degree=degree,
                gate_select=gate_select, gumbel_tau=gumbel_tau, use_triton=use_triton))
            self.blocks.append(OrPool(2))
            c = n
            in_hw = in_hw // 2
        self.feat_dim = c * in_hw * in_hw
        if head_widths is None:
            head_widths = [head_width] * head_depth
        layers = []
        d_in = self.feat_dim
        for j, w in enumerate(head_widths):
            layers.append(LogicLayer(d_in, w, connectome=head_connect, k=head_k, node=node,
                                     gate_select=gate_select, use_triton=use_triton,
                                     seed=seed * 31 + j))
            d_in = w
        self.head_layers = nn.ModuleList(layers)
        self.head = build_decoder(decoder, head_widths[-1], num_classes, tau,
                                  feature_ste=decoder_ste)
        self.decoder_kind = decoder
        self._head_widths = head_widths
        self.wire_residual = wire_residual

    def _convs(self):
        return [self.blocks[i] for i in range(0, len(self.blocks), 2)]

    def _apply_blocks(self, x):
        for conv in self._convs():
            if self.wire_residual > 0:
                x_in = x
                y = conv(x)
                r = min(int(conv.n * self.wire_residual), x_in.shape[1])
                if r > 0:
                    y = torch.cat([x_in[:, :r], y[:, r:]], dim=1)
                x = ops.orpool(y, 2)
            else:
                x = conv.forward_pooled(x)
        return x

    def forward(self, x):
        ops.require_gpu(x)
        x = self._apply_blocks(x).flatten(1)
        if not _needs_grad(self, x):
            out = _soft_fc_stack(self.head_layers, self.head, x, 0)
            if out is not None:
                return out
        for layer in self.head_layers:
            x = layer(x)
        return self.head(x)

    @torch.no_grad()
    def forward_hard(self, x):
        ops.require_gpu(x)
        step = self._hard_step(x)
        if step is not None:
            return step(x)
        B, C, H, W = x.shape
        xp = ops.pack_bits(x.reshape(B, -1))                  # [C*H*W, nw] = [C,H,W,nw]
        return self.forward_hard_packed(xp, B, (C, H, W))

    def _hard_step(self, x):
        """The launch sequence of ``forward_hard`` for ``x``'s shape on the
        current stream (:class:`_HardStep`, cached per parameter
        version), or None where the general path runs."""
        if (x.dim() != 4 or x.dtype not in (torch.float32, torch.uint8) or not x.is_contiguous()
                or self.wire_residual > 0 or torch.compiler.is_compiling()):
            return None
        key = (derived.state_key(self), tuple(x.shape), x.dtype, x.get_device(),
               ops._stream(x).value)
        return derived.cached(self, "_derived_hard_step", key,
                              lambda: _HardStep.for_conv(self, x))

    @torch.no_grad()
    def forward_hard_packed(self, xp, B, chw):
        """``forward_hard`` on packed input ``[C*H*W, nw]`` (the layout of
        ``ops.pack_bits`` and ``data.binarize_packed`` for images, channel-
        major) for ``B`` samples of shape ``chw``: class counts ``[B, C]``."""
        ops.require_gpu(xp)
        C, H, W = chw
        xp = ops._words_for(xp, B, "forward_hard_packed")
        if xp.shape[0] != C * H * W:
            raise ValueError("forward_hard_packed: %d rows for C*H*W = %d" % (xp.shape[0], C * H * W))
        convs = list(self._convs())
        # the LDS-kernel trees of every block in one prep launch, generic
        # trees (walsh, deeper LUT trees) with their own per-node tables
        lds = [conv for conv in convs if not conv.generic]
        batched = iter(derived.cached(
            self, "_derived_conv_codes", derived.state_key(*lds),
            lambda: ops.conv_hard_prep_net([conv.hard_spec() for conv in lds])) if lds else [])
        params = [conv.hard_params() if conv.generic else next(batched) for conv in convs]
        for conv, prm in zip(convs, params):
            x_in = xp
            xp = conv.packed_forward(xp, (C, H, W), pool=True, params=prm)
            Ho, Wo = conv._hw_out(H, W)
            if self.wire_residual > 0:
                # the first r channels copy the input before the OR-pool
                # (models.py:252-261); pooling is channel-wise, so pool them
                r = min(int(conv.n * self.wire_residual), C)
                if r > 0:
                    nw = xp.shape[-1]
                    res = ops.packed_or_pool(x_in.reshape(C, H * W, nw)[:r].contiguous(), Ho, Wo)
                    xp.view(conv.n, -1, nw)[:r] = res
            C, H, W = conv.n, Ho // 2, Wo // 2
        xp = xp.view(-1, xp.shape[-1])                        # flatten (n, h, w)
        return _hard_fc_stack(self.head_layers, xp, ops.PACKED, B, xp.shape[0],
                              self.head.num_classes, 0)

    def gate_count(self, in_hw):
        total = 0
        hw = in_hw
        for blk in self.blocks:
            if isinstance(blk, ConvLogicTree):
                total += blk.n * hw * hw * blk.gates_per_output
            elif isinstance(blk, OrPool):
                hw = hw // 2
        total += sum(self._head_widths)
        return total


class _HardStep:
    """A network's ``forward_hard`` for one input shape on one stream as one
    C-ABI call (``slg_hard_step``): for a conv network packing, every conv
    block (pooled) and the fused head (which evaluates the last block itself
    where ``fuses_head`` is set); for an FC network the fused network on the
    rows. The per-call host
    work of the general path (parameter walks for each table, shape checks,
    wrapper calls, an allocation per intermediate, a C-ABI call per launch
    with its argument conversion) is done once here, into a
    ``slg_hard_step_t`` descriptor: the intermediate words live in buffers
    this object keeps (the launches run in stream order, so a call's packing
    cannot overtake the previous call's reads of them) and a call allocates
    only its logits. The tables are the general path's own, so the logits
    are the same bits."""

    def __init__(self, step, out_shape, st, bufs, tables):
        from . import _lib
        self.step, self.out_shape, self.st = step, out_shape, st
        self.bufs, self.tables = bufs, tables          # kept alive for the pointers
        self.fn, self.ref = _lib.lib().slg_hard_step, ctypes.byref(step)
        # 1: the one-layer head evaluates the last conv block, 2: the fused head network does
        self.fuses_head = int(_lib.lib().slg_hard_step_fuses_head(self.ref))
        # the descriptor's buffers are shared by every call: a second host
        # thread's packing must not land between this call's packing and
        # the launches that read it
        self.lock = threading.Lock()

    @staticmethod
    def _head(step, head_in, head_kind, in_dim, codes, n_cls, wire_r):
        """The fused head's fields, as ``ops.fc_hard_net`` passes them."""
        if codes.plan is not None and (wire_r or in_dim != codes.in_dim):
            raise ValueError("forward_hard: type-placed codes take inputs %s wide and no wire "
                             "residual (got %d, wire_r %d)" % (codes.in_dim, in_dim, wire_r))
        step.head_in, step.head_in_kind, step.head_in_dim = head_in, head_kind, in_dim
        step.n_layers, step.n_classes, step.wire_r = len(codes), n_cls, int(wire_r)
        step.widths = ctypes.cast(codes.widths, ctypes.c_void_p)
        step.codes = ctypes.cast(codes.ptrs, ctypes.c_void_p)
        step.plan = ops._p(codes.plan) if codes.plan is not None else None

    @staticmethod
    def for_fc(model, x):
        """LogicNet: the fused network on rows (packed inside it); None for
        LUT layers or widths past LDS."""
        from . import _lib
        layers, n_cls = list(model.layers), model.head.num_classes
        B, in_dim = x.shape
        lut, widths, spw, typable = _hard_fc_plan(layers, in_dim, n_cls)
        if lut or not spw:
            return None
        wire_r = model.wire_r
        codes = _hard_fc_net_codes(layers, in_dim, wire_r, bool(not wire_r and typable))
        kind = 1 if x.dtype == torch.uint8 else 0
        step = _lib.HardStep()
        step.dtype, step.B, step.pack = kind, B, 0
        _HardStep._head(step, None, kind, in_dim, codes, n_cls, wire_r)
        return _HardStep(step, (B, n_cls), ops._stream(x), [], [codes])

    @staticmethod
    def for_conv(model, x):
        """LogicConvNet: packing, the pooled conv blocks, the fused head, all
        on word-major words (one 64-sample column of an image contiguous).
        The images between blocks keep a zero border as wide as the next
        block's padding (cleared here, once; the kernels write only the
        interiors), so the conv kernels read every leaf unconditionally.
        None for generic trees, LUT head layers, head widths past LDS or more
        blocks than the descriptor holds."""
        from . import _lib
        convs = list(model._convs())
        if not convs or any(conv.generic for conv in convs) or \
                len(convs) > _lib.STEP_MAX_CONV:
            return None
        B, C, H, W = x.shape
        nw = ops.n_words(B)
        dev = x.device
        pads = [conv.padding for conv in convs] + [0]
        xp = torch.zeros((nw, C, H + 2 * pads[0], W + 2 * pads[0]), device=dev, dtype=torch.int64)
        step = _lib.HardStep()
        step.pack, step.dtype, step.B = 1, 1 if x.dtype == torch.uint8 else 0, B
        step.C, step.H, step.W, step.pack_pad, step.packed = C, H, W, pads[0], ops._p(xp)
        bufs, tables = [xp], []
        params = derived.cached(
            model, "_derived_conv_codes", derived.state_key(*convs),
            lambda: ops.conv_hard_prep_net([conv.hard_spec() for conv in convs]))
        cur = xp
        for i, (conv, (leaf, tt)) in enumerate(zip(convs, params)):
            k, pad, opad = conv.kh, conv.padding, pads[i + 1]
            Hf, Wf = H + 2 * pad - k + 1, W + 2 * pad - k + 1
            Ho, Wo = Hf // 2, Wf // 2                     # every block is OR-pooled
            out = torch.zeros((nw, conv.n, Ho + 2 * opad, Wo + 2 * opad), device=dev,
                              dtype=torch.int64)
            step.conv[i] = _lib.StepConv(ops._p(cur), ops._p(out), C, H, W, conv.n,
                                         conv._kind(), conv.d, conv.node_arity, k, pad, opad,
                                         ops._p(leaf), ops._p(tt))
            bufs.append(out)
            tables += [leaf, tt]
            cur, (C, H, W) = out, (conv.n, Ho, Wo)
        step.n_conv = len(convs)
        in_dim, n_cls, layers = C * H * W, model.head.num_classes, list(model.head_layers)
        if not layers:
            return None
        lut, widths, spw, typable = _hard_fc_plan(layers, in_dim, n_cls)
        if lut or not spw:
            return None
        codes = _hard_fc_net_codes(layers, in_dim, 0, bool(typable))
        tables.append(codes)
        _HardStep._head(step, ops._p(cur), ops.PACKED_WORD_MAJOR, in_dim, codes, n_cls, 0)
        return _HardStep(step, (B, n_cls), ops._stream(x), bufs, tables)

    def __call__(self, x):
        from . import _lib
        out = torch.empty(self.out_shape, device=x.device, dtype=torch.float32)
        with self.lock:
            _lib.check(self.fn(self.ref, x.data_ptr(), out.data_ptr(), self.st), "slg_hard_step")
        return out


class LogicTreeNet(LogicConvNet):
    """Convolutional logic-gate-tree network preset (Top-K wiring)."""
