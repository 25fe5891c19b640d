"""End-to-end bit-packed inference (silogic/bitpacking/packed_model.py) on the
HIP kernels.

:class:`BitpackedNet` mirrors a LogicNet on ``[B, in_dim]`` {0,1} inputs and
:class:`BitpackedConvNet` a LogicConvNet on ``[B, C, H, W]`` inputs; both
return ``[B, num_classes]`` float32 logits divided by the GroupSum ``tau``
(packed_model.py:34-128, 131-283). Where the layers fit the fused kernels
(every FC layer two-input, inputs at most 16384 wide, the widths within
LDS; conv blocks with stride 1, 'same' padding, OR-pool 2 and a gate16 tree
of depth <= 4 or a one-level LUT) the whole FC stack is one launch and each
conv block one launch; other layers run the per-layer packed kernels. Inputs
may be numpy (copied to the GPU, logits returned as numpy) or torch tensors
(logits returned as a tensor on the same GPU).
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np
import torch

from .. import ops as _ops
from ..functional import TT_CODES
from .ops import divide_by_tau, like_input, mask_last_word, to_device
from .packed_layer import (
    BitpackedConvLUTLayer,
    BitpackedConvTreeLayer,
    BitpackedFCLayer,
    BitpackedGroupSumHead,
    BitpackedLUTLayer,
    pack_conv_input,
    packed_or_pool,
    packed_unfold,
    unpack_conv_output,
)

_COMPACT_MAX = 1 << 14


def _compact_codes(layer: BitpackedFCLayer, device) -> torch.Tensor:
    """Fused-network code ``b | a << 14 | tt << 28`` per output (inputs at most
    16384 wide)."""
    def make(d):
        tt = np.asarray(TT_CODES, dtype=np.int64)[layer.gate_types.astype(np.int64)]
        c = (layer.b_idx.astype(np.int64) | (layer.a_idx.astype(np.int64) << 14) | (tt << 28))
        return torch.from_numpy(c.astype(np.uint32).view(np.int32).copy()).to(d)
    return layer._codes.get(("compact", str(device)), lambda _: make(device))


def _fused_fc_ok(layers, in_dim, head) -> bool:
    if not isinstance(head, BitpackedGroupSumHead) or not layers:
        return False
    if not all(isinstance(l, BitpackedFCLayer) for l in layers):
        return False
    widths = [l.out_dim for l in layers]
    w_in = [in_dim] + widths[:-1]
    if max(w_in) > _COMPACT_MAX or any(l.max_idx >= w for l, w in zip(layers, w_in)):
        return False
    if widths[-1] % head.num_classes:
        return False
    return bool(_ops.fc_hard_net_supported(in_dim, widths, head.num_classes))


def _run_fc(layers, packed, B, head, wire_r, fallback, device):
    """FC stack on packed ``[dim, nw]`` activations, then the head."""
    if _fused_fc_ok(layers, packed.shape[0], head):
        codes = [_compact_codes(l, device) for l in layers]
        counts = _ops.fc_hard_net(packed, _ops.PACKED, B, packed.shape[0], codes,
                                  head.num_classes, wire_r)
        return divide_by_tau(counts, head.tau)
    for i, layer in enumerate(layers):
        if layer is None:
            bits = _ops.unpack_bits(packed, B)
            with torch.no_grad():
                out = fallback[i].forward_hard(bits)
            packed = _ops.pack_bits(out)
            continue
        prev = packed
        packed = layer.forward(packed)
        if wire_r and prev.shape[0] == packed.shape[0]:
            packed[:wire_r] = prev[:wire_r]
    mask_last_word(packed, B)
    return head.forward(packed, B)


class BitpackedNet:
    """Bit-packed LogicNet (packed_model.py:34-128): ``packed_layers``
    (BitpackedFCLayer / BitpackedLUTLayer, or None for a layer run through
    ``fallback_torch_layers[i].forward_hard``), a GroupSum head and the
    wire-residual width ``wire_r``."""

    def __init__(self, packed_layers: List, head, wire_r: int = 0,
                 fallback_torch_layers: Optional[Dict[int, object]] = None,
                 device=None) -> None:
        self.packed_layers = packed_layers
        self.head = head
        self.wire_r = int(wire_r)
        self.fallback = fallback_torch_layers or {}
        self.device = device
        self.num_layers = len(packed_layers)

    def _dev(self, x):
        if self.device is not None:
            return torch.device(self.device)
        return x.device if isinstance(x, torch.Tensor) and x.is_cuda else None

    def forward(self, x):
        """``[B, in_dim]`` {0,1} uint8/bool/float -> ``[B, num_classes]`` float32."""
        t = to_device(x, device=self._dev(x))
        if t.dim() != 2:
            raise ValueError("BitpackedNet: x must be [B, in_dim]")
        B, in_dim = t.shape
        if t.dtype == torch.bool:
            t = t.to(torch.uint8)
        layers = self.packed_layers
        if (t.dtype == torch.uint8 and _fused_fc_ok(layers, in_dim, self.head)):
            # rows straight into the fused kernel: packing happens inside it
            codes = [_compact_codes(l, t.device) for l in layers]
            out = divide_by_tau(_ops.fc_hard_net(t, _ops.ROWS_U8, B, in_dim, codes,
                                                 self.head.num_classes, self.wire_r),
                                self.head.tau)
        else:
            packed = _ops.pack_bits(t)
            out = _run_fc(layers, packed, B, self.head, self.wire_r, self.fallback, t.device)
        return like_input(out, x)

    __call__ = forward

    def layer_summary(self) -> list:
        rows = []
        for i, layer in enumerate(self.packed_layers):
            if layer is None:
                rows.append({"layer": i, "mode": "uint8-fallback"})
            elif isinstance(layer, BitpackedFCLayer):
                hist = layer.gate_histogram
                top = sorted(hist.items(), key=lambda kv: -kv[1])[:3]
                rows.append({"layer": i, "mode": "gate16", "out_dim": layer.out_dim,
                             "n_gate_types": len(hist), "top_gates": top})
            else:
                rows.append({"layer": i, "mode": "lut", "out_dim": layer.out_dim,
                             "arity": layer.arity})
        return rows


class BitpackedConvNet:
    """Bit-packed LogicConvNet (packed_model.py:131-283): per (conv, pool)
    block a BitpackedConvTreeLayer / BitpackedConvLUTLayer (None = run the
    block's ``forward_hard``), then the packed FC head layers and the head.
    Activations stay B-packed ``[dim, L, nw_B]`` from the input pack to the
    head's GroupSum."""

    def __init__(self, conv_blocks, bp_conv_layers: Optional[List], packed_head_layers: List,
                 head, fallback_head_torch: Optional[Dict[int, object]] = None,
                 wire_residual: float = 0.0, device=None) -> None:
        self.conv_blocks = conv_blocks
        self.bp_conv_layers = bp_conv_layers or []
        self.packed_head_layers = packed_head_layers
        self.head = head
        self.fallback_head = fallback_head_torch or {}
        self.wire_residual = wire_residual
        self.device = device

    def _block(self, i, x3, C, H, W, B):
        """One (conv, pool) block on packed ``x3`` [C, H*W, nw] -> pooled
        ``[n, Ho', Wo', nw]`` flattened to ``[n, L', nw]``, with its sizes."""
        conv = self.conv_blocks[2 * i]
        pool = self.conv_blocks[2 * i + 1]
        ps = getattr(pool, "size", 2)
        bp = self.bp_conv_layers[i] if i < len(self.bp_conv_layers) else None
        nw = x3.shape[-1]
        if bp is not None:
            Ho = (H + 2 * bp.padding - bp.kh) // bp.stride + 1
            Wo = (W + 2 * bp.padding - bp.kw) // bp.stride + 1
            r = min(int(bp.n_out * self.wire_residual), C) if self.wire_residual > 0 else 0
            if bp.fused_ok() and ps == 2:
                leaf, tt, kind, depth, arity = bp.fused_params(x3.device)
                y = _ops.conv_hard(x3, (C, H, W), leaf, tt, kind, depth, arity, bp.kh,
                                   bp.padding, True)                       # [n, Ho/2, Wo/2, nw]
                y = y.view(bp.n_out, -1, nw)
                if r > 0:   # channel-wise copy before the pool = pooled copy
                    y[:r] = packed_or_pool(x3[:r, :Ho * Wo].contiguous(), Ho, Wo, 2)
            else:
                xu = packed_unfold(x3, bp.kh, bp.kw, bp.stride, bp.padding, H, W)
                y3 = bp.forward_packed(xu)                                 # [n, Ho*Wo, nw]
                if r > 0:
                    y3[:r] = x3[:r, :Ho * Wo]
                y = packed_or_pool(y3, Ho, Wo, ps)
            return y, bp.n_out, Ho // ps, Wo // ps
        # block without a packed layer: its own forward_hard on unpacked bits
        xb = unpack_conv_output(x3, B, H, W)
        with torch.no_grad():
            y = conv.forward_hard(xb)
            if self.wire_residual > 0:
                r = min(int(conv.n * self.wire_residual), xb.shape[1])
                if r > 0:
                    y = torch.cat([xb[:, :r], y[:, r:]], dim=1)
            pooled = pool.forward_hard(y)
        n, Hp, Wp = pooled.shape[1:]
        return pack_conv_input(pooled), n, Hp, Wp

    def forward(self, x):
        """``[B, C, H, W]`` (or ``[B, in_dim]``) {0,1} -> ``[B, num_classes]`` float32."""
        dev = torch.device(self.device) if self.device is not None else None
        t = to_device(x, device=dev)
        if t.dtype == torch.bool:
            t = t.to(torch.uint8)
        B = t.shape[0]
        if t.dim() == 4:
            _, C, H, W = t.shape
            x3 = pack_conv_input(t)
            for i in range(len(self.bp_conv_layers)):
                x3, C, H, W = self._block(i, x3, C, H, W, B)
            packed = x3.reshape(-1, x3.shape[-1]).contiguous()             # flatten (n, h, w)
        else:
            packed = _ops.pack_bits(t)
        out = _run_fc(self.packed_head_layers, packed, B, self.head, 0, self.fallback_head,
                      t.device)
        return like_input(out, x)

    __call__ = forward


# ── GPU helpers and the GPU network (all of the above already runs on the GPU) ──

def packed_unfold_gpu(x_3d: torch.Tensor, kh: int, kw: int, stride: int, padding: int,
                      H_in: int, W_in: int) -> torch.Tensor:
    """Spatial unfold of B-packed activations on the GPU (packed_model.py:287-341)."""
    return packed_unfold(x_3d, kh, kw, stride, padding, H_in, W_in)


def packed_or_pool_gpu(x_3d: torch.Tensor, H: int, W: int, pool_size: int = 2) -> torch.Tensor:
    """OR-pool of B-packed activations on the GPU (packed_model.py:344-383)."""
    return packed_or_pool(x_3d, H, W, pool_size)


class BitpackedConvGPUNet:
    """GPU bit-packed LogicConvNet (packed_model.py:388-631). Built from a
    :class:`BitpackedConvNet` with :meth:`from_conv_net`; every block and the
    head run on the GPU ``device``."""

    def __init__(self, bp_conv_net: BitpackedConvNet, block_spatial: list, device="cuda") -> None:
        self.bp_conv_net = bp_conv_net
        self.block_spatial = block_spatial
        self.head = bp_conv_net.head
        self.device = device
        self.gpu_conv_layers = bp_conv_net.bp_conv_layers
        self.gpu_head_layers = bp_conv_net.packed_head_layers

    @classmethod
    def from_conv_net(cls, bp_conv_net: BitpackedConvNet, H_in: int, W_in: int,
                      device="cuda") -> "BitpackedConvGPUNet":
        spatial = []
        cur_H, cur_W = H_in, W_in
        for i, bp in enumerate(bp_conv_net.bp_conv_layers):
            conv = bp_conv_net.conv_blocks[2 * i]
            ps = getattr(bp_conv_net.conv_blocks[2 * i + 1], "size", 2)
            k = bp.kh if bp is not None else conv.kh
            pad = bp.padding if bp is not None else conv.padding
            stride = bp.stride if bp is not None else conv.stride
            Ho = (cur_H + 2 * pad - k) // stride + 1
            Wo = (cur_W + 2 * pad - k) // stride + 1
            spatial.append((cur_H, cur_W, Ho, Wo, ps))
            cur_H, cur_W = Ho // ps, Wo // ps
        net = BitpackedConvNet(bp_conv_net.conv_blocks, bp_conv_net.bp_conv_layers,
                               bp_conv_net.packed_head_layers, bp_conv_net.head,
                               bp_conv_net.fallback_head, bp_conv_net.wire_residual,
                               device=device)
        return cls(net, spatial, device)

    def forward(self, x):
        return self.bp_conv_net.forward(x)

    __call__ = forward
