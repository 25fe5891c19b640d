"""Convert silogic_amd models to bit-packed inference (silogic/bitpacking/convert.py).

* LogicLayer (two-input gate16 / walsh / multilinear nodes, top-k or fixed
  wiring) -> :class:`BitpackedFCLayer`.
* ConvLogicTree with gate16 trees -> :class:`BitpackedConvTreeLayer`; with
  one-level multilinear LUT nodes -> :class:`BitpackedConvLUTLayer`.
* LogicNet -> :class:`BitpackedNet`; LogicConvNet -> :class:`BitpackedConvNet`.

The hard parameters (argmax wiring, gate types, LUT truth tables) come from
the same HIP prep kernels that ``forward_hard`` uses, so a converted network
returns ``forward_hard``'s GroupSum counts divided by ``tau``
(convert.py:165-402 semantics: argmax of the wiring logits, argmax gate,
sign of the LUT logits, Walsh truth table from the node's own sum).
"""
from __future__ import annotations

import numpy as np
import torch

from .. import ops as _ops
from .ops import code_to_gate16
from .packed_layer import (
    BitpackedConvLUTLayer,
    BitpackedConvTreeLayer,
    BitpackedFCLayer,
    BitpackedGroupSumHead,
    BitpackedLUTLayer,
)
from .packed_model import BitpackedConvNet, BitpackedNet


def convert_layer(layer):
    """One LogicLayer -> :class:`BitpackedFCLayer` (gate16 / walsh / arity-2
    multilinear, convert.py:165-214) or :class:`BitpackedLUTLayer` (hybrid
    and multilinear LUT layers of any arity, convert.py:84-120)."""
    if getattr(layer, "is_lut", False):
        with torch.no_grad():
            idx, tt = layer.lut_hard_codes()                            # HIP prep
            idx = idx.cpu().numpy().astype(np.int32)
            words = tt.cpu().numpy().astype(np.uint64)
        n = idx.shape[1]
        tables = ((words[:, None] >> np.arange(1 << n, dtype=np.uint64)[None, :]) & 1).astype(bool)
        return BitpackedLUTLayer(tables, idx)
    with torch.no_grad():
        codes = layer.hard_codes().cpu().numpy().astype(np.int64)      # [OUT, 2]
    a_idx = codes[:, 0].astype(np.int32)
    hi = codes[:, 1] & 0xFFFFFFFF
    b_idx = (hi & 0x0FFFFFFF).astype(np.int32)
    gates = code_to_gate16()[(hi >> 28) & 15]
    return BitpackedFCLayer(gates, a_idx, b_idx)


def convert_conv_tree_layer(layer):
    """One ConvLogicTree -> :class:`BitpackedConvTreeLayer` (gate16) or
    :class:`BitpackedConvLUTLayer` (multilinear LUT) (convert.py:219-296)."""
    with torch.no_grad():
        leaf, tt = layer.hard_params()                                  # HIP prep
        leaf = leaf.cpu().numpy().astype(np.int64)
        tt = tt.cpu().numpy().astype(np.int64)
    kh, kw = layer.kh, layer.kw
    cm, ch, cw = leaf >> 8, (leaf >> 4) & 15, leaf & 15
    leaf_idx = (cm * kh * kw + ch * kw + cw).astype(np.int32)           # flat unfold rows
    kw_args = dict(kh=kh, kw=kw, stride=layer.stride, padding=layer.padding, cin=layer.cin)
    n = layer.n
    if layer._kind() == _ops.GATE16:
        lut = code_to_gate16()
        per_level, nb, cnt = [], 0, layer.leaves // 2
        while cnt >= 1:
            codes = np.stack([(tt >> (4 * (nb + m))) & 15 for m in range(cnt)], axis=1)
            per_level.append(lut[codes].astype(np.int32))               # [n, cnt]
            nb += cnt
            cnt //= 2
        return BitpackedConvTreeLayer(leaf_idx, per_level, **kw_args)
    arity = layer.node_arity
    bits = ((tt[:, None] >> np.arange(2 ** arity)[None, :]) & 1).astype(bool)  # [n, 2^arity]
    return BitpackedConvLUTLayer(leaf_idx, [bits], arity, **kw_args)


def convert_head(head) -> BitpackedGroupSumHead:
    """GroupSum -> :class:`BitpackedGroupSumHead` (convert.py:301-309)."""
    from ..heads import GroupSum
    if isinstance(head, GroupSum):
        return BitpackedGroupSumHead(head.num_classes, head.tau)
    raise TypeError(f"Unsupported head type: {type(head)}")


def _device_of(model):
    for p in list(model.parameters()) + list(model.buffers()):
        if p.is_cuda:
            return p.device
    return None


def convert_logic_net(model) -> BitpackedNet:
    """LogicNet -> :class:`BitpackedNet` (convert.py:336-366)."""
    layers = [convert_layer(l) for l in model.layers]
    return BitpackedNet(layers, convert_head(model.head), wire_r=getattr(model, "wire_r", 0),
                        device=_device_of(model))


def convert_logic_conv_net(model) -> BitpackedConvNet:
    """LogicConvNet -> :class:`BitpackedConvNet` (convert.py:369-402)."""
    from ..layers import ConvLogicTree
    bp_conv = []
    for i in range(0, len(model.blocks), 2):
        conv = model.blocks[i]
        bp_conv.append(convert_conv_tree_layer(conv) if isinstance(conv, ConvLogicTree) else None)
    head_layers = [convert_layer(l) for l in model.head_layers]
    return BitpackedConvNet(model.blocks, bp_conv, head_layers, convert_head(model.head),
                            wire_residual=getattr(model, "wire_residual", 0.0),
                            device=_device_of(model))
