"""Bit-packed layers (silogic/bitpacking/packed_layer.py) on the HIP kernels.

FC layers take ``[dim, n_words]`` int64 activations; conv layers take the
B-packed ``[dim, L, nw_B]`` layout with ``L = H * W`` (packed_layer.py:1-17).
The constructors take the same arrays as the reference's (gate types,
operand indices, truth tables); ``forward`` runs one HIP launch. Inputs may
be numpy (copied to the GPU and back) or torch tensors on the GPU.
"""
from __future__ import annotations

from typing import List

import numpy as np
import torch

from .. import ops as _ops
from .ops import layer_codes, like_input, pack_bits, to_device, unpack_bits, group_sum_packed
from ..functional import TT_CODES


def _tt_word(bits) -> int:
    """Signed int64 value of a truth table given as a 0/1 sequence (entry e at
    bit e, at most 64 entries)."""
    v = 0
    for e, bit in enumerate(np.asarray(bits).reshape(-1)):
        if bit:
            v |= 1 << e
    return v - (1 << 64) if v >= (1 << 63) else v


def gate16_lut_word(gate: int) -> int:
    """A gate16 node as an arity-2 LUT word: LUT entry p = c0 | c1 << 1 of the
    children (c0 the first) is the gate's output at address (c0 << 1) | c1."""
    code = TT_CODES[int(gate)]
    v = 0
    for p in range(4):
        c0, c1 = p & 1, p >> 1
        if (code >> ((c0 << 1) | c1)) & 1:
            v |= 1 << p
    return v


class _DeviceCache:
    """Device copies of a layer's tables, made on first use per device."""

    def __init__(self):
        self._cache = {}

    def get(self, device, make):
        key = str(device)
        if key not in self._cache:
            self._cache[key] = make(device)
        return self._cache[key]


# ── two-input gate layer ─────────────────────────────────────────────────────

class BitpackedFCLayer:
    """Hard, bit-packed two-input LogicLayer (packed_layer.py:29-116):
    ``out[o] = gate_types[o](x[a_idx[o]], x[b_idx[o]])``, one launch of the
    packed layer kernel (the reference groups outputs by gate type for numpy;
    the kernel evaluates any gate per output)."""

    def __init__(self, gate_types: np.ndarray, a_idx: np.ndarray, b_idx: np.ndarray) -> None:
        self.out_dim = len(gate_types)
        self.gate_types = np.asarray(gate_types).astype(np.int32)
        self.a_idx = np.asarray(a_idx).astype(np.int32)
        self.b_idx = np.asarray(b_idx).astype(np.int32)
        if not (self.gate_types.shape == self.a_idx.shape == self.b_idx.shape):
            raise ValueError("BitpackedFCLayer: gate_types, a_idx, b_idx must have one entry per output")
        if self.out_dim and (self.gate_types.min() < 0 or self.gate_types.max() > 15):
            raise ValueError("BitpackedFCLayer: gate types must lie in 0..15")
        self.max_idx = int(max(self.a_idx.max(initial=0), self.b_idx.max(initial=0)))
        self._codes = _DeviceCache()

    @property
    def gate_histogram(self) -> dict:
        g, n = np.unique(self.gate_types, return_counts=True)
        return {int(a): int(b) for a, b in zip(g, n)}

    def codes(self, device):
        """``[OUT, 2]`` int32 ``(a, b | tt << 28)`` codes on ``device``."""
        return self._codes.get(device, lambda d: layer_codes(self.gate_types, self.a_idx,
                                                             self.b_idx, d))

    def forward(self, x):
        """``[in_dim, n_words]`` int64 -> ``[out_dim, n_words]`` int64."""
        t = to_device(x, dtype=torch.int64)
        if t.dim() != 2 or self.max_idx >= t.shape[0]:
            raise ValueError("BitpackedFCLayer: input has %d rows, operands reach row %d"
                             % (t.shape[0] if t.dim() else 0, self.max_idx))
        return like_input(_ops.fc_hard_layer(t, self.codes(t.device)), x)

    __call__ = forward


# ── n-input LUT layer ───────────────────────────────────────────────────────

class BitpackedLUTLayer:
    """Bit-packed n-input LUT layer (packed_layer.py:121-178): output ``o``
    reads inputs ``input_indices[o]`` and returns ``truth_tables[o][addr]``
    with ``addr = sum_j x_j << j`` (arity <= 6, one launch)."""

    def __init__(self, truth_tables: np.ndarray, input_indices: np.ndarray) -> None:
        tt = np.asarray(truth_tables).astype(bool)
        out_dim, lut_size = tt.shape
        self.out_dim = out_dim
        self.arity = int(np.log2(lut_size))
        if 1 << self.arity != lut_size or not 1 <= self.arity <= 6:
            raise ValueError("BitpackedLUTLayer: truth tables must have 2^arity entries, arity <= 6")
        self.truth_tables = tt
        self.input_indices = np.asarray(input_indices).astype(np.int32)
        if self.input_indices.shape != (out_dim, self.arity):
            raise ValueError("BitpackedLUTLayer: input_indices must be [out_dim, arity]")
        self.max_idx = int(self.input_indices.max(initial=0))
        self._words = np.array([_tt_word(r) for r in tt], dtype=np.int64)
        self._dev = _DeviceCache()

    def tables(self, device):
        return self._dev.get(device, lambda d: (
            torch.from_numpy(self.input_indices.copy()).to(d),
            torch.from_numpy(self._words.copy()).to(d)))

    def forward(self, x):
        """``[in_dim, n_words]`` int64 -> ``[out_dim, n_words]`` int64."""
        t = to_device(x, dtype=torch.int64)
        if t.dim() != 2 or self.max_idx >= t.shape[0]:
            raise ValueError("BitpackedLUTLayer: input has too few rows")
        idx, words = self.tables(t.device)
        return like_input(_ops.fc_lut_hard(t, idx, words), x)

    __call__ = forward


# ── conv spatial helpers ────────────────────────────────────────────────────

def pack_conv_input(x, nw_B: int = None):
    """``[B, C, H, W]`` uint8 -> ``[C, H*W, nw_B]`` int64, the batch packed
    (packed_layer.py:184-210)."""
    t = to_device(x)
    B, C, H, W = t.shape
    if nw_B is not None and nw_B != (B + 63) // 64:
        raise ValueError("pack_conv_input: nw_B = %d for B = %d" % (nw_B, B))
    packed = _ops.pack_bits(t.reshape(B, C * H * W) if t.dtype != torch.bool
                            else t.to(torch.uint8).reshape(B, -1))
    return like_input(packed.view(C, H * W, -1), x)


def unpack_conv_output(x_3d, B: int, H: int, W: int):
    """``[C, H*W, nw_B]`` int64 -> ``[B, C, H, W]`` uint8 (packed_layer.py:213-221)."""
    t = to_device(x_3d, dtype=torch.int64)
    C, L, nw = t.shape
    bits = _ops.unpack_bits(t.reshape(C * L, nw), int(B))
    return like_input(bits.view(int(B), C, H, W), x_3d)


def packed_unfold(x_3d, kh: int, kw: int, stride: int, padding: int, H_in: int, W_in: int):
    """``[C, L_in, nw_B]`` -> ``[C*kh*kw, L_out, nw_B]``, the unrolled receptive
    field in ``F.unfold`` row order, zero outside the image
    (packed_layer.py:224-283)."""
    t = to_device(x_3d, dtype=torch.int64)
    return like_input(_ops.packed_unfold(t, kh, kw, stride, padding, H_in, W_in), x_3d)


def packed_or_pool(x_3d, H: int, W: int, pool_size: int = 2):
    """``[C, H*W, nw_B]`` -> ``[C, (H//ps)*(W//ps), nw_B]`` OR over windows
    (packed_layer.py:286-319)."""
    t = to_device(x_3d, dtype=torch.int64)
    return like_input(_ops.packed_or_pool(t, H, W, pool_size), x_3d)


def _leaf_fields(leaf_idx, kh, kw):
    """Flat receptive-field indices c*kh*kw + dy*kw + dx as the fused conv
    kernel's packed leaves c << 8 | dy << 4 | dx."""
    li = np.asarray(leaf_idx, dtype=np.int64)
    c, q = li // (kh * kw), li % (kh * kw)
    return (c << 8) | ((q // kw) << 4) | (q % kw)


class _ConvTreeBase:
    def __init__(self, leaf_idx, kh, kw, stride, padding, cin):
        self.n_out = leaf_idx.shape[0]
        self.n_leaves = leaf_idx.shape[1]
        self.leaf_idx = np.asarray(leaf_idx).astype(np.int32)
        self.kh, self.kw, self.stride, self.padding, self.cin = kh, kw, stride, padding, cin
        self._dev = _DeviceCache()

    def _tree(self, device):
        return self._dev.get(device, lambda d: (
            torch.from_numpy(self.leaf_idx.copy()).to(d),
            torch.from_numpy(self._tables.copy()).to(d)))

    def forward_packed(self, x_3d):
        """``[P, L, nw_B]`` unfolded input -> ``[n_out, L, nw_B]``."""
        t = to_device(x_3d, dtype=torch.int64)
        if t.dim() != 3 or int(self.leaf_idx.max(initial=0)) >= t.shape[0]:
            raise ValueError("%s: unfolded input has too few rows" % type(self).__name__)
        leaf, tables = self._tree(t.device)
        return like_input(_ops.lut_tree_hard(t, leaf, self.node_arity, self.depth, tables), x_3d)

    def fused_ok(self):
        """True when the fused conv + OR-pool kernel runs this layer: stride 1,
        'same' padding, and a gate16 tree of depth <= 4 or a one-level LUT."""
        return (self.stride == 1 and self.kh == self.kw == 2 * self.padding + 1
                and self.kh <= 15 and self._fused_tt is not None)

    def fused_params(self, device):
        """``(leaf, tt, node_kind, depth, arity)`` for the fused kernel."""
        leaf, tt = self._dev.get(("fused", str(device)), lambda _: (
            torch.from_numpy(_leaf_fields(self.leaf_idx, self.kh, self.kw).astype(np.int32))
            .to(device),
            torch.from_numpy(self._fused_tt.copy()).to(device)))
        return leaf, tt, self._fused_kind, self.depth, self.node_arity


# ── convolutional gate-tree layer ───────────────────────────────────────────

class BitpackedConvTreeLayer(_ConvTreeBase):
    """Bit-packed gate16 tree for B-packed conv inputs (packed_layer.py:324-432):
    ``leaf_idx`` [n_out, n_leaves] flat indices into the unfolded input,
    ``gate_types_per_level`` one [n_out, nodes] array per level (leaves'
    level first); node m combines values 2m (a) and 2m+1 (b)."""

    node_arity = 2

    def __init__(self, leaf_idx: np.ndarray, gate_types_per_level: List[np.ndarray], kh: int,
                 kw: int, stride: int, padding: int, cin: int) -> None:
        super().__init__(np.asarray(leaf_idx), kh, kw, stride, padding, cin)
        self.depth = len(gate_types_per_level)
        self.gate_types_per_level = [np.asarray(g).astype(np.int32) for g in gate_types_per_level]
        if self.n_leaves != 2 ** self.depth:
            raise ValueError("BitpackedConvTreeLayer: %d leaves for depth %d"
                             % (self.n_leaves, self.depth))
        gt = np.concatenate([g.reshape(self.n_out, -1) for g in self.gate_types_per_level], axis=1)
        lut = np.array([gate16_lut_word(g) for g in range(16)], dtype=np.int64)
        self._tables = lut[gt]                                   # [n_out, nodes]
        if self.depth <= 4:   # fused kernel: node j's 4-bit gate code at bits 4j..4j+3
            codes = np.asarray(TT_CODES, dtype=np.int64)[gt]
            self._fused_tt = np.zeros(self.n_out, dtype=np.int64)
            for j in range(gt.shape[1]):
                self._fused_tt |= codes[:, j] << (4 * j)
            self._fused_kind = _ops.GATE16
        else:
            self._fused_tt = None


# ── convolutional LUT-tree layer ────────────────────────────────────────────

class BitpackedConvLUTLayer(_ConvTreeBase):
    """Bit-packed k-ary LUT tree for B-packed conv inputs (packed_layer.py:437-540):
    ``truth_tables_per_level[i]`` is [n_out * nodes_i, 2^k] bool with node
    ``m`` of output ``n`` at row ``n * nodes_i + m``; entry address
    ``sum_j x_j << j``."""

    def __init__(self, leaf_idx: np.ndarray, truth_tables_per_level: List[np.ndarray],
                 node_arity: int, kh: int, kw: int, stride: int, padding: int, cin: int) -> None:
        super().__init__(np.asarray(leaf_idx), kh, kw, stride, padding, cin)
        self.node_arity = int(node_arity)
        self.depth = len(truth_tables_per_level)
        if self.n_leaves != self.node_arity ** self.depth or not 2 <= self.node_arity <= 6:
            raise ValueError("BitpackedConvLUTLayer: %d leaves for arity %d depth %d"
                             % (self.n_leaves, self.node_arity, self.depth))
        per_level = []
        for tt in truth_tables_per_level:
            tt = np.asarray(tt).astype(bool)
            words = np.array([_tt_word(r) for r in tt], dtype=np.int64)
            per_level.append(words.reshape(self.n_out, -1))
        self._tables = np.concatenate(per_level, axis=1)         # [n_out, nodes]
        if self.depth == 1:   # fused kernel: the LUT word itself
            self._fused_tt = self._tables[:, 0].copy()
            self._fused_kind = _ops.MULTILINEAR2
        else:
            self._fused_tt = None


# ── heads ────────────────────────────────────────────────────────────────────

class BitpackedGroupSumHead:
    """GroupSum on packed activations, logits divided by ``tau``
    (packed_layer.py:546-572, ops.py:66-104)."""

    def __init__(self, num_classes: int, tau: float = 1.0) -> None:
        self.num_classes = num_classes
        self.tau = tau

    def forward(self, x, B: int):
        """``[width, n_words]`` int64 -> ``[B, num_classes]`` float32."""
        return group_sum_packed(x, B, self.num_classes, self.tau)

    __call__ = forward
