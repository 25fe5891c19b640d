"""Bit-packing primitives (silogic/bitpacking/ops.py) on the HIP kernels.

Layout: activations are int64 arrays ``[dim, n_words]`` with
``n_words = ceil(B / 64)``; bit ``p`` of word ``w`` in row ``d`` holds
dimension ``d`` of sample ``b = 64*w + p`` (ops.py:1-9). Every function takes
numpy arrays or torch tensors: numpy inputs are copied to the GPU, computed
there and copied back, torch tensors stay on their device. All arithmetic
runs in the HIP library; there is no CPU path.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import ops as _ops
from ..functional import TT_CODES


def default_device():
    """The GPU the package computes on when handed numpy arrays."""
    return torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() \
        else torch.device("cuda")


def to_device(x, device=None, dtype=None):
    """``x`` (numpy or torch) as a contiguous tensor on ``device`` (the GPU)."""
    if isinstance(x, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(x))
    elif isinstance(x, torch.Tensor):
        t = x
    else:
        t = torch.as_tensor(x)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    dev = device if device is not None else (t.device if t.is_cuda else default_device())
    return t.to(dev).contiguous()


def like_input(t, ref):
    """Return ``t`` as numpy when ``ref`` was numpy, else as the tensor."""
    return t.cpu().numpy() if isinstance(ref, np.ndarray) else t


def n_words(B: int) -> int:
    """Number of 64-bit words that hold ``B`` samples (ops.py:27-29)."""
    return (int(B) + 63) >> 6


def pack_bits(x):
    """``[B, dim]`` uint8/bool -> ``[dim, ceil(B/64)]`` int64, sample ``b`` at
    bit ``b % 64`` of word ``b // 64``, zero padding (ops.py:32-49)."""
    t = to_device(x)
    if t.dtype == torch.bool:
        t = t.to(torch.uint8)
    if t.dim() != 2:
        raise ValueError("pack_bits: x must be [B, dim], got %s" % (tuple(t.shape),))
    return like_input(_ops.pack_bits(t), x)


def unpack_bits(packed, B: int):
    """``[dim, n_words]`` int64 -> ``[B, dim]`` uint8 (ops.py:52-63)."""
    t = to_device(packed, dtype=torch.int64)
    return like_input(_ops.unpack_bits(t, int(B)), packed)


def divide_by_tau(counts: torch.Tensor, tau: float) -> torch.Tensor:
    """``counts / tau`` rounded once, as numpy's float32 division
    (ops.py:104): a divisor on the device (torch turns a host-scalar divisor
    into a multiplication by its reciprocal, which can differ in the last
    bit)."""
    return counts / torch.tensor(float(tau), dtype=counts.dtype, device=counts.device)


def group_sum_packed(x_packed, B: int, num_classes: int, tau: float = 1.0):
    """GroupSum class logits from packed activations: class ``c`` counts the
    ones of rows ``[c*gs, (c+1)*gs)`` with ``gs = dim // num_classes``,
    divided by ``tau`` -> ``[B, num_classes]`` float32 (ops.py:66-104)."""
    t = to_device(x_packed, dtype=torch.int64)
    dim = t.shape[0]
    gs = dim // num_classes
    if gs == 0:
        raise ValueError("group_sum_packed: %d rows for %d classes" % (dim, num_classes))
    counts = _ops.groupsum_packed(t[:gs * num_classes], int(B), int(num_classes))
    return like_input(divide_by_tau(counts, tau), x_packed)


def mask_last_word(packed, B: int):
    """Zero the padding bits of the last word, in place (ops.py:107-115)."""
    rem = int(B) % 64
    if rem == 0:
        return packed
    mask = (1 << rem) - 1
    if isinstance(packed, np.ndarray):
        packed[:, -1] &= np.int64(mask)
    else:
        packed[:, -1] &= mask
    return packed


def code_to_gate16() -> np.ndarray:
    """16-entry lookup ``code -> gate16 index``, code = sum_i TT[g][i] << i
    over input addresses i = (a << 1) | b (ops.py:146-165)."""
    lut = np.zeros(16, dtype=np.int32)
    for g, code in enumerate(TT_CODES):
        lut[code] = g
    return lut


def gate16_code(gate):
    """Truth-table code of gate16 index ``gate`` (inverse of code_to_gate16)."""
    return TT_CODES[int(gate)]


def layer_codes(gate_types, a_idx, b_idx, device):
    """``[OUT, 2]`` int32 codes ``(a, b | tt << 28)`` of the packed layer
    kernel, from gate16 indices and operand rows (host arrays)."""
    g = np.asarray(gate_types, dtype=np.int64)
    tt = np.asarray(TT_CODES, dtype=np.int64)[g]
    a = np.asarray(a_idx, dtype=np.int64)
    b = np.asarray(b_idx, dtype=np.int64)
    if a.min(initial=0) < 0 or b.min(initial=0) < 0 or b.max(initial=0) >= (1 << 28):
        raise ValueError("layer_codes: operand indices must lie in [0, 2^28)")
    hi = (b | (tt << 28)).astype(np.uint32).view(np.int32)
    codes = np.stack([a.astype(np.int32), hi], axis=1)
    return torch.from_numpy(np.ascontiguousarray(codes)).to(device)


def apply_gate(a, b, gate: int):
    """One of the 16 two-input gates on packed words of any shape
    (ops.py:123-170); bit i of the gate's truth-table code is its output at
    address (a << 1) | b."""
    ta = to_device(a, dtype=torch.int64)
    tb = to_device(b, device=ta.device, dtype=torch.int64)
    if ta.shape != tb.shape:
        raise ValueError("apply_gate: operand shapes differ")
    x = torch.stack([ta.reshape(-1), tb.reshape(-1)])          # [2, n] words
    codes = layer_codes([gate], [0], [1], ta.device)
    out = _ops.fc_hard_layer(x, codes).reshape(ta.shape)
    return like_input(out, a)
