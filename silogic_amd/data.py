"""Input encoders of ``silogic.data`` on the GPU (data.py:15-131): the
thermometer codes ``binarize`` / ``binarize_spatial`` and the edge-detector
bits ``edge_bits``, with the reference's names, threshold lists and output
layouts (uint8), plus packed forms that feed the hard kernels directly
(``binarize_packed``: ``[T*D, nw]`` rows or ``[nw, T*D]`` words, the former
also the conv layout ``[C*T, H*W, nw]``). The dataset loaders (torchvision,
disk caches) are not part of this build."""
import torch

from . import _lib, ops

MNIST_THRESH = [0.25]
SEVEN_THRESH = [0.125, 0.25, 0.375, 0.5, 0.625, 0.75, 0.875]
FOUR_THRESH = [0.2, 0.4, 0.6, 0.8]
CIFAR3_THRESH = [0.25, 0.5, 0.75]
FIVE_THRESH = [1 / 6, 2 / 6, 3 / 6, 4 / 6, 5 / 6]
EDGE_THRESH = [0.12, 0.25]


_THR_CACHE = {}


def _thr(thresholds, device):
    """Thresholds as an fp32 device tensor; a list's copy is kept per device
    so repeated calls issue no host-to-device copy."""
    if isinstance(thresholds, torch.Tensor):
        t = thresholds.detach().reshape(-1).to(device=device, dtype=torch.float32)
        if t.numel() == 0:
            raise ValueError("thresholds: a non-empty list of floats")
        return t.contiguous()
    key = (tuple(float(v) for v in thresholds), str(device))
    t = _THR_CACHE.get(key)
    if t is None:
        if not key[0]:
            raise ValueError("thresholds: a non-empty list of floats")
        t = torch.tensor(key[0], dtype=torch.float32).to(device)
        _THR_CACHE[key] = t
    return t


def _encode(x, thr, learned, layout, T):
    """x [B, D] fp32, or uint8 pixel bytes (value x / 255)."""
    B, D = x.shape
    dtype = 1 if x.dtype == torch.uint8 else 0
    if layout == 2:
        out = torch.empty((B, D * T), device=x.device, dtype=torch.uint8)
    else:
        nw = ops.n_words(B)
        shape = (D * T, nw) if layout == 0 else (nw, D * T)
        out = torch.empty(shape, device=x.device, dtype=torch.int64)
    _lib.call("slg_encode_thermometer", ops._p(x), dtype, B, D, ops._p(thr), T, int(learned),
              layout, ops._p(out), ops._stream(x))
    return out


def binarize(x, thresholds):
    """``[N, C, H, W]`` (or ``[N, D]``) in [0, 1] -> uint8 ``[N, D*T]``: one
    bit ``x >= t`` per threshold, the threshold planes concatenated
    (data.py:23-40)."""
    ops.require_gpu(x)
    xf = ops._as_f32(x.reshape(x.shape[0], -1))
    thr = _thr(thresholds, x.device)
    return _encode(xf, thr, False, 2, thr.numel())


def binarize_spatial(x, thresholds):
    """``[N, C, H, W]`` -> uint8 ``[N, C*T, H, W]`` (channel ``t*C + c``,
    data.py:75-89)."""
    ops.require_gpu(x)
    N, C, H, W = x.shape
    thr = _thr(thresholds, x.device)
    return _encode(ops._as_f32(x.reshape(N, -1)), thr, False, 2, thr.numel()).view(
        N, C * thr.numel(), H, W)


def binarize_packed(x, thresholds, word_major=False):
    """The bits of :func:`binarize` packed 64 samples per word: ``[T*D, nw]``
    (``word_major``: ``[nw, T*D]``, the fused FC network's input). For image
    input the rows are the conv layout ``[C*T, H*W, nw]`` of
    :func:`binarize_spatial`. ``x`` may be fp32 in [0, 1] or the uint8 pixel
    bytes of a dataset (value ``x / 255`` as the reference's loaders compute
    it, data.py:49-57), read directly."""
    ops.require_gpu(x)
    x2 = x.reshape(x.shape[0], -1)
    xf = x2.contiguous() if x2.dtype == torch.uint8 else ops._as_f32(x2)
    thr = _thr(thresholds, x.device)
    return _encode(xf, thr, False, 1 if word_major else 0, thr.numel())


def edge_bits(x, edge_thr=None):
    """``[N, C, H, W]`` in [0, 1] -> uint8 ``[N, C*3*2*T, H, W]``: per colour
    the Sobel-x, Sobel-y and Laplacian responses (zero padding), each
    thresholded at ``> t`` and ``< -t`` (data.py:102-131)."""
    ops.require_gpu(x)
    if edge_thr is None:
        edge_thr = EDGE_THRESH
    N, C, H, W = x.shape
    thr = _thr(edge_thr, x.device)
    T = thr.numel()
    out = torch.empty((N, C * 3 * 2 * T, H, W), device=x.device, dtype=torch.uint8)
    _lib.call("slg_edge_bits", ops._p(ops._as_f32(x)), N, C, H, W, ops._p(thr), T, ops._p(out),
              ops._stream(x))
    return out
