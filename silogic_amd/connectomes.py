"""Input wiring ("connectomes") of the FC logic layers — the candidate-based
kinds the HIP kernels consume: ``topk``, ``blocktopk`` and ``fixed`` (= one
candidate per slot, K = 1).

Construction draws from the generator in the reference's order
(silogic/connectomes.py:37-43, 46-56, 94-111, 186-202), so a given ``seed``
yields the same wiring and the same ``state_dict``. ``dense`` and the
sum-threshold kinds (``st``, ``stw``, ``stt``) are not part of the gate-layer
hot path and are rejected at construction.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

_ALIASES = {
    "f": "fixed", "fixed": "fixed",
    "l": "dense", "dense": "dense",
    "topk": "topk", "blocktopk": "blocktopk",
    "st": "st", "stw": "stw", "stt": "stt",
}
SUPPORTED = ("fixed", "topk", "blocktopk")


def _candidates(in_dim, out_dim, arity, k, gen):
    """``[out, arity, k]``: for each output, for each slot, the first k of a
    fresh permutation of the inputs."""
    rows = []
    for _ in range(out_dim):
        rows.append(torch.stack([torch.randperm(in_dim, generator=gen)[:k]
                                 for _ in range(arity)]))
    return torch.stack(rows)


class FixedConnectome(nn.Module):
    """One fixed random wire per (node, slot); exposed to the kernels as K=1."""

    def __init__(self, in_dim, out_dim, arity, gen=None):
        super().__init__()
        self.in_dim, self.out_dim, self.arity = in_dim, out_dim, arity
        idx = torch.randint(0, in_dim, (out_dim, arity), generator=gen)
        self.register_buffer("idx", idx)
        self.register_buffer("cand_i32", idx.unsqueeze(-1).to(torch.int32))
        self.k = 1

    def candidates_i32(self):
        return self.cand_i32

    def weights(self):
        return torch.ones(self.out_dim, self.arity, 1, device=self.idx.device)

    def hard_inputs(self):
        """(wiring tensor, conn or None) for the hard-code prep kernel."""
        return self.idx.to(torch.int32), None


class TopKConnectome(nn.Module):
    """Each slot picks among ``k`` random candidates through a softmax.

    ``block=True`` draws the candidates of output ``o`` from a contiguous
    window that slides with ``o`` (cache-local wiring)."""

    def __init__(self, in_dim, out_dim, arity, k, gen=None, block=False, window=0):
        super().__init__()
        self.in_dim, self.out_dim, self.arity = in_dim, out_dim, arity
        kk = min(k, in_dim)
        self.k = kk
        if block:
            W = min(in_dim, window if window else max(4 * kk, 256))
            starts = (torch.arange(out_dim).float() / max(1, out_dim)
                      * max(1, in_dim - W)).long()
            cand = torch.stack([
                torch.stack([starts[o] + torch.randperm(W, generator=gen)[:kk]
                             for _ in range(arity)])
                for o in range(out_dim)])
        else:
            cand = _candidates(in_dim, out_dim, arity, kk, gen)
        self.register_buffer("cand", cand)
        self.register_buffer("cand_i32", cand.to(torch.int32))
        self.conn = nn.Parameter(torch.randn(out_dim, arity, kk, generator=gen))
        self.ste = False   # one-hot forward / softmax gradient selection

    def weights(self):
        w = F.softmax(self.conn, dim=2)
        if self.ste:
            hard = F.one_hot(self.conn.argmax(dim=2), w.shape[-1]).to(w.dtype)
            w = hard + w - w.detach()
        return w

    def candidates_i32(self):
        return self.cand_i32

    def hard_inputs(self):
        return self.cand_i32, self.conn


def build_connectome(kind, in_dim, out_dim, arity=2, k=8, seed=None, window=0):
    """Construct a connectome by name (``topk``, ``blocktopk``, ``fixed``/``F``)."""
    key = _ALIASES.get(str(kind).lower())
    if key is None:
        raise ValueError(f"unknown connectome {kind!r}")
    if key not in SUPPORTED:
        raise NotImplementedError(
            f"connectome {kind!r} is not on the MI355X gate-layer path "
            f"(supported: {', '.join(SUPPORTED)})")
    gen = torch.Generator().manual_seed(seed) if seed is not None else None
    if key == "fixed":
        return FixedConnectome(in_dim, out_dim, arity, gen)
    if key == "topk":
        return TopKConnectome(in_dim, out_dim, arity, k, gen)
    return TopKConnectome(in_dim, out_dim, arity, k, gen, block=True, window=window)
