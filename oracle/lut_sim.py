"""Brute-force per-node LUT evaluation of hard FC networks (small cases only).

Restates silogic/fpga/circuit.py: ``extract_logic_net`` (150-214) lowers every
node to ``(input wires, truth table over address sum_j in_j << j)`` and
``simulate`` (219-248) evaluates node by node with integer arithmetic, then
sums each class block. The reference's own test requires these scores to be
``np.array_equal`` to ``forward_hard`` (tests/test_fpga.py:53-63), which is
what pins hard logits as exact integer popcounts.

Truth tables are taken by evaluating the oracle's per-node hard function at
every corner (convert.py:100-123 does the same through ``node.forward_hard``),
so this module checks the network plumbing (wiring, layer order, class blocks)
independently of the vectorised paths.

Test infrastructure only (see :mod:`oracle`).
"""
import numpy as np
import torch

from . import torch_ref


def extract(spec, sd):
    """Return ``(layers, num_classes)``; layer = list of ``(idx list, tt list)``."""
    st = torch_ref.structure(spec)
    assert st["kind"] == "fc"
    layers = []
    for L in st["layers"]:
        idx = torch_ref.hard_indices(L, sd).numpy()
        n = idx.shape[1]
        corners = torch_ref.corner_bits(n)                    # [P, n], bit j of p
        tts = []
        for p in range(2 ** n):
            ops = corners[p].view(1, 1, n).expand(1, L["d_out"], n).to(torch.uint8)
            tts.append(torch_ref.node_hard(L, sd, ops)[0].numpy())
        tt = np.stack(tts, axis=1)                            # [out, P]
        layers.append([(list(idx[o]), list(tt[o])) for o in range(idx.shape[0])])
    return layers, st["head"]["C"]


def simulate(layers, C, x):
    """``[B, in] {0,1}`` -> integer scores ``[B, C]`` (circuit.py:219-248)."""
    cur = (np.asarray(x) != 0).astype(np.int64)
    for layer in layers:
        out = np.empty((cur.shape[0], len(layer)), dtype=np.int64)
        for o, (idx, tt) in enumerate(layer):
            addr = np.zeros(cur.shape[0], dtype=np.int64)
            for j, wi in enumerate(idx):
                addr |= cur[:, wi] << j
            out[:, o] = np.asarray(tt, dtype=np.int64)[addr]
        cur = out
    g = cur.shape[1] // C
    return cur.reshape(cur.shape[0], C, g).sum(axis=2)
