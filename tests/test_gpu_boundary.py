"""The entry points whose signatures are the reference's own, called the way
the reference calls its fused ops, against the oracle (GPU):

* ``slg_dense_logic_fwd`` / ``slg_warp_logic_fwd`` take separate ``ca``,
  ``cb``, ``wa``, ``wb`` arrays ``[OUT, K]`` (kernels/dense.py:123-125,
  warp.py:104-105, called at layers.py:121-123);
* ``slg_tree_conv_fwd`` takes ``coef [N, 2^d-1, 4]`` and, for Top-K leaves,
  ``w/cm/ch/cw [N, 2^d, K]`` (kernels/conv_topk.py:175-189), for fixed
  leaves ``cm/ch/cw [N, 2^d]`` with no weights (kernels/conv.py:399-400).

Each is called once through ctypes directly and once through the
``silogic_amd.kernels`` drop-in (which now reaches these entry points), with
a gradient check of the drop-in against autograd through the oracle.
"""
import ctypes

import pytest
import torch
import torch.nn.functional as F

import silogic_amd as sl
from conftest import build_product
from oracle import torch_ref
from silogic_amd import _lib, kernels

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-5, 1e-6


def _close(got, ref, what, rtol=RTOL, atol=ATOL):
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    bad = (got - ref).abs() > rtol * ref.abs() + atol
    assert not bad.any(), f"{what}: {int(bad.sum())} values outside tolerance"


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _fc_arrays(sd, L):
    """The reference's dispatch arguments (layers.py:111-123): per-operand
    candidate and weight arrays and the node coefficients."""
    p = L["prefix"]
    cand = sd[p + "_conn.cand"].to(torch.int32)
    w = torch.softmax(sd[p + "_conn.conn"], dim=2)
    if L["node"] == "gate16":
        coef = torch.softmax(sd[p + "node.gate_logits"], dim=1) @ torch_ref.BASIS
    else:
        t = sd[p + "node.theta"]
        coef = torch.stack([t[:, 0] - t[:, 1] - t[:, 2] + t[:, 3], 2 * (t[:, 1] - t[:, 3]),
                            2 * (t[:, 2] - t[:, 3]), 4 * t[:, 3]], dim=1)
    parts = [cand[:, 0], cand[:, 1], w[:, 0], w[:, 1], coef]
    return [t.contiguous().to(DEV) for t in parts]


@pytest.mark.parametrize("node", ["gate16", "walsh"])
@pytest.mark.parametrize("K", [8, 4, 3])
def test_dense_and_warp_entry_points_with_separate_arrays(node, K):
    spec = ("LogicNet", dict(in_dim=500, width=330, depth=1, k=K, node=node, node_tau=0.7))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    L = torch_ref.structure(spec)["layers"][0]
    x = torch.rand(70, 500, generator=torch.Generator().manual_seed(K))
    ref = torch_ref.fc_layer_soft(L, sd, x)
    ca, cb, wa, wb, coef = _fc_arrays(sd, L)
    xd = x.to(DEV)
    y = torch.empty(70, 330, device=DEV)
    lib = _lib.lib()
    if node == "gate16":
        rc = lib.slg_dense_logic_fwd(_p(xd), 70, 500, 330, K, _p(ca), _p(cb), _p(wa), _p(wb),
                                     _p(coef), _p(y), _stream())
        drop = kernels.dense_logic(xd, ca, cb, wa, wb, coef)
    else:
        inv_tau = 1.0 / 0.7
        rc = lib.slg_warp_logic_fwd(_p(xd), 70, 500, 330, K, _p(ca), _p(cb), _p(wa), _p(wb),
                                    _p(coef), inv_tau, _p(y), _stream())
        drop = kernels.warp_logic(xd, ca, cb, wa, wb, coef, inv_tau)
    _lib.check(rc, "dense/warp entry point")
    _close(y, ref, f"{node} K={K} ctypes")
    assert torch.equal(drop.cpu(), y.cpu())


@pytest.mark.parametrize("node", ["gate16", "walsh"])
def test_dense_dropin_gradients(node):
    spec = ("LogicNet", dict(in_dim=200, width=120, depth=1, k=8, node=node))
    model = build_product(spec)
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    L = torch_ref.structure(spec)["layers"][0]
    ca, cb, wa, wb, coef = _fc_arrays(sd, L)
    x = torch.rand(33, 200, generator=torch.Generator().manual_seed(5))
    gy = torch.randn(33, 120, generator=torch.Generator().manual_seed(6))
    xd = x.to(DEV).requires_grad_(True)
    wad, wbd, cd = (t.clone().requires_grad_(True) for t in (wa, wb, coef))
    fn = kernels.dense_logic if node == "gate16" else (
        lambda *a: kernels.warp_logic(*a, 1.0))
    fn(xd, ca, cb, wad, wbd, cd).backward(gy.to(DEV))
    # autograd through the same expression on the CPU
    xc = x.clone().requires_grad_(True)
    wac, wbc, cc = (t.detach().cpu().clone().requires_grad_(True) for t in (wa, wb, coef))
    a = (xc[:, ca.long().cpu()] * wac).sum(-1)
    b = (xc[:, cb.long().cpu()] * wbc).sum(-1)
    z = cc[:, 0] + cc[:, 1] * a + cc[:, 2] * b + cc[:, 3] * (a * b)
    (torch.sigmoid(z) if node == "walsh" else z).backward(gy)
    for got, ref, what in ((xd.grad, xc.grad, "x"), (wad.grad, wac.grad, "wa"),
                           (wbd.grad, wbc.grad, "wb"), (cd.grad, cc.grad, "coef")):
        scale = ref.abs().max().item()
        _close(got, ref, f"{node} grad {what}", rtol=0, atol=1e-4 * scale)


def _tree_args(conv, sd, prefix, fixed):
    coef = torch.cat([torch.softmax(sd[f"{prefix}gate_logits.{i}"], dim=2) @ torch_ref.BASIS
                      for i in range(conv.d)], dim=1)
    if fixed:
        cm, ch, cw = sd[prefix + "cm_idx"], sd[prefix + "ch_idx"], sd[prefix + "cw_idx"]
        w = None
    else:
        cm, ch, cw = sd[prefix + "lc_cm"], sd[prefix + "lc_ch"], sd[prefix + "lc_cw"]
        w = torch.softmax(sd[prefix + "conn"], dim=2)
    return [None if t is None else t.contiguous().to(DEV) for t in (coef, w, cm, ch, cw)]


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("depth", [1, 2, 3])
def test_tree_conv_entry_point(fixed, depth):
    conv = sl.ConvLogicTree(5, 12, kernel=3, tree_depth=depth, connect="fixed" if fixed else "topk",
                            k=4, n_chan=2, residual_init=False, seed=depth)
    sd = {k: v.clone() for k, v in conv.state_dict().items()}
    blk = dict(prefix="", cin=5, n=12, kernel=3, depth=depth, stride=1, padding=1,
               connect="fixed" if fixed else "topk", k=conv.k, node="gate16", node_arity=2,
               leaves=2 ** depth)
    x = (torch.rand(6, 5, 11, 9, generator=torch.Generator().manual_seed(depth)) > 0.4).float()
    ref = torch_ref.conv_soft(blk, sd, x)
    coef, w, cm, ch, cw = _tree_args(conv, sd, "", fixed)
    K = 1 if fixed else conv.k
    xd = x.to(DEV)
    out = torch.empty(6, 12, 11, 9, device=DEV)
    rc = _lib.lib().slg_tree_conv_fwd(_p(xd), 6, 5, 11, 9, 12, depth, K, _p(coef),
                                      None if w is None else _p(w), _p(cm), _p(ch), _p(cw), 1, 1,
                                      11, 9, _p(out), _stream())
    _lib.check(rc, "slg_tree_conv_fwd")
    _close(out, ref, f"tree_conv depth {depth} fixed={fixed}")
    if fixed:
        drop = kernels.tree_conv(xd, coef, cm, ch, cw, depth, 1, 1, 11, 9)
    else:
        drop = kernels.tree_conv_topk(xd, coef, w, cm, ch, cw, depth, K, 1, 1, 11, 9)
    assert torch.equal(drop.cpu(), out.cpu())
    # a gradient through the drop-in reaches x, the weights and coef
    if not fixed:
        xg, wg, cg = (t.clone().requires_grad_(True) for t in (xd, w, coef))
        kernels.tree_conv_topk(xg, cg, wg, cm, ch, cw, depth, K, 1, 1, 11, 9).sum().backward()
        xc, wc, ccf = (t.detach().cpu().clone().requires_grad_(True) for t in (x, w, coef))
        patches = F.unfold(xc, 3, padding=1)
        flat = (cm.long() * 9 + ch.long() * 3 + cw.long()).reshape(-1).cpu()
        vals = (patches[:, flat, :].view(6, 12, 2 ** depth, K, -1) *
                wc.view(1, 12, 2 ** depth, K, 1)).sum(3)
        nb, cnt = 0, 2 ** depth
        while cnt > 1:
            c = ccf[:, nb:nb + cnt // 2, :].unsqueeze(0).unsqueeze(-1)
            a, b = vals[:, :, 0::2, :], vals[:, :, 1::2, :]
            vals = c[:, :, :, 0] + c[:, :, :, 1] * a + c[:, :, :, 2] * b + c[:, :, :, 3] * (a * b)
            nb += cnt // 2
            cnt //= 2
        vals.sum().backward()
        for got, ref_g, what in ((xg.grad, xc.grad, "x"), (wg.grad, wc.grad, "w"),
                                 (cg.grad, ccf.grad, "coef")):
            _close(got, ref_g, f"tree_conv grad {what}", rtol=0,
                   atol=1e-4 * ref_g.abs().max().item())
