"""The ``torch.ops.silogic_hip`` custom operators on the GPU:
``torch.library.opcheck`` (schema, fake implementation against the kernel,
autograd registration, AOT dispatch), and the ``silogic_amd.kernels``
drop-ins that call them give the same values and gradients as the layer
path's autograd functions."""
import pytest
import torch

import silogic_amd as sl
from silogic_amd import kernels, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
CHECKS = ("test_schema", "test_autograd_registration", "test_faketensor",
          "test_aot_dispatch_dynamic")


def _fc_args(node, B=37, IN=150, OUT=70, K=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(B, IN, generator=g).to(DEV).requires_grad_()
    cand = torch.randint(0, IN, (OUT, 2, K), generator=g, dtype=torch.int32).to(DEV)
    w = torch.softmax(torch.randn(OUT, 2, K, generator=g), -1).to(DEV).requires_grad_()
    npar = torch.randn(OUT, 4, generator=g).to(DEV).requires_grad_()
    return (x, cand, w, npar, node, 0.7 if node == ops.WALSH else 1.0)


@pytest.mark.parametrize("node", [ops.GATE16, ops.WALSH, ops.MULTILINEAR2])
def test_opcheck_fc_soft(node):
    torch.library.opcheck(torch.ops.silogic_hip.fc_soft.default, _fc_args(node),
                          test_utils=CHECKS)


def test_opcheck_fc_lut_soft():
    g = torch.Generator().manual_seed(1)
    x = torch.rand(21, 90, generator=g).to(DEV).requires_grad_()
    cand = torch.randint(0, 90, (33, 4, 4), generator=g, dtype=torch.int32).to(DEV)
    w = torch.softmax(torch.randn(33, 4, 4, generator=g), -1).to(DEV).requires_grad_()
    s = torch.rand(33, 16, generator=g).to(DEV).requires_grad_()
    for hybrid in (False, True):
        torch.library.opcheck(torch.ops.silogic_hip.fc_lut_soft.default, (x, cand, w, s, hybrid),
                              test_utils=CHECKS)


@pytest.mark.parametrize("pool", [True, False])
def test_opcheck_conv_soft(pool):
    g = torch.Generator().manual_seed(2)
    x = torch.rand(3, 5, 9, 9, generator=g).to(DEV).requires_grad_()
    N, leaves, K = 6, 4, 3
    cm = torch.randint(0, 5, (N, leaves, K), generator=g, dtype=torch.int32).to(DEV)
    ch = torch.randint(0, 3, (N, leaves, K), generator=g, dtype=torch.int32).to(DEV)
    cw = torch.randint(0, 3, (N, leaves, K), generator=g, dtype=torch.int32).to(DEV)
    w = torch.softmax(torch.randn(N, leaves, K, generator=g), -1).to(DEV).requires_grad_()
    npar = torch.randn(N, leaves - 1, 4, generator=g).to(DEV).requires_grad_()
    torch.library.opcheck(torch.ops.silogic_hip.conv_soft.default,
                          (x, npar, w, cm, ch, cw, ops.GATE16, 2, 2, K, 1, pool), test_utils=CHECKS)


def test_dropins_match_the_layer_path_bitwise():
    x, cand, w, npar, node, inv_tau = _fc_args(ops.WALSH, seed=3)
    ca, cb = cand[:, 0].contiguous(), cand[:, 1].contiguous()
    wa = w.detach()[:, 0].clone().requires_grad_()
    wb = w.detach()[:, 1].clone().requires_grad_()
    y = kernels.warp_logic(x, ca, cb, wa, wb, npar, inv_tau)
    gy = torch.randn_like(y)
    gx, gwa, gwb, gn = torch.autograd.grad(y, [x, wa, wb, npar], gy)
    x2 = x.detach().clone().requires_grad_()
    w2 = torch.stack([wa.detach(), wb.detach()], 1).requires_grad_()
    n2 = npar.detach().clone().requires_grad_()
    y2 = ops.fc_soft(x2, cand, w2, n2, ops.WALSH, inv_tau)
    gx2, gw2, gn2 = torch.autograd.grad(y2, [x2, w2, n2], gy)
    assert torch.equal(y, y2) and torch.equal(gx, gx2) and torch.equal(gn, gn2)
    assert torch.equal(gwa, gw2[:, 0]) and torch.equal(gwb, gw2[:, 1])


def test_hard_ops_match_the_module_path():
    net = sl.LogicNet(64, 200, 3, k=8).to(DEV).eval()
    x = (torch.rand(150, 64, generator=torch.Generator().manual_seed(4)) < 0.5).float().to(DEV)
    with torch.no_grad():
        codes = ops.fc_hard_codes_net([l.hard_spec() for l in net.layers], compact=True)
        ref = net.forward_hard(x)
        y = torch.ops.silogic_hip.fc_hard_net(x, ops.ROWS_F32, 150, 64, codes, 10, 0)
        assert torch.equal(y, ref)
        xp = torch.ops.silogic_hip.pack_bits(x, False)
        assert torch.equal(xp, ops.pack_bits(x))
        gs = torch.ops.silogic_hip.groupsum_packed(ops.pack_bits((x[:, :60] > 0.5).float()), 150, 10)
        assert torch.equal(gs, ops.groupsum_packed(ops.pack_bits(x[:, :60]), 150, 10))
