"""The ``torch.ops.silogic_hip`` custom operators without a GPU: every entry
is registered, the fake implementations give the kernels' output shapes and
dtypes, and a traced forward + backward is a graph of those operators (the
HIP backward op included) rather than a break at the ctypes call."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import silogic_amd  # noqa: F401  (registers the ops)
from silogic_amd import kernels, ops

OPS = ["fc_soft", "fc_soft_bwd", "dense_logic", "fc_lut_soft", "fc_lut_soft_bwd", "conv_soft",
       "conv_soft_bwd", "tree_conv", "groupsum_soft", "orpool", "pack_bits", "fc_hard_net",
       "groupsum_packed"]


def test_every_op_is_registered():
    for name in OPS:
        assert hasattr(torch.ops.silogic_hip, name), name


def test_fake_shapes():
    with FakeTensorMode():
        d = "cuda"
        x = torch.empty(8, 100, device=d)
        cand = torch.empty(40, 2, 8, dtype=torch.int32, device=d)
        w = torch.empty(40, 2, 8, device=d)
        npar = torch.empty(40, 4, device=d)
        assert torch.ops.silogic_hip.fc_soft(x, cand, w, npar, ops.GATE16, 1.0).shape == (8, 40)
        gx, gw, gn = torch.ops.silogic_hip.fc_soft_bwd(x, cand, w, npar, ops.GATE16, 1.0,
                                                       torch.empty(8, 40, device=d), True, False,
                                                       True)
        assert gx.shape == x.shape and gw.shape == (0,) and gn.shape == npar.shape
        s = torch.empty(40, 16, device=d)
        lc = torch.empty(40, 4, 8, dtype=torch.int32, device=d)
        assert torch.ops.silogic_hip.fc_lut_soft(x, lc, torch.empty(40, 4, 8, device=d), s,
                                                 True).shape == (8, 40)
        xi = torch.empty(2, 7, 28, 28, device=d)
        cm = torch.empty(64, 4, 4, dtype=torch.int32, device=d)
        cp = torch.empty(64, 3, 4, device=d)
        wc = torch.empty(64, 4, 4, device=d)
        for pool, shape in ((True, (2, 64, 14, 14)), (False, (2, 64, 28, 28))):
            y = torch.ops.silogic_hip.conv_soft(xi, cp, wc, cm, cm, cm, ops.GATE16, 2, 2, 4, 1, pool)
            assert y.shape == shape and y.dtype == torch.float32
        xb = torch.empty(100, 784, device=d)
        assert torch.ops.silogic_hip.pack_bits(xb, False).shape == (784, 2)
        assert torch.ops.silogic_hip.pack_bits(xb, True).shape == (2, 784)
        assert torch.ops.silogic_hip.pack_bits(xb, True).dtype == torch.int64
        codes = [torch.empty(200, dtype=torch.int32, device=d)] * 2
        assert torch.ops.silogic_hip.fc_hard_net(xb, ops.ROWS_F32, 100, 784, codes, 10,
                                                 0).shape == (100, 10)
        assert torch.ops.silogic_hip.groupsum_packed(torch.empty(200, 2, dtype=torch.int64,
                                                                 device=d), 100, 10).shape == (100, 10)


def test_traced_forward_and_backward_is_a_graph_of_the_ops():
    def step(x, ca, cb, wa, wb, coef):
        y = kernels.dense_logic(x, ca, cb, wa, wb, coef)
        return torch.autograd.grad(y.sum(), [x, wa, coef])

    def args():
        d = "meta"   # the fake implementations serve meta tensors; no device needed
        x = torch.empty(8, 100, device=d, requires_grad=True)
        ca = torch.empty(40, 8, dtype=torch.int32, device=d)
        wa = torch.empty(40, 8, device=d, requires_grad=True)
        coef = torch.empty(40, 4, device=d, requires_grad=True)
        return x, ca, ca, wa, torch.empty(40, 8, device=d), coef

    gm = make_fx(step)(*args())
    text = str(gm.graph)
    # the reference's separate-array op, then the HIP backward op
    assert "silogic_hip.dense_logic.default" in text and "silogic_hip.fc_soft_bwd.default" in text
    # x, wa and coef gradients are asked for: the weight gradient (wa's half) and coef
    bwd = [n for n in gm.graph.nodes if "fc_soft_bwd" in str(n.target)]
    assert len(bwd) == 1 and bwd[0].args[-3:] == (True, True, True)
