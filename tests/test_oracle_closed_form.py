"""Pin the oracle with what the mathematics fixes, independently of the golden
vectors: closed forms, exhaustive brute force on tiny inputs, invariants —
and check that planted mistakes (in the oracle, on the CPU) are caught."""
import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import silogic_amd
from conftest import load_fixture, random_bits
from oracle import lut_sim, packed_ref, torch_ref


def _sixteen(a, b):
    """The 16 two-input functions written out independently of the basis table."""
    ab = a * b
    return torch.stack([torch.zeros_like(a), ab, a - ab, a, b - ab, b, a + b - 2 * ab,
                        a + b - ab, 1 - a - b + ab, 1 - a - b + 2 * ab, 1 - b, 1 - b + ab,
                        1 - a, 1 - a + ab, 1 - ab, torch.ones_like(a)], dim=0)


def test_truth_tables_are_the_basis_at_the_corners():
    bits = torch.tensor([[0., 0], [0, 1], [1, 0], [1, 1]])
    f = _sixteen(bits[:, 0], bits[:, 1])                       # [16, 4]
    for tt in (torch_ref.TRUTH, silogic_amd.TRUTH_TABLES):
        assert torch.equal(tt, f.round().to(torch.uint8))
    # named gates at address (a<<1)|b
    assert torch_ref.TRUTH[1].tolist() == [0, 0, 0, 1]        # AND
    assert torch_ref.TRUTH[6].tolist() == [0, 1, 1, 0]        # XOR
    assert torch_ref.TRUTH[2].tolist() == [0, 0, 1, 0]        # A and not B
    assert silogic_amd.functional.TT_CODES[1] == 0b1000


def test_basisproj_equals_full_mixture():
    """gate16 soft node == sum_g softmax_g * f_g(a, b) (nodes.py:86-98)."""
    L = dict(prefix="", node="gate16", arity=2)
    gl = torch.randn(30, 16)
    ops = torch.rand(8, 30, 2)
    y = torch_ref.node_soft(L, {"node.gate_logits": gl}, ops)
    p = F.softmax(gl, dim=1)
    full = torch.einsum("ibo,oi->bo", _sixteen(ops[..., 0], ops[..., 1]), p)
    assert (y - full).abs().max() < 1e-5


def test_walsh_change_of_variables():
    """theta form on u = 2x-1 equals the (a, b) coefficient form used by the
    kernels (nodes.py:129-143)."""
    L = dict(prefix="", node="walsh", arity=2, node_tau=1.0)
    th = torch.randn(12, 4)
    ops = torch.rand(5, 12, 2)
    y = torch_ref.node_soft(L, {"node.theta": th}, ops)
    node = silogic_amd.WARPLayer(16, 12, k=4, seed=0).node
    with torch.no_grad():
        node.theta.copy_(th)
        c = node.coef()
    a, b = ops[..., 0], ops[..., 1]
    z = c[:, 0] + c[:, 1] * a + c[:, 2] * b + c[:, 3] * (a * b)
    assert (torch.sigmoid(z) - y).abs().max() < 1e-6


def test_multilinear_interpolates_its_truth_table():
    """At cube corners the soft multilinear node equals sigmoid(logit) of the
    corner (boundary consistency) and the hard node equals logit > 0; it is
    affine in each input (nodes.py:165-189)."""
    n = 4
    logits = torch.randn(3, 2 ** n)
    corners = torch_ref.corner_bits(n)
    for p in range(2 ** n):
        ops = corners[p].view(1, 1, n).expand(1, 3, n)
        soft = torch_ref.multilinear_f(ops, logits, n)[0]
        hard = torch_ref.multilinear_hard(ops.to(torch.uint8), logits, n)[0]
        assert torch.allclose(soft, torch.sigmoid(logits[:, p]), atol=1e-6)
        assert torch.equal(hard, (logits[:, p] > 0).to(torch.uint8))
    a = torch.rand(1, 3, n)
    for j in range(n):
        lo, hi = a.clone(), a.clone()
        lo[..., j], hi[..., j] = 0.0, 1.0
        t = a[..., j]
        lin = (1 - t) * torch_ref.multilinear_f(lo, logits, n) + t * torch_ref.multilinear_f(hi, logits, n)
        assert torch.allclose(torch_ref.multilinear_f(a, logits, n), lin, atol=1e-6)


def test_hybrid_is_the_lut_at_the_thresholded_address_with_multilinear_gradient():
    """Hybrid node (nodes.py:198-206): its value is sigmoid(logit) of the
    corner the operands round to (a LUT lookup, written here as a plain index
    computation; exact, as the reference's fused kernels return it, where its
    PyTorch form adds and subtracts the soft value), and its gradient is the
    multilinear node's."""
    n = 5
    L = dict(prefix="", node="hybrid", arity=n)
    Lm = dict(prefix="", node="multilinear", arity=n)
    logits = torch.randn(4, 2 ** n)
    ops = torch.rand(7, 4, n)
    ops[0, 0, 0] = 0.5                                       # the threshold itself rounds up
    addr = ((ops >= 0.5).long() * (2 ** torch.arange(n))).sum(2)        # [B, out]
    want = torch.sigmoid(logits)[torch.arange(4)[None, :].expand(7, 4), addr]
    sd = {"node.logits": logits.clone().requires_grad_(True)}
    a = ops.clone().requires_grad_(True)
    y = torch_ref.node_soft(L, sd, a)
    assert torch.equal(y.detach(), want)
    # the reference's PyTorch form equals it up to fp32 rounding
    f_soft = torch_ref.multilinear_f(ops, logits, n)
    assert torch.allclose(want + f_soft - f_soft, want, rtol=0, atol=1e-6)
    g = torch.randn(7, 4)
    (y * g).sum().backward()
    sdm = {"node.logits": logits.clone().requires_grad_(True)}
    am = ops.clone().requires_grad_(True)
    (torch_ref.node_soft(Lm, sdm, am) * g).sum().backward()
    assert torch.equal(a.grad, am.grad)
    assert torch.equal(sd["node.logits"].grad, sdm["node.logits"].grad)


def _hardened_fc(spec):
    torch.manual_seed(0)
    model = getattr(silogic_amd, spec[0])(seed=0, **spec[1])
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    for k in list(sd):
        if k.endswith("_conn.conn"):
            c = sd[k]
            sd[k] = F.one_hot(c.argmax(2), c.shape[2]).float() * 30.0
        if k.endswith("gate_logits"):
            g = sd[k]
            sd[k] = F.one_hot(g.argmax(1), 16).float() * 30.0
        if k.endswith("node.logits"):
            sd[k] = torch.where(sd[k] > 0, 30.0, -30.0)
    return sd


@pytest.mark.parametrize("node", ["gate16", "multilinear"])
def test_hardened_soft_equals_hard(node):
    """One-hot parameters make the relaxed forward the Boolean circuit
    (tests/test_model.py:53-63 of the reference)."""
    spec = ("LogicNet", dict(in_dim=24, width=40, depth=3, num_classes=4, node=node, k=4,
                             decoder_ste=False))
    sd = _hardened_fc(spec)
    x = random_bits(16, 24)
    st = torch_ref.structure(spec)
    soft = torch_ref.forward_features(st, sd, x, hard=False)
    hard = torch_ref.forward_features(st, sd, x, hard=True)
    assert (soft - hard.float()).abs().max() < 1e-3


def test_exhaustive_brute_force_small_net():
    """All 2^10 inputs of a 3-layer net: torch oracle == packed oracle == per-
    node LUT simulation, and a hand loop over the truth tables agrees."""
    spec = ("LogicNet", dict(in_dim=10, width=20, depth=3, num_classes=4, k=4))
    torch.manual_seed(0)
    model = silogic_amd.LogicNet(seed=0, **spec[1])
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    x = torch.tensor(list(itertools.product([0, 1], repeat=10)), dtype=torch.float32)
    a = torch_ref.forward_hard(spec, sd, x).numpy()
    b = packed_ref.forward_hard(spec, sd, x.numpy())
    layers, C = lut_sim.extract(spec, sd)
    c = lut_sim.simulate(layers, C, x.numpy())
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a, c)
    # plain-Python evaluation of one sample from the raw parameters
    sample = x[777].long().tolist()
    cur = sample
    for i in range(3):
        cand, conn = sd[f"layers.{i}._conn.cand"], sd[f"layers.{i}._conn.conn"]
        gate = sd[f"layers.{i}.node.gate_logits"].argmax(1)
        nxt = []
        for o in range(20):
            ia = int(cand[o, 0, int(conn[o, 0].argmax())])
            ib = int(cand[o, 1, int(conn[o, 1].argmax())])
            nxt.append(int(torch_ref.TRUTH[gate[o], (cur[ia] << 1) | cur[ib]]))
        cur = nxt
    counts = [sum(cur[c * 5:(c + 1) * 5]) for c in range(4)]
    assert counts == a[777].astype(int).tolist()


def test_wire_residual_fc_three_ways():
    """Wire residual (models.py:88-94; packed_model.py:104-108): the torch
    oracle, the packed oracle and a plain loop over all 2^8 inputs agree."""
    spec = ("LogicNet", dict(in_dim=8, width=12, depth=3, num_classes=4, k=4,
                             wire_residual=0.25))
    torch.manual_seed(0)
    model = silogic_amd.LogicNet(seed=0, **spec[1])
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    x = torch.tensor(list(itertools.product([0, 1], repeat=8)), dtype=torch.float32)
    a = torch_ref.forward_hard(spec, sd, x).numpy()
    b = packed_ref.forward_hard(spec, sd, x.numpy())
    np.testing.assert_array_equal(a, b)
    wire_r = 3
    for s_i in (0, 77, 255):
        cur = x[s_i].long().tolist()
        for i in range(3):
            cand, conn = sd[f"layers.{i}._conn.cand"], sd[f"layers.{i}._conn.conn"]
            gate = sd[f"layers.{i}.node.gate_logits"].argmax(1)
            nxt = []
            for o in range(12):
                ia = int(cand[o, 0, int(conn[o, 0].argmax())])
                ib = int(cand[o, 1, int(conn[o, 1].argmax())])
                nxt.append(int(torch_ref.TRUTH[gate[o], (cur[ia] << 1) | cur[ib]]))
            if len(cur) == len(nxt):          # the first wire_r outputs copy the inputs
                nxt[:wire_r] = cur[:wire_r]
            cur = nxt
        assert [sum(cur[c * 3:(c + 1) * 3]) for c in range(4)] == a[s_i].astype(int).tolist()
    # the residual changes the result (the check is not vacuous)
    st_off = dict(spec[1], wire_residual=0.0)
    assert not np.array_equal(a, torch_ref.forward_hard(("LogicNet", st_off), sd, x).numpy())


def test_wire_residual_conv_packed_equals_torch():
    spec = ("LogicConvNet", dict(in_channels=4, in_hw=6, channels=[4, 4], head_widths=[20],
                                 num_classes=4, connect="topk", k=4, kernel=3, tree_depth=2,
                                 n_chan=2, wire_residual=0.5))
    torch.manual_seed(0)
    model = silogic_amd.LogicConvNet(seed=0, **spec[1])
    sd = {k: v.clone() for k, v in model.state_dict().items()}
    x = (torch.rand(70, 4, 6, 6, generator=torch.Generator().manual_seed(3)) > 0.5).float()
    a = torch_ref.forward_hard(spec, sd, x).numpy()
    np.testing.assert_array_equal(a, packed_ref.forward_hard(spec, sd, x.numpy()))
    off = ("LogicConvNet", dict(spec[1], wire_residual=0.0))
    assert not np.array_equal(a, torch_ref.forward_hard(off, sd, x).numpy())


@pytest.mark.parametrize("B,dim", [(1, 1), (63, 8), (64, 64), (65, 256), (200, 784)])
def test_pack_roundtrip_and_layout(B, dim):
    rng = np.random.default_rng(0)
    x = rng.integers(0, 2, (B, dim), dtype=np.uint8)
    xp = packed_ref.pack_bits(x)
    assert xp.shape == (dim, packed_ref.n_words(B)) and xp.dtype == np.int64
    assert (packed_ref.unpack_bits(xp, B) == x).all()
    u = xp.view(np.uint64)
    for b in (0, B // 2, B - 1):
        for d in (0, dim - 1):
            assert int((int(u[d, b // 64]) >> (b % 64)) & 1) == int(x[b, d])


def test_n_words():
    assert [packed_ref.n_words(b) for b in (1, 64, 65, 128, 129)] == [1, 1, 2, 2, 3]


def test_group_sum_packed_matches_naive():
    rng = np.random.default_rng(1)
    B, W, C = 137, 100, 10
    x = rng.integers(0, 2, (B, W), dtype=np.uint8)
    out = packed_ref.group_sum_packed(packed_ref.pack_bits(x), B, C)
    np.testing.assert_array_equal(out, x.reshape(B, C, W // C).sum(2).astype(np.float32))


def test_packed_conv_unfold_matches_torch_unfold():
    rng = np.random.default_rng(2)
    x = rng.integers(0, 2, (70, 3, 5, 6), dtype=np.uint8)
    un = packed_ref.packed_unfold(packed_ref.pack_conv_input(x), 3, 1, 1, 5, 6)
    ref = F.unfold(torch.from_numpy(x).float(), 3, padding=1).to(torch.uint8)   # [B, 27, L]
    got = packed_ref.unpack_bits(un.reshape(-1, un.shape[2]), 70).reshape(70, 27, -1)
    np.testing.assert_array_equal(got, ref.numpy())


def test_orpool_is_max_of_window():
    x = torch.rand(2, 3, 7, 5)
    ref = torch.stack([x[:, :, 0:6:2, 0:4:2], x[:, :, 1:6:2, 0:4:2],
                       x[:, :, 0:6:2, 1:4:2], x[:, :, 1:6:2, 1:4:2]]).amax(0)
    assert torch.equal(torch_ref.orpool_soft(x), ref)


# ---- planted mistakes: each must make a golden check fail -----------------
def test_planted_swapped_gate_address_is_caught(monkeypatch):
    fx = load_fixture("fc_gate16")
    bad = torch_ref.TRUTH[:, [0, 2, 1, 3]].contiguous()      # (b<<1)|a instead of (a<<1)|b
    monkeypatch.setattr(torch_ref, "TRUTH", bad)
    out = torch_ref.forward_hard(fx.spec, fx.sd, fx.x)
    assert not torch.equal(out, fx.arrays["logits_hard"])


def test_planted_missing_tau_is_caught():
    fx = load_fixture("fc_gate16")
    st = torch_ref.structure(fx.spec)
    feats = torch_ref.forward_features(st, fx.sd, fx.x, hard=False)
    head = dict(st["head"], tau=1.0)
    assert not torch.equal(torch_ref.groupsum_soft(head, feats), fx.arrays["logits_soft"])


def test_planted_wrong_walsh_sign_is_caught():
    fx = load_fixture("warp")
    sd = dict(fx.sd)
    for k in [k for k in sd if k.endswith("node.theta")]:
        sd[k] = sd[k][:, [0, 2, 1, 3]]                          # swap the u0 / u1 terms
    out = torch_ref.forward_hard(fx.spec, sd, fx.x)
    assert not torch.equal(out, fx.arrays["logits_hard"])


def test_planted_wrong_leaf_pairing_is_caught(monkeypatch):
    fx = load_fixture("conv_gate16")
    orig = torch_ref.conv_leaves_soft

    def swapped(blk, sd, patches):
        v = orig(blk, sd, patches)
        return v[:, :, [1, 0, 3, 2]]                             # pair (1,0) instead of (0,1)
    monkeypatch.setattr(torch_ref, "conv_leaves_soft", swapped)
    tr = {}
    torch_ref.forward(fx.spec, fx.sd, fx.x, ste=False, trace=tr)
    # caught by the first conv map (the error shrinks through the later layers
    # of a random-init net, so end-to-end soft logits alone would miss it)
    assert (tr["conv/0"] - fx.arrays["conv/0"]).abs().max() > 1e-4


def test_oracle_gumbel_draws_follow_the_gumbel_law():
    """torch_ref.gumbel: -log(-log u) of clamped uniforms has the standard
    Gumbel mean (Euler-Mascheroni) and variance pi^2 / 6, and re-seeding
    repeats the draws."""
    import math
    torch.manual_seed(3)
    a = torch_ref.gumbel((200000,), "cpu")
    torch.manual_seed(3)
    b = torch_ref.gumbel((200000,), "cpu")
    assert torch.equal(a, b)
    assert abs(a.mean().item() - 0.5772156649) < 0.01
    assert abs(a.var().item() - math.pi ** 2 / 6) < 0.03
    assert a.max().item() <= -math.log(-math.log(1 - 1e-6)) + 1e-4
