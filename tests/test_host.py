"""Host-side checks that need no GPU: RNG-faithful construction and
``state_dict`` layout against the reference's golden vectors, the C ABI
library loads and exports every declared entry point, and the product path
refuses to compute on the CPU."""
import ctypes
import hashlib
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

import silogic_amd
from conftest import GOLDEN, ROOT, build_product
from silogic_amd import _lib, synthetic


def test_tiny_construction_matches_reference_state_dict(fixture):
    model = build_product(fixture.spec)
    sd = model.state_dict()
    assert set(sd) == set(fixture.sd), set(sd) ^ set(fixture.sd)
    for k, v in fixture.sd.items():
        assert sd[k].dtype == v.dtype and torch.equal(sd[k], v), k


@pytest.mark.slow
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_full_size_construction_matches_reference_hashes(cfg):
    """Exact construction of the five BASELINE configs (SHA-256 of every
    state_dict tensor of the reference-built model)."""
    with open(os.path.join(GOLDEN, "construct_sha256.json")) as fh:
        ref = json.load(fh)[f"cfg{cfg}"]
    ctor, args = synthetic.CONFIGS[cfg]
    assert ref["ctor"] == ctor and ref["args"] == json.loads(json.dumps(args))
    model = synthetic.build_config(cfg)
    sd = model.state_dict()
    assert set(sd) == set(ref["tensors"])
    for k, v in sd.items():
        a = np.ascontiguousarray(v.detach().cpu().numpy())
        assert list(a.shape) == ref["tensors"][k]["shape"], k
        assert hashlib.sha256(a.tobytes()).hexdigest() == ref["tensors"][k]["sha256"], k


def _declared_symbols():
    with open(os.path.join(ROOT, "include", "silogic_hip.h")) as fh:
        text = fh.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(slg_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    path = _lib.library_path()
    if not os.path.exists(path):
        pytest.fail(f"{path} missing: run __graft_entry__.build()")
    h = ctypes.CDLL(path)
    declared = _declared_symbols()
    assert len(declared) >= 20
    missing = [s for s in declared if not hasattr(h, s)]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)
    assert h.slg_version() >= 1


def test_entry_points_reject_bad_arguments_without_a_gpu():
    """Argument validation runs before any device work and reports a message."""
    L = _lib.lib()
    rc = L.slg_fc_soft_fwd(None, 4, 8, 8, 8, None, None, 0, None, 1.0, None, 0, 0, None)
    assert rc == -1 and b"null" in L.slg_last_error()
    rc = L.slg_groupsum_soft(ctypes.c_void_p(16), 4, 25, 10, 1.0, 1, ctypes.c_void_p(16), None)
    assert rc == -2 and b"divisible" in L.slg_last_error()
    # a gate16 tree of depth 6 (64 leaves) is beyond every conv kernel
    rc = L.slg_conv_soft_fwd(ctypes.c_void_p(16), 1, 1, 4, 4, 1, 0, 6, 2, 1, ctypes.c_void_p(16),
                             None, ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                             1, 1, ctypes.c_void_p(16), None)
    assert rc == -3
    # records built for 1000 inputs, x only 999 wide: rejected before any launch
    fake = ctypes.c_void_p(256)
    rc = L.slg_fc_soft_fwd_records(fake, 4, 999, 64, 8, fake, 1000, 0, 1.0, fake, 0, 0, None)
    assert rc == -2 and b"built for 1000" in L.slg_last_error()
    rc = L.slg_fc_soft_fwd_groupsum(fake, 4, 999, 60, 8, fake, 1000, 0, 1.0, 10, 1.0, fake,
                                    None)
    assert rc == -2 and b"built for 1000" in L.slg_last_error()
    # the backward takes rows wider than 16-bit record indices (slab staging),
    # and refuses fan-ins beyond 16
    assert L.slg_fc_soft_bwd_workspace(8, 65537, 16, 8) > 0
    assert L.slg_fc_soft_bwd_workspace(8, 1 << 20, 16, 8) > 0
    assert L.slg_fc_soft_bwd_workspace(8, 1000, 16, 17) == -1


def test_hard_step_descriptor_layout_matches_the_header(tmp_path):
    """``slg_hard_step_t`` / ``slg_step_conv_t`` as ctypes lays them out, field
    by field, against the header compiled by the host C compiler; and the
    entry point's argument checks (before any launch)."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    fields = {"slg_step_conv_t": _lib.StepConv, "slg_hard_step_t": _lib.HardStep}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "silogic_hip.h"',
             "int main(void) {"]
    for cname, cls in fields.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            cf = "in" if f == "inp" else f
            lines.append(f'  printf("{cname}.{f} %zu\\n", offsetof({cname}, {cf}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True,
                                                        text=True, check=True).stdout.split("\n")
               if l)
    for cname, cls in fields.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(cls, f).offset, (cname, f)
    L = _lib.lib()
    step = _lib.HardStep()
    assert L.slg_hard_step(None, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -1
    assert b"null" in L.slg_last_error()
    step.B = 5
    assert L.slg_hard_step(ctypes.byref(step), None, ctypes.c_void_p(16), None) == -1
    step.B = 0                        # an empty batch launches nothing
    assert L.slg_hard_step(ctypes.byref(step), None, None, None) == 0
    step.n_conv = _lib.STEP_MAX_CONV + 1
    assert L.slg_hard_step(ctypes.byref(step), ctypes.c_void_p(16), ctypes.c_void_p(16),
                           None) == -1


def test_cpu_inputs_are_refused():
    net = silogic_amd.LogicNet(16, 20, 2, k=4)
    x = torch.zeros(3, 16)
    with pytest.raises(RuntimeError, match="GPU only"):
        net(x)
    with pytest.raises(RuntimeError, match="GPU only"):
        net.forward_hard(x)


def test_missing_library_fails_loudly():
    code = ("import silogic_amd, silogic_amd._lib as L\n"
            "try:\n    L.lib()\nexcept ImportError as e:\n    print('IMPORT_ERROR', e)\n"
            "print('HAS_DENSE', silogic_amd.kernels.HAS_DENSE)\n")
    env = dict(os.environ, SILOGIC_HIP_LIB="/nonexistent/libsilogic_hip.so")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=120)
    assert "IMPORT_ERROR" in r.stdout and "HAS_DENSE False" in r.stdout, r.stdout + r.stderr


def test_unsupported_components_are_rejected_at_construction():
    with pytest.raises(NotImplementedError):
        silogic_amd.LogicLayer(8, 8, connectome="dense")
    with pytest.raises(NotImplementedError):
        silogic_amd.LogicLayer(8, 8, node="linear")
    # hybrid and n-input multilinear layers construct (the LUT kernels)
    assert silogic_amd.LogicLayer(8, 8, node="hybrid", arity=4).is_lut
    assert silogic_amd.LogicLayer(8, 8, node="multilinear", arity=3).is_lut
    assert not silogic_amd.LogicLayer(8, 8, node="multilinear", arity=2).is_lut
    with pytest.raises(NotImplementedError):
        silogic_amd.LogicNet(8, 20, 2, decoder="linear")


def test_public_api_names_mirror_the_reference():
    for name in ["LogicLayer", "LogicNet", "WARPNet", "WARPLayer", "LogicConvNet",
                 "LogicTreeNet", "ConvLogicTree", "ConvLogicLayer", "OrPool", "GroupSum",
                 "BASIS_COEFFS", "TRUTH_TABLES", "build_connectome", "build_node",
                 "build_decoder", "gate_probs", "binarize_ste", "WARPLayerN", "LUTkLayer",
                 "LUTNodeLayer", "WARPNetN", "LUTkNet", "LUTNodeNet"]:
        assert hasattr(silogic_amd, name), name
    for name in ["dense_logic", "warp_logic", "tree_conv", "tree_conv_topk", "tree_conv_af",
                 "build_inverse_map", "multilinear_logic", "conv_hybrid", "HAS_DENSE",
                 "HAS_WARP", "HAS_CONV", "HAS_CONV_TOPK", "HAS_MULTILINEAR", "HAS_CONV_HYBRID"]:
        assert hasattr(silogic_amd.kernels, name), name


def test_presets_are_their_generic_constructors():
    """The presets (layers.py:162-224, models.py:117-147) are the generic
    constructors with fixed arguments: same parameters for the same seed."""
    def sd(ctor, *a, **k):
        torch.manual_seed(0)
        return ctor(*a, **k).state_dict()

    def same(a, b):
        assert a.keys() == b.keys() and all(torch.equal(a[k], b[k]) for k in a)

    same(sd(silogic_amd.LUTkNet, 30, 40, 2, k=3, cand_k=4, tau=4.0, seed=1),
         sd(silogic_amd.LogicNet, 30, 40, 2, node="multilinear", arity=3, k=4, tau=4.0, seed=1))
    same(sd(silogic_amd.LUTNodeNet, 30, 40, 2, arity=4, relaxation="hybrid", k=6, seed=2),
         sd(silogic_amd.LogicNet, 30, 40, 2, node="hybrid", arity=4, k=6, tau=10.0, seed=2))
    same(sd(silogic_amd.WARPNetN, 30, 40, 2, arity=5, k=8, seed=3),
         sd(silogic_amd.LogicNet, 30, 40, 2, node="walsh", arity=5, k=8, tau=20.0, seed=3))
    same(sd(silogic_amd.LUTkLayer, 30, 40, k=3, cand_k=5, seed=4),
         sd(silogic_amd.LogicLayer, 30, 40, node="multilinear", arity=3, k=5, seed=4))
    same(sd(silogic_amd.WARPLayerN, 30, 40, arity=4, seed=5),
         sd(silogic_amd.LogicLayer, 30, 40, node="walsh", arity=4, k=8, seed=5))
    lut = silogic_amd.LUTkLayer(30, 40, k=3, cand_k=5, learn_conn=False, seed=4)
    assert lut.k == 3 and lut.lut.shape == (40, 8) and lut.is_lut
    assert silogic_amd.WARPNetN(30, 40, 2, arity=5).head.tau == 20.0
    assert silogic_amd.LUTkNet(30, 40, 2, k=3).num_luts() == 80
    assert silogic_amd.WARPLayerN(30, 40, arity=4).is_walsh_n


def test_inverse_map_matches_the_reference_layout():
    """build_inverse_map (kernels/conv.py:247-265): channel buckets in
    ascending (n, l) order, checked against a plain loop."""
    g = torch.Generator().manual_seed(0)
    cm = torch.randint(0, 5, (7, 4), generator=g)
    ch = torch.randint(0, 3, (7, 4), generator=g)
    cw = torch.randint(0, 3, (7, 4), generator=g)
    off, en, el, edy, edx = silogic_amd.kernels.build_inverse_map(cm, ch, cw, 6)
    rows = [(n, l, int(ch[n, l]), int(cw[n, l])) for c in range(6) for n in range(7)
            for l in range(4) if int(cm[n, l]) == c]
    assert [tuple(int(t[i]) for t in (en, el, edy, edx)) for i in range(len(en))] == rows
    counts = [sum(1 for n in range(7) for l in range(4) if int(cm[n, l]) == c) for c in range(6)]
    assert off.tolist() == [sum(counts[:c]) for c in range(7)]
    assert off.dtype == en.dtype == torch.int32


def test_bitpacking_api_names_and_host_tables():
    from silogic_amd import bitpacking as bp
    from silogic_amd.bitpacking.ops import layer_codes
    from silogic_amd.bitpacking.packed_layer import _tt_word, gate16_lut_word
    from oracle import packed_ref
    for name in ["convert_logic_net", "convert_logic_conv_net", "convert_layer", "convert_head",
                 "BitpackedNet", "BitpackedConvNet", "BitpackedConvGPUNet", "packed_unfold_gpu",
                 "packed_or_pool_gpu", "pack_bits", "unpack_bits", "n_words", "HAS_TRITON"]:
        assert hasattr(bp, name), name
    assert np.array_equal(bp.code_to_gate16(), packed_ref.code_to_gate16())
    # gate16 as a LUT: entry c0 | c1 << 1 is the gate at address (c0 << 1) | c1
    for g in range(16):
        word = gate16_lut_word(g)
        for c0 in (0, 1):
            for c1 in (0, 1):
                a = np.array([-1 if c0 else 0], dtype=np.int64)
                b = np.array([-1 if c1 else 0], dtype=np.int64)
                want = int(packed_ref.GATE_OPS[g](a, b)[0] & 1)
                assert (word >> (c0 | c1 << 1)) & 1 == want, (g, c0, c1)
    assert _tt_word([0] * 63 + [1]) == -(1 << 63) and _tt_word([1, 0, 1]) == 5
    codes = layer_codes([1, 15], [3, 7], [5, (1 << 28) - 1], torch.device("cpu")).numpy()
    code_and = packed_ref.code_to_gate16().tolist().index(1)          # AND's truth-table code
    assert codes[0, 0] == 3 and (int(codes[0, 1]) & 0xFFFFFFFF) == 5 | (code_and << 28)
    assert (codes[1, 1].astype(np.int64) & 0xFFFFFFFF) >> 28 == 15
    with pytest.raises(ValueError):
        layer_codes([0], [0], [1 << 28], torch.device("cpu"))


def test_bitpacking_without_a_gpu_raises():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from silogic_amd import bitpacking as bp
    with pytest.raises((RuntimeError, AssertionError)):
        bp.pack_bits(np.zeros((4, 3), dtype=np.uint8))


def test_derived_cache_follows_parameter_versions():
    """Tables derived from parameters are rebuilt exactly when a parameter or
    buffer changes in place, moves, or the cache is cleared."""
    from silogic_amd import derived
    m = torch.nn.Linear(3, 2)
    m.register_buffer("idx", torch.arange(4))
    calls = []

    def get():
        return derived.cached(m, "_derived_t", derived.state_key(m),
                              lambda: calls.append(1) or len(calls))
    assert get() == 1 and get() == 1
    with torch.no_grad():
        m.weight.add_(1.0)                  # in-place update: version bump
    assert get() == 2 and get() == 2
    m.idx[0] = 7                            # buffer write
    assert get() == 3
    m.weight = torch.nn.Parameter(m.weight.detach().clone())   # new storage
    assert get() == 4
    derived.clear(m)
    assert get() == 5
    m.idx = torch.arange(5)                 # buffer replaced by assignment
    assert get() == 6
    m.double()                              # Module._apply: new buffer objects in _buffers
    assert get() == 7 and get() == 7


def test_derived_cache_follows_the_module_tree():
    """The key's tensors come from a list of the module tree's dictionaries
    kept per module: a child module replaced, added to a ModuleList or set
    to None, and a parameter registered on a child, all change the key."""
    from silogic_amd import derived
    net = torch.nn.Module()
    net.a = torch.nn.Linear(3, 2)
    net.seq = torch.nn.ModuleList([torch.nn.Linear(2, 2)])
    k0 = derived.state_key(net)
    assert derived.state_key(net) == k0
    net.a = torch.nn.Linear(3, 2)                     # child replaced
    k1 = derived.state_key(net)
    assert k1 != k0
    net.seq.append(torch.nn.Linear(2, 2))             # child added
    k2 = derived.state_key(net)
    assert len(k2) == len(k1) + 2
    net.seq[0].extra = torch.nn.Parameter(torch.ones(1))   # parameter on a child
    k3 = derived.state_key(net)
    assert len(k3) == len(k2) + 1
    net.a = None                                      # child removed
    assert len(derived.state_key(net)) == len(k3) - 2
    # the same tensors as a full walk, in the same order
    ts = []
    derived._tensors(net, ts)
    assert derived.state_key(net) == tuple((t.data_ptr(), t._version) for t in ts
                                           if t is not None)
