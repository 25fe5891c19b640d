"""Write the golden vectors that pin what no closed form can: the reference's
RNG-faithful parameter construction and its exact fp32 soft outputs.

This script is the ONLY place the reference is executed, and only in the
development container (``/root/reference`` does not exist on the GPU box). It
imports the reference's hot-path modules (``functional``, ``nodes``,
``connectomes``, ``heads``, ``layers``, ``models``) directly: the package's
``__init__`` is bypassed because it also imports the dataset module, whose
torchvision dependency is absent here and which is not on the path.

Output (committed, numpy ``.npz`` with ``allow_pickle=False`` semantics):

* ``tiny_<name>.npz`` — a tiny model per BASELINE config family: its full
  ``state_dict``, the input batch, every layer's soft activation, soft logits
  with and without the feature STE, and the hard logits.
* ``construct_sha256.json`` — SHA-256 of every ``state_dict`` tensor of the
  FULL-size configs 1-5 (exact construction pin without storing megabytes).

Run: ``python tests/golden/make_golden.py`` (takes about a minute);
``--only=name,...`` writes just those tiny fixtures, ``--no-full`` skips the
hashes.
"""
import hashlib
import json
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference/silogic"
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # repo root

if "silogic" not in sys.modules:
    pkg = types.ModuleType("silogic")
    pkg.__path__ = [REF]
    sys.modules["silogic"] = pkg

from silogic.models import LogicNet, WARPNet, WARPNetN, LogicConvNet, LogicTreeNet  # noqa: E402
from silogic.heads import GroupSum  # noqa: E402

from silogic_amd.synthetic import (bernoulli_inputs, cfg3_images,  # noqa: E402
                                   cfg5_images)

torch.set_num_threads(4)


def _sd_arrays(model):
    out = {}
    for k, v in model.state_dict().items():
        out["sd/" + k] = v.detach().cpu().numpy()
    return out


def _soft_trace_fc(model, x):
    acts = {}
    h = x
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            h = layer(h)
            acts[f"act/{i}"] = h.numpy().copy()
        logits = model.head(h)
        nste = GroupSum(model.head.num_classes, model.head.tau, feature_ste=False)(h)
    return acts, logits, nste


def _soft_trace_conv(model, x):
    acts = {}
    h = x
    with torch.no_grad():
        for i in range(0, len(model.blocks), 2):
            conv, pool = model.blocks[i], model.blocks[i + 1]
            y = conv(h)
            acts[f"conv/{i // 2}"] = y.numpy().copy()
            h = pool(y)
            acts[f"pool/{i // 2}"] = h.numpy().copy()
        h = h.flatten(1)
        for j, layer in enumerate(model.head_layers):
            h = layer(h)
            acts[f"act/{j}"] = h.numpy().copy()
        logits = model.head(h)
        nste = GroupSum(model.head.num_classes, model.head.tau, feature_ste=False)(h)
    return acts, logits, nste


def _hard_trace_fc(model, x):
    acts = {}
    h = x
    with torch.no_grad():
        for i, layer in enumerate(model.layers):
            h = layer.forward_hard(h)
            acts[f"hact/{i}"] = h.numpy().copy()
    return acts


def _hard_trace_conv(model, x):
    acts = {}
    h = x
    with torch.no_grad():
        for i in range(0, len(model.blocks), 2):
            conv, pool = model.blocks[i], model.blocks[i + 1]
            y = conv.forward_hard(h)
            acts[f"hconv/{i // 2}"] = y.numpy().copy()
            h = pool.forward_hard(y)
        h = h.flatten(1)
        for j, layer in enumerate(model.head_layers):
            h = layer.forward_hard(h)
            acts[f"hact/{j}"] = h.numpy().copy()
    return acts


def _save(name, model, x, kind, meta):
    model.eval()
    if kind == "fc":
        acts, logits, nste = _soft_trace_fc(model, x)
        hacts = _hard_trace_fc(model, x)
    else:
        acts, logits, nste = _soft_trace_conv(model, x)
        hacts = _hard_trace_conv(model, x)
    with torch.no_grad():
        logits_fwd = model(x)
        hard = model.forward_hard(x)
    assert torch.equal(logits_fwd, logits)
    arrays = dict(_sd_arrays(model))
    arrays.update(acts)
    arrays.update(hacts)
    arrays["x"] = x.numpy()
    arrays["logits_soft"] = logits.numpy()
    arrays["logits_soft_noste"] = nste.numpy()
    arrays["logits_hard"] = hard.numpy()
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    path = os.path.join(HERE, f"tiny_{name}.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


# --- tiny versions of the five configs (same constructors, small shapes) ----
TINY = {
    # config 1/2 family: FC gate16 TopK k=8 GroupSum tau=10
    "fc_gate16": dict(kind="fc", ctor="LogicNet",
                      args=dict(in_dim=64, width=200, depth=3, num_classes=10,
                                node="gate16", connectome="topk", k=8, tau=10.0),
                      B=96, p=0.5),
    "fc_gate16_in784": dict(kind="fc", ctor="LogicNet",
                            args=dict(in_dim=784, width=400, depth=2, num_classes=10,
                                      node="gate16", connectome="topk", k=8, tau=10.0),
                            B=130, p=0.2),
    "fc_gate16_fixed": dict(kind="fc", ctor="LogicNet",
                            args=dict(in_dim=48, width=60, depth=2, num_classes=10,
                                      node="gate16", connectome="fixed", tau=10.0),
                            B=70, p=0.5),
    # config 4 family: WARPNet walsh arity 2 TopK k=8, head tau=20
    "warp": dict(kind="fc", ctor="WARPNet",
                 args=dict(in_dim=64, width=120, depth=3, num_classes=10, k=8),
                 B=70, p=0.5),
    # config 3 family: LogicTreeNet gate16 depth-2 trees, topk k=4, OrPool
    "conv_gate16": dict(kind="conv", ctor="LogicTreeNet",
                        args=dict(in_channels=7, in_hw=14, channels=[8, 16], kernel=3,
                                  tree_depth=2, node="gate16", connect="topk", k=4,
                                  n_chan=2, num_classes=10, head_widths=[40, 40],
                                  residual_init=False),
                        B=20, images="cfg3"),
    "conv_gate16_resinit": dict(kind="conv", ctor="LogicTreeNet",
                                args=dict(in_channels=7, in_hw=8, channels=[8, 16],
                                          kernel=3, tree_depth=2, node="gate16",
                                          connect="topk", k=4, n_chan=2, num_classes=10,
                                          head_widths=[40]),
                                B=10, images="cfg3"),
    # config 5 family: LogicConvNet multilinear arity-6 depth-1, OrPool, head
    "conv_lut6": dict(kind="conv", ctor="LogicConvNet",
                      args=dict(in_channels=9, in_hw=8, channels=[8, 16],
                                head_widths=[40], num_classes=10, node="multilinear",
                                arity=6, tree_depth=1, connect="topk", k=4, n_chan=2,
                                residual_init=False),
                      B=12, images="cfg5"),
    # node trees beyond the configs (the reference's own test shapes,
    # tests/test_conv.py:58-75, test_bitpacking.py:172-220): walsh trees,
    # deeper multilinear / hybrid LUT trees, n-input walsh FC nodes
    "conv_walsh": dict(kind="conv", ctor="LogicConvNet",
                       args=dict(in_channels=3, in_hw=8, channels=[8, 16], head_widths=[40],
                                 num_classes=10, node="walsh", tree_depth=2, connect="topk",
                                 k=4, n_chan=2, node_tau=0.5, residual_init=False),
                       B=12, images="cfg5_3"),
    "conv_ml2_d3": dict(kind="conv", ctor="LogicConvNet",
                        args=dict(in_channels=3, in_hw=8, channels=[8, 16], head_widths=[40],
                                  num_classes=10, node="multilinear", arity=2, tree_depth=3,
                                  connect="fixed", n_chan=2, residual_init=False),
                        B=12, images="cfg5_3"),
    "conv_ml4_d2": dict(kind="conv", ctor="LogicConvNet",
                        args=dict(in_channels=6, in_hw=10, channels=[8, 16], head_widths=[40],
                                  num_classes=10, node="multilinear", arity=4, tree_depth=2,
                                  connect="topk", k=4, n_chan=2, residual_init=False),
                        B=6, images="bits6"),
    "conv_hybrid3_d2": dict(kind="conv", ctor="LogicConvNet",
                            args=dict(in_channels=6, in_hw=10, channels=[8, 16],
                                      head_widths=[40], num_classes=10, node="hybrid", arity=3,
                                      tree_depth=2, connect="topk", k=4, n_chan=2,
                                      residual_init=False),
                            B=6, images="bits6"),
    "warp_n4": dict(kind="fc", ctor="WARPNetN",
                    args=dict(in_dim=64, width=120, depth=2, arity=4, num_classes=10, k=8),
                    B=70, p=0.5),
}

# --- full-size configs (Appendix B choices) ------
FULL = {
    "cfg1": ("LogicNet", dict(in_dim=784, width=2000, depth=4, num_classes=10,
                              node="gate16", connectome="topk", k=8, tau=10.0)),
    "cfg2": ("LogicNet", dict(in_dim=784, width=10000, depth=6, num_classes=10,
                              node="gate16", connectome="topk", k=8, tau=10.0)),
    "cfg3": ("LogicTreeNet", dict(in_channels=7, in_hw=28, channels=[64, 128, 256],
                                  kernel=3, tree_depth=2, node="gate16", connect="topk",
                                  k=4, n_chan=2, num_classes=10, head_widths=[2560, 2560],
                                  residual_init=False)),
    "cfg4": ("WARPNet", dict(in_dim=4096, width=16380, depth=4, num_classes=10, k=8)),
    "cfg5": ("LogicConvNet", dict(in_channels=9, in_hw=32, channels=[128, 256],
                                  head_widths=[1280], num_classes=10, node="multilinear",
                                  arity=6, tree_depth=1, connect="topk", k=4, n_chan=2,
                                  residual_init=False)),
}

CTORS = {"LogicNet": LogicNet, "WARPNet": WARPNet, "WARPNetN": WARPNetN,
         "LogicConvNet": LogicConvNet, "LogicTreeNet": LogicTreeNet}


def make_tiny(only=None):
    for name, spec in TINY.items():
        if only and name not in only:
            continue
        torch.manual_seed(0)
        model = CTORS[spec["ctor"]](seed=0, **spec["args"])
        g = torch.Generator().manual_seed(1)
        if spec["kind"] == "fc":
            x = bernoulli_inputs(spec["B"], spec["args"]["in_dim"], spec["p"], g)
        elif spec["images"] == "cfg3":
            x = cfg3_images(spec["B"], spec["args"]["in_hw"], g)
        elif spec["images"] == "cfg5_3":     # 3 of the 9 threshold planes
            x = cfg5_images(spec["B"], spec["args"]["in_hw"], g)[:, :3].contiguous()
        elif spec["images"] == "bits6":      # 6 random bit planes
            hw = spec["args"]["in_hw"]
            x = bernoulli_inputs(spec["B"], 6 * hw * hw, 0.5, g).view(spec["B"], 6, hw, hw)
        else:
            x = cfg5_images(spec["B"], spec["args"]["in_hw"], g)
        meta = dict(ctor=spec["ctor"], args=spec["args"], kind=spec["kind"],
                    seed=0, torch_manual_seed=0, input_seed=1, B=spec["B"])
        _save(name, model, x, spec["kind"], meta)


def make_full_hashes():
    out = {}
    for name, (ctor, args) in FULL.items():
        torch.manual_seed(0)
        model = CTORS[ctor](seed=0, **args)
        h = {}
        for k, v in model.state_dict().items():
            a = np.ascontiguousarray(v.detach().cpu().numpy())
            h[k] = dict(sha256=hashlib.sha256(a.tobytes()).hexdigest(),
                        shape=list(a.shape), dtype=str(a.dtype))
        out[name] = dict(ctor=ctor, args=args, tensors=h)
        print(f"hashed {name}: {len(h)} tensors")
    path = os.path.join(HERE, "construct_sha256.json")
    with open(path, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
    print(f"wrote {path}")


if __name__ == "__main__":
    only = None
    for a in sys.argv[1:]:
        if a.startswith("--only="):
            only = set(a[len("--only="):].split(","))
    make_tiny(only)
    if "--no-full" not in sys.argv and only is None:
        make_full_hashes()
