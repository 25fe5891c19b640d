"""Benchmark of the silogic gate-layer hot path on one MI355X.

Workload ("config 2"): LogicNet(784 -> 10000 x 6,
gate16, TopK k=8, GroupSum 10 classes, tau 10), seeded random parameters
(torch.manual_seed(0), seed=0), synthetic Bernoulli(0.2) inputs. One step =
``forward_hard`` on B = 65536 samples (bit-packed circuit, 64 samples per
word); the soft ``forward`` on the first 4096 of them is timed the same way
in a region of its own. Inputs are resident in HBM before timing starts. HIP
events at the two ends of each region (K steps between synchronisations)
give the time per step.

``value`` = hard-circuit Ggate-evals/s = 65536 * 60000 / t_hard (the
reference's gate count, models.py:103-104); the soft rate is reported beside
it (``soft_samples_per_s``). ``cpu_baseline`` times the oracle (the
reference's PyTorch CPU path restated) on a bounded sample on this host.

Before the timed regions, after the ``--warmup`` steps, a settle phase runs
untimed steps for 300 ms of wall time (``settle_ms``), so a short warm-up
does not time the GPU while its clocks are still rising.

Every launch is then timed alone with HIP events on its stream:
``hard_kernels`` lists each launch of ``forward_hard`` (packing, conv blocks,
fused networks) with its algorithmic bytes and bit-ops and both fractions;
``soft_kernels`` each timed stage of the soft forward (the FC hidden layer,
or every conv block with its OrPool and the FC head). Bit-ops count one per
two-input gate and 2^k - 1 per arity-k LUT node, plus three ORs per pooled
output.
* ``roofline`` (config 2: the fused hard network) = ``roofline_hard``: for FC
  networks the launches from fp32 rows to logits (HBM-bound on the input
  read); for conv networks the conv block that takes the most time
  (VALU-bound, bit-ops against 1.258e15/s).
* ``roofline_soft``: the soft stage with the largest share of the forward's
  time (HBM for FC layers; FP32 against 157.3 TFLOP/s for conv blocks).
* ``roofline_valu``: bit-ops of the whole eager hard step.

The default run measures all five BASELINE configs the same way and adds
them under ``configs`` (the headline keys stay config 2's). ``--config N``
measures config N alone; ``--kernels-only`` runs every launch three times
for counter passes; ``--param-change`` times ``forward_hard``'s first call
after a parameter change (the one-time re-derivation of its tables).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config N] [--no-cpu]
"""
import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0                      # MI355X HBM3E
VALU_BITOPS_PEAK = 256 * 64 * 2.4e9 * 32   # CUs x lanes x clock x bits = 1.258e15


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _events_ms(fn, reps, settle_ms=60.0):
    """Average device time of ``fn`` on the current stream (HIP events), after
    ``settle_ms`` of untimed calls: a launch timed straight after host work
    (building a plan, capturing a graph) otherwise starts on lowered clocks."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        fn()
    e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


# bounded CPU samples (hard samples, soft samples) per config: about 10-30 s of
# CPU work at most, chunk sizes as BASELINE.md's CPU plan suggests
CPU_SAMPLE = {1: (256, 256), 2: (4096, 512), 3: (64, 16), 4: (512, 128), 5: (64, 4)}


def cpu_baseline(cfg, sd, x_hard, x_soft, gates):
    """Oracle (reference PyTorch CPU path) on bounded samples of the workload."""
    from oracle import torch_ref
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    from silogic_amd.synthetic import CONFIGS
    spec = CONFIGS[cfg]
    nh, ns = CPU_SAMPLE[cfg]
    nh, ns = min(nh, x_hard.shape[0]), min(ns, x_soft.shape[0])
    xh, xs = x_hard[:nh].contiguous(), x_soft[:ns].contiguous()

    def timed(fn, reps=3):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), max(ts) - min(ts)

    th, sh = timed(lambda: torch_ref.forward_hard(spec, sd, xh))
    tsft, ss = timed(lambda: torch_ref.forward(spec, sd, xs))
    cpu = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        cpu = next((l.split(":", 1)[1].strip() for l in out.splitlines()
                    if l.startswith("Model name")), cpu)
    except Exception:
        pass
    return {
        "value": round(nh * gates / th / 1e9, 4), "unit": "Ggate-evals/s",
        "cores": threads, "kind": "port",
        "sample": (f"oracle forward_hard on {nh} of the {x_hard.shape[0]} hard samples (median "
                   f"of 3 after 1 warm-up, spread {sh:.3f}s, {th:.3f}s each); soft forward on "
                   f"{ns} samples: {ns / tsft:.1f} samples/s ({tsft:.3f}s, spread {ss:.3f}s)"),
        "soft_samples_per_s": round(ns / tsft, 2),
        "host": {"cpu": cpu, "os_cpu_count": os.cpu_count(), "torch": torch.__version__,
                 "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
                 "python": platform.python_version()},
    }


def load_traffic(cfg):
    """HBM bytes per launch of config ``cfg``'s launches, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over ``--kernels-only`` and
    scaled by the same counters' reading for a plain copy of known size
    (profiles/hbm_traffic.json: per config, launch name -> bytes)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as fh:
        return json.load(fh).get(f"cfg{cfg}", {})


def kernels_only(reps=3, cfgs=(1, 2, 3, 4, 5)):
    """Workload for counter passes: a 256 MiB device copy (calibration), then,
    per config of ``cfgs`` at the bench's batch sizes, ``reps`` launches each of every
    launch of ``forward_hard`` (packing, conv blocks, fused networks) and of
    every stage of the soft forward the bench times. Each group of ``reps``
    launches runs after one untimed launch and between two one-byte
    ``bitwise_not_`` launches (no other code here runs that op), so that a
    trace can assign its dispatches to the group; the groups' names, in
    order, are printed as one JSON line on stdout (``cfgN | <launch name>``,
    the names the bench's per-launch records use)."""
    import silogic_amd as sl
    from silogic_amd.synthetic import BATCHES, build_config, config_inputs
    dev = torch.device("cuda:0")
    marker = torch.zeros(1, device=dev, dtype=torch.uint8)
    groups = []

    def group(label, fn, nbytes, work):
        fn()
        torch.cuda.synchronize()
        marker.bitwise_not_()
        for _ in range(reps):
            fn()
        marker.bitwise_not_()
        torch.cuda.synchronize()
        groups.append({"launch": label, "algorithmic_bytes": nbytes, "work": work})

    src = torch.ones(64 << 20, device=dev)          # 256 MiB
    dst = torch.empty_like(src)
    group("calibration | 256 MiB copy", lambda: dst.copy_(src), 2 * src.numel() * 4, None)
    del src, dst
    for cfg in cfgs:
        model = build_config(cfg, sl).eval().to(dev)
        B_soft, B_hard = BATCHES[cfg][:2]
        x_hard = config_inputs(cfg, B_hard).to(dev)
        x_soft = x_hard[:B_soft].contiguous()
        with torch.no_grad():
            for name, fn, nbytes, bops in hard_launches(cfg, model, x_hard):
                group(f"cfg{cfg} | {name}", fn, nbytes, {"bitops": bops})
            for name, fn, nbytes, flops, _, _ in soft_stages(cfg, model, B_soft, x_soft, dev):
                group(f"cfg{cfg} | {name}", fn, nbytes, {"flops": flops})
        log(f"kernels-only: config {cfg} done")
        del model, x_hard, x_soft
        torch.cuda.empty_cache()
    print(json.dumps({"kernels_only_groups": groups, "reps": reps}), flush=True)
    log("kernels-only done")


def param_change(cfg, reps=5):
    """The one-time cost of ``forward_hard`` after a parameter change on
    config ``cfg``: after a settle phase of steady calls, ``reps`` times an
    in-place update of the first layer's first parameter (the new
    parameter version makes every derived table stale: hard codes, the
    type-uniform placement, launch plans) followed by one timed call, then
    the steady call time. Prints one JSON line (wall and HIP-event times)."""
    import silogic_amd as sl
    from silogic_amd.synthetic import BATCHES, build_config, config_inputs
    dev = torch.device("cuda:0")
    model = build_config(cfg, sl).eval().to(dev)
    B_hard = BATCHES[cfg][1]
    x = config_inputs(cfg, B_hard).to(dev)
    first = model.layers[0] if hasattr(model, "layers") else model._convs()[0]
    param = next(first.parameters())     # the connection logits

    def call():
        with torch.no_grad():
            model.forward_hard(x)

    settle(call, 200.0)

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3, e0.elapsed_time(e1)

    after = []
    for _ in range(reps):
        with torch.no_grad():
            param.add_(0.0)            # a new version of the same values
        after.append(timed(call))
        for _ in range(3):
            call()
    steady = [timed(call) for _ in range(20)]
    wall = sorted(a[0] for a in after)[len(after) // 2]
    gpu = sorted(a[1] for a in after)[len(after) // 2]
    swall = sorted(a[0] for a in steady)[len(steady) // 2]
    sgpu = sorted(a[1] for a in steady)[len(steady) // 2]
    print(json.dumps({
        "config": cfg, "what": "forward_hard after a parameter change (median of %d)" % reps,
        "after_change_wall_ms": round(wall, 3), "after_change_gpu_ms": round(gpu, 3),
        "steady_wall_ms": round(swall, 3), "steady_gpu_ms": round(sgpu, 3),
        "overhead_wall_ms": round(wall - swall, 3)}), flush=True)


def train_step(cfg, steps, warmup):
    """One training step of config ``cfg`` at its soft batch: soft forward,
    cross-entropy on synthetic labels, backward through the HIP kernels
    (FC and conv soft backward, GroupSum), Adam update. Prints one JSON line
    (samples per second); not the headline metric."""
    import silogic_amd as sl
    from silogic_amd.synthetic import BATCHES, build_config, config_inputs
    dev = torch.device("cuda:0")
    B = BATCHES[cfg][0]
    model = build_config(cfg, sl).train().to(dev)
    x = config_inputs(cfg, B).to(dev)
    labels = torch.randint(0, 10, (B,), generator=torch.Generator().manual_seed(2)).to(dev)
    opt = torch.optim.Adam(model.parameters(), lr=1e-3)

    def step():
        opt.zero_grad(set_to_none=True)
        loss = torch.nn.functional.cross_entropy(model(x), labels)
        loss.backward()
        opt.step()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    print(json.dumps({"metric": "train_samples_per_s", "value": B * 1e3 / ms,
                      "unit": "samples/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
                      "ms_per_step": ms, "higher_is_better": True, "dtype": "fp32",
                      "data": "synthetic", "config": {"workload": WORKLOADS[cfg],
                                                      "global_batch": B}}), flush=True)


WORKLOADS = {
    1: "cfg1: LogicNet(784, 2000, 4, gate16, TopK k=8, GroupSum 10, tau=10); forward_hard + "
       "soft forward, B=256 Bernoulli(0.5)",
    2: "cfg2: LogicNet(784, 10000, 6, gate16, TopK k=8, GroupSum 10, tau=10); forward_hard "
       "B=65536 Bernoulli(0.2) + soft forward B=4096",
    3: "cfg3: LogicTreeNet 28x28x7 (5 thermometer + 2 edge planes), channels [64,128,256], "
       "gate16 trees depth 2, TopK k=4, OrPool, head [2560,2560], GroupSum 10; B=1024",
    4: "cfg4: WARPNet(4096, 16380, 4, walsh, TopK k=8, GroupSum 10, tau=20); forward_hard + "
       "soft forward, B=4096 Bernoulli(0.5)",
    5: "cfg5: LogicConvNet 32x32x9 (3 channels x 3 thresholds), channels [128,256], "
       "multilinear LUT6 trees depth 1, TopK k=4, OrPool, head [1280], GroupSum 10; B=512",
}


FP32_PEAK_TFLOPS = 157.3                   # MI355X vector fp32 (spec, packed)


def conv_flops_per_position(conv):
    """FP32 operations of one pre-pool output position of a conv tree: the
    leaf sums (K FMAs a leaf) and the nodes (gate16: c0 + c1 a + c2 b + c3 ab
    = 7; LUT: the 2^n - 1 FMAs of a lerp tree), FMAs counted as 2."""
    K = conv.k if conv.connect != "fixed" else 1
    leaf = conv.leaves * K * 2
    if conv.node_name in ("gate16", "walsh"):
        return leaf + 7 * (conv.leaves - 1)
    return leaf + 2 * ((2 ** conv.node_arity) - 1) * conv.gates_per_output


def node_bitops(name, arity):
    """Bit-operations of one hard node on one sample: a two-input gate
    (gate16, or walsh hardened to its truth table) is one; an arity-k LUT
    node (multilinear, hybrid) is a Shannon tree of 2^k - 1 two-to-one muxes."""
    if name in ("gate16", "walsh") and arity == 2:
        return 1
    return (1 << arity) - 1


def conv_geometry(model, in_hw):
    """``[(conv, H, W, Ho, Wo)]`` per block (square inputs, every block pooled 2x2)."""
    out, hw = [], in_hw
    for conv in model._convs():
        Hf = hw + 2 * conv.padding - conv.kh + 1
        out.append((conv, hw, hw, Hf // 2, Hf // 2))
        hw = Hf // 2
    return out


def conv_block_bitops(conv, H, W, Ho, Wo):
    """Bit-ops per sample of one hard conv block: the reference's gate count
    for it (n * H * W * gates_per_output, models.py:277-288) times the node's
    bit-ops, plus the 2x2 OR-pool's three ORs per pooled output."""
    return (conv.n * H * W * conv.gates_per_output * node_bitops(conv.node_name, conv.node_arity)
            + 3 * conv.n * Ho * Wo)


def fc_bitops(layers):
    return sum(l.out_dim * node_bitops(l._node_name, l.arity) for l in layers)


def hard_units(cfg, model):
    """Gate evaluations per sample (the reference's counts, models.py:103-104, 277-288)."""
    if hasattr(model, "layers"):
        return model.num_gates()
    from silogic_amd.synthetic import CONFIGS
    return model.gate_count(CONFIGS[cfg][1]["in_hw"])


def hard_bitops(cfg, model):
    """Bit-ops per sample of the whole hard circuit (gate-evals x bit-ops per node,
    plus the OR-pools)."""
    if hasattr(model, "layers"):
        return fc_bitops(model.layers)
    from silogic_amd.synthetic import CONFIGS
    geo = conv_geometry(model, CONFIGS[cfg][1]["in_hw"])
    return sum(conv_block_bitops(*g) for g in geo) + fc_bitops(model.head_layers)


def soft_stages(cfg, model, B_soft, x_soft, dev):
    """The launches of config ``cfg``'s soft forward that can be timed alone:
    ``[(name, fn, bytes, flops, count, extra)]``. FC networks: the widest hidden
    layer on records (``count`` = how many such layers the forward runs;
    HBM-bound: bytes), or the one-launch network. Conv networks: every conv
    block with its OrPool on its real input (FP32-bound: flops, bytes
    beside) and the FC head."""
    from silogic_amd import ops
    stages = []
    if hasattr(model, "layers"):
        with torch.no_grad():
            model(x_soft)                      # builds (or reuses) the forward's launch plan
        slot = model.layers[0].__dict__.get("_derived_soft_plan")
        plan = slot[1] if slot else None
        K = model.layers[0].n_candidates
        if plan is not None and plan.net is not None:
            # the forward is one launch for the whole network (with its
            # head): activations stay in LDS. Its bytes are counted as the
            # per-layer schedule moves them (every layer reads its input
            # rows, writes its outputs and reads its records; the head is
            # fused in the last layer), beside the HBM bytes it moves (the
            # input rows, the logits and each layer's records once) and
            # the record stream from L2 (every tile reads every record)
            C = model.head.num_classes
            rec_b = [-(-l.out_dim // 64) * 64 * 16 * ops.record_quads(K)
                     for l in model.layers]
            sched, w = 0, x_soft.shape[1]
            for i, l in enumerate(model.layers):
                out_w = C if (i + 1 == len(model.layers) and plan.head is not None) else l.out_dim
                sched += B_soft * (w + out_w) * 4 + rec_b[i]
                w = l.out_dim
            moved = B_soft * (x_soft.shape[1] + C) * 4 + sum(rec_b)
            maxw = max([x_soft.shape[1]] + [l.out_dim for l in model.layers])
            S = 4 if (plan.net_kind == 1 or maxw * 16 + 16 * C <= 160 * 1024) else 2
            stream = -(-B_soft // S) * sum(rec_b)
            kname = "fc_soft_rec_net_kernel" if plan.net_kind == 2 else "fc_soft_net_kernel"
            name = (f"{kname} ({len(model.layers)} layers + GroupSum, "
                    f"{model.layers[0]._node_name}, K={K}, B={B_soft}, {S}-sample tiles)")
            extra = {"hbm_bytes_moved": moved, "l2_record_stream_bytes": stream,
                     "bytes_counted_as": "per-layer schedule (input rows + outputs + records "
                                         "per layer, head fused)"}
            return [(name, lambda: plan(x_soft), sched, None, 1, extra)]
        L = model.layers[1] if len(model.layers) > 1 else model.layers[0]
        x_mid = torch.rand(B_soft, L.in_dim, device=dev)
        rec = ops.fc_soft_records([L.record_spec()], L.n_candidates)[0]
        OUT = L.out_dim
        fn = lambda: ops.fc_soft_rec(x_mid, rec, L.in_dim, OUT, K, L.node.kind, L._inv_tau())  # noqa: E731
        # input rows read once, output rows written once, one record per output
        nbytes = B_soft * (L.in_dim + OUT) * 4 + OUT * 16 * ops.record_quads(K)
        name = f"fc_soft_kernel ({L._node_name}, K={K}, IN={L.in_dim}, OUT={OUT}, B={B_soft})"
        n_same = sum(1 for l in model.layers[1:] if l.in_dim == L.in_dim and l.out_dim == OUT)
        return [(name, fn, nbytes, None, max(1, n_same), {})]
    x = x_soft
    with torch.no_grad():
        for i, conv in enumerate(model._convs()):
            B, C, H, W = x.shape
            xin = x
            fn = (lambda c=conv, t=xin: c.forward_pooled(t))
            y = fn()
            nbytes = xin.numel() * 4 + y.numel() * 4
            flops = B * conv.n * H * W * conv_flops_per_position(conv)
            name = (f"conv_soft block {i}: {C}->{conv.n} channels, {H}x{W}, "
                    f"{conv.node_name}, pooled, B={B}")
            stages.append((name, fn, nbytes, flops, 1, {}))
            x = y
        feats = x.flatten(1).contiguous()
        from silogic_amd.models import _soft_fc_stack
        fn = lambda: _soft_fc_stack(model.head_layers, model.head, feats, 0)  # noqa: E731
        fn()
        nbytes = feats.numel() * 4 + B_soft * model.head.num_classes * 4 + sum(
            l.out_dim * 16 * ops.record_quads(l.n_candidates) for l in model.head_layers)
        stages.append((f"head: {len(model.head_layers)} FC layers + GroupSum, B={B_soft}",
                       fn, nbytes, None, 1, {}))
    return stages


def hard_launches(cfg, model, x_hard):
    """The C-ABI launches of ``forward_hard`` on ``x_hard`` (the cached
    ``slg_hard_step`` descriptor), each with what it moves and computes:
    ``[(name, fn, bytes, bitops)]``. ``fn`` re-launches that one kernel on the
    descriptor's own buffers."""
    import ctypes
    from silogic_amd import ops
    from silogic_amd.synthetic import CONFIGS
    with torch.no_grad():
        model.forward_hard(x_hard)
    slot = model.__dict__.get("_derived_hard_step")
    step = slot[1] if slot else None
    if step is None:
        return []
    out = torch.empty(step.out_shape, device=x_hard.device)
    B = x_hard.shape[0]
    nw = ops.n_words(B)
    isz = x_hard.element_size()
    # the descriptor's launches as separate C-ABI calls (what slg_hard_step
    # makes), each on the descriptor's own buffers
    from silogic_amd import _lib
    L, d, st = _lib.lib(), step.step, step.st
    xv, ov = ctypes.c_void_p(x_hard.data_ptr()), ctypes.c_void_p(out.data_ptr())
    calls = []
    if d.pack == 1:
        calls.append((L.slg_pack_image_wm, "slg_pack_image_wm",
                      [xv, d.dtype, B, d.C, d.H, d.W, d.pack_pad, d.packed, st]))
    elif d.pack == 2:
        calls.append((L.slg_pack_bits, "slg_pack_bits",
                      [xv, d.dtype, B, d.C * d.H * d.W, 1, d.packed, st]))
    # a one-layer head at a small batch evaluates the last conv block itself
    fused = step.fuses_head
    for c in d.conv[:d.n_conv - (1 if fused else 0)]:
        calls.append((L.slg_conv_hard_fwd_wm, "slg_conv_hard_fwd_wm",
                      [c.inp, B, c.C, c.H, c.W, c.N, c.node_kind, c.depth, c.arity, c.leaf, c.tt,
                       c.kernel, c.pad, c.out, c.out_pad, st]))
    hin = d.head_in if d.head_in else xv
    if fused == 1:
        c = d.conv[d.n_conv - 1]
        width = ctypes.cast(d.widths, ctypes.POINTER(ctypes.c_int64))[0]
        codes0 = ctypes.cast(d.codes, ctypes.POINTER(ctypes.c_void_p))[0]
        calls.append((L.slg_conv_hard_head_wm, "slg_conv_hard_head_wm",
                      [c.inp, B, c.C, c.H, c.W, c.N, c.node_kind, c.depth, c.arity, c.leaf, c.tt,
                       c.kernel, c.pad, width, codes0, d.plan, d.n_classes, ov, st]))
    elif fused == 2:
        c = d.conv[d.n_conv - 1]
        calls.append((L.slg_conv_hard_net_wm, "slg_conv_hard_net_wm",
                      [c.inp, B, c.C, c.H, c.W, c.N, c.node_kind, c.depth, c.arity, c.leaf, c.tt,
                       c.kernel, c.pad, d.n_layers, d.widths, d.codes, d.plan, d.n_classes, ov,
                       st]))
    elif d.plan:
        calls.append((L.slg_fc_hard_net_typed, "slg_fc_hard_net_typed",
                      [hin, d.head_in_kind, B, d.head_in_dim, d.n_layers, d.widths, d.codes,
                       d.plan, d.n_classes, ov, st]))
    else:
        calls.append((L.slg_fc_hard_net, "slg_fc_hard_net",
                      [hin, d.head_in_kind, B, d.head_in_dim, d.n_layers, d.widths, d.codes,
                       d.n_classes, d.wire_r, ov, st]))
    res = []
    geo = None if hasattr(model, "layers") else conv_geometry(model, CONFIGS[cfg][1]["in_hw"])
    conv_i = 0
    for fn, name, a in calls:
        launch = (lambda f=fn, aa=a: f(*aa))
        if name in ("slg_pack_bits", "slg_pack_image_wm"):
            D = x_hard[0].numel()
            res.append(("pack_kernel", launch, B * D * isz + D * nw * 8, 0))
        elif name in ("slg_conv_hard_fwd", "slg_conv_hard_fwd_wm"):
            conv, H, W, Ho, Wo = geo[conv_i]
            Cin = a[1] if name == "slg_conv_hard_fwd" else a[2]
            nbytes = (Cin * H * W + conv.n * Ho * Wo) * nw * 8
            res.append((f"conv_hard block {conv_i}: {Cin}->{conv.n} channels, {H}x{W}, "
                        f"{conv.node_name} arity {conv.node_arity}, pooled",
                        launch, nbytes, B * conv_block_bitops(conv, H, W, Ho, Wo)))
            conv_i += 1
        elif name in ("slg_conv_hard_head_wm", "slg_conv_hard_net_wm"):
            # counted as the launches it replaces: the whole conv block and the head
            conv, H, W, Ho, Wo = geo[conv_i]
            layers, C = list(model.head_layers), model.head.num_classes
            nbytes = a[2] * H * W * nw * 8 + B * C * 4 + sum(l.out_dim for l in layers) * 4
            what = (f"conv block {conv_i}: {a[2]}->{conv.n} channels, {H}x{W}, "
                    f"{conv.node_name} arity {conv.node_arity}, pooled, evaluated inside the")
            kname = (f"conv_head_kernel ({what} 1-layer head + GroupSum, {nw} words x {C} "
                     "classes)" if name == "slg_conv_hard_head_wm" else
                     f"conv_net_kernel ({what} {len(layers)}-layer head + GroupSum, {nw} words)")
            res.append((kname, launch, nbytes,
                        B * (conv_block_bitops(conv, H, W, Ho, Wo) + fc_bitops(layers))))
            conv_i += 1
        else:
            layers = model.layers if hasattr(model, "layers") else model.head_layers
            in_dim, C = a[3], model.head.num_classes
            widths = [l.out_dim for l in layers]
            codes = sum(widths) * 4
            cus = torch.cuda.get_device_properties(x_hard.device).multi_processor_count
            if a[1] in (0, 1):       # rows: packing inside
                nbytes = B * in_dim * isz + B * C * 4 + codes
                spw = ops.fc_hard_net_supported(in_dim, widths, C)
                if in_dim <= 1024 and spw == 64 and 4 * nw > cus:
                    kname = f"fc_hard_net_rows_kernel (packing + {len(widths)} layers + GroupSum)"
                else:                # a tile per workgroup, packed in LDS
                    kname = (f"fc_hard_net_packed_kernel (packing per tile + {len(widths)} "
                             "layers + GroupSum)")
            elif len(widths) == 1 and 2 * nw < cus and widths[0] // C <= 8192:
                # one layer, few words: a workgroup per (word, class)
                nbytes = in_dim * nw * 8 + B * C * 4 + codes
                kname = f"fc_hard_head_kernel (1 layer + GroupSum, {nw} words x {C} classes)"
            else:
                nbytes = in_dim * nw * 8 + B * C * 4 + codes
                kname = f"fc_hard_net_packed_kernel ({len(widths)} layers + GroupSum)"
            res.append((kname, launch, nbytes, B * fc_bitops(layers)))
    return res


def settle(step, ms=300.0):
    """Untimed steps until ``ms`` of wall time has passed (synchronising every
    few steps), so the timed region starts at the clocks the GPU keeps under
    load whatever the warm-up count. Returns (wall ms, steps)."""
    t0, n = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            step()
        n += 8
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3, n


def _roof_hbm(name, nbytes, t, traffic=None, **extra):
    gbs = nbytes / t / 1e9
    d = {"kernel": name, "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
         "algorithmic_bytes": nbytes, "avg_kernel_us": round(t * 1e6, 2)}
    d.update(extra)
    return d


def measure_config(cfg, steps, warmup, with_cpu):
    """Time config ``cfg``: ``steps`` steps of forward_hard (hard batch) +
    soft forward (soft batch) after ``warmup`` untimed ones and a settle
    phase, then every hard launch and soft stage alone with HIP events, then
    (optionally) the CPU baseline. Returns the config's result dict."""
    import silogic_amd as sl
    from silogic_amd.synthetic import build_config, config_inputs, BATCHES

    dev = torch.device("cuda:0")
    log(f"config {cfg}: building (seeded construction) ...")
    model = build_config(cfg, sl).eval()
    sd_cpu = {k: v.clone() for k, v in model.state_dict().items()} if with_cpu else None
    model = model.to(dev)
    B_soft, B_hard, _, _ = BATCHES[cfg]
    x_hard_cpu = config_inputs(cfg, B_hard)
    x_hard = x_hard_cpu.to(dev)
    x_soft = x_hard[:B_soft].contiguous()
    gates = hard_units(cfg, model)
    bitops_ps = hard_bitops(cfg, model)
    torch.cuda.synchronize()

    def step():
        with torch.no_grad():
            model.forward_hard(x_hard)
            model(x_soft)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    settle_ms, settle_steps = settle(step)

    # ---- timed regions: exactly `steps` steps between synchronisations ----
    # A step is forward_hard on the batch (the metric's unit of work); the
    # soft forward is timed the same way in a region of its own. Events go
    # only at the two ends of a region: an event's queue marker holds the
    # next kernel back by about 5 us, which a per-step event would charge to
    # every step.
    stream = torch.cuda.current_stream()

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            e0.record(stream)
            for _ in range(steps):
                fn()
            e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return e0.elapsed_time(e1) / 1e3 / steps, wall

    t_hard, wall = timed(lambda: model.forward_hard(x_hard))
    t_soft, _ = timed(lambda: model(x_soft))
    # the same hard step replayed from a captured graph (no per-call host
    # work): where the eager loop is host-bound, this is the GPU's rate
    from silogic_amd.graphs import CapturedForward
    captured = CapturedForward(model.forward_hard, x_hard)
    for _ in range(warmup):
        captured()
    t_hard_graph, _ = timed(captured)
    del captured
    log(f"config {cfg}: hard step {t_hard * 1e6:.1f} us (wall {wall / steps * 1e6:.1f} us, "
        f"graph replay {t_hard_graph * 1e6:.1f} us); soft forward {t_soft * 1e6:.1f} us")

    # ---- every launch alone, HIP events on the launch stream ----
    reps = 20
    traffic = load_traffic(cfg)
    with torch.no_grad():
        hard_k = []
        for name, fn, nbytes, bops in hard_launches(cfg, model, x_hard):
            fn()
            t = _events_ms(fn, reps) / 1e3
            hard_k.append({"kernel": name, "avg_kernel_us": round(t * 1e6, 2),
                           "algorithmic_bytes": nbytes,
                           "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                           "bitops": bops,
                           "valu_frac": round(bops / t / VALU_BITOPS_PEAK, 4),
                           "traffic": traffic.get(name)})
        soft_k = []
        for name, fn, nbytes, flops, count, extra in soft_stages(cfg, model, B_soft, x_soft, dev):
            fn()
            t = _events_ms(fn, reps) / 1e3
            rec = {"kernel": name, "avg_kernel_us": round(t * 1e6, 2), "launches_per_forward": count,
                   "algorithmic_bytes": nbytes,
                   "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                   "traffic": traffic.get(name)}
            rec.update(extra)
            if "l2_record_stream_bytes" in extra:
                rec["l2_record_GBps"] = round(extra["l2_record_stream_bytes"] / t / 1e9, 1)
            if flops is not None:
                rec["algorithmic_flops"] = flops
                rec["fp32_frac"] = round(flops / t / 1e12 / FP32_PEAK_TFLOPS, 4)
            soft_k.append(rec)

    res = {
        "workload": WORKLOADS[cfg], "hard_batch": B_hard, "soft_batch": B_soft,
        "gates_per_sample": gates, "bitops_per_sample": bitops_ps,
        "hard_Ggate_evals_per_s": round(B_hard * gates / t_hard / 1e9, 3),
        "soft_samples_per_s": round(B_soft / t_soft, 1),
        "t_hard_us": round(t_hard * 1e6, 2), "t_soft_us": round(t_soft * 1e6, 2),
        "t_hard_graph_us": round(t_hard_graph * 1e6, 2),
        "ms_per_step": round(t_hard * 1e3, 4),
        "settle_ms": round(settle_ms, 1), "settle_steps": settle_steps,
        "hard_kernels": hard_k, "soft_kernels": soft_k,
    }
    # soft roofline: the stage with the largest share of the forward's time
    dom = max(soft_k, key=lambda r: r["avg_kernel_us"] * r["launches_per_forward"])
    t_dom = dom["avg_kernel_us"] / 1e6
    if "algorithmic_flops" in dom:
        tflops = dom["algorithmic_flops"] / t_dom / 1e12
        res["roofline_soft"] = {
            "kernel": dom["kernel"], "bound": "fp32", "achieved": round(tflops, 2),
            "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
            "traffic": traffic.get(dom["kernel"]),
            "algorithmic_flops": dom["algorithmic_flops"],
            "algorithmic_bytes": dom["algorithmic_bytes"], "hbm_frac": dom["hbm_frac"],
            "avg_kernel_us": dom["avg_kernel_us"],
            "share_of_forward": round(dom["avg_kernel_us"] / (t_soft * 1e6), 3)}
    else:
        extra = {k: dom[k] for k in ("hbm_bytes_moved", "l2_record_stream_bytes",
                                     "l2_record_GBps", "bytes_counted_as") if k in dom}
        res["roofline_soft"] = _roof_hbm(
            dom["kernel"], dom["algorithmic_bytes"], t_dom,
            traffic.get(dom["kernel"]),
            share_of_forward=round(dom["avg_kernel_us"] * dom["launches_per_forward"]
                                   / (t_soft * 1e6), 3), **extra)
    # hard roofline. FC networks: the launches from the fp32 rows to the
    # logits (packing, where it is a launch of its own, plus the fused
    # network), HBM-bound on the input read. Conv networks: the conv block
    # that takes the most time, VALU-bound (bit-ops).
    if hard_k:
        if hasattr(model, "layers"):
            t = sum(r["avg_kernel_us"] for r in hard_k) / 1e6
            nbytes = B_hard * x_hard.shape[1] * 4 + B_hard * model.head.num_classes * 4 + \
                sum(l.out_dim for l in model.layers) * 4
            name = " + ".join(r["kernel"] for r in hard_k)
            moved = [traffic.get(r["kernel"]) for r in hard_k]
            res["roofline_hard"] = _roof_hbm(
                name, nbytes, t, None if None in moved else sum(moved),
                valu_frac=round(B_hard * bitops_ps / t / VALU_BITOPS_PEAK, 4))
        else:
            convs = [r for r in hard_k if r["kernel"].startswith("conv_hard")]
            d = max(convs, key=lambda r: r["avg_kernel_us"])
            t = d["avg_kernel_us"] / 1e6
            res["roofline_hard"] = {
                "kernel": d["kernel"], "bound": "valu",
                "achieved": d["bitops"] / t, "peak": VALU_BITOPS_PEAK, "unit": "bit-ops/s",
                "frac": d["valu_frac"], "traffic": traffic.get(d["kernel"]),
                "algorithmic_bitops": d["bitops"], "algorithmic_bytes": d["algorithmic_bytes"],
                "hbm_frac": d["hbm_frac"], "avg_kernel_us": d["avg_kernel_us"]}
    bitops = B_hard * bitops_ps / t_hard
    res["roofline_valu"] = {"kernel": "forward_hard (whole packed circuit, eager step)",
                            "achieved_bitops_per_s": bitops, "peak": VALU_BITOPS_PEAK,
                            "frac": round(bitops / VALU_BITOPS_PEAK, 6)}
    if with_cpu:
        log(f"config {cfg}: cpu baseline (oracle on host cores) ...")
        res["cpu_baseline"] = cpu_baseline(cfg, sd_cpu, x_hard_cpu, x_hard_cpu[:B_soft], gates)
    del model, x_hard, x_soft
    torch.cuda.empty_cache()
    return res


def bench_line(head_cfg, res, steps, warmup, configs=None):
    """The driver's JSON line: BASELINE.json's metric on config ``head_cfg``
    (value = hard Ggate-evals/s, soft samples/s beside it), plus per-config
    records when measured."""
    roof = res.get("roofline_hard", res["roofline_soft"])
    line = {
        "metric": "hard-circuit Ggate-evals/s + soft fwd samples/s; % HBM/VALU roofline, 1 GPU",
        "value": res["hard_Ggate_evals_per_s"],
        "unit": "Ggate-evals/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {"workload": res["workload"], "hard_batch": res["hard_batch"],
                   "soft_batch": res["soft_batch"], "gates_per_sample": res["gates_per_sample"]},
        "soft_samples_per_s": res["soft_samples_per_s"],
        "soft_dtype": "f32",
        "t_hard_us": res["t_hard_us"],
        "t_hard_graph_us": res["t_hard_graph_us"],
        "t_soft_us": res["t_soft_us"],
        "settle_ms": res["settle_ms"],
        "roofline": roof,
        "roofline_soft": res["roofline_soft"],
        "roofline_valu": res["roofline_valu"],
        "hard_kernels": res["hard_kernels"],
        "soft_kernels": res["soft_kernels"],
    }
    if "cpu_baseline" in res:
        line["cpu_baseline"] = res["cpu_baseline"]
    if configs:
        line["configs"] = configs
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # the GPU runs at lower clocks after the idle of each config's build:
    # a timed block after 5 warm-up steps measured up to 20% slower than after 50
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=0, choices=[0, 1, 2, 3, 4, 5],
                    help="measure only BASELINE config N (default: the headline config 2 "
                         "plus a record of every config)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--kernels-only", action="store_true",
                    help="run only the copy calibration and the dominant kernels (for --pmc)")
    ap.add_argument("--param-change", action="store_true",
                    help="time forward_hard's first call after a parameter change instead")
    ap.add_argument("--train-step", action="store_true",
                    help="time a training step (soft forward + backward + Adam) instead")
    args = ap.parse_args()
    if args.kernels_only:
        kernels_only(cfgs=(args.config,) if args.config else (1, 2, 3, 4, 5))
        return
    if args.param_change:
        param_change(args.config or 2)
        return
    if args.train_step:
        train_step(args.config or 2, args.steps, args.warmup)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the workload would shard by batch, one slice per GPU). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.config:
        res = measure_config(args.config, args.steps, args.warmup, not args.no_cpu)
        print(json.dumps(bench_line(args.config, res, args.steps, args.warmup)), flush=True)
        return
    # default: every config, the headline line on config 2
    configs = {}
    for cfg in (1, 2, 3, 4, 5):
        configs[str(cfg)] = measure_config(cfg, args.steps, args.warmup, not args.no_cpu)
    print(json.dumps(bench_line(2, configs["2"], args.steps, args.warmup, configs)), flush=True)


if __name__ == "__main__":
    main()
