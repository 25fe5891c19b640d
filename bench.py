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
it (``soft_samples_per_s``). ``roofline`` is that of the fused hard-network
kernel (HBM: it must read the fp32 input), with the bit-op view in
``roofline_valu``; ``roofline_soft`` is the soft Top-K layer kernel's.
``cpu_baseline`` times the oracle (the reference's PyTorch CPU path restated)
on a bounded sample on this host.

The default run measures all five BASELINE configs the same way and adds
them under ``configs`` (the headline keys stay config 2's): each one's
forward_hard and soft forward at the config's batch sizes, its dominant soft
kernel (the widest FC layer, HBM-bound; or the first conv block with its
OrPool, FP32-bound against 157.3 TFLOP/s), for FC networks the fused
hard-network kernel, and the CPU baseline. ``--config N`` measures config N
alone.

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


def _events_ms(fn, reps):
    """Average device time of ``fn`` on the current stream (HIP events)."""
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
    """HBM bytes per launch of config ``cfg``'s dominant kernels, measured with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE and scaled by the same counters'
    reading for a plain copy of known size (profiles/hbm_traffic.json, keyed
    by config; see --kernels-only)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as fh:
        return json.load(fh).get(f"cfg{cfg}", {})


def hard_net_codes(ops, model, in_dim):
    """The codes LogicNet.forward_hard runs on unpacked rows: the type-uniform
    layout where it applies, else the bank-aware order."""
    codes = ops.fc_hard_codes_net([l.hard_spec() for l in model.layers], compact=True)
    if ops.fc_hard_type_slots(in_dim, [l.out_dim for l in model.layers]) > 0:
        return ops.fc_hard_type_place_net(codes, in_dim)
    return ops.NetCodes(ops.fc_hard_place_net(codes))


def kernels_only(reps=3):
    """Workload for counter passes: a 256 MiB copy (calibration), then
    ``reps`` times each: config 2's fused hard network and one soft hidden
    layer, config 4's walsh hidden layer, and the first conv block (with its
    OrPool) of configs 3 and 5, at the bench's batch sizes."""
    import silogic_amd as sl
    from silogic_amd import ops
    from silogic_amd.synthetic import BATCHES, build_config, config_inputs
    dev = torch.device("cuda:0")
    src = torch.ones(64 << 20, device=dev)          # 256 MiB
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    model = build_config(2, sl).eval().to(dev)
    xh = config_inputs(2, 65536).to(dev)
    with torch.no_grad():
        codes = hard_net_codes(ops, model, 784)
        for _ in range(reps):
            ops.fc_hard_net(xh, ops.ROWS_F32, 65536, 784, codes, 10)
        for cfg in (2, 4):
            m = model if cfg == 2 else build_config(cfg, sl).eval().to(dev)
            L = m.layers[1]
            x_mid = torch.rand(BATCHES[cfg][0], L.in_dim, device=dev)
            rec = ops.fc_soft_records([L.record_spec()], L.n_candidates)[0]
            for _ in range(reps):
                ops.fc_soft_rec(x_mid, rec, L.in_dim, L.out_dim, L.n_candidates, L.node.kind,
                                L._inv_tau())
        for cfg in (3, 5):
            m = build_config(cfg, sl).eval().to(dev)
            x = config_inputs(cfg, BATCHES[cfg][0]).to(dev)
            conv = m._convs()[0]
            for _ in range(reps):
                conv.forward_pooled(x)
    torch.cuda.synchronize()
    log("kernels-only done")


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


def dominant_soft_kernel(cfg, model, B_soft, x_soft, dev):
    """(name, launch function, roofline dict builder inputs) of the soft
    kernel that dominates config ``cfg``'s forward: the widest FC layer on
    records (HBM-bound: bytes), or the first (largest) conv block with its
    OrPool (FP32-bound: flops, with its bytes beside)."""
    from silogic_amd import ops
    if hasattr(model, "layers"):
        with torch.no_grad():
            model(x_soft)                      # builds (or reuses) the forward's launch plan
        slot = model.layers[0].__dict__.get("_derived_soft_plan")
        plan = slot[1] if slot else None
        if plan is not None and plan.net is not None:
            # small batch, narrow layers: the forward is one launch for the
            # whole network (with its head); that launch is the kernel
            K = model.layers[0].n_candidates
            fn = lambda: plan(x_soft)  # noqa: E731
            C = model.head.num_classes
            nbytes = (B_soft * (x_soft.shape[1] + C) * 4 +
                      sum(l.out_dim * 16 * ops.record_quads(K) for l in model.layers))
            name = (f"fc_soft_net_kernel ({len(model.layers)} layers + GroupSum, "
                    f"{model.layers[0]._node_name}, K={K}, B={B_soft})")
            return name, fn, nbytes, None
        L = model.layers[1] if len(model.layers) > 1 else model.layers[0]
        x_mid = torch.rand(B_soft, L.in_dim, device=dev)
        rec = ops.fc_soft_records([L.record_spec()], L.n_candidates)[0]
        K, OUT = L.n_candidates, L.out_dim
        fn = lambda: ops.fc_soft_rec(x_mid, rec, L.in_dim, OUT, K, L.node.kind, L._inv_tau())  # noqa: E731
        # input rows read once, output rows written once, one record per output
        nbytes = B_soft * (L.in_dim + OUT) * 4 + OUT * 16 * ops.record_quads(K)
        name = f"fc_soft_kernel ({L._node_name}, K={K}, IN={L.in_dim}, OUT={OUT}, B={B_soft})"
        return name, fn, nbytes, None
    conv = model._convs()[0]
    B, C, H, W = x_soft.shape
    fn = lambda: conv.forward_pooled(x_soft)  # noqa: E731
    nbytes = B * C * H * W * 4 + B * conv.n * (H // 2) * (W // 2) * 4
    flops = B * conv.n * H * W * conv_flops_per_position(conv)
    name = (f"conv_soft_kernel (block 0: {C}->{conv.n} channels, {H}x{W}, "
            f"{conv.node_name}, pooled, B={B})")
    return name, fn, nbytes, flops


def hard_units(cfg, model):
    """Gate evaluations per sample (the reference's counts, models.py:103-104, 277-288)."""
    if hasattr(model, "layers"):
        return model.num_gates()
    from silogic_amd.synthetic import CONFIGS
    return model.gate_count(CONFIGS[cfg][1]["in_hw"])


def measure_config(cfg, steps, warmup, with_cpu):
    """Time config ``cfg``: ``steps`` steps of forward_hard (hard batch) +
    soft forward (soft batch) after ``warmup`` untimed ones, then the
    dominant kernels alone with HIP events, then (optionally) the CPU
    baseline. Returns the config's result dict."""
    import silogic_amd as sl
    from silogic_amd import ops
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
    torch.cuda.synchronize()

    def step():
        with torch.no_grad():
            model.forward_hard(x_hard)
            model(x_soft)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

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

    # ---- dominant kernels alone, HIP events on the launch stream ----
    reps = 20
    hard = None
    with torch.no_grad():
        if hasattr(model, "layers"):
            widths = [l.out_dim for l in model.layers]
            C = model.head.num_classes
            in_dim = x_hard.shape[1]
            if ops.fc_hard_net_supported(in_dim, widths, C) == 64 and in_dim <= 1024:
                codes = hard_net_codes(ops, model, in_dim)
                fn_net = lambda: ops.fc_hard_net(x_hard, ops.ROWS_F32, B_hard, in_dim, codes, C)  # noqa: E731
                fn_net()
                k_hard = _events_ms(fn_net, reps) / 1e3
                hard_bytes = B_hard * in_dim * 4 + sum(w * 4 for w in widths) + B_hard * C * 4
                hard = ("fc_hard_net_rows_kernel (packing + %d layers + GroupSum)" % len(widths),
                        k_hard, hard_bytes)
        name, fn_soft, soft_bytes, soft_flops = dominant_soft_kernel(cfg, model, B_soft, x_soft,
                                                                     dev)
        fn_soft()
        k_soft = _events_ms(fn_soft, reps) / 1e3
    soft_gbs = soft_bytes / k_soft / 1e9
    traffic = load_traffic(cfg)
    bitops = B_hard * gates / t_hard

    res = {
        "workload": WORKLOADS[cfg], "hard_batch": B_hard, "soft_batch": B_soft,
        "gates_per_sample": gates,
        "hard_Ggate_evals_per_s": round(B_hard * gates / t_hard / 1e9, 3),
        "soft_samples_per_s": round(B_soft / t_soft, 1),
        "t_hard_us": round(t_hard * 1e6, 2), "t_soft_us": round(t_soft * 1e6, 2),
        "t_hard_graph_us": round(t_hard_graph * 1e6, 2),
        "ms_per_step": round(t_hard * 1e3, 4),
    }
    if soft_flops is None:
        soft_roof = {"kernel": name, "bound": "hbm", "achieved": round(soft_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(soft_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("fc_soft_kernel"), "algorithmic_bytes": soft_bytes,
                     "avg_kernel_us": round(k_soft * 1e6, 2)}
    else:
        tflops = soft_flops / k_soft / 1e12
        soft_roof = {"kernel": name, "bound": "fp32", "achieved": round(tflops, 2),
                     "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
                     "traffic": traffic.get("conv_soft_kernel"),
                     "algorithmic_flops": soft_flops, "algorithmic_bytes": soft_bytes,
                     "hbm_frac": round(soft_gbs / HBM_PEAK_GBS, 4),
                     "avg_kernel_us": round(k_soft * 1e6, 2)}
    res["roofline_soft"] = soft_roof
    if hard is not None:
        hname, k_hard, hard_bytes = hard
        hard_gbs = hard_bytes / k_hard / 1e9
        res["roofline_hard"] = {"kernel": hname, "bound": "hbm", "achieved": round(hard_gbs, 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(hard_gbs / HBM_PEAK_GBS, 4),
                                "traffic": traffic.get("fc_hard_net_rows_kernel"),
                                "algorithmic_bytes": hard_bytes,
                                "avg_kernel_us": round(k_hard * 1e6, 2)}
    res["roofline_valu"] = {"kernel": "forward_hard (whole packed circuit)",
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
        "roofline": roof,
        "roofline_soft": res["roofline_soft"],
        "roofline_valu": res["roofline_valu"],
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
    ap.add_argument("--train-step", action="store_true",
                    help="time a training step (soft forward + backward + Adam) instead")
    args = ap.parse_args()
    if args.kernels_only:
        kernels_only()
        return
    if args.train_step:
        train_step(args.config or 2, args.steps, args.warmup)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the workload shards by batch; see DESIGN.md). Run with --gpus 1.",
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
