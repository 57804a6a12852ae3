"""Benchmark of the MoE SwiGLU layer on one MI355X (the metric and configs of BASELINE.json).

A step is one pass of the layer over one batch of seeded synthetic tokens, inputs resident in HBM:
  c1            forward at the tiny C1 shape (512 tokens, d=256, 8 experts, top-2, h=512); its CPU baseline is the
                reference's fp32 CPU path on the whole workload
  c5 (default)  training step at the C3 shape: forward + backward (16384 tokens, d=1536, 16 experts, top-2, h=4096)
  c3            forward only at the same shape
  c4            forward only, Zipf(1.2)-biased router logits, 2 experts never routed
  c2            forward only, 2048 tokens, d=1024, 8 experts, top-2, h=2048
  bailing       forward of the BailingMoeV2 block at its real shape (PoziomkaMoE: 8192 tokens, d=2048, 128 int8
                experts, sigmoid group-limited top-8 of 8 groups keeping 2, h=320, one shared expert h=320)
value = algorithmic grouped-GEMM TFLOP/s of the layer step (routed rows only: 6*M*d*h forward, 18*M*d*h forward +
backward) / measured step time; ms_per_step is the layer time of the eager step (with --graph: of replays of the
step captured once as a HIP graph, eager_ms_per_step beside it).  The roofline kernel's launch time comes from HIP
events around its launches in the eager timed pass.  With the default c5 workload the same run also times c2, c3,
c4 and bailing (--extras) and reports each under other_workloads (layer µs, grouped-GEMM TFLOP/s, per-op µs).  One
JSON line is printed.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
PEAK_HBM_GBS = 8000.0
METRIC = "MoE layer µs + grouped-GEMM TFLOP/s (% bf16 MFMA peak) at 16k tokens, 1 GPU"

WORKLOADS = {
    "c1": dict(T=512, d=256, E=8, k=2, h=512, backward=False, zipf=False, cpu_dtype="fp32", cpu_tokens=512,
               desc="C1: tiny MoE layer forward, 512 tokens, d_model=256, 8 experts, top-2, SwiGLU hidden=512 (the "
                    "reference's CPU path runs it in fp32 at full size; the GPU runs the bf16 layer)"),
    "c2": dict(T=2048, d=1024, E=8, k=2, h=2048, backward=False, zipf=False,
               desc="C2: MoE layer forward, 8 images x 256 tokens = 2048 tokens, d_model=1024, 8 experts, top-2, "
                    "SwiGLU hidden=2048"),
    "c3": dict(T=16384, d=1536, E=16, k=2, h=4096, backward=False, zipf=False,
               desc="C3: MoE layer forward, 4 images x 4096 tokens = 16384 tokens, d_model=1536, 16 experts, top-2, "
                    "SwiGLU hidden=4096"),
    "c4": dict(T=16384, d=1536, E=16, k=2, h=4096, backward=False, zipf=True,
               desc="C4: MoE layer forward, 16384 packed tokens, d_model=1536, 16 experts, top-2, SwiGLU hidden=4096, "
                    "Zipf(1.2) expert bias with 2 experts never routed"),
    "c5": dict(T=16384, d=1536, E=16, k=2, h=4096, backward=True, zipf=False,
               desc="C5: MoE layer training step (forward + backward) at the C3 shape: 16384 tokens, d_model=1536, "
                    "16 experts, top-2, SwiGLU hidden=4096"),
    "bailing": dict(T=8192, d=2048, E=128, k=8, h=320, backward=False, zipf=False, poziomka=True, shared_h=320,
                    n_group=8, topk_group=2, scaling=2.5,
                    desc="BailingMoeV2 block forward (PoziomkaMoE, aurora/hf_pipeline.py:332-370): 8192 tokens, "
                         "d_model=2048, 128 int8 experts, sigmoid router with expert bias, top-8 within the best 2 "
                         "of 8 groups, SwiGLU hidden=320, one shared expert hidden=320"),
}


def gemm_flops(w):
    M = w["T"] * w["k"]
    f = (18 if w["backward"] else 6) * M * w["d"] * w["h"]
    if w.get("poziomka"):
        f += 6 * w["T"] * w["d"] * w["shared_h"]  # the shared expert: every token
    return f


def zipf_bias(E, seed=0, s=1.2, n_empty=2):
    """Per-expert logit bias: a seeded permutation of the experts; rank r (1-based) gets -s*ln(r), the last n_empty
    get -inf (never routed)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    b = np.empty(E, np.float32)
    for r, e in enumerate(perm):
        b[e] = -np.inf if r >= E - n_empty else np.float32(-s * np.log(r + 1.0))
    return b


PROBE_STRIDE = 8


def time_steps(step, steps, warmup, graph, probe_kernel, probe_every=1, probe_first=0):
    """The timed region.  graph: the step is captured once as a HIP graph (graphs.StepGraph, after the warm-ups) and
    the timed region replays it `steps` times; an eager pass of the same number of steps follows, with events
    around the probe kernel's launches on its stream in every PROBE_STRIDE-th step (its average launch time, for the
    roofline) and its own wall time (eager_ms).  Without graph the timed region is that eager pass.  Returns (ms per step, eager ms per step,
    probe kernel ms per launch)."""
    import torch

    from trenowanie_generatora_obrazkow_amd import ops
    from trenowanie_generatora_obrazkow_amd.graphs import StepGraph

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ms = None
    if graph:
        g = StepGraph(step)
        for _ in range(max(warmup, 3)):  # the first replays of a new graph carry one-time setup
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        del g
    # the probe's two event records cost the stream a few microseconds each, so every PROBE_STRIDE-th step carries
    # them (the first step always).  A forward without gradient runs as one C call (ops.moe_forward) except in the
    # steps that carry the probe, which launch the same kernels op by op so that the events can sit between them
    probes = {probe_kernel: []}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ops.probe = probes if i % PROBE_STRIDE == 0 else None
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / steps
    ops.probe = probes
    # every probe_every-th launch of the probe kernel from launch probe_first on (the BailingMoeV2 block launches it
    # twice per step: for the shared expert and the routed experts)
    dom = [a.elapsed_time(b) for a, b in ops.probe[probe_kernel][probe_first::probe_every]]
    ops.probe = None
    return (ms if graph else eager_ms), eager_ms, statistics.mean(dom)


def run_gpu(w, steps, warmup, graph=False, probe_kernel="gate_up_swiglu"):
    import torch

    from trenowanie_generatora_obrazkow_amd import moe_swiglu, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(0)
    T, d, E, h, k = w["T"], w["d"], w["E"], w["h"], w["k"]
    x = torch.randn(T, d, generator=g).bfloat16().to(dev)
    wr = (torch.randn(E, d, generator=g) * 0.02).bfloat16().to(dev)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.02).bfloat16().to(dev)
    wd = (torch.randn(E, h, d, generator=g) * 0.02).bfloat16().to(dev)
    dout = torch.randn(T, d, generator=g).bfloat16().to(dev)
    bias = torch.zeros(E, dtype=torch.float32)
    if w["zipf"]:
        bias = torch.from_numpy(zipf_bias(E, seed=0))
    bias = bias.to(dev)
    if w["backward"]:
        for t in (x, wr, wgu, wd):
            t.requires_grad_(True)

    def step():
        if w["backward"]:
            for t in (x, wr, wgu, wd):
                t.grad = None
            out, _, _ = moe_swiglu(x, wr, wgu, wd, k, logit_bias=bias)
            out.backward(dout)
        else:
            with torch.no_grad():
                moe_swiglu(x, wr, wgu, wd, k, logit_bias=bias)

    ms, eager_ms, dom = time_steps(step, steps, warmup, graph, probe_kernel)

    # per-kernel breakdown: a second pass with events around every op (reported, not the headline)
    names = ["route_topk", "dispatch", "gate_up_swiglu", "down_scatter", "combine", "combine_bwd",
             "down_dgrad_swiglu", "grouped_wgrad", "gate_up_dgrad", "router_bwd", "unpermute_bwd"]
    ops.probe = {n: [] for n in names}
    nb = max(3, min(steps, 10))
    for _ in range(nb):
        step()
    torch.cuda.synchronize()
    kern = {}
    for n in names:
        ts = [a.elapsed_time(b) * 1e3 for a, b in ops.probe[n]]
        if not ts:
            continue
        if n == "grouped_wgrad":  # two calls per step: down (first) then gate/up
            kern["wgrad_down"] = statistics.median(ts[0::2])
            kern["wgrad_gate_up"] = statistics.median(ts[1::2])
        else:
            kern[n] = statistics.median(ts)
    ops.probe = None
    return ms, eager_ms, dom, kern


def _poziomka_block(w, g):
    """PoziomkaMoE with seeded N(0, 0.02) weights (experts quantised to int8 with per-column scales), bf16, on GPU."""
    import torch

    from trenowanie_generatora_obrazkow_amd.hf_compat import _quant_int8
    from trenowanie_generatora_obrazkow_amd.poziomka import PoziomkaMoE
    d, E, h, sh = w["d"], w["E"], w["h"], w["shared_h"]
    m = PoziomkaMoE(d, h, E, w["k"], w["n_group"], w["topk_group"], w["scaling"], sh)
    with torch.no_grad():
        m.gate.weight.copy_(torch.randn(E, d, generator=g) * 0.02)
        m.gate.expert_bias.copy_(torch.randn(E, generator=g) * 0.01)
        for lin in (m.shared_experts.gate_proj, m.shared_experts.up_proj, m.shared_experts.down_proj):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.02)
        for name, shape in (("_wgu", (E, d, 2 * h)), ("_wd", (E, h, d))):
            q, s = _quant_int8(torch.randn(shape, generator=g) * 0.02)
            getattr(m, name).copy_(q)
            getattr(m, name + "_s").copy_(s)
    return m.to(torch.bfloat16)


def run_gpu_poziomka(w, steps, warmup, graph=False):
    """Forward of the BailingMoeV2 block; the dominant kernel is the routed gate/up GEMM (int8 experts).  A step
    launches the gate/up and down GEMMs twice: the shared expert's first when it runs on its side stream
    (overlap_shared, the default), else the routed experts' first.  With the shared expert overlapping, the routed
    GEMMs' event times include the CUs they share with it."""
    import torch

    from trenowanie_generatora_obrazkow_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(0)
    m = _poziomka_block(w, g).to(dev)
    x = torch.randn(w["T"], w["d"], generator=g).bfloat16().to(dev)

    def step():
        m(x)

    routed = 1 if m.overlap_shared else 0  # position of the routed launch among a step's two
    ms, eager_ms, dom = time_steps(step, steps, warmup, graph, "gate_up_swiglu", probe_every=2, probe_first=routed)
    names = ["route_topk", "dispatch", "gate_up_swiglu", "down_scatter", "combine"]
    ops.probe = {n: [] for n in names}
    nb = max(3, min(steps, 10))
    for _ in range(nb):
        step()
    torch.cuda.synchronize()
    kern = {}
    for n in names:
        ts = [a.elapsed_time(b) * 1e3 for a, b in ops.probe[n]]
        if n in ("gate_up_swiglu", "down_scatter"):  # the routed experts' and the shared expert's launches
            kern[n] = statistics.median(ts[routed::2])
            kern[n + "_shared"] = statistics.median(ts[1 - routed::2])
        else:
            kern[n] = statistics.median(ts)
    ops.probe = None
    return ms, eager_ms, dom, kern


def cpu_threads():
    """CPU threads for the baseline: the CPUs this process may run on (len(os.sched_getaffinity(0))), capped by
    OMP_NUM_THREADS where the host sets it (a GPU box's CPU share); torch is set to that many threads.  Returns
    (threads used, affinity CPUs)."""
    import torch
    aff = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    n = min(aff, int(cap)) if cap.isdigit() and int(cap) > 0 else aff
    torch.set_num_threads(n)
    return n, aff


def time_cpu(step, budget_s, warmup=3, min_reps=10, max_reps=30):
    """3 warm-ups, then the median of at least 10 timed runs (more while the budget lasts)."""
    for _ in range(warmup):
        step()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (len(times) < max_reps and time.perf_counter() < t_end):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline_poziomka(w, budget_s=15.0):
    """The reference block's own forward (oracle/cpu_path.py: aurora/hf_pipeline.py:348-370) on CPU, on a bounded
    sample of the same workload: the full d, E, k, h with fewer tokens."""
    import torch

    from oracle import cpu_path

    threads, aff = cpu_threads()
    T = 512
    g = torch.Generator().manual_seed(0)
    m = _poziomka_block(w, g)
    x = torch.randn(T, w["d"], generator=g).bfloat16()
    sh = m.shared_experts
    args = (x, m.gate.weight, m.gate.expert_bias, m._wgu, m._wgu_s, m._wd, m._wd_s, sh.gate_proj.weight,
            sh.up_proj.weight, sh.down_proj.weight, w["k"], w["n_group"], w["topk_group"], w["scaling"])

    def step():
        with torch.no_grad():
            cpu_path.poziomka_forward(*args)

    med, reps = time_cpu(step, budget_s)
    flops = gemm_flops(dict(w, T=T))
    return {"value": flops / med / 1e12, "unit": "TFLOP/s", "cores": threads, "affinity_cpus": aff, "kind": "port",
            "us_per_layer": round(med * 1e6, 1),
            "sample": f"{T} tokens of the same block shape (d={w['d']}, E={w['E']}, top-{w['k']}, h={w['h']}, shared "
                      f"h={w['shared_h']}), bf16 activations, int8 experts, torch CPU forward with {threads} threads; "
                      f"median of {reps} runs after 3 warm-ups; {med * 1e3:.1f} ms per sample step"}


def cpu_baseline(w, budget_s=15.0):
    """The reference's PyTorch CPU path (oracle/cpu_path.py: router + _fused_moe_infer's `grouped` branch, autograd
    for the backward) on a bounded sample of the same workload: the full d, E, k, h with fewer tokens."""
    import torch

    from oracle import cpu_path

    threads, aff = cpu_threads()
    T = w.get("cpu_tokens", 2048)
    fp32 = w.get("cpu_dtype") == "fp32"
    dt = torch.float32 if fp32 else torch.bfloat16
    d, E, h, k = w["d"], w["E"], w["h"], w["k"]
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, d, generator=g).to(dt)
    wr = (torch.randn(E, d, generator=g) * 0.02).to(dt)
    wgu = (torch.randn(E, d, 2 * h, generator=g) * 0.02).to(dt)
    wd = (torch.randn(E, h, d, generator=g) * 0.02).to(dt)
    dout = torch.randn(T, d, generator=g).to(dt)
    bias = torch.from_numpy(zipf_bias(E, seed=0)) if w["zipf"] else None

    def step():
        if w["backward"]:
            ts = [t.clone().requires_grad_(True) for t in (x, wr, wgu, wd)]
            cpu_path.training_step(*ts, k, dout, bias=bias)
        else:
            with torch.no_grad():
                cpu_path.layer_forward(x, wr, wgu, wd, k, bias=bias)

    med, reps = time_cpu(step, budget_s)
    flops = (18 if w["backward"] else 6) * T * k * d * h
    what = "the whole workload" if T == w["T"] else f"{T} tokens of the same layer shape"
    return {"value": flops / med / 1e12, "unit": "TFLOP/s", "cores": threads, "affinity_cpus": aff, "kind": "port",
            "us_per_layer": round(med * 1e6, 1),
            "sample": f"{what} (d={d}, E={E}, top-{k}, h={h}), {'fp32' if fp32 else 'bf16'}, torch CPU "
                      f"{'forward+backward' if w['backward'] else 'forward'} with {threads} threads; median of {reps} "
                      f"runs after 3 warm-ups; {med * 1e3:.1f} ms per sample step"}


def library_ceiling(M, N, K, reps=10):
    """Dense bf16 (M, K) @ (K, N) through torch.matmul (the vendor BLAS, hipBLASLt on gfx950) on the same GPU: the
    practical ceiling the grouped GEMM is compared with (same M, N, K; no gather, no expert boundaries, no fused
    epilogue)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(1)
    a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16, generator=g)
    b = torch.randn(K, N, device="cuda", dtype=torch.bfloat16, generator=g)
    # warm for a quarter of a second first: a library GEMM of a new shape runs up to 20% slow over its first few dozen
    # launches (862 -> 749 -> 724 us over three 13-launch batches at the C5 gate/up shape), so a short warm-up
    # understates the library
    t_end = time.perf_counter() + 0.25
    while time.perf_counter() < t_end:
        for _ in range(4):
            c = a @ b
        torch.cuda.synchronize()
    runs = []
    for _ in range(3):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            c = a @ b
        e.record()
        torch.cuda.synchronize()
        runs.append(s.elapsed_time(e) * 1e3 / reps)
    us = sorted(runs)[1]  # the median of three timed batches
    del a, b, c
    blas = str(torch.backends.cuda.preferred_blas_library()).split(".")[-1]
    blas = {"Cublaslt": "hipBLASLt", "Cublas": "rocBLAS"}.get(blas, blas)  # torch's enum names on ROCm
    return {"kernel": f"torch.matmul bf16, dense ({M} x {K}) @ ({K} x {N}), BLAS backend {blas}",
            "M": M, "N": N, "K": K, "avg_launch_us": round(us, 2), "tflops": round(2 * M * N * K / us / 1e6, 2)}


def load_traffic(workload):
    p = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 30 warm-up steps: the step time settles over the first ~100 ms of work (clocks), 5 left it 2-4% high
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--workload", default="c5", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of the step captured once as a HIP graph instead of the eager step (kernels "
                         "launched from Python op by op); measured alternately in one process the two are within "
                         "noise at every workload here")
    ap.add_argument("--extras", default="c2,c3,c4,bailing",
                    help="with the default c5 workload, also time these workloads (comma-separated, 'none' for "
                         "none) with --extra-steps timed steps each and report them under other_workloads; value "
                         "and metric stay those of the main workload")
    ap.add_argument("--extra-steps", type=int, default=20)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of 256 MiB three times (the known-size reference for the "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        src = torch.empty(128 * 1024 * 1024, dtype=torch.bfloat16, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 2, "launches": 3}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {args.gpus} requested); the MoE layer has no "
              f"multi-GPU path here", file=sys.stderr)
        sys.exit(2)
    w = WORKLOADS[args.workload]
    pz = bool(w.get("poziomka"))
    ms, eager_ms, dom_ms, kern = (run_gpu_poziomka if pz else run_gpu)(w, args.steps, args.warmup,
                                                                     graph=args.graph)
    flops = gemm_flops(w)
    tflops = flops / (ms * 1e-3) / 1e12
    M = w["T"] * w["k"]
    dom_flops = 4 * M * w["d"] * w["h"]  # gate/up: 2 * M * d * (2h)
    dom_tflops = dom_flops / (dom_ms * 1e-3) / 1e12
    traffic = load_traffic(args.workload)
    lib = library_ceiling(M, 2 * w["h"], w["d"])
    lib["achieved_over_library"] = round(dom_tflops / lib["tflops"], 4)
    res = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) tokens and upstream gradient, N(0,0.02) router and expert weights "
                "(torch CPU generator, seed 0, fp32 then bf16" + ("; experts quantised to int8 with per-column bf16 "
                                                                  "scales)" if pz else ")"),
        "config": {"workload": w["desc"], "tokens": w["T"], "d_model": w["d"], "experts": w["E"], "top_k": w["k"],
                   "hidden": w["h"], "pass": "forward+backward" if w["backward"] else "forward"},
        "layer_us": round(ms * 1e3, 1),
        "execution": "hip_graph" if args.graph else "eager",
        "eager_ms_per_step": round(eager_ms, 4),
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "gemm_flops_per_step": flops,
        "roofline": {"bound": "mfma", "kernel": "hmoe gate/up grouped GEMM + fused SwiGLU (grouped_gemm_kernel, "
                                                "EPI_SWIGLU" + (", int8 weights" if pz else "") + ")",
                     "achieved": round(dom_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(dom_tflops / PEAK_BF16_TFLOPS, 4),
                     "flops_per_launch": dom_flops, "avg_launch_us": round(dom_ms * 1e3, 2),
                     "traffic": traffic.get("bytes_per_launch") if traffic else None,
                     "library_ceiling": lib},
        "kernels_us": {k_: round(v, 1) for k_, v in kern.items()},
    }
    if pz:
        res["config"].update(shared_hidden=w["shared_h"], n_group=w["n_group"], topk_group=w["topk_group"],
                             weights="int8 experts, bf16 router and shared expert")
    if args.workload == "c5" and args.extras != "none":
        res["other_workloads"] = {n: run_extra(n, args.extra_steps) for n in args.extras.split(",") if n}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = (cpu_baseline_poziomka if pz else cpu_baseline)(w)
    print(json.dumps(res), flush=True)


def run_extra(name, steps):
    """One more workload timed in the same process (eager, steps timed steps after 5 warm-ups: the GPU is warm
    from the main workload): layer time, grouped-GEMM rate and the per-op breakdown."""
    if name not in WORKLOADS:
        raise SystemExit(f"bench.py: unknown extra workload {name!r}")
    w = WORKLOADS[name]
    pz = bool(w.get("poziomka"))
    ms, _, dom_ms, kern = (run_gpu_poziomka if pz else run_gpu)(w, steps, 5)
    flops = gemm_flops(w)
    tflops = flops / (ms * 1e-3) / 1e12
    M = w["T"] * w["k"]
    dom_tflops = 4 * M * w["d"] * w["h"] / (dom_ms * 1e-3) / 1e12
    return {"config": w["desc"], "pass": "forward+backward" if w["backward"] else "forward", "steps": steps,
            "layer_us": round(ms * 1e3, 1), "gemm_tflops": round(tflops, 2),
            "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
            "gate_up_frac": round(dom_tflops / PEAK_BF16_TFLOPS, 4),
            "kernels_us": {k_: round(v, 1) for k_, v in kern.items()}}


if __name__ == "__main__":
    main()
