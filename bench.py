#!/usr/bin/env python3
"""Benchmark: causal GQA attention forward + backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config qwen7b_s512]
    python bench.py --precision fp32      # the fp32-operand mode (fp32 tensors and MFMAs)
    python bench.py --component proj      # the q/k/v projections with LoRA adapters
    python bench.py --component norm      # the residual add + RMSNorm

One step = the attention layer's forward (RoPE, QK^T, causal softmax, PV,
saving the row log-sum-exp) followed by its backward (dP, softmax gradient,
dQ/dK/dV with the GQA reduction, inverse RoPE) on device-resident bf16
tensors: BASELINE.json configs[1] (Qwen2.5-7B: B=1, S=512, 28 Q / 4 KV heads,
head_dim 128, theta 1e6).  Prints ONE JSON line.

value  = algorithmic FLOPs per step / wall time per step, where algorithmic
         FLOPs = 12 * D * Hq * sum_b L_b (L_b + 1) / 2 (4 D per unmasked
         (query, key, head) triple forward, 8 D backward; no credit for the
         score recompute, softmax or RoPE).
roofline = the dominant kernel (largest share of device time), its average
         duration from events that its own launches timestamp (on the stream
         it runs on), against the 2.5 PFLOP/s dense bf16 MFMA peak of MI355X;
         traffic = its HBM bytes per launch measured with rocprofv3 counters
         (profiles/attn_kernels_<config>[_fp32]_pmc.md).
cpu_baseline = the C restatement of the reference CPU path (oracle/), fp32,
         on this host's cores, over a bounded sample.
timing = before the W warmup steps the step runs untimed for --settle-ms of
         wall clock (default 200 ms), so that the K timed steps see the GPU's
         steady state after sustained work, not its ramp from idle (at
         --steps 20 --warmup 5 the headline read 39.5-39.8 us per step without
         it, 36.6-37.2 us with 100-300 ms of it); the timed region is exactly
         the K steps either way, and timing.settle reports the steps it ran.

--precision fp32 runs the same step in the fp32-operand mode (fp32 device
tensors, v_mfma_f32_16x16x4f32 with fp32 accumulation) and prices it against
the 157.3 TFLOP/s dense fp32 MFMA peak.

--component proj measures the projection step instead (include/glacier_qkv.h):
one step = glacier_proj_forward + glacier_proj_backward of the q, k and v
projections of Qwen2.5-7B (T=512, hidden 3584 -> 3584, 512, 512, with bias)
with rank-16 LoRA adapters (alpha 32) on all three, bf16 tensors.

--component norm measures the residual add + RMSNorm (include/glacier_norm.h):
one step = glacier_rmsnorm_forward (x1 = x + delta, y = RMSNorm(x1) w) +
glacier_rmsnorm_backward (dx = RMSNormBackward(dy; x1, w) + d_residual) at
Qwen2.5-7B (T=512, hidden 3584, eps 1e-6), bf16 tensors; value = algorithmic
HBM bytes (each input row read once, each output row written once) per second.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "glacier.tune_amd"))

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
METRIC = "causal GQA attn fwd+bwd TFLOP/s + % bf16 MFMA peak, Qwen2.5-7B shape S=512"

# The shape each config is (BASELINE.json's configs index where it is one).
CONFIG_LABEL = {
    "qwen7b_s512": ("Qwen2.5-7B shape S=512", "BASELINE.json configs[1]"),
    "qwen05b_s512": ("Qwen2.5-0.5B shape S=512", "BASELINE.json configs[0]'s shape"),
    "qwen7b_s4096": ("Qwen2.5-7B shape S=4096", "BASELINE.json configs[3]"),
    "llama3_b2_s2048": ("Llama-3-8B shape B=2 S=2048", "BASELINE.json configs[4]"),
    "qwen7b_ckpt28_varlen": ("Qwen2.5-7B 28-layer checkpointed step, 4 packed sequences",
                             "BASELINE.json configs[2]"),
}


def settle(step, ms, sync):
    """Runs step() untimed for ms of wall clock (batches of 16, one sync per
    batch so the device stays busy while the host enqueues the next batch);
    returns the steps run.  The timed steps then see the GPU's steady state."""
    n = 0
    if ms > 0:
        t_end = time.perf_counter() + ms / 1e3
        while time.perf_counter() < t_end and n < 100000:
            for _ in range(16):
                step()
            n += 16
            sync()
    return n


def metric_name(config, precision):
    """BASELINE.json's metric for its own config and mode; the same form,
    naming the shape and the peak priced against, for the others."""
    if config == "qwen7b_s512" and precision == "bf16":
        return METRIC
    return (f"causal GQA attn fwd+bwd TFLOP/s + % {precision} MFMA peak, "
            f"{CONFIG_LABEL[config][0]}")

CONFIGS = {
    # name: (lengths, Hq, Hkv, D, theta, layers).  layers == 1: one attention
    # layer's forward + backward; layers > 1: a checkpointed training step,
    # where every layer runs forward (no save), then, in reverse layer order,
    # the recompute forward (saving lse, q_rot, k_rot) and the backward.
    "qwen7b_s512": ([512], 28, 4, 128, 1.0e6, 1),
    "qwen05b_s512": ([512], 14, 2, 64, 1.0e6, 1),
    "qwen7b_s4096": ([4096], 28, 4, 128, 1.0e6, 1),
    "llama3_b2_s2048": ([2048, 2048], 32, 8, 128, 5.0e5, 1),
    # 28 layers, 4 packed sequences with lengths
    # drawn from U[64, 512] by numpy.random.default_rng(5).integers(64, 513, 4)
    "qwen7b_ckpt28_varlen": ([365, 425, 74, 426], 28, 4, 128, 1.0e6, 28),
}

# Algorithmic FLOPs per unmasked (query, key, head) triple, per kernel: the
# forward does QK^T and PV (4 D); the backward kernel dP, dV, dK and dQ (8 D);
# rope_k, the backward's row stats and the dK/dV head reduction are credited
# with none.  Sum: 12 D.
FLOPS_PER_PAIR = {"attn_fwd": 4, "attn_bwd": 8, "rope_k": 0, "attn_bwd_reduce": 0,
                  "attn_bwd_stats": 0}


# HBM bytes per launch of each kernel, per config and mode, from two
# rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) scaled by a plain copy of
# known size; profiles/attn_kernels_<config>[_fp32]_pmc.md gives the commands
# and the calibration.
def measured_traffic(config, kernel, precision="bf16"):
    path = os.path.join(ROOT, "profiles", f"attn_kernels_{config}"
                        f"{'_fp32' if precision == 'fp32' else ''}_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes" and f[1] == kernel:
            return int(f[2])
    return None


def pairs(lengths):
    return sum(L * (L + 1) // 2 for L in lengths)


def host_cpu():
    """What the CPU baseline runs on: model name, ISA level, CPU counts."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "model name" and model == "unknown":
                    model = val.strip()
                elif key == "flags" and not flags:
                    flags = set(val.split())
    except OSError:
        pass
    isa = "AVX-512" if "avx512f" in flags else "AVX2" if "avx2" in flags else "x86-64"
    return {"model": model, "isa": isa, "cpus_usable": len(os.sched_getaffinity(0)),
            "cpu_count": os.cpu_count()}


def cpu_threads(Hq):
    """Threads for the CPU leg: the reference's Parallel.For over the query
    heads (CausalAttentionKernel.cs:26,102) uses up to Hq, capped by the CPUs
    this process may use (and OMP_NUM_THREADS where the host sets a share)."""
    n = min(len(os.sched_getaffinity(0)), Hq)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def native_oracle(oracle):
    """Builds the oracle for this host's ISA (-march=native: AVX-512 where the
    host has it) outside the tree, checks it against the portable build on a
    small layer bit for bit, and loads it.  Returns (path, bitwise_equal)."""
    import subprocess
    import tempfile

    import numpy as np

    out = os.path.join(tempfile.mkdtemp(prefix="glacier_oracle_"), "liboracle_native.so")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "native",
                    f"NATIVE_OUT={out}"], check=True)
    S, Hq, Hkv, D = 96, 4, 2, 64
    args = (oracle.fill_normal((S, Hq, D), 11), oracle.fill_normal((S, Hkv, D), 12),
            oracle.fill_normal((S, Hkv, D), 13), oracle.fill_normal((S, Hq, D), 14, 0.0, 0.01))
    ref = oracle.layer_fwd_bwd(*args, 1.0e6)
    oracle.use_library(out)
    got = oracle.layer_fwd_bwd(*args, 1.0e6)
    same = all(np.array_equal(ref[k], got[k]) for k in ref)
    return out, same


def cpu_baseline(lengths, Hq, Hkv, D, theta, budget_s=12.0):
    """Times oracle.layer_fwd_bwd (fp32, the reference CPU path restated),
    built for this host's ISA, over the query heads on this host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    cpu = host_cpu()
    _, same = native_oracle(oracle)
    threads = cpu_threads(Hq)
    oracle.set_threads(threads)
    S = lengths[0]
    q = oracle.fill_normal((S, Hq, D), 1)
    k = oracle.fill_normal((S, Hkv, D), 2)
    v = oracle.fill_normal((S, Hkv, D), 3)
    dO = oracle.fill_normal((S, Hq, D), 4, 0.0, 0.01)
    oracle.layer_fwd_bwd(q, k, v, dO, theta)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        oracle.layer_fwd_bwd(q, k, v, dO, theta)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    flops = 12.0 * D * Hq * pairs([S])
    return {
        "value": round(flops / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu": cpu["model"],
        "isa": cpu["isa"],
        "build": "gcc -O3 -march=native -ffp-contract=off (built on this host)",
        "bitwise_equal_to_portable_build": same,
        "cpus_usable": cpu["cpus_usable"],
        "cpu_count": cpu["cpu_count"],
        "sample": (f"median of {len(times)} full layer fwd+bwd passes (RoPE, attention fwd "
                   f"materialising P, attention bwd, inverse RoPE) at S={S}, Hq={Hq}, "
                   f"Hkv={Hkv}, D={D}, fp32; {med * 1e3:.1f} ms each; OpenMP over the "
                   f"{Hq} query heads on {threads} threads (min of usable CPUs, Hq and "
                   f"OMP_NUM_THREADS)"),
    }


PROJ_SHAPE = (512, 3584, (3584, 512, 512), 16, 2.0)  # T, hidden, q/k/v outs, rank, alpha/rank


def proj_flops(T, n_in, outs, rank):
    """Algorithmic FLOPs of one projection forward + backward: the base
    products X W^T and dY W, and per adapter X A, (XA) B, dY B^T, (XA)^T dY,
    X^T dL and dL A^T (2 flop per multiply-add; no credit for recomputing X A)."""
    base = 2 * 2.0 * T * n_in * sum(outs)
    lora = sum(2.0 * T * rank * (3 * n_in + 3 * o) for o in outs)
    return base + lora


def cpu_proj_baseline(T, n_in, outs, rank, s, budget_s=20.0):
    """Times oracle.proj_forward + proj_backward for the three projections."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = cpu_threads(1 << 30)
    oracle.set_threads(threads)
    x = oracle.fill_normal((T, n_in), 1)
    projs = []
    for i, o in enumerate(outs):
        projs.append((oracle.fill_normal((o, n_in), 10 + i, 0.0, n_in ** -0.5),
                      oracle.fill_normal((o,), 20 + i, 0.0, 0.1),
                      oracle.fill_normal((n_in, rank), 30 + i, 0.0, n_in ** -0.5),
                      oracle.fill_normal((rank, o), 40 + i, 0.0, 0.1),
                      oracle.fill_normal((T, o), 50 + i, 0.0, 0.01)))

    def one():
        dx = np.zeros((T, n_in), np.float32)
        for w, b, a, bb, dy in projs:
            oracle.proj_forward(x, w, b, a, bb, s)
            oracle.proj_backward(x, dy, w, a, bb, s, dx=dx)

    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(proj_flops(T, n_in, outs, rank) / med / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"median of {len(times)} full q/k/v projection fwd+bwd passes "
                   f"(LoraAdapter.Forward/Backward restated, fp32) at T={T}, hidden={n_in}, "
                   f"outs={list(outs)}, rank={rank}; {med * 1e3:.0f} ms each; OpenMP over rows"),
    }


def run_proj(args):
    import torch

    import glacier_attn as ga

    T, n_in, outs, rank, s = PROJ_SHAPE
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    rnd = lambda *shape: torch.randn(*shape, device=dev, generator=g)
    x = rnd(T, n_in).bfloat16()
    projs = []
    for o in outs:
        projs.append({"w": (rnd(o, n_in) / n_in ** 0.5).bfloat16(), "bias": 0.1 * rnd(o),
                      "a": rnd(n_in, rank) / n_in ** 0.5, "b": 0.1 * rnd(rank, o), "scaling": s,
                      "y": torch.empty(T, o, device=dev, dtype=torch.bfloat16),
                      "dy": (0.01 * rnd(T, o)).bfloat16(),
                      "grad_a": torch.zeros(n_in, rank, device=dev),
                      "grad_b": torch.zeros(rank, o, device=dev)})
    dx = torch.empty_like(x)
    eng = ga.GpuAttentionEngine(0, ga.PREC_BF16)

    def step():
        eng.proj_forward(x, projs, rank)
        eng.proj_backward(x, projs, rank, dx=dx)

    settle_steps = settle(step, args.settle_ms, torch.cuda.synchronize)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    flops = proj_flops(T, n_in, outs, rank)
    tflops = flops / (ms * 1e-3) / 1e12
    cpu = None if args.no_cpu else cpu_proj_baseline(T, n_in, outs, rank, s)
    res = {
        "metric": "q/k/v projection + LoRA fwd+bwd TFLOP/s + % bf16 MFMA peak, Qwen2.5-7B shape T=512",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 3),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded normal x, W, bias, adapters, dY; device-resident)",
        "config": {
            "workload": "qkv_proj_qwen7b_t512: q/k/v projections with bias and rank-16 LoRA, fwd+bwd",
            "tokens": T, "hidden": n_in, "out_features": list(outs), "lora_rank": rank,
            "lora_scaling": s, "io": "bf16 x/W/y/dY/dX, fp32 bias/adapters/gradients",
            "parallelism": "1 GPU", "algorithmic_gflop_per_step": round(flops / 1e9, 4),
        },
        "roofline": {"bound": "mfma", "kernel": "whole step (the library's own q/k/v GEMMs "
                     "and low-rank kernels)", "achieved": round(tflops, 3), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 5),
                     "traffic": None},
        "cpu_baseline": cpu,
        "timing": {"settle": {"ms": args.settle_ms, "steps": settle_steps}},
    }
    print(json.dumps(res), flush=True)
    eng.close()


NORM_SHAPE = (512, 3584, 1.0e-6)  # Qwen2.5-7B: tokens, hidden, rms_norm_eps
PEAK_HBM_GBS = 8000.0
NORM_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "rmsnorm_qwen7b_t512_pmc.md")


def norm_bytes(T, n, esz):
    """Algorithmic bytes per launch: forward reads x, delta and writes x1, y;
    backward reads dy, x1, d_residual and writes dx; both read the weight."""
    return {"rmsnorm_fwd": 4 * T * n * esz + 4 * n, "rmsnorm_bwd": 4 * T * n * esz + 4 * n}


def norm_traffic(kernel):
    if not os.path.exists(NORM_TRAFFIC_FILE):
        return None
    for line in open(NORM_TRAFFIC_FILE):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes" and f[1] == kernel:
            return int(f[2])
    return None


def cpu_norm_baseline(T, n, eps, nbytes, budget_s=15.0):
    """Times oracle.rmsnorm_forward (with delta) + rmsnorm_backward (with
    d_residual), fp32, OpenMP over rows; the rate is the bf16 step's
    algorithmic bytes over the CPU time."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = cpu_threads(1 << 30)
    oracle.set_threads(threads)
    x, delta = oracle.fill_normal((T, n), 1), oracle.fill_normal((T, n), 2, 0.0, 0.5)
    dy, dres = oracle.fill_normal((T, n), 3), oracle.fill_normal((T, n), 4, 0.0, 0.3)
    w = oracle.fill_normal((n,), 5, 1.0, 0.2)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 200 and (len(times) < 5 or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        x1, _ = oracle.rmsnorm_forward(x, w, eps, delta=delta)
        oracle.rmsnorm_backward(dy, x1, w, eps, d_residual=dres)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"median of {len(times)} fwd+bwd passes (RMSNorm/RMSNormBackward and the "
                      f"residual adds restated, fp32) at T={T}, hidden={n}; {med * 1e3:.2f} ms "
                      "each; OpenMP over rows; rate = the bf16 step's algorithmic bytes / time"}


def run_norm(args):
    import torch

    import glacier_attn as ga

    T, n, eps = NORM_SHAPE
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    rnd = lambda *shape: torch.randn(*shape, device=dev, generator=g)
    x, delta = rnd(T, n).bfloat16(), (0.5 * rnd(T, n)).bfloat16()
    dy, dres = rnd(T, n).bfloat16(), (0.3 * rnd(T, n)).bfloat16()
    w = 1.0 + 0.2 * rnd(n)
    x1, y, dx = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)
    eng = ga.GpuAttentionEngine(0, ga.PREC_BF16)

    def fwd():
        eng.rmsnorm_forward(x, w, eps, delta=delta, x1=x1, y=y)

    def bwd():
        eng.rmsnorm_backward(dy, x1, w, eps, d_residual=dres, dx=dx)

    def both():
        fwd(); bwd()

    settle_steps = settle(both, args.settle_ms, torch.cuda.synchronize)
    for _ in range(args.warmup):
        both()
    torch.cuda.synchronize()

    def timed(fn):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / args.steps

    ms = timed(lambda: (fwd(), bwd()))
    # per-kernel device time: events that each launch timestamps itself on the
    # stream it runs on, in a separate pass
    eng.set_kernel_timing(True)
    for _ in range(args.steps):
        fwd(); bwd()
    times = eng.kernel_times()
    eng.set_kernel_timing(False)
    per = {k: times[k][0] / times[k][1] for k in ("rmsnorm_fwd", "rmsnorm_bwd")}
    nb = norm_bytes(T, n, 2)
    step_bytes = nb["rmsnorm_fwd"] + nb["rmsnorm_bwd"]
    gbs = step_bytes / (ms * 1e-3) / 1e9
    dom = max(per, key=per.get)
    achieved = nb[dom] / (per[dom] * 1e-3) / 1e9
    cpu = None if args.no_cpu else cpu_norm_baseline(T, n, eps, step_bytes)
    res = {
        "metric": "residual add + RMSNorm fwd+bwd GB/s (algorithmic HBM bytes), Qwen2.5-7B shape T=512",
        "value": round(gbs, 3),
        "unit": "GB/s",
        "pct_hbm_peak": round(100.0 * gbs / PEAK_HBM_GBS, 3),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded normal x, delta, dy, d_residual, weight; device-resident)",
        "config": {
            "workload": "rmsnorm_qwen7b_t512: x1 = x + delta, y = RMSNorm(x1) w, and dx = "
                        "RMSNormBackward(dy; x1, w) + d_residual",
            "tokens": T, "hidden": n, "eps": eps, "io": "bf16 activations, fp32 weight",
            "parallelism": "1 GPU", "algorithmic_bytes_per_step": step_bytes,
            "kernel_us": {k: round(v * 1e3, 3) for k, v in per.items()},
        },
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 3),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 5), "traffic": norm_traffic(dom)},
        "cpu_baseline": cpu,
        "timing": {"settle": {"ms": args.settle_ms, "steps": settle_steps}},
    }
    print(json.dumps(res), flush=True)
    eng.close()


def run_host(args):
    """The drop-in host entry points (glacier_attn_forward_host /
    backward_host, fp32 host arrays as the C# engine passes them): every call
    copies its tensors host -> device and back, so this rate includes PCIe.
    It is reported beside the device-resident headline, never as it."""
    import time

    import numpy as np

    import glacier_attn as ga

    lengths, Hq, Hkv, D, theta, _ = CONFIGS[args.config]
    if len(lengths) != 1:
        sys.exit("the host entry points take one sequence per call")
    S = lengths[0]
    rng = np.random.default_rng(0)
    q0 = rng.standard_normal((S, Hq, D), dtype=np.float32)
    k0 = rng.standard_normal((S, Hkv, D), dtype=np.float32)
    v = rng.standard_normal((S, Hkv, D), dtype=np.float32)
    dO = (0.01 * rng.standard_normal((S, Hq, D))).astype(np.float32)
    q, k = np.empty_like(q0), np.empty_like(k0)
    out = np.empty_like(q0)
    lse = np.empty((Hq, S), np.float32)
    dq, dk, dv = np.empty_like(q0), np.empty_like(k0), np.empty_like(v)
    flops = 12 * D * Hq * pairs(lengths)  # the headline convention: 4 D fwd + 8 D bwd per pair
    res = {}
    for name, prec in (("bf16", ga.PREC_BF16), ("fp32", ga.PREC_FP32)):
        eng = ga.GpuAttentionEngine(0, prec)
        total = 0.0
        for it in range(args.warmup + args.steps):
            np.copyto(q, q0)  # the forward overwrites q, k with their post-RoPE values
            np.copyto(k, k0)
            t0 = time.perf_counter()
            eng.forward_attention(0, q, k, v, out, lse, S, Hq, Hkv, D, theta)
            eng.backward_attention(0, dO, q, k, v, out, lse, dq, dk, dv, S, Hq, Hkv, D, theta)
            dt = time.perf_counter() - t0
            if it >= args.warmup:
                total += dt
        eng.close()
        ms = total / args.steps * 1e3
        res[name] = {"ms_per_step": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 3)}
    print(json.dumps({
        "metric": "PCIe-inclusive causal GQA attn fwd+bwd TFLOP/s through the host entry points "
                  "(glacier_attn_forward_host + backward_host, fp32 host arrays)",
        "unit": "TFLOP/s", "steps": args.steps, "warmup": args.warmup,
        "config": {"workload": args.config, "seq_len": S, "n_heads_q": Hq, "n_heads_kv": Hkv,
                   "head_dim": D, "host_memory": "pageable numpy arrays"},
        "algorithmic_gflop_per_step": round(flops / 1e9, 4), "modes": res}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed steps for this long before the warmup steps (0: none)")
    ap.add_argument("--config", default="qwen7b_s512", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--precision", default="bf16", choices=["bf16", "fp32"],
                    help="attention: bf16 tensors on bf16 MFMAs (the headline) or the "
                         "fp32-operand mode (fp32 tensors and MFMAs)")
    ap.add_argument("--component", default="attention",
                    choices=["attention", "proj", "norm", "host"],
                    help="attention (the headline), the q/k/v projections with LoRA adapters, "
                         "the residual add + RMSNorm, or the attention's PCIe-inclusive host "
                         "entry points")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run 5 plain device copies of MIB MiB (a known-size kernel that "
                         "calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; use --gpus 1 "
                                   "(the path shards by KV-head group)"}))
        sys.exit(2)
    if args.copy_probe > 0:
        import torch

        src = torch.ones(args.copy_probe << 18, device="cuda:0", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.component == "proj":
        run_proj(args)
        return
    if args.component == "norm":
        run_norm(args)
        return
    if args.component == "host":
        run_host(args)
        return

    import numpy as np
    import torch

    import glacier_attn as ga

    lengths, Hq, Hkv, D, theta, layers = CONFIGS[args.config]
    fp32 = args.precision == "fp32"
    tdt = torch.float32 if fp32 else torch.bfloat16
    peak = PEAK_FP32_TFLOPS if fp32 else PEAK_BF16_TFLOPS
    T = sum(lengths)
    cu = None if len(lengths) == 1 else np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)

    class Layer:
        """One layer's device tensors (each layer has its own activations)."""

        def __init__(self):
            self.q = torch.randn(T, Hq, D, device=dev, generator=g).to(tdt)
            self.k = torch.randn(T, Hkv, D, device=dev, generator=g).to(tdt)
            self.v = torch.randn(T, Hkv, D, device=dev, generator=g).to(tdt)
            self.dO = (0.01 * torch.randn(T, Hq, D, device=dev, generator=g)).to(tdt)
            self.out = torch.empty_like(self.q)
            self.lse = torch.empty(Hq, T, device=dev, dtype=torch.float32)
            self.q_rot = torch.empty_like(self.q)
            self.k_rot = torch.empty_like(self.k)
            self.dq = torch.empty_like(self.q)
            self.dk = torch.empty_like(self.k)
            self.dv = torch.empty_like(self.v)

    net = [Layer() for _ in range(layers)]
    eng = ga.GpuAttentionEngine(0, ga.PREC_FP32 if fp32 else ga.PREC_BF16)

    # Every call with its arguments checked and converted once
    # (eng.bind_forward / bind_backward / bind_step), so each timed call is
    # one C call.  One layer: forward + backward.  Several layers: the
    # checkpointed step (forward without saving through every layer, then
    # per layer from the last: the recompute forward that saves, and the
    # backward).
    if layers == 1:
        L0 = net[0]
        bound = eng.bind_step(dict(q=L0.q, k=L0.k, v=L0.v, out=L0.out, lse=L0.lse,
                                   q_rot=L0.q_rot, k_rot=L0.k_rot),
                              dict(d_out=L0.dO, dq=L0.dq, dk=L0.dk, dv=L0.dv), theta,
                              cu_seqlens=cu)
        calls = [bound]
    else:
        fwd_plain = [eng.bind_forward(L.q, L.k, L.v, L.out, theta, cu_seqlens=cu) for L in net]
        fwd_save = [eng.bind_forward(L.q, L.k, L.v, L.out, theta, cu_seqlens=cu, lse=L.lse,
                                     q_rot=L.q_rot, k_rot=L.k_rot) for L in net]
        bwd = [eng.bind_backward(L.dO, L.q_rot, L.k_rot, L.v, L.out, L.lse, L.dq, L.dk, L.dv,
                                 theta, cu_seqlens=cu) for L in net]
        calls = fwd_plain + [c for i in reversed(range(layers)) for c in (fwd_save[i], bwd[i])]
        bound = calls[0]  # rebind() binds the engine's stream for every bound call

    def step():
        for c in calls:
            c()

    # Settle: the step itself, untimed, for args.settle_ms of wall clock
    # before the W warmup steps, so that the timed steps see the GPU's
    # steady state (its clocks and caches after sustained work) rather than
    # its ramp from idle: with W = 30 the headline read 37.7-38.1 us per step,
    # after ~0.1 s of steps 36.5-36.7 us, same library and box.  Batches of
    # steps keep the device busy while the host enqueues the next batch.
    settle_steps = settle(step, args.settle_ms, torch.cuda.synchronize)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Eager: the K steps enqueued from Python (ctypes); host_ms is the time
    # the enqueueing itself takes per step.
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    host_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    stop.record()
    torch.cuda.synchronize()
    ms_eager = start.elapsed_time(stop) / args.steps

    # Graph replay: one step (every launch of the forward and the backward)
    # captured once and replayed K times, so the host path cannot bound the
    # measured rate.  This is the timed region of `value`.
    ms_graph, graph_error = None, None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            bound.rebind()  # enqueue on the capture stream
            step()
        bound.rebind()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        ms_graph = start.elapsed_time(stop) / args.steps
    except Exception as e:  # capture unsupported: report the eager rate
        graph_error = f"{type(e).__name__}: {e}"
        torch.cuda.synchronize()
    # The measured rate is the eager one unless the graph replay of the same
    # step is faster: the eager loop is then bound by the host (the enqueue
    # itself, or the device idling between bursts of it), which the replay
    # cannot be.
    host_bound = host_ms >= ms_eager
    use_graph = ms_graph is not None and ms_graph < ms_eager
    ms = ms_graph if use_graph else ms_eager

    # 12 D flop per unmasked (query, key, head) per layer, plus 4 D for the
    # checkpoint recompute forward in the multi-layer step.
    flops = (12.0 if layers == 1 else 16.0) * D * Hq * pairs(lengths) * layers
    tflops = flops / (ms * 1e-3) / 1e12

    # Per-kernel device time (events timestamped by each launch itself on the
    # stream it runs on), in a separate pass so timing does not perturb `ms`.
    eng.set_kernel_timing(True)
    for _ in range(args.steps):
        step()
    times = eng.kernel_times()
    eng.set_kernel_timing(False)
    avg = {name: (tot / n if n else 0.0) for name, (tot, n) in times.items()}
    dom = max(FLOPS_PER_PAIR, key=lambda n: times[n][0])
    dom_flops = FLOPS_PER_PAIR[dom] * D * Hq * pairs(lengths)
    achieved = dom_flops / (avg[dom] * 1e-3) / 1e12
    roofline = {
        "bound": "mfma",
        "kernel": dom,
        "achieved": round(achieved, 3),
        "peak": peak,
        "unit": "TFLOP/s",
        "frac": round(achieved / peak, 5),
        "traffic": measured_traffic(args.config, dom, args.precision),
        "kernel_avg_us": {n: round(avg[n] * 1e3, 3) for n in FLOPS_PER_PAIR},
    }

    cpu = None
    if not args.no_cpu and len(lengths) == 1:
        cpu = cpu_baseline(lengths, Hq, Hkv, D, theta)

    res = {
        "metric": metric_name(args.config, args.precision),
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        f"pct_{args.precision}_peak": round(100.0 * tflops / peak, 3),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if fp32 else "bf16",
        "data": "synthetic (seeded normal q/k/v, dO*0.01; device-resident)",
        "config": {
            "workload": f"{args.config}: {CONFIG_LABEL[args.config][0]}, causal GQA attention "
                        f"{'layer fwd+bwd' if layers == 1 else 'fwd, recompute fwd, bwd per layer'} "
                        f"({CONFIG_LABEL[args.config][1]})",
            "seq_lens": lengths, "n_heads_q": Hq, "n_heads_kv": Hkv, "head_dim": D,
            "rope_theta": theta, "parallelism": "1 GPU",
            "io": ("fp32 device tensors, fp32 MFMAs (fp32-operand mode), fp32 lse" if fp32 else
                   "bf16 device tensors, bf16 MFMAs with fp32 accumulation, fp32 lse"),
            "algorithmic_gflop_per_step": round(flops / 1e9, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "timing": {
            "method": ("hipGraph replay of one captured step (faster than the eager loop, "
                       "which the host bounds)"
                       if use_graph else
                       "eager: K steps enqueued back to back between two events (faster than "
                       "the graph replay of the same step)"),
            "graph_error": graph_error,
            "settle": {"ms": args.settle_ms, "steps": settle_steps},
            "ms_per_step_graph": None if ms_graph is None else round(ms_graph, 6),
            "ms_per_step_eager": round(ms_eager, 6),
            "host_enqueue_ms_per_step": round(host_ms, 6),
            "host_bound": host_bound,
            "kernel_sum_ms_per_step": round(sum(times[n][0] for n in FLOPS_PER_PAIR) / args.steps, 6),
        },
    }
    print(json.dumps(res), flush=True)
    eng.close()


if __name__ == "__main__":
    main()
