#!/usr/bin/env python3
"""Benchmark: causal GQA attention forward + backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config qwen7b_s512]

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
         (profiles/attn_kernels_qwen7b_s512_pmc.md).
cpu_baseline = the C restatement of the reference CPU path (oracle/), fp32,
         on this host's cores, over a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "glacier.tune_amd"))

PEAK_BF16_TFLOPS = 2500.0
METRIC = "causal GQA attn fwd+bwd TFLOP/s + % bf16 MFMA peak, Qwen2.5-7B shape S=512"

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
# rope_k and the dK/dV head reduction are credited with none.  Sum: 12 D.
FLOPS_PER_PAIR = {"attn_fwd": 4, "attn_bwd": 8, "rope_k": 0, "attn_bwd_reduce": 0}


# HBM bytes per launch of each kernel at qwen7b_s512, from two rocprofv3 --pmc
# runs (FETCH_SIZE, WRITE_SIZE) scaled by a plain copy of known size; the file
# gives the commands and the calibration.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attn_kernels_qwen7b_s512_pmc.md")


def measured_traffic(config, kernel):
    if config != "qwen7b_s512" or not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes" and f[1] == kernel:
            return int(f[2])
    return None


def pairs(lengths):
    return sum(L * (L + 1) // 2 for L in lengths)


def cpu_baseline(lengths, Hq, Hkv, D, theta, budget_s=12.0):
    """Times oracle.layer_fwd_bwd (fp32, the reference CPU path restated)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = max(1, min(16, os.cpu_count() or 1, Hq))
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
        "sample": (f"median of {len(times)} full layer fwd+bwd passes (RoPE, attention fwd "
                   f"materialising P, attention bwd, inverse RoPE) at S={S}, Hq={Hq}, "
                   f"Hkv={Hkv}, D={D}, fp32; {med * 1e3:.1f} ms each; OpenMP over query heads"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="qwen7b_s512", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run 5 plain device copies of MIB MiB (a known-size kernel that "
                         "calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; use --gpus 1 "
                                   "(the path shards by KV-head group, see DESIGN.md)"}))
        sys.exit(2)

    import numpy as np
    import torch

    import glacier_attn as ga

    lengths, Hq, Hkv, D, theta, layers = CONFIGS[args.config]
    T = sum(lengths)
    cu = None if len(lengths) == 1 else np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    dev = torch.device("cuda:0")
    if args.copy_probe > 0:
        src = torch.ones(args.copy_probe << 18, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    g = torch.Generator(device=dev).manual_seed(0)

    class Layer:
        """One layer's device tensors (each layer has its own activations)."""

        def __init__(self):
            self.q = torch.randn(T, Hq, D, device=dev, generator=g).bfloat16()
            self.k = torch.randn(T, Hkv, D, device=dev, generator=g).bfloat16()
            self.v = torch.randn(T, Hkv, D, device=dev, generator=g).bfloat16()
            self.dO = (0.01 * torch.randn(T, Hq, D, device=dev, generator=g)).bfloat16()
            self.out = torch.empty_like(self.q)
            self.lse = torch.empty(Hq, T, device=dev, dtype=torch.float32)
            self.q_rot = torch.empty_like(self.q)
            self.k_rot = torch.empty_like(self.k)
            self.dq = torch.empty_like(self.q)
            self.dk = torch.empty_like(self.k)
            self.dv = torch.empty_like(self.v)

    net = [Layer() for _ in range(layers)]
    eng = ga.GpuAttentionEngine(0, ga.PREC_BF16)

    def fwd(L, save):
        if save:
            eng.forward(L.q, L.k, L.v, theta, cu_seqlens=cu, out=L.out, lse=L.lse,
                        q_rot=L.q_rot, k_rot=L.k_rot)
        else:
            eng.forward(L.q, L.k, L.v, theta, cu_seqlens=cu, out=L.out, save=False)

    def bwd(L):
        eng.backward(L.dO, L.q_rot, L.k_rot, L.v, L.out, L.lse, theta, cu_seqlens=cu,
                     dq=L.dq, dk=L.dk, dv=L.dv)

    def step():
        if layers == 1:
            fwd(net[0], True)
            bwd(net[0])
            return
        for L in net:
            fwd(L, False)
        for L in reversed(net):
            fwd(L, True)
            bwd(L)

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
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 5),
        "traffic": measured_traffic(args.config, dom),
        "kernel_avg_us": {n: round(a * 1e3, 3) for n, a in avg.items()},
    }

    cpu = None
    if not args.no_cpu and len(lengths) == 1:
        cpu = cpu_baseline(lengths, Hq, Hkv, D, theta)

    res = {
        "metric": METRIC,
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
        "data": "synthetic (seeded normal q/k/v, dO*0.01; device-resident)",
        "config": {
            "workload": f"{args.config}: causal GQA attention layer fwd+bwd (BASELINE.json configs[1])"
            if args.config == "qwen7b_s512" else f"{args.config}: causal GQA attention layer fwd+bwd",
            "seq_lens": lengths, "n_heads_q": Hq, "n_heads_kv": Hkv, "head_dim": D,
            "rope_theta": theta, "io": "bf16 device tensors, fp32 lse", "parallelism": "1 GPU",
            "algorithmic_gflop_per_step": round(flops / 1e9, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    eng.close()


if __name__ == "__main__":
    main()
