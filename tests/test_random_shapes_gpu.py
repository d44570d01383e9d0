"""Seeded random packed batches through the C ABI against the CPU oracle
(oracle/attn_oracle.c: CausalAttentionKernel.Forward/Backward and
RoPEKernel, per packed segment as the reference runs one sequence per call).

Each case draws 1-4 sequences (half of the lengths at tile edges: 1, 15-17,
31-33, 63-65, 127-129, 191, 255-257, 383-385, 511-513; the rest uniform in
[1, 600]), or, one case in ten, a single sequence of 1000-3000 tokens (the
long-sequence backward kernels), a (Hq, Hkv) pair with Hq % Hkv == 0, a head
size (1 to 256; sizes the kernels are not built for run on padded rows), a
RoPE base and one mode:
  fp32         fp32 device tensors, fp32 math: gate 1e-4 on O, lse, dQ, dK,
               dV; post-RoPE q and k bit-exact
  bf16         bf16 device tensors, bf16 MFMA math (inputs rounded to bf16
               for the oracle too): gate 2e-2
  bf16_f32io   fp32 device tensors of bf16-rounded values, bf16 math: 2e-2
  rows16/32,   bf16 device tensors with each bf16 backward kernel pinned
  mfma32,      (head sizes 64 and 128 only; mfma32_pairs: the wide kernel
  mfma32_pairs with dK/dV tiles over head pairs) and 64-query forward
               workgroups: 2e-2
The same seed always gives the same cases; each prints its draw first.
GLACIER_RANDOM_CASES and GLACIER_RANDOM_SEED (default 60 and 20261202)
draw a larger or another sweep.
"""
import os
import sys

import numpy as np
import pytest

import glacier_attn as ga
import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FP32_GATE = 1e-4
BF16_GATE = 2e-2

EDGE_LENS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 191, 255, 256, 257, 383,
             384, 385, 511, 512, 513]
HEADS = [(1, 1), (2, 1), (3, 3), (4, 2), (6, 3), (7, 1), (8, 2), (12, 3), (14, 2), (28, 4),
         (32, 8), (40, 8), (21, 3), (16, 16)]
DIMS = [32, 64, 96, 128, 256, 80, 112, 72, 1, 7, 48, 100, 127, 200]
MODES = ["fp32", "bf16", "bf16_f32io", "rows16", "rows32", "mfma32", "mfma32_pairs"]


def _draw_cases(n=60, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        if rng.random() < 0.1:
            lens = [int(rng.integers(1000, 3001))]
        else:
            lens = [int(rng.choice(EDGE_LENS)) if rng.random() < 0.5 else int(rng.integers(1, 601))
                    for _ in range(int(rng.integers(1, 5)))]
        hq, hkv = HEADS[int(rng.integers(len(HEADS)))]
        d = DIMS[int(rng.integers(len(DIMS)))]
        mode = MODES[i % len(MODES)]
        if mode == "fp32" and d > 128:
            d = 128  # fp32 operands stop at 128
        if mode in ("rows16", "rows32", "mfma32", "mfma32_pairs") and d not in (64, 128):
            d = 64 if d < 128 else 128  # the pinned kernels' head sizes
        if d >= 200 and hq > 8:
            hq, hkv = 8, 2  # keeps the oracle's share of the run short
        if sum(lens) > 1000 and hq > 16:
            hq, hkv = 16, 2  # likewise
        base = [1.0e4, 5.0e5, 1.0e6][int(rng.integers(3))]
        cases.append((i, tuple(lens), hq, hkv, d, base, mode))
    return cases


CASES = _draw_cases(int(os.environ.get("GLACIER_RANDOM_CASES", "60")),
                    int(os.environ.get("GLACIER_RANDOM_SEED", "20261202")))


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def engines():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    made = {"fp32": ga.GpuAttentionEngine(0, ga.PREC_FP32),
            "bf16": ga.GpuAttentionEngine(0, ga.PREC_BF16)}
    # the pinned-backward engines also pin 64-query forward workgroups, which
    # "auto" replaces by 32-query ones on most of these small launches
    keys = ("GLACIER_ATTN_BWD", "GLACIER_ATTN_FWD_ROWS", "GLACIER_ATTN_BWD_PAIRS")
    old = {key: os.environ.get(key) for key in keys}
    try:
        os.environ["GLACIER_ATTN_FWD_ROWS"] = "64"
        for name in ("rows16", "rows32", "mfma32", "mfma32_pairs"):
            os.environ["GLACIER_ATTN_BWD"] = "mfma32" if name == "mfma32_pairs" else name
            os.environ["GLACIER_ATTN_BWD_PAIRS"] = "1" if name == "mfma32_pairs" else "0"
            made[name] = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    finally:
        for key, val in old.items():
            if val is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = val
    yield made
    for e in made.values():
        e.close()


def _inputs(T, hq, hkv, d, seed, bf16):
    q = oracle.fill_normal((T, hq, d), seed * 10 + 1)
    k = oracle.fill_normal((T, hkv, d), seed * 10 + 2)
    v = oracle.fill_normal((T, hkv, d), seed * 10 + 3)
    dO = oracle.fill_normal((T, hq, d), seed * 10 + 4, 0.0, 0.01)
    if bf16:
        q, k, v, dO = (oracle.round_bf16(x) for x in (q, k, v, dO))
    return q, k, v, dO


def _run(eng, q, k, v, dO, base, dtype, cu):
    dev = lambda x: torch.from_numpy(x).to("cuda:0", dtype).contiguous()  # noqa: E731
    tq, tk, tv, tdo = (dev(x) for x in (q, k, v, dO))
    out, lse, q_rot, k_rot = eng.forward(tq, tk, tv, base, cu_seqlens=cu, save=True)
    dq, dk, dv = eng.backward(tdo, q_rot, k_rot, tv, out, lse, base, cu_seqlens=cu)
    torch.cuda.synchronize()
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    return dict(out=f(out), lse=f(lse), q_rot=f(q_rot), k_rot=f(k_rot), dq=f(dq), dk=f(dk),
                dv=f(dv))


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"c{c[0]}-{c[6]}")
def test_random_packed_batch_matches_oracle(engines, case):
    i, lens, hq, hkv, d, base, mode = case
    _say(f"[random] case {i}: mode={mode} lens={list(lens)} Hq={hq} Hkv={hkv} D={d} base={base:g}")
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    bf = mode != "fp32"
    q, k, v, dO = _inputs(T, hq, hkv, d, 100 + i, bf)
    ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    eng = engines["fp32" if mode == "fp32" else "bf16" if mode in ("bf16", "bf16_f32io") else mode]
    dtype = torch.float32 if mode in ("fp32", "bf16_f32io") else torch.bfloat16
    got = _run(eng, q, k, v, dO, base, dtype, cu)
    err = {key: oracle.max_rel_err(got[key], ref[key]) for key in ("out", "lse", "dq", "dk", "dv")}
    _say(f"  errors {err}")
    gate = FP32_GATE if mode == "fp32" else BF16_GATE
    assert all(e <= gate for e in err.values()), err
    if mode == "fp32":
        assert np.array_equal(got["q_rot"], ref["q_rot"])
        assert np.array_equal(got["k_rot"], ref["k_rot"])
