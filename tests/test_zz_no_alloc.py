"""glacier_attn_backward_noalloc (the backward without device allocation)
against glacier_attn_backward, through the C ABI.

Both entry points run the same kernels; the allocation-free one takes its
tables and partial buffers from the library's fixed device scratch array, so
the gradients must be bitwise equal.  Each case makes two calls in a row, the
second with a smaller input (a different sequence layout and head_dim, so the
scratch's tables are rebuilt and its regions move).
"""
import ctypes
import os
import sys

import numpy as np
import pytest

import glacier_attn as ga

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _engine(kernel, precision):
    """kernel: a GLACIER_ATTN_BWD value, or mfma32_pairs (the wide kernel with
    dK/dV tiles over head pairs)."""
    env = {"GLACIER_ATTN_BWD": "mfma32" if kernel == "mfma32_pairs" else kernel,
           "GLACIER_ATTN_BWD_PAIRS": "1" if kernel == "mfma32_pairs" else "0"}
    old = {key: os.environ.get(key) for key in env}
    try:
        os.environ.update(env)
        return ga.GpuAttentionEngine(0, precision)
    finally:
        for key, val in old.items():
            if val is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = val


def _inputs(lens, hq, hkv, d, dtype, seed):
    T = int(sum(lens))
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(T, hq, d, device="cuda", generator=g).to(dtype)
    k = torch.randn(T, hkv, d, device="cuda", generator=g).to(dtype)
    v = torch.randn(T, hkv, d, device="cuda", generator=g).to(dtype)
    dO = (0.01 * torch.randn(T, hq, d, device="cuda", generator=g)).to(dtype)
    cu = None if len(lens) == 1 else np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return q, k, v, dO, cu


def backward_noalloc(eng, d_out, q_rot, k_rot, v, out, lse, base, precision, cu, dq, dk, dv):
    """glacier_attn_backward_noalloc on torch's current stream; returns the status."""
    T, hq, d = q_rot.shape
    desc, _keep = eng._desc(T, hq, k_rot.shape[1], d, base, precision, eng._io_of(q_rot), cu)
    eng._bind_stream()
    p = eng._ptr
    return ga.load().glacier_attn_backward_noalloc(eng._h, ctypes.byref(desc), p(d_out),
                                                   p(q_rot), p(k_rot), p(v), p(out), p(lse),
                                                   p(dq), p(dk), p(dv))


# (backward kernel pin, precision, tensor dtype)
MODES = [
    ("auto", ga.PREC_BF16, torch.bfloat16),
    ("rows32", ga.PREC_BF16, torch.bfloat16),
    ("auto", ga.PREC_BF16, torch.float32),
    ("auto", ga.PREC_FP32, torch.float32),
]
# two calls in a row per mode: the second input is smaller
CALLS = [
    ([300, 77, 1, 130], 14, 2, 128, 1.0e6),
    ([100], 4, 2, 64, 1.0e4),
]


@pytest.mark.parametrize("kernel,precision,dtype", MODES)
def test_noalloc_backward_matches_backward_bitwise(kernel, precision, dtype):
    eng = _engine(kernel, precision)
    try:
        for i, (lens, hq, hkv, d, base) in enumerate(CALLS):
            _say(f"[noalloc] {kernel} prec={precision} {dtype} call {i}: lens={lens} "
                 f"Hq={hq} Hkv={hkv} D={d}")
            q, k, v, dO, cu = _inputs(lens, hq, hkv, d, dtype, 40 + i)
            out, lse, q_rot, k_rot = eng.forward(q, k, v, base, cu_seqlens=cu)
            ref = eng.backward(dO, q_rot, k_rot, v, out, lse, base, cu_seqlens=cu)
            got = [torch.full_like(t, float("nan")) for t in ref]
            rc = backward_noalloc(eng, dO, q_rot, k_rot, v, out, lse, base, precision, cu, *got)
            assert rc == ga.OK, ga.load().glacier_attn_last_error()
            torch.cuda.synchronize()
            for name, a, b in zip(("dq", "dk", "dv"), ref, got):
                assert torch.equal(a, b), name
    finally:
        eng.close()


# long sequences of bf16 tensors: both entry points take the wide backward
# (128-row tiles from the scratch's own table); two calls, the second smaller
CALLS_LONG = [
    ([1100, 7], 14, 2, 128, 1.0e6),
    ([2050], 4, 1, 64, 1.0e4),
]


@pytest.mark.parametrize("kernel", ["auto", "mfma32", "mfma32_pairs"])
def test_noalloc_backward_long_sequences_match_backward_bitwise(kernel):
    eng = _engine(kernel, ga.PREC_BF16)
    try:
        for i, (lens, hq, hkv, d, base) in enumerate(CALLS_LONG):
            _say(f"[noalloc long] {kernel} call {i}: lens={lens} Hq={hq} Hkv={hkv} D={d}")
            q, k, v, dO, cu = _inputs(lens, hq, hkv, d, torch.bfloat16, 60 + i)
            out, lse, q_rot, k_rot = eng.forward(q, k, v, base, cu_seqlens=cu)
            ref = eng.backward(dO, q_rot, k_rot, v, out, lse, base, cu_seqlens=cu)
            got = [torch.full_like(t, float("nan")) for t in ref]
            rc = backward_noalloc(eng, dO, q_rot, k_rot, v, out, lse, base, ga.PREC_BF16, cu, *got)
            assert rc == ga.OK, ga.load().glacier_attn_last_error()
            torch.cuda.synchronize()
            for name, a, b in zip(("dq", "dk", "dv"), ref, got):
                assert torch.equal(a, b), name
    finally:
        eng.close()


def test_noalloc_backward_allocates_no_device_memory():
    """A fresh context: the allocation-free call leaves the device's free
    memory where it was (the same call through glacier_attn_backward would
    allocate the context's scratch)."""
    lens, hq, hkv, d, base = [512], 28, 4, 128, 1.0e6
    eng = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    try:
        q, k, v, dO, cu = _inputs(lens, hq, hkv, d, torch.bfloat16, 7)
        with _engine("auto", ga.PREC_BF16) as fwd:
            out, lse, q_rot, k_rot = fwd.forward(q, k, v, base)
        dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(3):
            rc = backward_noalloc(eng, dO, q_rot, k_rot, v, out, lse, base, ga.PREC_BF16, cu,
                                  dq, dk, dv)
            assert rc == ga.OK, ga.load().glacier_attn_last_error()
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0
        assert torch.isfinite(dq).all() and torch.isfinite(dk).all() and torch.isfinite(dv).all()
    finally:
        eng.close()


def test_noalloc_backward_rejects_calls_beyond_its_scratch():
    """T * Hq * D too large for the fixed array: a clear error, outputs untouched."""
    T, hq, hkv, d = 8192, 32, 8, 128  # 134 MB of dK/dV partials alone
    eng = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    try:
        q = torch.zeros(T, hq, d, device="cuda", dtype=torch.bfloat16)
        k = torch.zeros(T, hkv, d, device="cuda", dtype=torch.bfloat16)
        lse = torch.zeros(hq, T, device="cuda")
        dq = torch.full_like(q, 3.0)
        dk = torch.full_like(k, 3.0)
        dv = torch.full_like(k, 3.0)
        rc = backward_noalloc(eng, q, q, k, k, q, lse, 1.0e4, ga.PREC_BF16, None, dq, dk, dv)
        msg = ga.load().glacier_attn_last_error().decode()
        assert rc == ga.ERR_UNSUPPORTED and "scratch" in msg, msg
        torch.cuda.synchronize()
        assert bool((dq == 3.0).all()) and bool((dk == 3.0).all()) and bool((dv == 3.0).all())
    finally:
        eng.close()
