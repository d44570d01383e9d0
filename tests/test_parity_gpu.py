"""GPU parity: libglacier_attn.so (through its C ABI) against the CPU oracle.

Gates, normwise max relative error
max|gpu - ref| / max|ref| per tensor:
  fp32-operand mode  <= 1e-4 on O, lse, dQ, dK, dV; post-RoPE q/k bit-exact
  bf16-MFMA mode     <= 2e-2 on O, dQ, dK, dV (inputs rounded to bf16 on the
                     host first; the oracle runs on the same rounded values)
Configs: BASELINE.json configs[0] (Qwen2.5-0.5B, S=512, 14/2, D=64) and
configs[1] (Qwen2.5-7B, S=512, 28/4, D=128) against the oracle; configs[2]
(packed varlen) against the oracle per segment; configs[3] (S=4096) and
configs[4] (Llama-3-8B B=2 S=2048) against the oracle on the same seeded
SplitMix inputs in both modes (about 7-15 s of oracle time each on 8-16
host threads), and again, with other large shapes, against a float32 torch
reference on the GPU; plus edge cases.
"""
import functools
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


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def engines():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    e32 = ga.GpuAttentionEngine(0, ga.PREC_FP32)
    e16 = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    yield {ga.PREC_FP32: e32, ga.PREC_BF16: e16}
    e32.close()
    e16.close()


BWD_KERNELS = ("rows16", "rows32", "mfma32", "mfma32_pairs")
# the environment that pins each (read when an engine is created);
# mfma32_pairs: the wide kernel with dK/dV tiles over head pairs
BWD_ENV = {
    "rows16": {"GLACIER_ATTN_BWD": "rows16", "GLACIER_ATTN_BWD_PAIRS": "0"},
    "rows32": {"GLACIER_ATTN_BWD": "rows32", "GLACIER_ATTN_BWD_PAIRS": "0"},
    "mfma32": {"GLACIER_ATTN_BWD": "mfma32", "GLACIER_ATTN_BWD_PAIRS": "0"},
    "mfma32_pairs": {"GLACIER_ATTN_BWD": "mfma32", "GLACIER_ATTN_BWD_PAIRS": "1"},
}


def pinned_engine(name, precision=None):
    """An engine created under BWD_ENV[name]."""
    env = BWD_ENV[name]
    old = {key: os.environ.get(key) for key in env}
    try:
        os.environ.update(env)
        return ga.GpuAttentionEngine(0, ga.PREC_BF16 if precision is None else precision)
    finally:
        for key, val in old.items():
            if val is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = val


@pytest.fixture(scope="module")
def bf16_kernels():
    """bf16-mode engines pinned to each backward kernel for bf16 tensors."""
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    made = {name: pinned_engine(name) for name in BWD_KERNELS}
    yield made
    for e in made.values():
        e.close()


def make_inputs(S, Hq, Hkv, D, seed=1, bf16=False):
    q = oracle.fill_normal((S, Hq, D), seed * 10 + 1)
    k = oracle.fill_normal((S, Hkv, D), seed * 10 + 2)
    v = oracle.fill_normal((S, Hkv, D), seed * 10 + 3)
    dO = oracle.fill_normal((S, Hq, D), seed * 10 + 4, 0.0, 0.01)
    if bf16:
        q, k, v, dO = (oracle.round_bf16(x) for x in (q, k, v, dO))
    return q, k, v, dO


@functools.lru_cache(maxsize=8)
def oracle_case(S, Hq, Hkv, D, base, seed, bf16):
    q, k, v, dO = make_inputs(S, Hq, Hkv, D, seed, bf16)
    return (q, k, v, dO), oracle.layer_fwd_bwd(q, k, v, dO, base)


def run_host(eng, q, k, v, dO, base):
    """The C# call sequence: ForwardAttention (saving) then BackwardAttention."""
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    q = q.copy(); k = k.copy()
    out = np.empty_like(q)
    lse = np.empty((Hq, S), np.float32)
    eng.forward_attention(0, q, k, v, out, lse, S, Hq, Hkv, D, base)
    dq = np.zeros_like(q); dk = np.zeros_like(k); dv = np.zeros_like(v)
    eng.backward_attention(0, dO, q, k, v, out, lse, dq, dk, dv, S, Hq, Hkv, D, base)
    return dict(q_rot=q, k_rot=k, out=out, lse=lse, dq=dq, dk=dk, dv=dv)


def errors(got, ref, keys=("out", "lse", "dq", "dk", "dv")):
    return {key: oracle.max_rel_err(got[key], ref[key]) for key in keys}


CONFIGS = {
    "qwen05b_s512": (512, 14, 2, 64, 1.0e6),
    "qwen7b_s512": (512, 28, 4, 128, 1.0e6),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_fp32_mode_matches_oracle(engines, name):
    S, Hq, Hkv, D, base = CONFIGS[name]
    _say(f"[fp32 parity] {name} S={S} Hq={Hq} Hkv={Hkv} D={D}")
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 1, False)
    got = run_host(engines[ga.PREC_FP32], q, k, v, dO, base)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= FP32_GATE for e in err.values()), err
    # post-RoPE write-back: the same fp32 operations as RoPEKernel.cs
    assert np.array_equal(got["q_rot"], ref["q_rot"])
    assert np.array_equal(got["k_rot"], ref["k_rot"])


@pytest.mark.parametrize("name", list(CONFIGS))
def test_bf16_mode_matches_oracle(engines, name):
    S, Hq, Hkv, D, base = CONFIGS[name]
    _say(f"[bf16 parity] {name}")
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 1, True)
    got = run_host(engines[ga.PREC_BF16], q, k, v, dO, base)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err
    assert np.array_equal(got["q_rot"], ref["q_rot"])


def _dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype).contiguous()


def run_device(eng, q, k, v, dO, base, dtype, cu=None):
    tq, tk, tv, tdo = (_dev(x, dtype) for x in (q, k, v, dO))
    out, lse, q_rot, k_rot = eng.forward(tq, tk, tv, base, cu_seqlens=cu, save=True)
    dq, dk, dv = eng.backward(tdo, q_rot, k_rot, tv, out, lse, base, cu_seqlens=cu)
    torch.cuda.synchronize()
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    return dict(out=f(out), lse=f(lse), q_rot=f(q_rot), k_rot=f(k_rot), dq=f(dq), dk=f(dk), dv=f(dv))


@pytest.mark.parametrize("name", list(CONFIGS))
def test_bf16_device_tensors_match_oracle(engines, name):
    S, Hq, Hkv, D, base = CONFIGS[name]
    _say(f"[bf16 device io] {name}")
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 1, True)
    got = run_device(engines[ga.PREC_BF16], q, k, v, dO, base, torch.bfloat16)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err


@pytest.mark.parametrize("kernel", BWD_KERNELS)
@pytest.mark.parametrize("name", list(CONFIGS))
def test_bf16_device_tensors_each_backward_kernel(bf16_kernels, name, kernel):
    S, Hq, Hkv, D, base = CONFIGS[name]
    _say(f"[bf16 device io, {kernel} backward] {name}")
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 1, True)
    got = run_device(bf16_kernels[kernel], q, k, v, dO, base, torch.bfloat16)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err


RAGGED = [
    (1, 2, 1, 64), (2, 4, 4, 128), (17, 7, 1, 128), (63, 4, 2, 64), (64, 2, 2, 64),
    (65, 6, 3, 128), (100, 8, 2, 64), (129, 14, 2, 128), (200, 2, 1, 64),
]


@pytest.mark.parametrize("S,Hq,Hkv,D", RAGGED)
@pytest.mark.parametrize("kernel", BWD_KERNELS)
def test_bf16_device_ragged_shapes_each_backward_kernel(bf16_kernels, S, Hq, Hkv, D, kernel):
    """Partial tiles, one-token sequences and every GQA ratio through both
    backward kernels of bf16 tensors."""
    base = 1.0e4
    _say(f"[bf16 device shape, {kernel}] S={S} Hq={Hq} Hkv={Hkv} D={D}")
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 3, True)
    got = run_device(bf16_kernels[kernel], q, k, v, dO, base, torch.bfloat16)
    err = errors(got, ref)
    assert all(e <= BF16_GATE for e in err.values()), err


@pytest.mark.parametrize("case", ["qwen05b_s512", "short_packed"])
def test_split_dkdv_tiles_match_whole_tiles(engines, case):
    """When the 16-row backward's grid leaves CUs idle (bf16 tensors, e.g. 14
    query heads at S=512) its longest dK/dV tiles run as two query halves
    whose partials the head reduction adds.  Against an engine with
    GLACIER_ATTN_BWD_SPLIT=0 (every tile whole): dq bit-identical (dQ tiles
    do not change), dk and dv within the bf16 gate of each other, both runs
    within the gate of the oracle.  The packed case has sequences of one tile
    or less, whose second halves visit no query tile and write zeros."""
    if case == "qwen05b_s512":
        S, Hq, Hkv, D, base = CONFIGS["qwen05b_s512"]
        (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 1, True)
        cu = None
    else:
        Hq, Hkv, D, base = 4, 2, 128, 1.0e4
        cu = np.array([0, 30, 94, 95, 195], np.int32)
        q, k, v, dO = make_inputs(int(cu[-1]), Hq, Hkv, D, 6, True)
        ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    _say(f"[split dK/dV] {case}")
    old = os.environ.get("GLACIER_ATTN_BWD_SPLIT")
    os.environ["GLACIER_ATTN_BWD_SPLIT"] = "0"
    try:
        whole = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    finally:
        if old is None:
            os.environ.pop("GLACIER_ATTN_BWD_SPLIT", None)
        else:
            os.environ["GLACIER_ATTN_BWD_SPLIT"] = old
    try:
        got_w = run_device(whole, q, k, v, dO, base, torch.bfloat16, cu=cu)
    finally:
        whole.close()
    got_s = run_device(engines[ga.PREC_BF16], q, k, v, dO, base, torch.bfloat16, cu=cu)
    err_s, err_w = errors(got_s, ref), errors(got_w, ref)
    _say(f"  split {err_s}\n  whole {err_w}")
    assert all(e <= BF16_GATE for e in err_s.values()), err_s
    assert all(e <= BF16_GATE for e in err_w.values()), err_w
    assert np.array_equal(got_s["dq"], got_w["dq"])
    for key in ("dk", "dv"):
        assert oracle.max_rel_err(got_s[key], got_w[key]) <= BF16_GATE, key


@pytest.mark.parametrize("case", ["s1100_g7", "packed_g4", "g1", "g3"])
def test_wide_backward_head_pairs_match_single_heads(bf16_kernels, case):
    """The wide backward with each dK/dV tile walking two query heads of its
    group (one partial per pair; the head reduction sums every second head)
    against one head per tile: dq bit-identical (the dQ tiles do not change),
    dk and dv within the bf16 gate of each other, both within the gate of the
    oracle.  Groups of 7 (a last head alone), 4, 1 (no pair) and 3; a packed
    batch with sequences shorter than one 128-row tile."""
    lens, Hq, Hkv, D, base = {
        "s1100_g7": ([1100], 14, 2, 128, 1.0e6),
        "packed_g4": ([300, 1, 77, 530], 8, 2, 64, 5.0e5),
        "g1": ([700], 2, 2, 128, 1.0e4),
        "g3": ([129, 385], 6, 2, 64, 1.0e4),
    }[case]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v, dO = make_inputs(int(cu[-1]), Hq, Hkv, D, 11, True)
    ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    _say(f"[wide backward head pairs] {case}")
    cuv = None if len(lens) == 1 else cu
    got_p = run_device(bf16_kernels["mfma32_pairs"], q, k, v, dO, base, torch.bfloat16, cu=cuv)
    got_1 = run_device(bf16_kernels["mfma32"], q, k, v, dO, base, torch.bfloat16, cu=cuv)
    err_p, err_1 = errors(got_p, ref), errors(got_1, ref)
    _say(f"  pairs {err_p}\n  single {err_1}")
    assert all(e <= BF16_GATE for e in err_p.values()), err_p
    assert all(e <= BF16_GATE for e in err_1.values()), err_1
    assert np.array_equal(got_p["dq"], got_1["dq"])
    for key in ("dk", "dv"):
        assert oracle.max_rel_err(got_p[key], got_1[key]) <= BF16_GATE, key


@pytest.fixture(scope="module")
def fwd_rows():
    """bf16-mode engines pinned to 16-, 32- and 64-query forward workgroups
    (GLACIER_ATTN_FWD_ROWS is read when an engine is created)."""
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    made = {}
    old = os.environ.get("GLACIER_ATTN_FWD_ROWS")
    try:
        for rows in ("16", "32", "64"):
            os.environ["GLACIER_ATTN_FWD_ROWS"] = rows
            made[rows] = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    finally:
        if old is None:
            os.environ.pop("GLACIER_ATTN_FWD_ROWS", None)
        else:
            os.environ["GLACIER_ATTN_FWD_ROWS"] = old
    yield made
    for e in made.values():
        e.close()


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("case", ["qwen05b_s512", "qwen7b_s512", "packed"])
def test_forward_narrow_workgroups_match_64_row_workgroups(fwd_rows, case, dtype):
    """The bf16 forward with two 32-query or four 16-query workgroups per
    64-query tile (taken when 64-row workgroups would leave CUs idle) against
    64-row workgroups.  A query's scores, probabilities and partial sums come
    from the same wave over the same key chunks in all three, and the chunks
    a larger workgroup walks past its first queries' diagonal are masked to
    exact zeros, so out, lse and q_rot are bit-identical (no rescue pass:
    N(0, 1) inputs).  All match the oracle.  The packed batch has a sequence
    of 70 tokens (its second tile's later workgroups have no queries and
    return) and one of a single token."""
    if case == "packed":
        Hq, Hkv, D, base = 14, 2, 128, 1.0e4
        cu = np.array([0, 70, 103, 233, 234], np.int32)
        q, k, v, dO = make_inputs(int(cu[-1]), Hq, Hkv, D, 8, True)
        ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    else:
        S, Hq, Hkv, D, base = CONFIGS[case]
        (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 1, True)
        cu = None
    _say(f"[forward rows 32 vs 64] {case} {dtype} tensors")
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    got = {rows: run_device(fwd_rows[rows], q, k, v, dO, base, tdt, cu=cu) for rows in ("16", "32", "64")}
    for rows, g in got.items():
        err = errors(g, ref)
        _say(f"  rows {rows}: {err}")
        assert all(e <= BF16_GATE for e in err.values()), (rows, err)
    for rows in ("16", "32"):
        for key in ("out", "lse", "q_rot"):
            assert np.array_equal(got[rows][key], got["64"][key]), (rows, key)


@pytest.mark.parametrize("kernel", BWD_KERNELS)
def test_bf16_device_backward_is_bitwise_repeatable(bf16_kernels, kernel):
    S, Hq, Hkv, D, base = 300, 14, 2, 128, 1.0e6
    _say(f"[determinism, bf16 device, {kernel}]")
    q, k, v, dO = make_inputs(S, Hq, Hkv, D, 7, True)
    a = run_device(bf16_kernels[kernel], q, k, v, dO, base, torch.bfloat16)
    b = run_device(bf16_kernels[kernel], q, k, v, dO, base, torch.bfloat16)
    for key in a:
        assert np.array_equal(a[key], b[key]), key


@pytest.mark.parametrize("S,Hq,Hkv,D", RAGGED)
@pytest.mark.parametrize("prec", [ga.PREC_FP32, ga.PREC_BF16])
def test_small_and_ragged_shapes(engines, S, Hq, Hkv, D, prec):
    base = 1.0e4
    bf = prec == ga.PREC_BF16
    _say(f"[shape] S={S} Hq={Hq} Hkv={Hkv} D={D} prec={prec}")
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 3, bf)
    got = run_host(engines[prec], q, k, v, dO, base)
    err = errors(got, ref)
    gate = BF16_GATE if bf else FP32_GATE
    assert all(e <= gate for e in err.values()), err


# sizes the kernels are built for (32, 96, 256: the generic 16-row kernels;
# 64 and 128 are covered above) and sizes that run on padded rows: odd ones
# (an unrotated last element), one element, and one in each padding range
HEAD_DIMS = [32, 96, 256, 1, 16, 48, 80, 100, 127, 200]


@pytest.mark.parametrize("mode", ["fp32", "bf16_host", "bf16_device"])
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_head_dims_match_oracle(engines, D, mode):
    """Head sizes other than 64 and 128: a ragged S=200 (three full tiles and
    a partial one), GQA 4:1, in each mode; the post-RoPE q and k bit-exact in
    the fp32 mode and q in the bf16 host mode, as at the built sizes.  fp32
    operands stop at a padded size of 128 (UNSUPPORTED above)."""
    S, Hq, Hkv, base = 200, 8, 2, 1.0e4
    bf = mode != "fp32"
    _say(f"[head_dim] D={D} mode={mode}")
    if D > 128 and not bf:  # padded to 256
        q = np.zeros((S, Hq, D), np.float32)
        with pytest.raises(ga.Unsupported):
            engines[ga.PREC_FP32].forward_attention(0, q, q[:, :Hkv].copy(), q[:, :Hkv].copy(),
                                                    np.empty_like(q), None, S, Hq, Hkv, D, base)
        return
    (q, k, v, dO), ref = oracle_case(S, Hq, Hkv, D, base, 4, bf)
    if mode == "bf16_device":
        got = run_device(engines[ga.PREC_BF16], q, k, v, dO, base, torch.bfloat16)
    else:
        got = run_host(engines[ga.PREC_BF16 if bf else ga.PREC_FP32], q, k, v, dO, base)
    err = errors(got, ref)
    _say(f"  errors {err}")
    gate = BF16_GATE if bf else FP32_GATE
    assert all(e <= gate for e in err.values()), err
    if mode == "fp32":
        assert np.array_equal(got["q_rot"], ref["q_rot"])
        assert np.array_equal(got["k_rot"], ref["k_rot"])
    elif mode == "bf16_host":
        assert np.array_equal(got["q_rot"], ref["q_rot"])


@pytest.mark.parametrize("D", [32, 96, 256, 80, 127])
def test_head_dims_packed_batch_matches_oracle(engines, D):
    """Packed sequences (a one-token one among them) at the new head sizes,
    bf16 device tensors, against the oracle per segment."""
    Hq, Hkv, base = 6, 3, 1.0e6
    lens = [70, 1, 129]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    _say(f"[head_dim varlen] D={D} lens={lens}")
    q, k, v, dO = make_inputs(T, Hq, Hkv, D, 12, True)
    ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    got = run_device(engines[ga.PREC_BF16], q, k, v, dO, base, torch.bfloat16, cu=cu)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err


def test_forward_without_save_leaves_qk_and_matches_saving_forward(engines):
    S, Hq, Hkv, D, base = 96, 4, 2, 64, 1.0e6
    _say("[no-save forward]")
    eng = engines[ga.PREC_BF16]
    q, k, v, _ = make_inputs(S, Hq, Hkv, D, 5, True)
    q0, k0 = q.copy(), k.copy()
    out_a = np.empty_like(q)
    eng.forward_attention(0, q, k, v, out_a, None, S, Hq, Hkv, D, base)
    assert np.array_equal(q, q0) and np.array_equal(k, k0)
    out_b = np.empty_like(q)
    lse = np.empty((Hq, S), np.float32)
    eng.forward_attention(0, q, k, v, out_b, lse, S, Hq, Hkv, D, base)
    assert np.array_equal(out_a, out_b)  # O does not depend on saving
    assert not np.array_equal(q, q0)     # q became post-RoPE


@pytest.mark.parametrize("prec", [ga.PREC_FP32, ga.PREC_BF16])
def test_recompute_and_backward_are_bitwise_repeatable(engines, prec):
    """Activation checkpointing re-runs the forward (GgufLoraModel.cs:521-527);
    the reference demands identical gradients (GradientAndGpuParityTests.cs:143-172)."""
    S, Hq, Hkv, D, base = 300, 14, 2, 128, 1.0e6
    _say(f"[determinism] prec={prec}")
    q, k, v, dO = make_inputs(S, Hq, Hkv, D, 7, prec == ga.PREC_BF16)
    a = run_host(engines[prec], q, k, v, dO, base)
    b = run_host(engines[prec], q, k, v, dO, base)
    for key in a:
        assert np.array_equal(a[key], b[key]), key


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_bound_calls_match_unbound_calls(engines, dtype):
    """bind_forward / bind_backward / bind_step (arguments checked once) give
    the bits of forward() / backward() on the same tensors: with and without
    saving, on a packed batch."""
    Hq, Hkv, D, base = 14, 2, 64, 1.0e6
    lens = [100, 37, 200]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    _say(f"[bound calls] {dtype} lens={lens}")
    eng = engines[ga.PREC_BF16]
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    q, k, v, dO = (_dev(x, tdt) for x in make_inputs(T, Hq, Hkv, D, 11, dtype == "bf16"))
    out, lse, q_rot, k_rot = eng.forward(q, k, v, base, cu_seqlens=cu)
    dq, dk, dv = eng.backward(dO, q_rot, k_rot, v, out, lse, base, cu_seqlens=cu)
    out_ns, _, _, _ = eng.forward(q, k, v, base, cu_seqlens=cu, save=False)

    e = torch.empty_like
    b_out_ns = e(out)
    eng.bind_forward(q, k, v, b_out_ns, base, cu_seqlens=cu)()
    b = dict(out=e(out), lse=e(lse), q_rot=e(q_rot), k_rot=e(k_rot), dq=e(dq), dk=e(dk), dv=e(dv))
    eng.bind_forward(q, k, v, b["out"], base, cu_seqlens=cu, lse=b["lse"], q_rot=b["q_rot"],
                     k_rot=b["k_rot"])()
    eng.bind_backward(dO, b["q_rot"], b["k_rot"], v, b["out"], b["lse"], b["dq"], b["dk"],
                      b["dv"], base, cu_seqlens=cu)()
    s = dict(out=e(out), lse=e(lse), q_rot=e(q_rot), k_rot=e(k_rot), dq=e(dq), dk=e(dk), dv=e(dv))
    eng.bind_step(dict(q=q, k=k, v=v, out=s["out"], lse=s["lse"], q_rot=s["q_rot"],
                       k_rot=s["k_rot"]),
                  dict(d_out=dO, dq=s["dq"], dk=s["dk"], dv=s["dv"]), base, cu_seqlens=cu)()
    torch.cuda.synchronize()
    ref = dict(out=out, lse=lse, q_rot=q_rot, k_rot=k_rot, dq=dq, dk=dk, dv=dv)
    assert torch.equal(b_out_ns, out_ns)
    for name, t in ref.items():
        assert torch.equal(b[name], t), name
        assert torch.equal(s[name], t), name
    with pytest.raises(ValueError):
        eng.bind_forward(q, k, v, e(out), base, cu_seqlens=cu, lse=e(lse))


def test_varlen_packed_batch_matches_oracle_per_segment(engines, bf16_kernels):
    """BASELINE configs[2] shape: 4 packed sequences, lengths U[64,512] (seed 5),
    block-diagonal causal mask, 7B heads, bf16."""
    Hq, Hkv, D, base = 28, 4, 128, 1.0e6
    rng = np.random.default_rng(5)
    lens = rng.integers(64, 513, size=4)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    _say(f"[varlen] lens={lens.tolist()}")
    q, k, v, dO = make_inputs(T, Hq, Hkv, D, 9, True)
    ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    for eng in (engines[ga.PREC_BF16], *bf16_kernels.values()):
        got = run_device(eng, q, k, v, dO, base, torch.bfloat16, cu=cu)
        err = errors(got, ref)
        _say(f"  errors {err}")
        assert all(e <= BF16_GATE for e in err.values()), err
    # fp32 device tensors with fp32 math on the same packing
    (q, k, v, dO) = make_inputs(T, Hq, Hkv, D, 9, False)
    ref = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    got = run_device(engines[ga.PREC_FP32], q, k, v, dO, base, torch.float32, cu=cu)
    err = errors(got, ref)
    assert all(e <= FP32_GATE for e in err.values()), err


# ---------------------------------------------------------------------------
# BASELINE configs[3] and [4] against the oracle.
# ---------------------------------------------------------------------------

LONG_ORACLE = {
    "qwen7b_s4096": ([4096], 28, 4, 128, 1.0e6),            # configs[3]
    "llama3_b2_s2048": ([2048, 2048], 32, 8, 128, 5.0e5),   # configs[4]
}


@functools.lru_cache(maxsize=2)
def long_oracle_case(name, bf16):
    lens, Hq, Hkv, D, base = LONG_ORACLE[name]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v, dO = make_inputs(int(cu[-1]), Hq, Hkv, D, 5, bf16)
    return (q, k, v, dO), cu, oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)


@pytest.mark.parametrize("name", list(LONG_ORACLE))
def test_long_configs_fp32_mode_match_oracle(engines, name):
    """fp32 tensors, fp32 math: 1e-4 on O, lse, dQ, dK, dV; the post-RoPE q
    and k bit-exact."""
    lens, Hq, Hkv, D, base = LONG_ORACLE[name]
    _say(f"[long oracle fp32] {name}")
    (q, k, v, dO), cu, ref = long_oracle_case(name, False)
    got = run_device(engines[ga.PREC_FP32], q, k, v, dO, base, torch.float32,
                     cu=None if len(lens) == 1 else cu)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= FP32_GATE for e in err.values()), err
    assert np.array_equal(got["q_rot"], ref["q_rot"])
    assert np.array_equal(got["k_rot"], ref["k_rot"])


@pytest.mark.parametrize("kernel", ("auto",) + BWD_KERNELS)
@pytest.mark.parametrize("name", list(LONG_ORACLE))
def test_long_configs_bf16_mode_match_oracle(engines, bf16_kernels, name, kernel):
    """bf16 tensors (inputs rounded to bf16 for the oracle too), bf16 MFMA
    math, through the automatic backward choice and each pinned one: 2e-2
    on O, lse, dQ, dK, dV."""
    lens, Hq, Hkv, D, base = LONG_ORACLE[name]
    _say(f"[long oracle bf16, {kernel} backward] {name}")
    (q, k, v, dO), cu, ref = long_oracle_case(name, True)
    eng = engines[ga.PREC_BF16] if kernel == "auto" else bf16_kernels[kernel]
    got = run_device(eng, q, k, v, dO, base, torch.bfloat16, cu=None if len(lens) == 1 else cu)
    err = errors(got, ref)
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err


# ---------------------------------------------------------------------------
# Large shapes: float32 torch reference on the GPU (plain matmul/softmax).
# ---------------------------------------------------------------------------

def torch_reference(q, k, v, dO, base, cu):
    """Float32 reference of the whole layer, per segment, with autograd."""
    D = q.shape[-1]
    half = D // 2
    r = q.shape[1] // k.shape[1]
    qd = q.detach().float().clone().requires_grad_(True)
    kd = k.detach().float().clone().requires_grad_(True)
    vd = v.detach().float().clone().requires_grad_(True)
    w = base ** (-(2.0 * np.arange(half)) / D)
    outs, lses = [], []
    for b in range(len(cu) - 1):
        s0, s1 = int(cu[b]), int(cu[b + 1])
        L = s1 - s0
        th = np.arange(L)[:, None] * w[None, :]
        c = torch.tensor(np.cos(th), dtype=torch.float32, device=q.device)[:, None, :]
        s = torch.tensor(np.sin(th), dtype=torch.float32, device=q.device)[:, None, :]

        def rot(x):
            return torch.cat([x[..., :half] * c - x[..., half:] * s,
                              x[..., :half] * s + x[..., half:] * c], dim=-1)

        qr = rot(qd[s0:s1]).permute(1, 0, 2).contiguous()                       # [Hq,L,D]
        kr = rot(kd[s0:s1]).repeat_interleave(r, dim=1).permute(1, 2, 0).contiguous()  # [Hq,D,L]
        vr = vd[s0:s1].repeat_interleave(r, dim=1).permute(1, 0, 2).contiguous()
        sc = torch.matmul(qr, kr) / np.sqrt(D)
        mask = torch.ones(L, L, dtype=torch.bool, device=q.device).tril()
        sc = sc.masked_fill(~mask, float("-inf"))
        lses.append(torch.logsumexp(sc, dim=-1))
        outs.append(torch.matmul(torch.softmax(sc, dim=-1), vr).permute(1, 0, 2))
    out = torch.cat(outs, 0)
    out.backward(dO.float())
    return dict(out=out.detach(), lse=torch.cat(lses, 1).detach(), dq=qd.grad, dk=kd.grad,
                dv=vd.grad)


@pytest.mark.parametrize("name,lens,Hq,Hkv,D,base", [
    ("long_s4096", [4096], 28, 4, 128, 1.0e6),
    ("llama3_b2_s2048", [2048, 2048], 32, 8, 128, 5.0e5),
    ("qwen05b_s2048", [2048], 14, 2, 64, 1.0e6),
    ("long_and_ragged", [1100, 7, 1, 65, 64], 28, 4, 128, 1.0e6),
])
def test_large_shapes_match_torch_fp32_reference(engines, name, lens, Hq, Hkv, D, base):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    _say(f"[large] {name} T={T}")
    g = torch.Generator(device="cuda").manual_seed(1234)
    q = torch.randn(T, Hq, D, device="cuda", generator=g).bfloat16()
    k = torch.randn(T, Hkv, D, device="cuda", generator=g).bfloat16()
    v = torch.randn(T, Hkv, D, device="cuda", generator=g).bfloat16()
    dO = (0.01 * torch.randn(T, Hq, D, device="cuda", generator=g)).bfloat16()
    eng = engines[ga.PREC_BF16]
    cuarg = None if len(lens) == 1 else cu
    out, lse, q_rot, k_rot = eng.forward(q, k, v, base, cu_seqlens=cuarg)
    dq, dk, dv = eng.backward(dO, q_rot, k_rot, v, out, lse, base, cu_seqlens=cuarg)
    torch.cuda.synchronize()
    ref = torch_reference(q, k, v, dO, base, cu)
    got = dict(out=out, lse=lse, dq=dq, dk=dk, dv=dv)
    err = {key: float((got[key].float() - ref[key]).abs().max() / ref[key].abs().max())
           for key in got}
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err


@pytest.mark.parametrize("S,D", [(16384, 128), (16384, 64)])
def test_long_sequence_matches_torch_fp32_reference(engines, S, D):
    """S=16384 (a quarter of GLACIER_ATTN_MAX_SEQ_LEN) through the 32-row
    backward at D=128 and D=64, few heads so the float32 reference's S x S
    scores fit: row indices, tile tables and causal masks far from the
    shapes above."""
    Hq, Hkv, base = 2, 1, 1.0e6
    cu = np.array([0, S], np.int32)
    _say(f"[long] S={S} D={D}")
    g = torch.Generator(device="cuda").manual_seed(99)
    q = torch.randn(S, Hq, D, device="cuda", generator=g).bfloat16()
    k = torch.randn(S, Hkv, D, device="cuda", generator=g).bfloat16()
    v = torch.randn(S, Hkv, D, device="cuda", generator=g).bfloat16()
    dO = (0.01 * torch.randn(S, Hq, D, device="cuda", generator=g)).bfloat16()
    eng = engines[ga.PREC_BF16]
    out, lse, q_rot, k_rot = eng.forward(q, k, v, base)
    dq, dk, dv = eng.backward(dO, q_rot, k_rot, v, out, lse, base)
    torch.cuda.synchronize()
    ref = torch_reference(q, k, v, dO, base, cu)
    got = dict(out=out, lse=lse, dq=dq, dk=dk, dv=dv)
    err = {key: float((got[key].float() - ref[key]).abs().max() / ref[key].abs().max())
           for key in got}
    _say(f"  errors {err}")
    assert all(e <= BF16_GATE for e in err.values()), err


@pytest.mark.parametrize("prec,S,Hq,Hkv,D", [
    (ga.PREC_BF16, 512, 28, 4, 128),
    (ga.PREC_BF16, 512, 14, 2, 64),
    (ga.PREC_BF16, 1536, 28, 4, 128),
    (ga.PREC_FP32, 512, 28, 4, 128),
])
def test_scores_growing_far_past_the_first_chunk(engines, prec, S, Hq, Hkv, D):
    """Keys from position 256 on score about 6.4e5 above the earlier ones
    (value 800 in the lowest-frequency RoPE pair, which barely rotates: more
    than 2^16 in the exponent at either head size), so every
    query past 256 sees its maxima grow far beyond those of its first key
    chunk: the bf16 forward's rescue pass (references re-taken from the
    maxima seen; without it the probabilities overflow) and the fp32
    forward's rescaling must give finite results that match the float32
    reference.  At scores near 6.4e5, fp32 resolves about 0.06 and a bf16
    operand of 800 about 4 (the big component's rotation, under 0.01, is
    rounded away), so the bf16 mode is held to 5e-2 on O and 5e-5 on lse
    (about 3 nats at lse ~ 5.7e4) and the fp32 mode to 5e-3 and 1e-6; the
    backward is checked for finite values only (its row sums of P (dP - D)
    cancel at that scale in every fp32 implementation, the reference's
    included)."""
    base = 1.0e6
    dim = D // 2 - 1  # the pair (dim, dim + D/2) rotates by at most S * 1.2e-6 rad
    cu = np.array([0, S], np.int32)
    _say(f"[stress] prec={prec} S={S} Hq={Hq} D={D}")
    g = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(S, Hq, D, device="cuda", generator=g)
    k = torch.randn(S, Hkv, D, device="cuda", generator=g)
    v = torch.randn(S, Hkv, D, device="cuda", generator=g)
    dO = 0.01 * torch.randn(S, Hq, D, device="cuda", generator=g)
    q[:, :, dim] = 800.0
    k[:, :, dim] = 0.0
    k[256:, :, dim] = 800.0
    if prec == ga.PREC_BF16:
        q, k, v, dO = (x.bfloat16() for x in (q, k, v, dO))
    prev_tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        eng = engines[prec]
        out, lse, q_rot, k_rot = eng.forward(q, k, v, base)
        dq, dk, dv = eng.backward(dO, q_rot, k_rot, v, out, lse, base)
        torch.cuda.synchronize()
        ref = torch_reference(q, k, v, dO, base, cu)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev_tf32
    got = dict(out=out, lse=lse, dq=dq, dk=dk, dv=dv)
    for key, t in got.items():
        assert torch.isfinite(t.float()).all(), f"{key} has non-finite values"
    err = {key: float((got[key].float() - ref[key]).abs().max() / ref[key].abs().max())
           for key in ("out", "lse")}
    _say(f"  errors {err}")
    gate_out, gate_lse = (5e-2, 5e-5) if prec == ga.PREC_BF16 else (5e-3, 1e-6)
    assert err["out"] <= gate_out and err["lse"] <= gate_lse, err


LARGE_FP32 = [
    ("long_s4096", [4096], 28, 4, 1.0e6),
    ("llama3_b2_s2048", [2048, 2048], 32, 8, 5.0e5),
]


@pytest.mark.parametrize("name,lens,Hq,Hkv,base", LARGE_FP32)
def test_large_shapes_fp32_mode_match_torch_fp32_reference(engines, name, lens, Hq, Hkv, base):
    """BASELINE configs[3] and [4] in the fp32-operand mode, fp32 tensors, at
    the 1e-4 gate (the float32 reference: plain matmul/softmax/autograd)."""
    D = 128
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    _say(f"[large fp32] {name} T={T}")
    prev_tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        g = torch.Generator(device="cuda").manual_seed(4321)
        q = torch.randn(T, Hq, D, device="cuda", generator=g)
        k = torch.randn(T, Hkv, D, device="cuda", generator=g)
        v = torch.randn(T, Hkv, D, device="cuda", generator=g)
        dO = 0.01 * torch.randn(T, Hq, D, device="cuda", generator=g)
        eng = engines[ga.PREC_FP32]
        cuarg = None if len(lens) == 1 else cu
        out, lse, q_rot, k_rot = eng.forward(q, k, v, base, cu_seqlens=cuarg)
        dq, dk, dv = eng.backward(dO, q_rot, k_rot, v, out, lse, base, cu_seqlens=cuarg)
        torch.cuda.synchronize()
        ref = torch_reference(q, k, v, dO, base, cu)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev_tf32
    got = dict(out=out, lse=lse, dq=dq, dk=dk, dv=dv)
    err = {key: float((got[key].float() - ref[key]).abs().max() / ref[key].abs().max())
           for key in got}
    _say(f"  errors {err}")
    assert all(e <= FP32_GATE for e in err.values()), err


# ---------------------------------------------------------------------------
# Error behaviour and special values
# ---------------------------------------------------------------------------

def test_invalid_arguments_raise(engines):
    eng = engines[ga.PREC_FP32]
    q = np.zeros((8, 3, 64), np.float32)
    k = np.zeros((8, 2, 64), np.float32)
    out = np.empty_like(q)
    with pytest.raises(ga.InvalidArgument):
        eng.forward_attention(0, q, k, k, out, None, 8, 3, 2, 64, 1e4)  # Hq % Hkv != 0
    q = np.zeros((8, 2, 300), np.float32)
    with pytest.raises(ga.Unsupported):
        eng.forward_attention(0, q, q, q, np.empty_like(q), None, 8, 2, 2, 300, 1e4)
    assert not ga.supports_attention(512, 300)
    assert ga.supports_attention(512, 128) and ga.supports_attention(512, 80)


def test_empty_sequence_is_a_no_op(engines):
    eng = engines[ga.PREC_BF16]
    q = torch.empty((0, 4, 64), device="cuda", dtype=torch.bfloat16)
    k = torch.empty((0, 2, 64), device="cuda", dtype=torch.bfloat16)
    out, lse, q_rot, k_rot = eng.forward(q, k, k, 1e4)
    assert out.shape == (0, 4, 64)


def test_nan_in_upstream_gradient_propagates(engines):
    S, Hq, Hkv, D, base = 70, 4, 2, 64, 1e4
    q, k, v, dO = make_inputs(S, Hq, Hkv, D, 11, True)
    dO[5, 1, 3] = np.nan
    got = run_host(engines[ga.PREC_BF16], q, k, v, dO, base)
    assert np.isfinite(got["out"]).all()
    assert np.isnan(got["dq"][5, 1]).any()
    assert np.isnan(got["dv"]).any()
