"""Pins of the CPU oracle (oracle/attn_oracle.c) before anything trusts it.

Each check is chosen so that a plausible restatement mistake fails it: a
dropped scale, +sin instead of -sin, swapped rotation halves, a transposed
GQA map, a wrong softmax-gradient term or a missed head in the group
reduction.  The last block plants such mistakes in copies of oracle outputs
to show the checks catch them.
"""
import os

import numpy as np
import pytest
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_golden.npz")


def _inputs(S, Hq, Hkv, D, seed=11, dstd=0.01):
    q = oracle.fill_normal((S, Hq, D), seed + 1)
    k = oracle.fill_normal((S, Hkv, D), seed + 2)
    v = oracle.fill_normal((S, Hkv, D), seed + 3)
    dO = oracle.fill_normal((S, Hq, D), seed + 4, 0.0, dstd)
    return q, k, v, dO


# --------------------------------------------------------------------------
# Invariants the reference's own tests assert (KernelTests.cs)
# --------------------------------------------------------------------------

def test_rope_forward_backward_restores_vectors():
    """KernelTests.cs:9-47: S=4, Hq=2, Hkv=1, D=64, base 1e4, U(-1,1); 4 decimals."""
    rng = np.random.default_rng(42)
    q = rng.uniform(-1, 1, (4, 2, 64)).astype(np.float32)
    k = rng.uniform(-1, 1, (4, 1, 64)).astype(np.float32)
    qf, kf = oracle.rope_forward(q, k, 1.0e4)
    qb, kb = oracle.rope_backward(qf, kf, 1.0e4)
    np.testing.assert_allclose(qb, q, atol=0.5e-4, rtol=0)
    np.testing.assert_allclose(kb, k, atol=0.5e-4, rtol=0)
    assert not np.allclose(qf, q)  # the forward did rotate


def test_causal_attention_upper_triangle_exactly_zero():
    """KernelTests.cs:99-131: S=4, H=1, D=8, U(0,1) inputs; P[i, j>i] == 0.0."""
    rng = np.random.default_rng(77)
    q, k, v = (rng.uniform(0, 1, (4, 1, 8)).astype(np.float32) for _ in range(3))
    _, P, _ = oracle.attn_forward(q, k, v)
    for i in range(4):
        for j in range(i + 1, 4):
            assert P[0, i, j] == 0.0


# --------------------------------------------------------------------------
# Golden vectors (torch float64, tests/golden/make_golden.py)
# --------------------------------------------------------------------------

def _golden_cases():
    g = np.load(GOLDEN, allow_pickle=False)
    return [str(c) for c in g["cases"]]


@pytest.mark.parametrize("name", _golden_cases())
def test_oracle_layer_matches_golden(name):
    g = np.load(GOLDEN, allow_pickle=False)
    f = lambda key: g[f"{name}/{key}"]  # noqa: E731
    res = oracle.layer_fwd_bwd(f("q"), f("k"), f("v"), f("dO"), float(f("base")))
    S = f("q").shape[0]
    # RoPE angles are formed in fp32 (pos * w rounded): abs error grows ~S ulp
    assert oracle.max_rel_err(res["q_rot"], f("q_rot")) < 2e-6 * max(S, 8)
    assert oracle.max_rel_err(res["k_rot"], f("k_rot")) < 2e-6 * max(S, 8)
    for key in ("out", "lse", "dq", "dk", "dv"):
        err = oracle.max_rel_err(res[key], f(key))
        assert err < 5e-5, (key, err)


def test_golden_cases_cover_gqa_mha_and_head_dims():
    g = np.load(GOLDEN, allow_pickle=False)
    shapes = {(g[f"{n}/q"].shape[1], g[f"{n}/k"].shape[1], g[f"{n}/q"].shape[2]) for n in _golden_cases()}
    ratios = {hq // hkv for hq, hkv, _ in shapes}
    assert {1, 2, 3, 7} & ratios and {64, 128} <= {d for _, _, d in shapes}


# --------------------------------------------------------------------------
# Closed forms and library routines
# --------------------------------------------------------------------------

def test_rope_matches_fp64_closed_form_and_pos0_identity():
    q, k, _, _ = _inputs(512, 4, 2, 128)
    qf, kf = oracle.rope_forward(q, k, 1.0e6)
    # pos*w is rounded to fp32 in the reference; at pos<=511 that is <=3e-5 rad
    assert np.max(np.abs(qf - oracle.rope_fp64(q, 1.0e6))) < 3e-4
    assert np.max(np.abs(kf - oracle.rope_fp64(k, 1.0e6))) < 3e-4
    assert np.array_equal(qf[0], q[0]) and np.array_equal(kf[0], k[0])
    # rotation preserves each pair's norm
    h = 64
    n0 = q[..., :h] ** 2 + q[..., h:] ** 2
    n1 = qf[..., :h] ** 2 + qf[..., h:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)


def test_rope_table_matches_rotation():
    S, D = 64, 32
    cs, sn = oracle.rope_table(S, D, 1.0e4)
    x = oracle.fill_normal((S, 1, D), 5)
    xf, _ = oracle.rope_forward(x, np.zeros((S, 1, D), np.float32), 1.0e4)
    h = D // 2
    ref0 = x[:, 0, :h] * cs - x[:, 0, h:] * sn
    ref1 = x[:, 0, :h] * sn + x[:, 0, h:] * cs
    assert np.array_equal(xf[:, 0, :h], ref0) and np.array_equal(xf[:, 0, h:], ref1)


@pytest.mark.parametrize("S,Hq,Hkv,D", [(1, 2, 1, 8), (9, 4, 2, 16), (31, 6, 3, 32), (40, 7, 1, 64)])
def test_forward_backward_vs_fp64_bruteforce(S, Hq, Hkv, D):
    q, k, v, dO = _inputs(S, Hq, Hkv, D, seed=S)
    out, P, lse = oracle.attn_forward(q, k, v)
    dq, dk, dv = oracle.attn_backward(dO, q, k, v, P)
    ref = oracle.attn_fp64(q, k, v, dO)
    assert oracle.max_rel_err(out, ref["out"]) < 2e-6
    assert oracle.max_rel_err(lse, ref["lse"]) < 2e-6
    assert oracle.max_rel_err(P, ref["P"]) < 2e-6
    for key, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert oracle.max_rel_err(got, ref[key]) < 2e-5, key


def test_forward_backward_vs_torch_sdpa_fp64():
    S, Hq, Hkv, D = 48, 8, 2, 32
    q, k, v, dO = _inputs(S, Hq, Hkv, D, seed=3)
    out, P, _ = oracle.attn_forward(q, k, v)
    dq, dk, dv = oracle.attn_backward(dO, q, k, v, P)
    t = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v)]
    o = torch.nn.functional.scaled_dot_product_attention(
        *[x.permute(1, 0, 2)[None] for x in t], is_causal=True, enable_gqa=True)[0].permute(1, 0, 2)
    o.backward(torch.tensor(dO, dtype=torch.float64))
    assert oracle.max_rel_err(out, o.detach().numpy()) < 2e-6
    for got, ref in ((dq, t[0].grad), (dk, t[1].grad), (dv, t[2].grad)):
        assert oracle.max_rel_err(got, ref.numpy()) < 2e-5


def test_single_token_output_is_v0():
    q, k, v, _ = _inputs(1, 4, 2, 16)
    out, P, lse = oracle.attn_forward(q, k, v)
    assert np.array_equal(out[0], np.repeat(v[0], 2, axis=0))
    assert np.all(P == 1.0)
    s = np.sum(q[0] * np.repeat(k[0], 2, axis=0), -1) / np.sqrt(16)
    np.testing.assert_allclose(lse[:, 0], s, rtol=1e-5, atol=1e-6)


def test_zero_query_gives_causal_running_mean():
    S, Hq, Hkv, D = 24, 4, 1, 16
    _, k, v, _ = _inputs(S, Hq, Hkv, D)
    q = np.zeros((S, Hq, D), np.float32)
    out, P, lse = oracle.attn_forward(q, k, v)
    mean = np.cumsum(v[:, 0].astype(np.float64), 0) / np.arange(1, S + 1)[:, None]
    for h in range(Hq):
        np.testing.assert_allclose(out[:, h], mean, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse[0], np.log(np.arange(1, S + 1)), rtol=1e-6)


def test_rows_of_p_sum_to_one_and_dv_is_pt_do():
    S, Hq, Hkv, D = 37, 6, 2, 32
    q, k, v, dO = _inputs(S, Hq, Hkv, D)
    out, P, _ = oracle.attn_forward(q, k, v)
    np.testing.assert_allclose(P.sum(-1), 1.0, rtol=1e-5)
    _, _, dv = oracle.attn_backward(dO, q, k, v, P)
    r = Hq // Hkv
    ref = np.einsum("hij,ihd->jhd", P.astype(np.float64), dO.astype(np.float64))
    ref = ref.reshape(S, Hkv, r, D).sum(2)
    assert oracle.max_rel_err(dv, ref) < 1e-5


def test_gqa_equals_mha_with_repeated_kv_heads():
    S, Hq, Hkv, D = 20, 6, 2, 16
    q, k, v, dO = _inputs(S, Hq, Hkv, D)
    r = Hq // Hkv
    out, P, _ = oracle.attn_forward(q, k, v)
    dq, dk, dv = oracle.attn_backward(dO, q, k, v, P)
    kk, vv = np.repeat(k, r, axis=1), np.repeat(v, r, axis=1)
    out2, P2, _ = oracle.attn_forward(q, kk, vv)
    dq2, dk2, dv2 = oracle.attn_backward(dO, q, kk, vv, P2)
    assert np.array_equal(out, out2) and np.array_equal(dq, dq2)
    # the group reduction (CausalAttentionKernel.cs:184-206) sums heads in order
    np.testing.assert_allclose(dk, dk2.reshape(S, Hkv, r, D).sum(2), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(dv, dv2.reshape(S, Hkv, r, D).sum(2), rtol=1e-5, atol=1e-7)


def test_finite_differences_of_layer_loss():
    """Central differences of L = sum(dO * O(q, k, v)) through RoPE, in the
    spirit of GradientAndGpuParityTests.cs:613-646 (eps 1e-3, rel 2.5e-2,
    abs 5e-3), on the float64 twin, which then pins the fp32 oracle."""
    S, Hq, Hkv, D, base = 6, 4, 2, 8, 1.0e4
    q, k, v, dO = _inputs(S, Hq, Hkv, D, dstd=1.0)
    ref = oracle.layer_fp64(q, k, v, dO, base)
    got = oracle.layer_fwd_bwd(q, k, v, dO, base)

    def loss(qq, kk, vv):
        o = oracle.attn_fp64(oracle.rope_fp64(qq, base), oracle.rope_fp64(kk, base), vv)["out"]
        return float(np.sum(o * dO))

    eps = 1e-3
    rng = np.random.default_rng(0)
    for name, idx_src in (("dq", q), ("dk", k), ("dv", v)):
        for _ in range(6):
            idx = tuple(rng.integers(0, n) for n in idx_src.shape)
            args = [q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)]
            which = {"dq": 0, "dk": 1, "dv": 2}[name]
            a = args[which].copy(); a[idx] += eps; args_p = list(args); args_p[which] = a
            b = args[which].copy(); b[idx] -= eps; args_m = list(args); args_m[which] = b
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            an = ref[name][idx]
            assert abs(fd - an) < 5e-3 or abs(fd - an) / max(abs(an), 1e-12) < 2.5e-2
            assert abs(got[name][idx] - an) < 1e-4 * max(1.0, abs(an))


def test_layer_returns_pre_rope_gradients():
    """dq_pre = R(-theta) dq_post (the inverse rotation is applied last)."""
    S, Hq, Hkv, D, base = 16, 4, 2, 32, 1.0e6
    q, k, v, dO = _inputs(S, Hq, Hkv, D)
    res = oracle.layer_fwd_bwd(q, k, v, dO, base)
    _, P, _ = oracle.attn_forward(res["q_rot"], res["k_rot"], v)
    dq_post, dk_post, _ = oracle.attn_backward(dO, res["q_rot"], res["k_rot"], v, P)
    np.testing.assert_allclose(res["dq"], oracle.rope_fp64(dq_post, base, inverse=True), atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(res["dk"], oracle.rope_fp64(dk_post, base, inverse=True), atol=1e-6, rtol=1e-5)


def test_thread_count_does_not_change_bits():
    S, Hq, Hkv, D = 64, 7, 1, 32
    q, k, v, dO = _inputs(S, Hq, Hkv, D)
    n0 = oracle.num_threads()
    try:
        oracle.set_threads(1)
        a = oracle.layer_fwd_bwd(q, k, v, dO, 1e6)
        oracle.set_threads(max(n0, 4))
        b = oracle.layer_fwd_bwd(q, k, v, dO, 1e6)
    finally:
        oracle.set_threads(n0)
    for key in ("out", "lse", "dq", "dk", "dv"):
        assert np.array_equal(a[key], b[key]), key


def test_varlen_is_block_diagonal_with_restarting_positions():
    Hq, Hkv, D, base = 4, 2, 16, 1.0e4
    lens = [5, 1, 9]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v, dO = _inputs(T, Hq, Hkv, D)
    res = oracle.layer_fwd_bwd_varlen(q, k, v, dO, cu, base)
    for b in range(len(lens)):
        s = slice(cu[b], cu[b + 1])
        ref = oracle.layer_fp64(q[s], k[s], v[s], dO[s], base)
        for key in ("out", "dq", "dk", "dv"):
            assert oracle.max_rel_err(res[key][s], ref[key]) < 2e-5, (b, key)
        assert oracle.max_rel_err(res["lse"][:, s], ref["lse"]) < 2e-6


def test_bf16_rounding_is_rne():
    x = np.array([1.0, 1.00390625, 1.005859375, -3.0e-5, 65504.0, np.float32(1 + 2**-8 + 2**-9)], np.float32)
    r = oracle.round_bf16(x)
    t = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(r, t)


# --------------------------------------------------------------------------
# Planted mistakes (in copies of oracle outputs, on the CPU): the checks above
# must reject each of them.
# --------------------------------------------------------------------------

def test_planted_mistakes_are_caught():
    S, Hq, Hkv, D, base = 12, 4, 2, 16, 1.0e4
    q, k, v, dO = _inputs(S, Hq, Hkv, D)
    ref = oracle.layer_fp64(q, k, v, dO, base)
    good = oracle.layer_fwd_bwd(q, k, v, dO, base)
    assert oracle.max_rel_err(good["dq"], ref["dq"]) < 2e-5
    # forward rotation applied where the inverse belongs (+sin instead of -sin)
    _, P, _ = oracle.attn_forward(good["q_rot"], good["k_rot"], v)
    dq_post, _, _ = oracle.attn_backward(dO, good["q_rot"], good["k_rot"], v, P)
    wrong, _ = oracle.rope_forward(dq_post, np.zeros_like(k), base)
    assert oracle.max_rel_err(wrong, ref["dq"]) > 1e-2
    # missing 1/sqrt(D) on the scores
    bad = oracle.attn_fp64(good["q_rot"] * np.sqrt(D), good["k_rot"], v)
    assert oracle.max_rel_err(bad["out"], ref["out"]) > 1e-2
    # transposed GQA map (kv head = h % Hkv instead of h // (Hq/Hkv))
    kk = np.ascontiguousarray(good["k_rot"][:, [h % Hkv for h in range(Hq)]])
    vv = np.ascontiguousarray(v[:, [h % Hkv for h in range(Hq)]])
    o2, _, _ = oracle.attn_forward(good["q_rot"], kk, vv)
    assert oracle.max_rel_err(o2, ref["out"]) > 1e-2
    # softmax gradient without the rowsum term: dS = P * dP * scale
    Pd = ref["P"]; kk64 = np.repeat(ref["k_rot"], Hq // Hkv, axis=1)
    dP = np.einsum("ihd,jhd->hij", dO.astype(np.float64), np.repeat(v, Hq // Hkv, axis=1))
    dq_bad = np.einsum("hij,jhd->ihd", Pd * dP / np.sqrt(D), kk64)
    assert oracle.max_rel_err(oracle.rope_fp64(dq_bad, base, inverse=True), ref["dq"]) > 1e-2
    # group reduction that drops the last head of each group
    r = Hq // Hkv
    dv_heads = np.einsum("hij,ihd->jhd", Pd, dO.astype(np.float64)).reshape(S, Hkv, r, D)
    assert oracle.max_rel_err(dv_heads[:, :, :-1].sum(2), ref["dv"]) > 1e-2


# --------------------------------------------------------------------------
# Projection + LoRA adapter (lora_oracle.c: LoraAdapter.Forward/Backward)
# --------------------------------------------------------------------------

def _proj_inputs(S, n_in, n_out, rank, seed=11):
    rng = np.random.default_rng(seed)
    f = lambda *shape: rng.standard_normal(shape).astype(np.float32)
    return (f(S, n_in), f(n_out, n_in) / np.sqrt(n_in), f(n_out), f(n_in, rank) / np.sqrt(n_in),
            f(rank, n_out), f(S, n_out))


def test_proj_forward_matches_matrix_products():
    """y = x W^T + bias + s (x A) B (LoraAdapter.cs:15) against numpy float64 products."""
    x, w, bias, a, b, _ = _proj_inputs(9, 40, 24, 4)
    ref = oracle.proj_fp64(x, w, bias, a, b, 2.0)
    assert oracle.max_rel_err(oracle.proj_forward(x, w, bias, a, b, 2.0), ref) < 1e-6
    # no adapter, no bias: the plain product
    assert oracle.max_rel_err(oracle.proj_forward(x, w), x.astype(np.float64) @ w.T) < 1e-6


def test_proj_forward_one_hot_rows_and_fresh_adapter():
    """x = e_k picks column k of W; a fresh adapter (B = 0, LoraAdapter.cs:106) adds
    nothing; a rank-1 adapter adds s A[k,0] B[0,:] to row e_k."""
    n_in, n_out = 12, 7
    _, w, bias, a, b, _ = _proj_inputs(1, n_in, n_out, 1)
    x = np.eye(n_in, dtype=np.float32)
    y = oracle.proj_forward(x, w, bias, a, b, 3.0)
    expect = w.T.astype(np.float64) + bias + 3.0 * a.astype(np.float64) @ b.astype(np.float64)
    assert oracle.max_rel_err(y, expect) < 1e-6
    y0 = oracle.proj_forward(x, w, bias, a, np.zeros_like(b), 3.0)
    assert np.array_equal(y0, oracle.proj_forward(x, w, bias))


def test_proj_backward_is_the_gradient_of_the_forward():
    """Central differences (float64) of L = sum dy * y w.r.t. x, A and B."""
    S, n_in, n_out, rank, s = 5, 8, 6, 3, 1.5
    x, w, bias, a, b, dy = _proj_inputs(S, n_in, n_out, rank, seed=3)
    dx, ga, gb = oracle.proj_backward(x, dy, w, a, b, s)
    X, A, B, DY = (t.astype(np.float64) for t in (x, a, b, dy))
    loss = lambda X_, A_, B_: float(np.sum(DY * oracle.proj_fp64(X_, w, bias, A_, B_, s)))
    eps = 1e-4
    for got, base, which in ((dx, X, 0), (ga, A, 1), (gb, B, 2)):
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            hi = [X.copy(), A.copy(), B.copy()]
            lo = [X.copy(), A.copy(), B.copy()]
            hi[which][idx] += eps
            lo[which][idx] -= eps
            num[idx] = (loss(*hi) - loss(*lo)) / (2 * eps)
        assert oracle.max_rel_err(got, num) < 1e-5, which


def test_proj_backward_accumulates():
    """dx, grad_a and grad_b are added to (the reference's Grad tensors and dXInput)."""
    x, w, _, a, b, dy = _proj_inputs(6, 10, 8, 2)
    dx, ga, gb = oracle.proj_backward(x, dy, w, a, b, 0.5)
    dx2, ga2, gb2 = oracle.proj_backward(x, dy, w, a, b, 0.5, dx.copy(), ga.copy(), gb.copy())
    for one, two in ((dx, dx2), (ga, ga2), (gb, gb2)):
        assert oracle.max_rel_err(two, 2.0 * one) < 1e-6
    # without an adapter only the base gradient dy W is formed
    dxb, ga0, gb0 = oracle.proj_backward(x, dy, w)
    assert ga0 is None and gb0 is None
    assert oracle.max_rel_err(dxb, dy.astype(np.float64) @ w) < 1e-6


def test_proj_planted_mistakes_are_caught():
    """Each plausible slip in the projection math changes the result beyond the
    parity tolerances, so the checks above would catch it."""
    S, n_in, n_out, rank, s = 7, 16, 16, 4, 2.0
    x, w, bias, a, b, dy = _proj_inputs(S, n_in, n_out, rank, seed=5)
    y = oracle.proj_forward(x, w, bias, a, b, s)
    slips = {
        "W not transposed": oracle.proj_fp64(x, w.T, bias, a, b, s),
        "bias dropped": oracle.proj_fp64(x, w, None, a, b, s),
        "scaling dropped": oracle.proj_fp64(x, w, bias, a, b, 1.0),
        "A, B swapped roles": oracle.proj_fp64(x, w, bias, b.T, a.T, s),
    }
    for name, bad in slips.items():
        assert oracle.max_rel_err(bad, y) > 1e-2, name
    dx, ga, gb = oracle.proj_backward(x, dy, w, a, b, s)
    X, A, B, DY = (t.astype(np.float64) for t in (x, a, b, dy))
    grad_slips = {
        "dx with W^T": (dx, DY @ w.T + s * (DY @ B.T) @ A.T),
        "grad_a without scaling": (ga, X.T @ (DY @ B.T)),
        "grad_b with the output index reversed": (gb, s * (X @ A).T @ DY[:, ::-1]),
    }
    for name, (got, bad) in grad_slips.items():
        assert oracle.max_rel_err(got, bad) > 1e-2, name


# --- residual + RMSNorm (oracle/norm_oracle.c) -------------------------------

def _norm_inputs(rows, n, seed=0):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    return f(rows, n), f(rows, n), (1.0 + 0.2 * f(n)).astype(np.float32), f(rows, n)


def _rmsnorm_fp64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def test_rmsnorm_forward_closed_forms():
    """Constant rows, one-hot rows and the mean-square invariant."""
    n, eps = 24, 1e-5
    w = (1.0 + 0.3 * np.random.default_rng(1).standard_normal(n)).astype(np.float32)
    c = np.array([[0.5], [-3.0], [1e-3]], np.float32)
    x = np.repeat(c, n, axis=1)
    _, y = oracle.rmsnorm_forward(x, w, eps)
    want = c.astype(np.float64) / np.sqrt(c.astype(np.float64) ** 2 + eps) * w
    assert oracle.max_rel_err(y, want) < 1e-6
    # one-hot row: only element k is non-zero
    x = np.zeros((1, n), np.float32); x[0, 7] = 2.5
    _, y = oracle.rmsnorm_forward(x, w, eps)
    r = 1.0 / np.sqrt(2.5 ** 2 / n + eps)
    assert abs(y[0, 7] - 2.5 * r * w[7]) < 1e-6 * abs(y[0, 7]) and np.count_nonzero(y) == 1
    # mean over i of (y_i / w_i)^2 = ms / (ms + eps)
    x, _, w, _ = _norm_inputs(5, 64, seed=2)
    _, y = oracle.rmsnorm_forward(x, w, eps)
    ms = np.mean(x.astype(np.float64) ** 2, axis=1)
    got = np.mean((y.astype(np.float64) / w) ** 2, axis=1)
    assert np.max(np.abs(got - ms / (ms + eps))) < 1e-5


def test_rmsnorm_forward_scale_invariance_and_residual():
    """With eps = 0, RMSNorm(a x) = sign(a) RMSNorm(x); the residual form is
    RMSNorm(x + delta) with x1 = x + delta exactly."""
    x, delta, w, _ = _norm_inputs(6, 40, seed=3)
    _, y = oracle.rmsnorm_forward(x, w, 0.0)
    for a in (4.0, -0.25):
        _, ya = oracle.rmsnorm_forward((a * x).astype(np.float32), w, 0.0)
        assert oracle.max_rel_err(ya, np.sign(a) * y) < 1e-6
    x1, y1 = oracle.rmsnorm_forward(x, w, 1e-6, delta=delta)
    assert np.array_equal(x1, x + delta)
    _, y2 = oracle.rmsnorm_forward(x + delta, w, 1e-6)
    assert np.array_equal(y1, y2)
    assert oracle.max_rel_err(y1, _rmsnorm_fp64(x + delta, w, 1e-6)) < 1e-6


def test_rmsnorm_backward_is_the_gradient_of_the_forward():
    """Central differences (float64) of L = sum g * RMSNorm(x) w.r.t. x and w;
    d_residual is added to dx and d_weight accumulates."""
    rows, n, eps = 3, 12, 1e-3
    x, dres, w, g = _norm_inputs(rows, n, seed=4)
    dw = np.zeros(n, np.float32)
    dx = oracle.rmsnorm_backward(g, x, w, eps, d_residual=dres, d_weight=dw)
    X, W, G = x.astype(np.float64), w.astype(np.float64), g.astype(np.float64)
    loss = lambda X_, W_: float(np.sum(G * _rmsnorm_fp64(X_, W_, eps)))
    h = 1e-5
    num_x = np.zeros_like(X)
    for idx in np.ndindex(X.shape):
        hi, lo = X.copy(), X.copy()
        hi[idx] += h; lo[idx] -= h
        num_x[idx] = (loss(hi, W) - loss(lo, W)) / (2 * h)
    num_w = np.zeros_like(W)
    for i in range(n):
        hi, lo = W.copy(), W.copy()
        hi[i] += h; lo[i] -= h
        num_w[i] = (loss(X, hi) - loss(X, lo)) / (2 * h)
    assert oracle.max_rel_err(dx - dres, num_x) < 1e-5
    assert oracle.max_rel_err(dw, num_w) < 1e-5
    dx2 = oracle.rmsnorm_backward(g, x, w, eps, d_weight=dw)
    assert np.array_equal(dx2 + dres, dx) or oracle.max_rel_err(dx2 + dres, dx) < 1e-7
    assert oracle.max_rel_err(dw, 2.0 * num_w) < 1e-5


def test_rmsnorm_backward_is_orthogonal_to_x_without_eps():
    """With eps = 0 the norm is scale-invariant, so sum_i x_i dx_i = 0."""
    x, _, w, g = _norm_inputs(4, 96, seed=5)
    dx = oracle.rmsnorm_backward(g, x, w, 0.0)
    dots = np.sum(x.astype(np.float64) * dx, axis=1)
    scale = np.linalg.norm(x, axis=1) * np.linalg.norm(dx, axis=1)
    assert np.max(np.abs(dots) / scale) < 1e-5


def test_rmsnorm_planted_mistakes_are_caught():
    """Each plausible slip changes the result beyond the parity tolerances."""
    rows, n, eps = 5, 32, 0.05
    x, _, w, g = _norm_inputs(rows, n, seed=6)
    X, W, G = x.astype(np.float64), w.astype(np.float64), g.astype(np.float64)
    _, y = oracle.rmsnorm_forward(x, w, eps)
    ms = np.mean(X * X, axis=1, keepdims=True)
    fwd_slips = {
        "eps outside the root": X / (np.sqrt(ms) + eps) * W,
        "sum instead of mean": X / np.sqrt(ms * n + eps) * W,
        "weight dropped": _rmsnorm_fp64(X, np.ones(n), eps),
    }
    for name, bad in fwd_slips.items():
        assert oracle.max_rel_err(y, bad) > 1e-3, name
    dx = oracle.rmsnorm_backward(g, x, w, eps)
    r = 1.0 / np.sqrt(ms + eps)
    c = np.sum(G * W * X, axis=1, keepdims=True)
    bwd_slips = {
        "r instead of r^3": r * G * W - r / n * c * X,
        "weight missing in the sum": r * G * W - r ** 3 / n * np.sum(G * X, axis=1, keepdims=True) * X,
        "second term sign": r * G * W + r ** 3 / n * c * X,
        "weight missing in the first term": r * G - r ** 3 / n * c * X,
    }
    for name, bad in bwd_slips.items():
        assert oracle.max_rel_err(dx, bad) > 1e-3, name


# --- LM-head cross-entropy (oracle/ce_oracle.c) ------------------------------

def _ce_inputs(T, H, V, seed=0, wscale=0.3):
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((T, H)).astype(np.float32)
    w = (wscale * rng.standard_normal((V, H))).astype(np.float32)
    return h, w


def test_ce_loss_is_mean_logsumexp_minus_target_logit():
    """Against scipy's logsumexp in float64 over the kept rows only (targets -100
    and >= V dropped), with targets either side of the 4096-wide vocab tiles."""
    from scipy.special import logsumexp

    T, H, V = 8, 24, 9000
    h, w = _ce_inputs(T, H, V, seed=1)
    tg = np.array([0, 4095, 4096, 8999, -100, 9000, 17, 8191], np.int32)
    loss, n, _ = oracle.ce_loss(h, tg, w, grad=False)
    keep = [i for i in range(T) if 0 <= tg[i] < V]
    logits = h.astype(np.float64) @ w.T.astype(np.float64)
    want = np.mean([logsumexp(logits[i]) - logits[i, tg[i]] for i in keep])
    assert n == len(keep) == 6
    assert abs(loss - want) < 1e-5 * abs(want)


def test_ce_loss_closed_forms():
    """W = 0: every logit is 0, the loss is log V and the gradient is 0.  A
    vocabulary of one: loss 0."""
    T, H, V = 5, 8, 777
    h, _ = _ce_inputs(T, H, V)
    tg = np.arange(T, dtype=np.int32)
    loss, n, d = oracle.ce_loss(h, tg, np.zeros((V, H), np.float32))
    assert n == T and abs(loss - np.log(V)) < 1e-6 * np.log(V)
    assert np.all(d == 0.0)
    loss1, _, d1 = oracle.ce_loss(h, np.zeros(T, np.int32), np.ones((1, H), np.float32))
    assert loss1 == 0.0 and np.all(d1 == 0.0)
    # no kept row: loss 0, gradient 0
    loss0, n0, d0 = oracle.ce_loss(h, np.full(T, -1, np.int32), np.ones((V, H), np.float32))
    assert loss0 == 0.0 and n0 == 0 and np.all(d0 == 0.0)


def test_ce_gradient_is_the_derivative_of_the_loss():
    """Central differences (float64) of the mean cross-entropy w.r.t. the hidden
    states; dropped rows get zero gradient."""
    from scipy.special import logsumexp

    T, H, V = 4, 6, 4500
    h, w = _ce_inputs(T, H, V, seed=2)
    tg = np.array([3, -100, 4321, 4096], np.int32)
    _, _, d = oracle.ce_loss(h, tg, w)
    W = w.astype(np.float64)
    keep = [i for i in range(T) if 0 <= tg[i] < V]

    def loss(Hm):
        l = Hm @ W.T
        return np.mean([logsumexp(l[i]) - l[i, tg[i]] for i in keep])

    Hm = h.astype(np.float64)
    num = np.zeros_like(Hm)
    eps = 1e-5
    for idx in np.ndindex(Hm.shape):
        hi, lo = Hm.copy(), Hm.copy()
        hi[idx] += eps; lo[idx] -= eps
        num[idx] = (loss(hi) - loss(lo)) / (2 * eps)
    assert np.all(d[1] == 0.0)
    assert oracle.max_rel_err(d, num) < 1e-4


def test_ce_large_logits_stay_finite_and_planted_mistakes_are_caught():
    """Logits near 1e3 (exp overflows without the max shift) stay finite, and
    plausible slips change the result beyond the parity tolerances."""
    from scipy.special import logsumexp, softmax

    T, H, V = 6, 8, 5000
    h, w = _ce_inputs(T, H, V, seed=3, wscale=150.0)
    tg = np.array([1, 2, 4999, 4096, -1, 77], np.int32)
    loss, n, d = oracle.ce_loss(h, tg, w)
    assert np.isfinite(loss) and np.all(np.isfinite(d))
    h, w = _ce_inputs(T, H, V, seed=4)
    loss, n, d = oracle.ce_loss(h, tg, w)
    keep = [i for i in range(T) if 0 <= tg[i] < V]
    L = h.astype(np.float64) @ w.T.astype(np.float64)
    W = w.astype(np.float64)
    P = softmax(L, axis=1)
    onehot = np.zeros_like(P)
    for i in keep:
        onehot[i, tg[i]] = 1.0
    mask = np.zeros((T, 1)); mask[keep] = 1.0
    good = ((P - onehot) * mask) @ W / len(keep)
    assert oracle.max_rel_err(d, good) < 1e-4
    slips = {
        "no -1 at the target": (P * mask) @ W / len(keep),
        "divided by T": ((P - onehot) * mask) @ W / T,
        "dropped rows kept": (P - onehot) @ W / len(keep),
    }
    for name, bad in slips.items():
        assert oracle.max_rel_err(d, bad) > 1e-3, name
    lse = np.array([logsumexp(L[i]) for i in range(T)])
    loss_slips = {
        "mean over T": np.sum([lse[i] - L[i, tg[i]] for i in keep]) / T,
        "max logit instead of lse": np.mean([L[i].max() - L[i, tg[i]] for i in keep]),
    }
    for name, bad in loss_slips.items():
        assert abs(loss - bad) > 1e-3 * abs(loss), name
