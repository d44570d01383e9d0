"""Parity of the residual add + RMSNorm entry points (glacier_rmsnorm_forward /
glacier_rmsnorm_backward, include/glacier_norm.h) against the CPU oracle
(oracle/norm_oracle.c), through the C ABI on device tensors, and of the block
segment they form with the O projection (glacier_proj_*, n_proj = 1, with a
LoRA adapter): x1 = x + OProj(attnOut), norm2X = RMSNorm(x1) and back
(TransformerBlock.cs:505-506, :524, :672-687).

Gates (the north star's): fp32 mode max-rel-err <= 1e-4, bf16 mode <= 2e-2,
normwise (max|x - ref| / max|ref|) per tensor.  In the bf16 mode the oracle
runs on the bf16-rounded inputs; x1 is rounded to bf16 as stored before it is
normalised, which the oracle reproduces by normalising round_bf16(x + delta).
"""
import sys

import numpy as np
import pytest

import glacier_attn as ga
import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FP32_GATE, BF16_GATE = 1e-4, 2e-2
EPS = 1e-6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def eng():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    e = ga.GpuAttentionEngine(0, ga.PREC_BF16)
    yield e
    e.close()


def _dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0", dt).contiguous()


SHAPES = {  # rows, n
    "qwen7b_t512": (512, 3584),
    "qwen05b_t256": (256, 896),
    "per_head_qk": (512 * 4, 128),  # the per-head K norm: rows = tokens x heads
    "ragged": (37, 100),
    "widest": (3, 8192),
    "one_row": (1, 4),
}


@pytest.mark.parametrize("shape", sorted(SHAPES))
@pytest.mark.parametrize("bf16", [False, True], ids=["fp32", "bf16"])
def test_rmsnorm_matches_oracle(eng, bf16, shape):
    rows, n = SHAPES[shape]
    _say(f"[norm] io={'bf16' if bf16 else 'fp32'} shape={shape} rows={rows} n={n}")
    rng = np.random.default_rng(11)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    x, delta, dy, dres = f(rows, n), 0.5 * f(rows, n), f(rows, n), 0.3 * f(rows, n)
    w = (1.0 + 0.2 * f(n)).astype(np.float32)
    if bf16:
        x, delta, dy, dres = (oracle.round_bf16(t) for t in (x, delta, dy, dres))
    io = torch.bfloat16 if bf16 else torch.float32
    xd, dd, dyd, drd, wd = _dev(x, io), _dev(delta, io), _dev(dy, io), _dev(dres, io), _dev(w, torch.float32)
    x1d, yd = eng.rmsnorm_forward(xd, wd, EPS, delta=dd)
    _, y0d = eng.rmsnorm_forward(xd, wd, EPS)
    dxd = eng.rmsnorm_backward(dyd, x1d, wd, EPS, d_residual=drd)
    torch.cuda.synchronize()
    x1_ref = x + delta
    if bf16:
        x1_ref = oracle.round_bf16(x1_ref)
    assert np.array_equal(x1d.float().cpu().numpy(), x1_ref), "x1 = x + delta, as stored"
    _, y_ref = oracle.rmsnorm_forward(x1_ref, w, EPS)
    _, y0_ref = oracle.rmsnorm_forward(x, w, EPS)
    dx_ref = oracle.rmsnorm_backward(dy, x1_ref, w, EPS, d_residual=dres)
    gate = BF16_GATE if bf16 else FP32_GATE
    errs = {"y": oracle.max_rel_err(yd.float().cpu().numpy(), y_ref),
            "y_no_residual": oracle.max_rel_err(y0d.float().cpu().numpy(), y0_ref),
            "dx": oracle.max_rel_err(dxd.float().cpu().numpy(), dx_ref)}
    _say("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()) + f" (gate {gate:g})")
    for k, v in errs.items():
        assert v <= gate, k


def test_rmsnorm_weight_gradient_aliasing_repeatability_and_empty(eng):
    """d_weight accumulates the oracle's sum; y may overwrite x and dx may
    overwrite dy with the same bits; repeated calls are bitwise equal; rows = 0
    is a no-op."""
    rows, n = 300, 1024
    rng = np.random.default_rng(5)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    dy = rng.standard_normal((rows, n)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    xd, dyd, wd = _dev(x, torch.float32), _dev(dy, torch.float32), _dev(w, torch.float32)
    dw = torch.zeros(n, device="cuda:0")
    dx1 = eng.rmsnorm_backward(dyd, xd, wd, EPS, d_weight=dw).clone()
    dx2 = eng.rmsnorm_backward(dyd, xd, wd, EPS, d_weight=dw)
    torch.cuda.synchronize()
    dw_ref = np.zeros(n, np.float32)
    oracle.rmsnorm_backward(dy, x, w, EPS, d_weight=dw_ref)
    _say(f"  d_weight err {oracle.max_rel_err(dw.cpu().numpy(), 2 * dw_ref):.2e}")
    assert oracle.max_rel_err(dw.cpu().numpy(), 2 * dw_ref) <= FP32_GATE
    assert torch.equal(dx1, dx2)
    # in place
    _, y = eng.rmsnorm_forward(xd, wd, EPS)
    xin = xd.clone()
    eng.rmsnorm_forward(xin, wd, EPS, y=xin)
    dyin = dyd.clone()
    eng.rmsnorm_backward(dyin, xd, wd, EPS, dx=dyin)
    torch.cuda.synchronize()
    assert torch.equal(xin, y) and torch.equal(dyin, dx1)
    # in place with the weight gradient: d_weight is formed from dy as passed
    # in, not from the dx that overwrote it
    dyin = dyd.clone()
    dw2 = torch.zeros(n, device="cuda:0")
    eng.rmsnorm_backward(dyin, xd, wd, EPS, dx=dyin, d_weight=dw2)
    torch.cuda.synchronize()
    assert torch.equal(dyin, dx1)
    assert oracle.max_rel_err(dw2.cpu().numpy(), dw_ref) <= FP32_GATE
    # empty
    e = torch.empty((0, n), device="cuda:0")
    _, ye = eng.rmsnorm_forward(e, wd, EPS)
    assert ye.shape == (0, n)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp32", "bf16"])
def test_o_projection_residual_rmsnorm_block(eng, bf16):
    """The block segment from the attention output to the FFN input and back,
    entirely on the device: x1 = x + attnOut Wo^T + bo + s (attnOut A) B,
    norm2X = RMSNorm(x1); backward dX1 = dOutput + RMSNormBackward(dNorm2X, x1),
    dAttnOut = dX1 Wo + s (dX1 B^T) A^T with the adapter gradients, against the
    oracle composition (Qwen2.5-0.5B attention width, rank-8 adapter on O)."""
    T, hidden, qdim, rank, s = 128, 896, 896, 8, 2.0
    rng = np.random.default_rng(21)
    f = lambda *sh: rng.standard_normal(sh).astype(np.float32)
    x, attn = f(T, hidden), f(T, qdim)
    wo, bo = f(hidden, qdim) / np.sqrt(qdim), 0.1 * f(hidden)
    a, b = f(qdim, rank) / np.sqrt(qdim), 0.1 * f(rank, hidden)
    wn = (1.0 + 0.2 * f(hidden)).astype(np.float32)
    d_out, d_norm2 = f(T, hidden), f(T, hidden)
    r = oracle.round_bf16 if bf16 else (lambda t: t)
    x, attn, wo, d_out, d_norm2 = (r(t) for t in (x, attn, wo, d_out, d_norm2))
    io = torch.bfloat16 if bf16 else torch.float32
    eng_p = ga.GpuAttentionEngine(0, ga.PREC_BF16 if bf16 else ga.PREC_FP32)
    try:
        xd, ad = _dev(x, io), _dev(attn, io)
        proj = {"w": _dev(wo, io), "bias": _dev(bo, torch.float32), "a": _dev(a, torch.float32),
                "b": _dev(b, torch.float32), "scaling": s,
                "grad_a": torch.zeros(qdim, rank, device="cuda:0"),
                "grad_b": torch.zeros(rank, hidden, device="cuda:0")}
        (po,) = eng_p.proj_forward(ad, [proj], rank)
        x1d, n2d = eng_p.rmsnorm_forward(xd, _dev(wn, torch.float32), EPS, delta=po)
        dx1d = eng_p.rmsnorm_backward(_dev(d_norm2, io), x1d, _dev(wn, torch.float32), EPS,
                                      d_residual=_dev(d_out, io))
        proj["dy"] = dx1d
        d_attn = eng_p.proj_backward(ad, [proj], rank)
        torch.cuda.synchronize()
        # oracle composition on the values the library stored between the steps
        po_ref = oracle.proj_forward(attn, wo, bo, a, b, s)
        x1_ref = r(x + r(po_ref))
        _, n2_ref = oracle.rmsnorm_forward(x1_ref, wn, EPS)
        dx1_ref = oracle.rmsnorm_backward(d_norm2, x1_ref, wn, EPS, d_residual=d_out)
        dattn_ref, ga_ref, gb_ref = oracle.proj_backward(attn, r(dx1_ref), wo, a, b, s)
        gate = BF16_GATE if bf16 else FP32_GATE
        errs = {"o_proj": oracle.max_rel_err(po.float().cpu().numpy(), po_ref),
                "norm2X": oracle.max_rel_err(n2d.float().cpu().numpy(), n2_ref),
                "dX1": oracle.max_rel_err(dx1d.float().cpu().numpy(), dx1_ref),
                "dAttnOut": oracle.max_rel_err(d_attn.float().cpu().numpy(), dattn_ref),
                "grad_A": oracle.max_rel_err(proj["grad_a"].cpu().numpy(), ga_ref),
                "grad_B": oracle.max_rel_err(proj["grad_b"].cpu().numpy(), gb_ref)}
        _say(f"  [o-block {'bf16' if bf16 else 'fp32'}] "
             + " ".join(f"{k}={v:.2e}" for k, v in errs.items()) + f" (gate {gate:g})")
        for k, v in errs.items():
            assert v <= gate, k
    finally:
        eng_p.close()
