"""Parity of the LM-head cross-entropy (glacier_lmhead_loss /
glacier_lmhead_loss_and_grad, include/glacier_lmhead.h) against the CPU oracle
(oracle/ce_oracle.c: FusedCrossEntropyLoss.ComputeLoss /
ComputeLossAndGradients), through the C ABI on device tensors.

Gates (the north star's): fp32 mode relative error <= 1e-4, bf16 mode <= 2e-2,
on the loss and normwise (max|x - ref| / max|ref|) on d_hidden.  In the bf16
mode hidden and W are bf16 tensors and the oracle runs on the same rounded
values in fp32.  At the Qwen2.5-7B shape, and past the 2 GB logits chunk, the
reference is float32 torch products on the GPU of the same (rounded) operands.
"""
import sys

import numpy as np
import pytest

import glacier_attn as ga
import oracle

torch = pytest.importorskip("torch")
pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="the device LM-head path is switched off: its first GPU run "
                            "(fp32, T=32, hidden 896, vocab 151936) faulted with an illegal memory "
                            "access and no cause has been shown yet"),
]

FP32_GATE, BF16_GATE = 1e-4, 2e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def engines():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    e = {ga.PREC_FP32: ga.GpuAttentionEngine(0, ga.PREC_FP32),
         ga.PREC_BF16: ga.GpuAttentionEngine(0, ga.PREC_BF16)}
    yield e
    for eng in e.values():
        eng.close()


def _problem(T, H, V, seed):
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((V, H)) / np.sqrt(H)).astype(np.float32)
    tg = rng.integers(0, V, T).astype(np.int32)
    # dropped rows (the reference's -100 padding and out-of-range ids), the
    # first and last ids, and ids either side of a 4096-wide tile boundary
    special = [-100, V, 0, V - 1, min(4095, V - 1), min(4096, V - 1)]
    tg[: min(T, len(special))] = special[: min(T, len(special))]
    return h, w, tg


def _rel(a, b):
    return abs(a - b) / max(abs(b), 1e-30)


SHAPES = {  # T, H, V
    "tiles_padded_row": (37, 128, 9001),  # 3 vocab tiles, the logits row padded to 9008
    "qwen05b_vocab": (32, 896, 151936),
}


@pytest.mark.parametrize("shape", sorted(SHAPES))
@pytest.mark.parametrize("prec", [ga.PREC_FP32, ga.PREC_BF16], ids=["fp32", "bf16"])
def test_lmhead_matches_oracle(engines, prec, shape):
    T, H, V = SHAPES[shape]
    bf16 = prec == ga.PREC_BF16
    _say(f"[lmhead] prec={'bf16' if bf16 else 'fp32'} shape={shape} T={T} H={H} V={V}")
    h, w, tg = _problem(T, H, V, seed=3)
    if bf16:
        h, w = oracle.round_bf16(h), oracle.round_bf16(w)
    io = torch.bfloat16 if bf16 else torch.float32
    hd = torch.from_numpy(h).to("cuda:0", io).contiguous()
    wd = torch.from_numpy(w).to("cuda:0", io).contiguous()
    eng = engines[prec]
    loss, nv, dh = eng.lmhead_loss_and_grad(hd, tg, wd)
    loss_only, nv2 = eng.lmhead_loss(hd, tg, wd)
    torch.cuda.synchronize()
    ref_loss, ref_nv, ref_dh = oracle.ce_loss(h, tg, w)
    gate = BF16_GATE if bf16 else FP32_GATE
    e_loss, e_dh = _rel(loss, ref_loss), oracle.max_rel_err(dh.float().cpu().numpy(), ref_dh)
    _say(f"  loss {loss:.6f} ref {ref_loss:.6f} err={e_loss:.2e} d_hidden err={e_dh:.2e} "
         f"n_valid={nv} (gate {gate:g})")
    assert nv == nv2 == ref_nv == T - 2
    assert loss_only == loss
    assert e_loss <= gate and e_dh <= gate
    assert torch.count_nonzero(dh[:2]).item() == 0, "dropped rows get zero gradient"


def _torch_ref(hd, tg, wd):
    """float32 torch products on the GPU: (loss, d_hidden)."""
    keep = torch.from_numpy(np.nonzero((tg >= 0) & (tg < wd.shape[0]))[0]).to("cuda:0")
    h = hd.float()[keep]
    W = wd.float()
    logits = h @ W.T
    t = torch.from_numpy(tg).to("cuda:0").long()[keep]
    lse = torch.logsumexp(logits, dim=1)
    loss = (lse - logits.gather(1, t[:, None])[:, 0]).mean().item()
    p = torch.softmax(logits, dim=1)
    p[torch.arange(len(keep), device="cuda:0"), t] -= 1.0
    g = torch.zeros_like(hd, dtype=torch.float32)
    g[keep] = (p @ W) / len(keep)
    return loss, g


@pytest.mark.parametrize("case", ["qwen7b_t512", "two_chunks_t2500"])
def test_lmhead_large_vs_torch(engines, case):
    """Qwen2.5-7B (T=512, hidden 3584, vocab 152064, bf16), and 2500 rows of a
    152064 vocabulary, whose logits take two 2 GB chunks (fp32 mode)."""
    T, H, V, prec = {"qwen7b_t512": (512, 3584, 152064, ga.PREC_BF16),
                     "two_chunks_t2500": (2500, 256, 152064, ga.PREC_FP32)}[case]
    bf16 = prec == ga.PREC_BF16
    _say(f"[lmhead] {case} prec={'bf16' if bf16 else 'fp32'}")
    g = torch.Generator(device="cuda:0").manual_seed(5)
    io = torch.bfloat16 if bf16 else torch.float32
    hd = torch.randn(T, H, device="cuda:0", generator=g).to(io).contiguous()
    wd = (torch.randn(V, H, device="cuda:0", generator=g) / H ** 0.5).to(io).contiguous()
    tg = np.random.default_rng(6).integers(0, V, T).astype(np.int32)
    tg[:7] = -100
    loss, nv, dh = engines[prec].lmhead_loss_and_grad(hd, tg, wd)
    torch.cuda.synchronize()
    ref_loss, ref_dh = _torch_ref(hd, tg, wd)
    gate = BF16_GATE if bf16 else FP32_GATE
    e_loss = _rel(loss, ref_loss)
    e_dh = ((dh.float() - ref_dh).abs().max() / ref_dh.abs().max()).item()
    _say(f"  loss {loss:.6f} ref {ref_loss:.6f} err={e_loss:.2e} d_hidden err={e_dh:.2e} (gate {gate:g})")
    assert nv == T - 7
    assert e_loss <= gate and e_dh <= gate


def test_lmhead_repeatable_and_edge_cases(engines):
    """Bitwise repeatable; no kept row gives loss 0 and a zero gradient; T = 0."""
    eng = engines[ga.PREC_BF16]
    T, H, V = 40, 64, 3000
    h, w, tg = _problem(T, H, V, seed=9)
    hd = torch.from_numpy(h).to("cuda:0", torch.bfloat16).contiguous()
    wd = torch.from_numpy(w).to("cuda:0", torch.bfloat16).contiguous()
    l1, _, d1 = eng.lmhead_loss_and_grad(hd, tg, wd)
    d1 = d1.clone()
    l2, _, d2 = eng.lmhead_loss_and_grad(hd, tg, wd)
    assert l1 == l2 and torch.equal(d1, d2)
    none = np.full(T, -100, np.int32)
    dz = torch.full_like(hd, 7.0)
    l0, n0, dz = eng.lmhead_loss_and_grad(hd, none, wd, d_hidden=dz)
    torch.cuda.synchronize()
    assert l0 == 0.0 and n0 == 0 and torch.count_nonzero(dz).item() == 0
    e = torch.empty((0, H), device="cuda:0", dtype=torch.bfloat16)
    assert eng.lmhead_loss(e, np.zeros(0, np.int32), wd) == (0.0, 0)
