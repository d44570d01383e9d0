"""Loss drift over 10 LoRA steps: the library's attention against the CPU oracle.

Gate: in the bf16-MFMA mode the training loss may
drift from the fp32 CPU path by at most 1e-3 over 10 LoRA steps.  The
reference trains LoRA adapters through this attention path
(TransformerBlock.cs:444-485 forward, 731-741 backward); here one attention
block at Qwen2.5-0.5B's attention shape (hidden 896, 14 Q / 2 KV heads,
head_dim 64, theta 1e6) is trained twice from the same seed:

    q = x (Wq + Aq Bq),  k = x Wk,  v = x (Wv + Av Bv)      rank-8 LoRA on q, v
    o = attention(q, k, v)                                   RoPE + causal GQA
    loss = mean((o Wo - target)^2)                           AdamW on Aq Bq Av Bv

once with attention through libglacier_attn.so on the GPU and once through the
fp32 oracle on the CPU.  Everything else (projections, loss, optimiser) is the
same float32 torch code on the CPU in both runs, so the loss difference at each
step measures the attention path alone, including how its errors feed back
through the weight updates.  Bq and Bv start at zero (the usual LoRA init), so
step 0's loss is the frozen model's.
"""
import sys

import numpy as np
import pytest

import glacier_attn as ga
import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DRIFT_GATE = 1e-3
STEPS = 10
HIDDEN, HQ, HKV, D, RANK, THETA = 896, 14, 2, 64, 8, 1.0e6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class OracleAttention(torch.autograd.Function):
    """The fp32 CPU path: oracle.layer_fwd_bwd_varlen on the packed rows."""

    @staticmethod
    def forward(ctx, q, k, v, cu):
        T = q.shape[0]
        qn = q.detach().reshape(T, HQ, D).numpy()
        kn = k.detach().reshape(T, HKV, D).numpy()
        vn = v.detach().reshape(T, HKV, D).numpy()
        res = oracle.layer_fwd_bwd_varlen(qn, kn, vn, np.zeros_like(qn), cu, THETA)
        ctx.inputs = (qn, kn, vn)
        ctx.cu = cu
        return torch.from_numpy(res["out"]).reshape(T, HQ * D)

    @staticmethod
    def backward(ctx, d_out):
        qn, kn, vn = ctx.inputs
        T = qn.shape[0]
        dO = np.ascontiguousarray(d_out.reshape(T, HQ, D).numpy(), dtype=np.float32)
        res = oracle.layer_fwd_bwd_varlen(qn, kn, vn, dO, ctx.cu, THETA)
        return (torch.from_numpy(res["dq"]).reshape(T, -1),
                torch.from_numpy(res["dk"]).reshape(T, -1),
                torch.from_numpy(res["dv"]).reshape(T, -1), None)


class LibraryAttention(torch.autograd.Function):
    """The library: forward (saving lse, q_rot, k_rot) and backward on the GPU,
    operands in the engine's I/O type (bf16 tensors in the bf16 mode)."""

    @staticmethod
    def forward(ctx, q, k, v, cu, eng, io_dtype):
        T = q.shape[0]
        dev = torch.device("cuda:0")
        qd = q.detach().reshape(T, HQ, D).to(dev, io_dtype).contiguous()
        kd = k.detach().reshape(T, HKV, D).to(dev, io_dtype).contiguous()
        vd = v.detach().reshape(T, HKV, D).to(dev, io_dtype).contiguous()
        out, lse, q_rot, k_rot = eng.forward(qd, kd, vd, THETA, cu_seqlens=cu, save=True)
        ctx.saved = (q_rot, k_rot, vd, out, lse)
        ctx.cu, ctx.eng, ctx.io_dtype = cu, eng, io_dtype
        return out.float().cpu().reshape(T, HQ * D)

    @staticmethod
    def backward(ctx, d_out):
        q_rot, k_rot, vd, out, lse = ctx.saved
        T = q_rot.shape[0]
        dO = d_out.reshape(T, HQ, D).to(q_rot.device, ctx.io_dtype).contiguous()
        dq, dk, dv = ctx.eng.backward(dO, q_rot, k_rot, vd, out, lse, THETA, cu_seqlens=ctx.cu)
        return (dq.float().cpu().reshape(T, -1), dk.float().cpu().reshape(T, -1),
                dv.float().cpu().reshape(T, -1), None, None, None)


def train(attention, T, seed=0):
    """10 AdamW steps on the LoRA adapters; returns the loss before each step."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(T, HIDDEN, generator=gen)
    Wq = torch.randn(HIDDEN, HQ * D, generator=gen) / HIDDEN ** 0.5
    Wk = torch.randn(HIDDEN, HKV * D, generator=gen) / HIDDEN ** 0.5
    Wv = torch.randn(HIDDEN, HKV * D, generator=gen) / HIDDEN ** 0.5
    Wo = torch.randn(HQ * D, HIDDEN, generator=gen) / (HQ * D) ** 0.5
    target = torch.randn(T, HIDDEN, generator=gen)
    Aq = (torch.randn(HIDDEN, RANK, generator=gen) / HIDDEN ** 0.5).requires_grad_()
    Av = (torch.randn(HIDDEN, RANK, generator=gen) / HIDDEN ** 0.5).requires_grad_()
    Bq = torch.zeros(RANK, HQ * D, requires_grad=True)
    Bv = torch.zeros(RANK, HKV * D, requires_grad=True)
    opt = torch.optim.AdamW([Aq, Bq, Av, Bv], lr=1e-2, weight_decay=0.01)
    losses = []
    for _ in range(STEPS):
        q = x @ (Wq + Aq @ Bq)
        k = x @ Wk
        v = x @ (Wv + Av @ Bv)
        o = attention(q, k, v)
        loss = ((o @ Wo - target) ** 2).mean()
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return np.array(losses)


@pytest.fixture(scope="module")
def engines():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    e = {ga.PREC_FP32: ga.GpuAttentionEngine(0, ga.PREC_FP32),
         ga.PREC_BF16: ga.GpuAttentionEngine(0, ga.PREC_BF16)}
    yield e
    for eng in e.values():
        eng.close()


LAYOUTS = {"single_s128": [128], "packed_37_91": [37, 91]}


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
@pytest.mark.parametrize("prec", [ga.PREC_BF16, ga.PREC_FP32], ids=["bf16", "fp32"])
def test_lora_loss_drift(engines, prec, layout):
    lengths = LAYOUTS[layout]
    T = sum(lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    cu_lib = None if len(lengths) == 1 else cu
    io_dtype = torch.bfloat16 if prec == ga.PREC_BF16 else torch.float32
    _say(f"[lora-drift] prec={'bf16' if prec == ga.PREC_BF16 else 'fp32'} layout={layout} "
         f"T={T} steps={STEPS}")
    eng = engines[prec]
    ref = train(lambda q, k, v: OracleAttention.apply(q, k, v, cu), T)
    got = train(lambda q, k, v: LibraryAttention.apply(q, k, v, cu_lib, eng, io_dtype), T)
    drift = np.abs(got - ref)
    _say(f"  oracle  losses {np.array2string(ref, precision=6)}")
    _say(f"  library losses {np.array2string(got, precision=6)}")
    _say(f"  max drift {drift.max():.3e} (gate {DRIFT_GATE:g})")
    assert np.all(np.isfinite(got))
    assert ref[-1] < ref[0], "the harness must actually train (loss falls)"
    assert drift.max() <= DRIFT_GATE


# --------------------------------------------------------------------------
# The whole block on the device: q/k/v projections with their LoRA adapters
# through glacier_proj_forward/backward (the device replacement of
# GpuLoraEngine.ForwardQKV + AddLoraDeltaHost and LoraAdapter.Backward),
# attention through the library, loss and AdamW in torch on the GPU; Q, K, V
# and their gradients never leave HBM.  Compared with the same CPU fp32 run as
# above (torch projections, oracle attention).
# --------------------------------------------------------------------------

class LibraryProjQKV(torch.autograd.Function):
    """q = x Wq^T + (x Aq) Bq, k = x Wk^T, v = x Wv^T + (x Av) Bv (scaling 1)."""

    @staticmethod
    def forward(ctx, x, Aq, Bq, Av, Bv, eng, io_dtype, w):
        xd = x.detach().to(io_dtype).contiguous()
        projs = [{"w": w["q"], "a": Aq.detach().contiguous(), "b": Bq.detach().contiguous(),
                  "scaling": 1.0},
                 {"w": w["k"]},
                 {"w": w["v"], "a": Av.detach().contiguous(), "b": Bv.detach().contiguous(),
                  "scaling": 1.0}]
        q, k, v = eng.proj_forward(xd, projs, RANK)
        ctx.xd, ctx.projs, ctx.eng, ctx.io_dtype = xd, projs, eng, io_dtype
        return q.float(), k.float(), v.float()

    @staticmethod
    def backward(ctx, dq, dk, dv):
        projs = ctx.projs
        for p, g in zip(projs, (dq, dk, dv)):
            p["dy"] = g.to(ctx.io_dtype).contiguous()
            if "a" in p:
                p["grad_a"] = torch.zeros_like(p["a"])
                p["grad_b"] = torch.zeros_like(p["b"])
        ctx.eng.proj_backward(ctx.xd, projs, RANK)
        return (None, projs[0]["grad_a"], projs[0]["grad_b"], projs[2]["grad_a"],
                projs[2]["grad_b"], None, None, None)


class LibraryAttentionDevice(torch.autograd.Function):
    """LibraryAttention with device tensors in and out."""

    @staticmethod
    def forward(ctx, q, k, v, cu, eng, io_dtype):
        T = q.shape[0]
        qd = q.detach().reshape(T, HQ, D).to(io_dtype).contiguous()
        kd = k.detach().reshape(T, HKV, D).to(io_dtype).contiguous()
        vd = v.detach().reshape(T, HKV, D).to(io_dtype).contiguous()
        out, lse, q_rot, k_rot = eng.forward(qd, kd, vd, THETA, cu_seqlens=cu, save=True)
        ctx.saved = (q_rot, k_rot, vd, out, lse)
        ctx.cu, ctx.eng, ctx.io_dtype = cu, eng, io_dtype
        return out.float().reshape(T, HQ * D)

    @staticmethod
    def backward(ctx, d_out):
        q_rot, k_rot, vd, out, lse = ctx.saved
        T = q_rot.shape[0]
        dO = d_out.reshape(T, HQ, D).to(ctx.io_dtype).contiguous()
        dq, dk, dv = ctx.eng.backward(dO, q_rot, k_rot, vd, out, lse, THETA, cu_seqlens=ctx.cu)
        return (dq.float().reshape(T, -1), dk.float().reshape(T, -1), dv.float().reshape(T, -1),
                None, None, None)


def train_device(eng, io_dtype, cu, T, seed=0):
    """train() with every tensor on the GPU and the block through the library."""
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(T, HIDDEN, generator=gen)
    Wq = torch.randn(HIDDEN, HQ * D, generator=gen) / HIDDEN ** 0.5
    Wk = torch.randn(HIDDEN, HKV * D, generator=gen) / HIDDEN ** 0.5
    Wv = torch.randn(HIDDEN, HKV * D, generator=gen) / HIDDEN ** 0.5
    Wo = torch.randn(HQ * D, HIDDEN, generator=gen) / (HQ * D) ** 0.5
    target = torch.randn(T, HIDDEN, generator=gen)
    Aq = torch.randn(HIDDEN, RANK, generator=gen) / HIDDEN ** 0.5
    Av = torch.randn(HIDDEN, RANK, generator=gen) / HIDDEN ** 0.5
    x, Wo, target = x.to(dev), Wo.to(dev), target.to(dev)
    # base weights as the GGUF row order [out][in], in the engine's I/O type
    w = {n: W.T.contiguous().to(dev, io_dtype) for n, W in (("q", Wq), ("k", Wk), ("v", Wv))}
    Aq = Aq.to(dev).requires_grad_()
    Av = Av.to(dev).requires_grad_()
    Bq = torch.zeros(RANK, HQ * D, device=dev, requires_grad=True)
    Bv = torch.zeros(RANK, HKV * D, device=dev, requires_grad=True)
    opt = torch.optim.AdamW([Aq, Bq, Av, Bv], lr=1e-2, weight_decay=0.01)
    losses = []
    for _ in range(STEPS):
        q, k, v = LibraryProjQKV.apply(x, Aq, Bq, Av, Bv, eng, io_dtype, w)
        o = LibraryAttentionDevice.apply(q, k, v, cu, eng, io_dtype)
        loss = ((o @ Wo - target) ** 2).mean()
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return np.array(losses)


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
@pytest.mark.parametrize("prec", [ga.PREC_BF16, ga.PREC_FP32], ids=["bf16", "fp32"])
def test_lora_block_on_device_loss_drift(engines, prec, layout):
    lengths = LAYOUTS[layout]
    T = sum(lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    cu_lib = None if len(lengths) == 1 else cu
    io_dtype = torch.bfloat16 if prec == ga.PREC_BF16 else torch.float32
    _say(f"[lora-drift device block] prec={'bf16' if prec == ga.PREC_BF16 else 'fp32'} "
         f"layout={layout} T={T} steps={STEPS}")
    ref = train(lambda q, k, v: OracleAttention.apply(q, k, v, cu), T)
    got = train_device(engines[prec], io_dtype, cu_lib, T)
    drift = np.abs(got - ref)
    _say(f"  cpu path     losses {np.array2string(ref, precision=6)}")
    _say(f"  device block losses {np.array2string(got, precision=6)}")
    _say(f"  max drift {drift.max():.3e} (gate {DRIFT_GATE:g})")
    assert np.all(np.isfinite(got))
    assert drift.max() <= DRIFT_GATE
