"""Loss drift over 10 LoRA steps: the library's attention against the CPU oracle.

Gate: in the bf16-MFMA mode the training loss may
drift from the fp32 CPU path by at most 1e-3 over 10 LoRA steps.  The
reference trains LoRA adapters through this attention path
(TransformerBlock.cs:444-485 forward, 731-741 backward; the loop is
GgufLoraModel.cs:436-557).  One attention block is trained twice from the
same seed:

    q = x (Wq + s Aq Bq),  k = x Wk,  v = x (Wv + s Av Bv)  LoRA on q, v
    o = attention(q, k, v)                                   RoPE + causal GQA
    loss = mean((o Wo - target)^2)                           (MSE harness), or
    loss = CE(o Wo, W_lm, targets)                           (cross-entropy harness)
    AdamW on Aq Bq Av Bv

once with attention through libglacier_attn.so on the GPU and once through the
fp32 oracle on the CPU.  Everything else (projections, loss, optimiser) is the
same float32 code on the CPU in both runs, so the loss difference at each step
measures the attention path alone, including how its errors feed back through
the weight updates.  Bq and Bv start at zero (the usual LoRA init), so step 0's
loss is the frozen model's.

Shapes: Qwen2.5-0.5B's attention (hidden 896, 14 Q / 2 KV heads, head_dim 64)
with the MSE loss (rank 8, s = 1, learning rate 1e-2), and Qwen2.5-7B's
(hidden 3584, 28 Q / 4 KV heads, head_dim 128) with the reference's
cross-entropy, the pinned oracle/ce_oracle.c (FusedCrossEntropyLoss.
ComputeLossAndGradients) over a 2048-token synthetic vocabulary (the
152064-row LM head of the real model is outside this path), at the
reference's default hyperparameters (LoraConfig.cs:9-10 rank 16, alpha 32;
TrainingArguments.cs:8,25 learning rate 2e-4, weight decay 0.01).

The checkpoint test writes the adapters at step 5 through the 'LORA' v1 file
(glacier_lora_save, names blk.0.attn_q.lora_a.weight ... as ITuneBlock.cs:32-33
writes them), reads them back through glacier_lora_open/_read into fresh
parameters and resumes: steps 6-10 must equal an uninterrupted run bit for bit.
The optimiser's moments are carried over in memory, since the reference's
adapter file holds only the adapters (GgufLoraModel.cs:607-664).
"""
import copy
import dataclasses
import functools
import sys

import numpy as np
import pytest

import glacier_attn as ga
from lora_harness import (DRIFT_GATE, QWEN05B, QWEN7B_CE, STEPS, Block, OracleAttention,  # noqa: F401
                          _cu, _weights, train)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class LibraryAttention(torch.autograd.Function):
    """The library: forward (saving lse, q_rot, k_rot) and backward on the GPU,
    operands in the engine's I/O type (bf16 tensors in the bf16 mode)."""

    @staticmethod
    def forward(ctx, q, k, v, cu, eng, io_dtype, blk):
        T = q.shape[0]
        dev = torch.device("cuda:0")
        qd = q.detach().reshape(T, blk.hq, blk.d).to(dev, io_dtype).contiguous()
        kd = k.detach().reshape(T, blk.hkv, blk.d).to(dev, io_dtype).contiguous()
        vd = v.detach().reshape(T, blk.hkv, blk.d).to(dev, io_dtype).contiguous()
        out, lse, q_rot, k_rot = eng.forward(qd, kd, vd, blk.theta, cu_seqlens=cu, save=True)
        ctx.saved = (q_rot, k_rot, vd, out, lse)
        ctx.cu, ctx.eng, ctx.io_dtype, ctx.blk = cu, eng, io_dtype, blk
        return out.float().cpu().reshape(T, blk.hq * blk.d)

    @staticmethod
    def backward(ctx, d_out):
        q_rot, k_rot, vd, out, lse = ctx.saved
        blk = ctx.blk
        T = q_rot.shape[0]
        dO = d_out.reshape(T, blk.hq, blk.d).to(q_rot.device, ctx.io_dtype).contiguous()
        dq, dk, dv = ctx.eng.backward(dO, q_rot, k_rot, vd, out, lse, blk.theta,
                                      cu_seqlens=ctx.cu)
        return (dq.float().cpu().reshape(T, -1), dk.float().cpu().reshape(T, -1),
                dv.float().cpu().reshape(T, -1), None, None, None, None)


@pytest.fixture(scope="module")
def engines():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    e = {ga.PREC_FP32: ga.GpuAttentionEngine(0, ga.PREC_FP32),
         ga.PREC_BF16: ga.GpuAttentionEngine(0, ga.PREC_BF16)}
    yield e
    for eng in e.values():
        eng.close()


LAYOUTS = {"single_s128": [128], "packed_37_91": [37, 91]}
LAYOUTS_7B = {"single_s256": [256], "packed_100_156": [100, 156]}


@functools.lru_cache(maxsize=4)
def oracle_run(blk, lengths):
    """The fp32 CPU path's losses (shared by the bf16 and fp32 library runs)."""
    cu = _cu(lengths)
    return train(lambda q, k, v: OracleAttention.apply(q, k, v, cu, blk), blk, int(cu[-1]))


def _check_drift(ref, got, what):
    drift = np.abs(got - ref)
    _say(f"  oracle  losses {np.array2string(ref, precision=6)}")
    _say(f"  {what} losses {np.array2string(got, precision=6)}")
    _say(f"  max drift {drift.max():.3e} (gate {DRIFT_GATE:g})")
    assert np.all(np.isfinite(got))
    assert ref[-1] < ref[0], "the harness must actually train (loss falls)"
    assert drift.max() <= DRIFT_GATE


def _drift_case(engines, blk, prec, lengths, tag):
    T = sum(lengths)
    cu = _cu(lengths)
    cu_lib = None if len(lengths) == 1 else cu
    io_dtype = torch.bfloat16 if prec == ga.PREC_BF16 else torch.float32
    _say(f"[{tag}] prec={'bf16' if prec == ga.PREC_BF16 else 'fp32'} lengths={lengths} "
         f"T={T} steps={STEPS}")
    eng = engines[prec]
    ref = oracle_run(blk, tuple(lengths))
    got = train(lambda q, k, v: LibraryAttention.apply(q, k, v, cu_lib, eng, io_dtype, blk),
                blk, T)
    _check_drift(ref, got, "library")


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
@pytest.mark.parametrize("prec", [ga.PREC_BF16, ga.PREC_FP32], ids=["bf16", "fp32"])
def test_lora_loss_drift(engines, prec, layout):
    _drift_case(engines, QWEN05B, prec, LAYOUTS[layout], f"lora-drift {layout}")


@pytest.mark.parametrize("layout", sorted(LAYOUTS_7B))
@pytest.mark.parametrize("prec", [ga.PREC_BF16, ga.PREC_FP32], ids=["bf16", "fp32"])
def test_lora_cross_entropy_drift_qwen7b_shape(engines, prec, layout):
    _drift_case(engines, QWEN7B_CE, prec, LAYOUTS_7B[layout], f"lora-drift CE 7B {layout}")


@pytest.mark.parametrize("layout", sorted(LAYOUTS_7B))
def test_lora_cross_entropy_drift_qwen7b_lr1e2_fp32_mode(engines, layout):
    """Learning rate 1e-2 (50 times the reference's default; the loss falls
    from 7.6 to about 0.01 in 10 steps): the fp32-operand mode within 1e-3.
    In the bf16 mode this case drifts 2-8e-3, and no bf16-tensor path can
    do better: the fp32 oracle itself, given the same bf16-rounded q, k, v
    and dO, drifts 2.1-5.0e-3 (test_lora_harness_cpu.py pins that floor)."""
    blk = dataclasses.replace(QWEN7B_CE, lr=1e-2)
    _drift_case(engines, blk, ga.PREC_FP32, LAYOUTS_7B[layout], f"lora-drift CE 7B lr 1e-2 {layout}")


@pytest.mark.parametrize("layout", sorted(LAYOUTS_7B))
def test_lora_cross_entropy_drift_qwen7b_lr1e3_bf16_mode(engines, layout):
    """Learning rate 1e-3 (5 times the reference's default): the bf16 mode
    within 1e-3 (measured 1.9e-4 and 4.7e-4; the bf16-operand floor of the
    fp32 oracle is 1.5-1.7e-4 here)."""
    blk = dataclasses.replace(QWEN7B_CE, lr=1e-3)
    _drift_case(engines, blk, ga.PREC_BF16, LAYOUTS_7B[layout], f"lora-drift CE 7B lr 1e-3 {layout}")


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
    def forward(ctx, x, Aq, Bq, Av, Bv, eng, io_dtype, w, rank):
        xd = x.detach().to(io_dtype).contiguous()
        projs = [{"w": w["q"], "a": Aq.detach().contiguous(), "b": Bq.detach().contiguous(),
                  "scaling": 1.0},
                 {"w": w["k"]},
                 {"w": w["v"], "a": Av.detach().contiguous(), "b": Bv.detach().contiguous(),
                  "scaling": 1.0}]
        q, k, v = eng.proj_forward(xd, projs, rank)
        ctx.xd, ctx.projs, ctx.eng, ctx.io_dtype, ctx.rank = xd, projs, eng, io_dtype, rank
        return q.float(), k.float(), v.float()

    @staticmethod
    def backward(ctx, dq, dk, dv):
        projs = ctx.projs
        for p, g in zip(projs, (dq, dk, dv)):
            p["dy"] = g.to(ctx.io_dtype).contiguous()
            if "a" in p:
                p["grad_a"] = torch.zeros_like(p["a"])
                p["grad_b"] = torch.zeros_like(p["b"])
        ctx.eng.proj_backward(ctx.xd, projs, ctx.rank)
        return (None, projs[0]["grad_a"], projs[0]["grad_b"], projs[2]["grad_a"],
                projs[2]["grad_b"], None, None, None, None)


class LibraryAttentionDevice(torch.autograd.Function):
    """LibraryAttention with device tensors in and out."""

    @staticmethod
    def forward(ctx, q, k, v, cu, eng, io_dtype, blk):
        T = q.shape[0]
        qd = q.detach().reshape(T, blk.hq, blk.d).to(io_dtype).contiguous()
        kd = k.detach().reshape(T, blk.hkv, blk.d).to(io_dtype).contiguous()
        vd = v.detach().reshape(T, blk.hkv, blk.d).to(io_dtype).contiguous()
        out, lse, q_rot, k_rot = eng.forward(qd, kd, vd, blk.theta, cu_seqlens=cu, save=True)
        ctx.saved = (q_rot, k_rot, vd, out, lse)
        ctx.cu, ctx.eng, ctx.io_dtype, ctx.blk = cu, eng, io_dtype, blk
        return out.float().reshape(T, blk.hq * blk.d)

    @staticmethod
    def backward(ctx, d_out):
        q_rot, k_rot, vd, out, lse = ctx.saved
        blk = ctx.blk
        T = q_rot.shape[0]
        dO = d_out.reshape(T, blk.hq, blk.d).to(ctx.io_dtype).contiguous()
        dq, dk, dv = ctx.eng.backward(dO, q_rot, k_rot, vd, out, lse, blk.theta,
                                      cu_seqlens=ctx.cu)
        return (dq.float().reshape(T, -1), dk.float().reshape(T, -1), dv.float().reshape(T, -1),
                None, None, None, None)


ADAPTER_NAMES = ("blk.0.attn_q.lora_a.weight", "blk.0.attn_q.lora_b.weight",
                 "blk.0.attn_v.lora_a.weight", "blk.0.attn_v.lora_b.weight")


def train_device(eng, io_dtype, cu, T, blk=QWEN05B, seed=0, checkpoint=None, at=5):
    """train() with every tensor on the GPU and the block through the library.
    checkpoint: a file path; after step `at` the adapters go through the
    'LORA' v1 file into fresh parameters and a fresh optimiser that takes the
    old one's state.  Returns (losses, final adapters on the host)."""
    dev = torch.device("cuda:0")
    w0 = _weights(blk, T, seed)
    x, Wo, target = w0["x"].to(dev), w0["Wo"].to(dev), w0["target"].to(dev)
    # base weights as the GGUF row order [out][in], in the engine's I/O type
    w = {n: w0[W].T.contiguous().to(dev, io_dtype) for n, W in (("q", "Wq"), ("k", "Wk"),
                                                                 ("v", "Wv"))}
    params = [w0["Aq"].to(dev), torch.zeros(blk.rank, blk.hq * blk.d, device=dev),
              w0["Av"].to(dev), torch.zeros(blk.rank, blk.hkv * blk.d, device=dev)]
    params = [p.requires_grad_() for p in params]
    opt = torch.optim.AdamW(params, lr=1e-2, weight_decay=0.01)
    losses = []
    for step in range(STEPS):
        if checkpoint is not None and step == at:
            saved = [p.detach().cpu().numpy() for p in params]
            ga.lora_save(checkpoint, 1, blk.rank, float(blk.rank),
                         list(zip(ADAPTER_NAMES, saved)))
            header, records = ga.lora_load(checkpoint)
            assert header == {"version": 1, "layer_count": 1, "rank": blk.rank,
                              "alpha": float(blk.rank), "tensor_count": 4}
            assert [n for n, _ in records] == list(ADAPTER_NAMES)
            for (_, a), s in zip(records, saved):
                assert a.shape == s.shape and np.array_equal(a, s)
            state = copy.deepcopy(opt.state_dict())
            params = [torch.from_numpy(a).to(dev).requires_grad_() for _, a in records]
            opt = torch.optim.AdamW(params, lr=1e-2, weight_decay=0.01)
            opt.load_state_dict(state)
        Aq, Bq, Av, Bv = params
        q, k, v = LibraryProjQKV.apply(x, Aq, Bq, Av, Bv, eng, io_dtype, w, blk.rank)
        o = LibraryAttentionDevice.apply(q, k, v, cu, eng, io_dtype, blk)
        loss = ((o @ Wo - target) ** 2).mean()
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    return np.array(losses), [p.detach().cpu().numpy() for p in params]


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
@pytest.mark.parametrize("prec", [ga.PREC_BF16, ga.PREC_FP32], ids=["bf16", "fp32"])
def test_lora_block_on_device_loss_drift(engines, prec, layout):
    lengths = LAYOUTS[layout]
    T = sum(lengths)
    cu = _cu(lengths)
    cu_lib = None if len(lengths) == 1 else cu
    io_dtype = torch.bfloat16 if prec == ga.PREC_BF16 else torch.float32
    _say(f"[lora-drift device block] prec={'bf16' if prec == ga.PREC_BF16 else 'fp32'} "
         f"layout={layout} T={T} steps={STEPS}")
    ref = oracle_run(QWEN05B, tuple(lengths))
    got, _ = train_device(engines[prec], io_dtype, cu_lib, T)
    _check_drift(ref, got, "device block")


@pytest.mark.parametrize("prec", [ga.PREC_BF16, ga.PREC_FP32], ids=["bf16", "fp32"])
def test_adapter_file_checkpoint_resumes_bitwise(engines, prec, tmp_path):
    """Save at step 5 through the 'LORA' v1 file, reload, resume: steps 6-10
    and the final adapters equal the uninterrupted run's bit for bit."""
    lengths = LAYOUTS["packed_37_91"]
    T = sum(lengths)
    cu = _cu(lengths)
    io_dtype = torch.bfloat16 if prec == ga.PREC_BF16 else torch.float32
    _say(f"[adapter checkpoint] prec={'bf16' if prec == ga.PREC_BF16 else 'fp32'} T={T}")
    straight, final_a = train_device(engines[prec], io_dtype, cu, T)
    path = tmp_path / "adapter_model.bin"
    resumed, final_b = train_device(engines[prec], io_dtype, cu, T, checkpoint=str(path))
    _say(f"  straight {np.array2string(straight, precision=6)}")
    _say(f"  resumed  {np.array2string(resumed, precision=6)}")
    assert path.exists()
    assert np.array_equal(straight, resumed)
    for a, b in zip(final_a, final_b):
        assert np.array_equal(a, b)
    # the file reads back the same through a directory path (LoadAdapter's
    # adapter_model.bin convention)
    _, records = ga.lora_load(str(tmp_path))
    assert [n for n, _ in records] == list(ADAPTER_NAMES)
