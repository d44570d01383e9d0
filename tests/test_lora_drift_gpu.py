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
import functools
import sys
from dataclasses import dataclass

import numpy as np
import pytest

import glacier_attn as ga
import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DRIFT_GATE = 1e-3
STEPS = 10


@dataclass(frozen=True)
class Block:
    hidden: int
    hq: int
    hkv: int
    d: int
    rank: int
    theta: float
    vocab: int = 0  # > 0: cross-entropy loss over this many tokens
    lr: float = 1e-2
    scaling: float = 1.0  # LoRA delta = scaling * A B


QWEN05B = Block(896, 14, 2, 64, 8, 1.0e6)
# the reference's defaults: LoraConfig rank 16, alpha 32 (scaling 2),
# TrainingArguments learning rate 2e-4, weight decay 0.01
QWEN7B_CE = Block(3584, 28, 4, 128, 16, 1.0e6, vocab=2048, lr=2e-4, scaling=2.0)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class OracleAttention(torch.autograd.Function):
    """The fp32 CPU path: oracle.layer_fwd_bwd_varlen on the packed rows."""

    @staticmethod
    def forward(ctx, q, k, v, cu, blk):
        T = q.shape[0]
        qn = q.detach().reshape(T, blk.hq, blk.d).numpy()
        kn = k.detach().reshape(T, blk.hkv, blk.d).numpy()
        vn = v.detach().reshape(T, blk.hkv, blk.d).numpy()
        res = oracle.layer_fwd_bwd_varlen(qn, kn, vn, np.zeros_like(qn), cu, blk.theta)
        ctx.inputs = (qn, kn, vn)
        ctx.cu, ctx.blk = cu, blk
        return torch.from_numpy(res["out"]).reshape(T, blk.hq * blk.d)

    @staticmethod
    def backward(ctx, d_out):
        qn, kn, vn = ctx.inputs
        blk = ctx.blk
        T = qn.shape[0]
        dO = np.ascontiguousarray(d_out.reshape(T, blk.hq, blk.d).numpy(), dtype=np.float32)
        res = oracle.layer_fwd_bwd_varlen(qn, kn, vn, dO, ctx.cu, blk.theta)
        return (torch.from_numpy(res["dq"]).reshape(T, -1),
                torch.from_numpy(res["dk"]).reshape(T, -1),
                torch.from_numpy(res["dv"]).reshape(T, -1), None, None)


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


class OracleCrossEntropy(torch.autograd.Function):
    """FusedCrossEntropyLoss.ComputeLossAndGradients through oracle/ce_oracle.c:
    mean over the rows of (logsumexp(h W^T) - target logit), and d loss / d h."""

    @staticmethod
    def forward(ctx, h, w_lm, targets):
        loss, n_valid, d_h = oracle.ce_loss(h.detach().numpy(), targets, w_lm)
        assert n_valid == h.shape[0]
        ctx.d_h = torch.from_numpy(d_h)
        return torch.tensor(loss, dtype=torch.float32)

    @staticmethod
    def backward(ctx, g):
        return ctx.d_h * g, None, None


def _weights(blk, T, seed):
    gen = torch.Generator().manual_seed(seed)
    H, q_out, kv_out = blk.hidden, blk.hq * blk.d, blk.hkv * blk.d
    w = {
        "x": torch.randn(T, H, generator=gen),
        "Wq": torch.randn(H, q_out, generator=gen) / H ** 0.5,
        "Wk": torch.randn(H, kv_out, generator=gen) / H ** 0.5,
        "Wv": torch.randn(H, kv_out, generator=gen) / H ** 0.5,
        "Wo": torch.randn(q_out, H, generator=gen) / q_out ** 0.5,
        "Aq": torch.randn(H, blk.rank, generator=gen) / H ** 0.5,
        "Av": torch.randn(H, blk.rank, generator=gen) / H ** 0.5,
    }
    if blk.vocab:
        # LM head [V][H] (GGUF row order) and next-token targets
        w["W_lm"] = np.ascontiguousarray(
            (torch.randn(blk.vocab, H, generator=gen) / H ** 0.5).numpy())
        w["targets"] = torch.randint(0, blk.vocab, (T,), generator=gen).numpy().astype(np.int32)
    else:
        w["target"] = torch.randn(T, H, generator=gen)
    return w


def _loss(blk, w, o):
    h = o @ w["Wo"]
    if blk.vocab:
        return OracleCrossEntropy.apply(h, w["W_lm"], w["targets"])
    return ((h - w["target"]) ** 2).mean()


def train(attention, blk, T, seed=0):
    """10 AdamW steps on the LoRA adapters; returns the loss before each step."""
    w = _weights(blk, T, seed)
    x = w["x"]
    Aq = w["Aq"].clone().requires_grad_()
    Av = w["Av"].clone().requires_grad_()
    Bq = torch.zeros(blk.rank, blk.hq * blk.d, requires_grad=True)
    Bv = torch.zeros(blk.rank, blk.hkv * blk.d, requires_grad=True)
    opt = torch.optim.AdamW([Aq, Bq, Av, Bv], lr=blk.lr, weight_decay=0.01)
    losses = []
    for _ in range(STEPS):
        q = x @ (w["Wq"] + blk.scaling * (Aq @ Bq))
        k = x @ w["Wk"]
        v = x @ (w["Wv"] + blk.scaling * (Av @ Bv))
        o = attention(q, k, v)
        loss = _loss(blk, w, o)
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
LAYOUTS_7B = {"single_s256": [256], "packed_100_156": [100, 156]}


def _cu(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


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
