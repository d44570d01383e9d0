"""The LoRA training harness of the loss-drift tests, shared by the GPU drift
tests and the CPU tests of the harness itself.

One attention block is trained for STEPS AdamW steps on its LoRA adapters:

    q = x (Wq + s Aq Bq),  k = x Wk,  v = x (Wv + s Av Bv)  LoRA on q, v
    o = attention(q, k, v)                                   RoPE + causal GQA
    loss = mean((o Wo - target)^2)                           (MSE harness), or
    loss = CE(o Wo, W_lm, targets)                           (cross-entropy harness)

with `attention` a torch autograd function (the CPU oracle's, or the
library's); everything else is the same float32 CPU code in every run.  The
reference trains LoRA adapters through this attention path
(TransformerBlock.cs:444-485 forward, 731-741 backward; the loop is
GgufLoraModel.cs:436-557; cross-entropy FusedCrossEntropyLoss.
ComputeLossAndGradients, restated in oracle/ce_oracle.c).
"""
from dataclasses import dataclass

import numpy as np
import torch

import oracle

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


def _cu(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
