"""Writes tests/golden/attn_golden.npz: known-answer vectors for the causal GQA
attention layer (RoPE -> causal softmax attention -> backward -> inverse RoPE).

The expected outputs come from torch's own float64 routines, an implementation
independent of both the reference and this repository's oracle:
  - torch.nn.functional.scaled_dot_product_attention(is_causal=True,
    enable_gqa=True) in float64 for the forward,
  - torch.autograd for every gradient (through the rotation as well),
  - torch.logsumexp over the causally masked scaled scores for lse,
  - the NeoX half-split rotation written out from its definition
    (x_i cos - x_{i+D/2} sin, x_i sin + x_{i+D/2} cos, w_i = base^(-2i/D)),
    with the angle pos * w_i computed in float64.
The reference ships no attention golden vectors (its tests only assert
invariants, KernelTests.cs:9-47 and :99-131), so these pin the oracle at
values.  Inputs are drawn with the oracle's SplitMix64/Box-Muller generator
and stored as float32; the float64 expectations are stored rounded to float32.

Run from the repo root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle  # noqa: E402  (input generator only)

# (name, S, Hq, Hkv, D, rope base)
CASES = [
    ("s4_h2x1_d8", 4, 2, 1, 8, 1.0e4),
    ("s7_h4x2_d16", 7, 4, 2, 16, 1.0e4),
    ("s16_h6x2_d32", 16, 6, 2, 32, 1.0e6),
    ("s24_h14x2_d64", 24, 14, 2, 64, 1.0e6),
    ("s12_h7x1_d128", 12, 7, 1, 128, 5.0e5),
]


def rope(x, base, S, D):
    half = D // 2
    pos = torch.arange(S, dtype=torch.float64)
    w = torch.tensor(base, dtype=torch.float64) ** (-(2.0 * torch.arange(half, dtype=torch.float64)) / D)
    th = pos[:, None] * w[None, :]
    c = torch.cos(th)[:, None, :]
    s = torch.sin(th)[:, None, :]
    x0, x1 = x[..., :half], x[..., half:]
    return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1)


def case(seed0, S, Hq, Hkv, D, base):
    q = oracle.fill_normal((S, Hq, D), seed0 + 1)
    k = oracle.fill_normal((S, Hkv, D), seed0 + 2)
    v = oracle.fill_normal((S, Hkv, D), seed0 + 3)
    dO = oracle.fill_normal((S, Hq, D), seed0 + 4, 0.0, 0.01)
    tq = torch.tensor(q, dtype=torch.float64, requires_grad=True)
    tk = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    tv = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    qr = rope(tq, base, S, D)
    kr = rope(tk, base, S, D)
    # SDPA wants [B, H, S, D]
    o = torch.nn.functional.scaled_dot_product_attention(
        qr.permute(1, 0, 2)[None], kr.permute(1, 0, 2)[None], tv.permute(1, 0, 2)[None],
        is_causal=True, enable_gqa=True)[0].permute(1, 0, 2)
    o.backward(torch.tensor(dO, dtype=torch.float64))
    r = Hq // Hkv
    kk = kr.detach().repeat_interleave(r, dim=1)
    sc = torch.einsum("ihd,jhd->hij", qr.detach(), kk) / np.sqrt(D)
    sc = sc.masked_fill(~torch.tril(torch.ones(S, S, dtype=torch.bool)), float("-inf"))
    lse = torch.logsumexp(sc, dim=-1)
    return dict(q=q, k=k, v=v, dO=dO, base=np.float64(base),
                q_rot=qr.detach().numpy(), k_rot=kr.detach().numpy(),
                out=o.detach().numpy(), lse=lse.numpy(),
                dq=tq.grad.numpy(), dk=tk.grad.numpy(), dv=tv.grad.numpy())


def main():
    data = {}
    for n, (name, S, Hq, Hkv, D, base) in enumerate(CASES):
        res = case(100 * (n + 1), S, Hq, Hkv, D, base)
        for key, val in res.items():
            # float64 results are stored rounded to float32 (a relative change
            # of at most 2^-24, far below every tolerance that reads them)
            if isinstance(val, np.ndarray) and val.dtype == np.float64:
                val = val.astype(np.float32)
            data[f"{name}/{key}"] = val
    data["cases"] = np.array([c[0] for c in CASES])
    path = os.path.join(HERE, "attn_golden.npz")
    np.savez_compressed(path, **data)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
