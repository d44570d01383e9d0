"""TEST INFRASTRUCTURE ONLY: ctypes front end of the C oracle (attn_oracle.c,
lora_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, always as the checker or the timed CPU baseline, never as part of
the product path.

Functions that call into liboracle.so follow the reference loop for loop:
  rope_forward / rope_backward  -> src/Glacier.Tune/Kernels/RoPEKernel.cs:12-105
  attn_forward                  -> src/Glacier.Tune/Kernels/CausalAttentionKernel.cs:17-77
  attn_backward                 -> src/Glacier.Tune/Kernels/CausalAttentionKernel.cs:79-213
  layer_fwd_bwd                 -> the CPU branch of TransformerBlock.cs:444-485 and :731-741
  proj_forward / proj_backward  -> LoraAdapter.Forward / Backward (lora_oracle.c)
The *_fp64 functions are independent brute-force twins in float64 used to pin
the C restatement (they are not a restatement of the reference's loops).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile liboracle.so with oracle/Makefile (gcc is the only tool used)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def use_library(path: str) -> None:
    """Loads the oracle from another build of the same sources (bench.py's
    -march=native copy for the timed CPU baseline) in place of liboracle.so."""
    global _lib, _LIB_PATH
    _LIB_PATH = path
    _lib = None
    lib()


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built: run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        i, f = ctypes.c_int, ctypes.c_float
        vp = ctypes.c_void_p
        L.oracle_rope_forward.argtypes = [_f32p, _f32p, i, i, i, i, f, f, i, vp]
        L.oracle_rope_backward.argtypes = [_f32p, _f32p, i, i, i, i, f, f, i, vp]
        L.oracle_rope_table.argtypes = [_f32p, _f32p, i, i, f]
        L.oracle_attn_forward_lse.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, vp, i, i, i, i]
        L.oracle_attn_backward.argtypes = [_f32p] * 8 + [i, i, i, i]
        L.oracle_attn_backward.restype = i
        L.oracle_layer_fwd_bwd.argtypes = [_f32p] * 10 + [i, i, i, i, f]
        L.oracle_layer_fwd_bwd.restype = i
        L.oracle_layer_fwd_bwd_varlen.argtypes = [_f32p] * 9 + [_i32p, i, i, i, i, f]
        L.oracle_layer_fwd_bwd_varlen.restype = i
        L.oracle_fill_normal.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64, f, f]
        L.oracle_num_threads.restype = i
        L.oracle_proj_forward.argtypes = [_f32p, _f32p, vp, vp, vp, f, _f32p, i, i, i, i]
        L.oracle_proj_backward.argtypes = [_f32p, _f32p, _f32p, vp, vp, f, vp, vp, vp, i, i, i, i]
        L.oracle_rmsnorm_forward.argtypes = [_f32p, vp, _f32p, f, vp, _f32p, i, i]
        L.oracle_rmsnorm_backward.argtypes = [_f32p, _f32p, _f32p, f, vp, _f32p, vp, i, i]
        L.oracle_ce_loss.argtypes = [_f32p, _i32p, _f32p, vp, i, i, i, ctypes.POINTER(ctypes.c_int)]
        L.oracle_ce_loss.restype = f
        L.oracle_set_num_threads.argtypes = [i]
        _lib = L
    return _lib


def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def fill_normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Seeded SplitMix64 -> Box-Muller fp32 samples (the bench/test input generator)."""
    x = np.empty(int(np.prod(shape)), dtype=np.float32)
    lib().oracle_fill_normal(x, x.size, seed, mean, std)
    return x.reshape(shape)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32, on the host."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    nan = np.isnan(x)
    out = r.astype(np.uint32).view(np.float32).reshape(np.shape(x)).copy()
    out[nan] = np.nan
    return out


def set_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def rope_forward(q, k, freq_base, freq_scale=1.0, rope_dim=-1):
    """RoPEKernel.ForwardSequence on copies of q [S,Hq,D], k [S,Hkv,D]."""
    q = _c(q).copy(); k = _c(k).copy()
    S, Hq, D = q.shape; Hkv = k.shape[1]
    lib().oracle_rope_forward(q, k, S, Hq, Hkv, D, freq_base, freq_scale, rope_dim, None)
    return q, k


def rope_backward(dq, dk, freq_base, freq_scale=1.0, rope_dim=-1):
    """RoPEKernel.BackwardSequence on copies of dq, dk."""
    dq = _c(dq).copy(); dk = _c(dk).copy()
    S, Hq, D = dq.shape; Hkv = dk.shape[1]
    lib().oracle_rope_backward(dq, dk, S, Hq, Hkv, D, freq_base, freq_scale, rope_dim, None)
    return dq, dk


def rope_table(S, D, freq_base):
    """cos/sin [S, D/2] exactly as RoPEKernel.cs:62-69 computes them."""
    cs = np.empty((S, D // 2), np.float32); sn = np.empty((S, D // 2), np.float32)
    lib().oracle_rope_table(cs, sn, S, D, freq_base)
    return cs, sn


def attn_forward(q, k, v, want_lse=True):
    """CausalAttentionKernel.Forward: returns (out [S,Hq,D], probs [Hq,S,S], lse [Hq,S])."""
    q = _c(q); k = _c(k); v = _c(v)
    S, Hq, D = q.shape; Hkv = k.shape[1]
    out = np.empty_like(q)
    probs = np.empty((Hq, S, S), np.float32)
    lse = np.empty((Hq, S), np.float32)
    lib().oracle_attn_forward_lse(q, k, v, out, probs, lse.ctypes.data if want_lse else None,
                                  S, Hq, Hkv, D)
    return out, probs, lse


def attn_backward(dO, q, k, v, probs):
    """CausalAttentionKernel.Backward: returns (dq, dk, dv), w.r.t. post-RoPE q/k."""
    dO = _c(dO); q = _c(q); k = _c(k); v = _c(v); probs = _c(probs)
    S, Hq, D = q.shape; Hkv = k.shape[1]
    dq = np.empty_like(q); dk = np.empty_like(k); dv = np.empty_like(v)
    rc = lib().oracle_attn_backward(dO, q, k, v, probs, dq, dk, dv, S, Hq, Hkv, D)
    if rc:
        raise MemoryError("oracle backward workspace allocation failed")
    return dq, dk, dv


def layer_fwd_bwd(q, k, v, dO, freq_base):
    """The reference CPU layer path (TransformerBlock.cs:444-485, 731-741).

    Returns a dict with q_rot, k_rot (post-RoPE, as saved in the state), out,
    lse, and dq, dk (w.r.t. the pre-RoPE inputs) and dv.
    """
    q = _c(q).copy(); k = _c(k).copy(); v = _c(v); dO = _c(dO)
    S, Hq, D = q.shape; Hkv = k.shape[1]
    out = np.empty_like(q); probs = np.empty((Hq, S, S), np.float32)
    lse = np.empty((Hq, S), np.float32)
    dq = np.empty_like(q); dk = np.empty_like(k); dv = np.empty_like(v)
    rc = lib().oracle_layer_fwd_bwd(q, k, v, dO, out, probs, lse, dq, dk, dv,
                                    S, Hq, Hkv, D, freq_base)
    if rc:
        raise MemoryError("oracle backward workspace allocation failed")
    return dict(q_rot=q, k_rot=k, out=out, lse=lse, probs=probs, dq=dq, dk=dk, dv=dv)


def layer_fwd_bwd_varlen(q, k, v, dO, cu_seqlens, freq_base):
    """Packed segments, each run through layer_fwd_bwd on its own rows."""
    q = _c(q).copy(); k = _c(k).copy(); v = _c(v); dO = _c(dO)
    T, Hq, D = q.shape; Hkv = k.shape[1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    out = np.empty_like(q); lse = np.empty((Hq, T), np.float32)
    dq = np.empty_like(q); dk = np.empty_like(k); dv = np.empty_like(v)
    rc = lib().oracle_layer_fwd_bwd_varlen(q, k, v, dO, out, lse, dq, dk, dv, cu,
                                           len(cu) - 1, Hq, Hkv, D, freq_base)
    if rc:
        raise MemoryError("oracle varlen allocation failed")
    return dict(q_rot=q, k_rot=k, out=out, lse=lse, dq=dq, dk=dk, dv=dv)


# ----------------------------------------------------------------------------
# Independent float64 brute force (checkers of the restatement, tiny shapes).
# ----------------------------------------------------------------------------

def rope_fp64(x, freq_base, inverse=False, positions=None):
    """NeoX half-split rotation in float64 from the closed form
    x'_i = x_i cos(p w_i) - x_{i+h} sin(p w_i), x'_{i+h} = x_i sin + x_{i+h} cos,
    w_i = base^(-2i/D)."""
    x = np.asarray(x, np.float64)
    S, H, D = x.shape
    half = D // 2
    pos = np.arange(S, dtype=np.float64) if positions is None else np.asarray(positions, np.float64)
    w = float(freq_base) ** (-(2.0 * np.arange(half)) / D)
    th = pos[:, None] * w[None, :]
    c = np.cos(th)[:, None, :]
    s = np.sin(th)[:, None, :] * (-1.0 if inverse else 1.0)
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


def attn_fp64(q, k, v, dO=None):
    """Causal GQA softmax attention and its exact gradients in float64.

    q [S,Hq,D], k/v [S,Hkv,D] (post-RoPE).  Returns dict(out, lse, P, dq, dk, dv)."""
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64); v = np.asarray(v, np.float64)
    S, Hq, D = q.shape; Hkv = k.shape[1]; r = Hq // Hkv
    scale = 1.0 / np.sqrt(D)
    kk = np.repeat(k, r, axis=1); vv = np.repeat(v, r, axis=1)       # [S,Hq,D]
    s = np.einsum("ihd,jhd->hij", q, kk) * scale                     # [Hq,S,S]
    mask = np.tril(np.ones((S, S), bool))
    s = np.where(mask[None], s, -np.inf)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    z = e.sum(-1, keepdims=True)
    P = e / z
    out = np.einsum("hij,jhd->ihd", P, vv)
    res = dict(out=out, lse=(m + np.log(z))[..., 0], P=P)
    if dO is not None:
        dO = np.asarray(dO, np.float64)
        dP = np.einsum("ihd,jhd->hij", dO, vv)
        Dr = (P * dP).sum(-1, keepdims=True)
        dS = P * (dP - Dr) * scale
        res["dq"] = np.einsum("hij,jhd->ihd", dS, kk)
        dkh = np.einsum("hij,ihd->jhd", dS, q)
        dvh = np.einsum("hij,ihd->jhd", P, dO)
        res["dk"] = dkh.reshape(S, Hkv, r, D).sum(2)
        res["dv"] = dvh.reshape(S, Hkv, r, D).sum(2)
    return res


def layer_fp64(q, k, v, dO, freq_base):
    """The full layer (RoPE, attention, backward, inverse RoPE) in float64."""
    qr = rope_fp64(q, freq_base); kr = rope_fp64(k, freq_base)
    res = attn_fp64(qr, kr, v, dO)
    res["q_rot"], res["k_rot"] = qr, kr
    res["dq"] = rope_fp64(res["dq"], freq_base, inverse=True)
    res["dk"] = rope_fp64(res["dk"], freq_base, inverse=True)
    return res


def _ptr(a):
    return None if a is None else a.ctypes.data


def proj_forward(x, w, bias=None, a=None, b=None, scaling=0.0):
    """LoraAdapter.Forward: y = x W^T + bias + scaling (x A) B.

    x [S,in], w [out,in], bias [out] or None, a [in,r], b [r,out] or None."""
    x = _c(x); w = _c(w)
    S, n_in = x.shape; n_out = w.shape[0]
    bias = None if bias is None else _c(bias)
    a = None if a is None else _c(a); b = None if b is None else _c(b)
    rank = 0 if a is None else a.shape[1]
    y = np.empty((S, n_out), np.float32)
    lib().oracle_proj_forward(x, w, _ptr(bias), _ptr(a), _ptr(b), scaling, y, S, n_in, n_out, rank)
    return y


def proj_backward(x, dy, w, a=None, b=None, scaling=0.0, dx=None, grad_a=None, grad_b=None):
    """LoraAdapter.Backward: dx += dy W + scaling (dy B^T) A^T, grad_a += scaling
    x^T (dy B^T), grad_b += scaling (x A)^T dy.  The accumulators are updated in
    place (zeros are made for those passed as None) and returned."""
    x = _c(x); dy = _c(dy); w = _c(w)
    S, n_in = x.shape; n_out = w.shape[0]
    a = None if a is None else _c(a); b = None if b is None else _c(b)
    rank = 0 if a is None else a.shape[1]
    dx = np.zeros((S, n_in), np.float32) if dx is None else dx
    if a is not None:
        grad_a = np.zeros((n_in, rank), np.float32) if grad_a is None else grad_a
        grad_b = np.zeros((rank, n_out), np.float32) if grad_b is None else grad_b
    for t in (dx, grad_a, grad_b):
        assert t is None or (t.dtype == np.float32 and t.flags["C_CONTIGUOUS"])
    lib().oracle_proj_backward(x, dy, w, _ptr(a), _ptr(b), scaling, _ptr(dx), _ptr(grad_a),
                               _ptr(grad_b), S, n_in, n_out, rank)
    return dx, grad_a, grad_b


def rmsnorm_forward(x, w, eps, delta=None):
    """x1 = x + delta (delta None: x1 = x); y = RMSNorm(x1) w.  x, delta [rows, n],
    w [n].  Returns (x1, y)."""
    x = _c(x); w = _c(w)
    rows, n = x.shape
    delta = None if delta is None else _c(delta)
    x1 = np.empty_like(x)
    y = np.empty_like(x)
    lib().oracle_rmsnorm_forward(x, _ptr(delta), w, eps, _ptr(x1), y, rows, n)
    return x1, y


def rmsnorm_backward(dy, x, w, eps, d_residual=None, d_weight=None):
    """dx = RMSNormBackward(dy; x, w) + d_residual; d_weight (if given) is
    accumulated in place.  Returns dx."""
    dy = _c(dy); x = _c(x); w = _c(w)
    rows, n = x.shape
    d_residual = None if d_residual is None else _c(d_residual)
    assert d_weight is None or (d_weight.dtype == np.float32 and d_weight.flags["C_CONTIGUOUS"])
    dx = np.empty_like(x)
    lib().oracle_rmsnorm_backward(dy, x, w, eps, _ptr(d_residual), dx, _ptr(d_weight), rows, n)
    return dx


def ce_loss(hidden, targets, w, grad=True):
    """FusedCrossEntropyLoss.ComputeLoss / ComputeLossAndGradients: hidden [T, H],
    targets [T] (rows outside [0, V) are dropped), w [V, H].  Returns (loss,
    n_valid, d_hidden or None)."""
    hidden = _c(hidden); w = _c(w)
    targets = np.ascontiguousarray(targets, np.int32)
    T, H = hidden.shape
    V = w.shape[0]
    d = np.empty((T, H), np.float32) if grad else None
    nv = ctypes.c_int(0)
    loss = lib().oracle_ce_loss(hidden, targets, w, _ptr(d), T, H, V, ctypes.byref(nv))
    return float(loss), nv.value, d


def proj_fp64(x, w, bias=None, a=None, b=None, scaling=0.0):
    """float64 twin of proj_forward (matrix products, not the reference's loops)."""
    x = np.asarray(x, np.float64); w = np.asarray(w, np.float64)
    y = x @ w.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    if a is not None:
        y = y + scaling * ((x @ np.asarray(a, np.float64)) @ np.asarray(b, np.float64))
    return y


def max_rel_err(x, ref) -> float:
    """Normwise max relative error max|x - ref| / max|ref| (the parity metric)."""
    x = np.asarray(x, np.float64); ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    if den == 0:
        return float(np.max(np.abs(x)))
    return float(np.max(np.abs(x - ref)) / den)
