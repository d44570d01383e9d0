"""Python front end of libglacier_attn.so (ctypes; no torch types cross the ABI).

`GpuAttentionEngine` mirrors the attention methods of Glacier.Tune's
GpuLoraEngine with the same names and argument meaning:

    supports_attention(seq_len, head_dim)            GpuLoraEngine.cs:111-112
    forward_attention(layer, q, k, v, out, lse, ...) GpuLoraEngine.Forward.cs:467-512
    backward_attention(layer, dO, q, k, v, out, lse, dq, dk, dv, ...)
                                                     GpuLoraEngine.Backward.cs:414-458

on host float32 numpy arrays, plus `forward` / `backward` on device-resident
torch tensors (passed to the library as raw pointers, enqueued on torch's
current stream), and `proj_forward` / `proj_backward`: the q/k/v projections
with LoRA adapters on the device (include/glacier_qkv.h; GpuLoraEngine.ForwardQKV,
GpuLoraEngine.Forward.cs:205-245, and LoraAdapter.Backward, LoraAdapter.cs:190-247).  Errors raise: InvalidArgument (a ValueError, where the C#
engine throws ArgumentOutOfRangeException), Unsupported (the shape stays on
the CPU path), DeviceError, OutOfMemory.  There is no fallback: if the
library is missing or the device fails, the call raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libglacier_attn.so")
HEADERS = [os.path.join(os.path.dirname(HERE), "include", h)
           for h in ("glacier_attn.h", "glacier_qkv.h", "glacier_norm.h", "glacier_lmhead.h",
                     "glacier_lora_file.h")]

OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_DEVICE, ERR_OUT_OF_MEMORY = 0, 1, 2, 3, 4
PREC_FP32, PREC_BF16 = 0, 1
IO_F32, IO_BF16 = 0, 1


class GlacierAttnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class InvalidArgument(GlacierAttnError, ValueError):
    pass


class Unsupported(GlacierAttnError):
    pass


class DeviceError(GlacierAttnError):
    pass


class OutOfMemory(GlacierAttnError, MemoryError):
    pass


class InvalidData(GlacierAttnError):
    """A file is missing, truncated or malformed (GLACIER_LORA_ERR_DATA)."""


_ERRORS = {ERR_INVALID_ARGUMENT: InvalidArgument, ERR_UNSUPPORTED: Unsupported,
           ERR_DEVICE: DeviceError, ERR_OUT_OF_MEMORY: OutOfMemory, 5: InvalidData}


class Desc(ctypes.Structure):
    _fields_ = [
        ("total_tokens", ctypes.c_int32),
        ("n_seqs", ctypes.c_int32),
        ("cu_seqlens", ctypes.POINTER(ctypes.c_int32)),
        ("n_heads_q", ctypes.c_int32),
        ("n_heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rope_freq_base", ctypes.c_float),
        ("precision", ctypes.c_int32),
        ("io_dtype", ctypes.c_int32),
    ]


class ProjDesc(ctypes.Structure):
    _fields_ = [
        ("total_tokens", ctypes.c_int32),
        ("in_features", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("io_dtype", ctypes.c_int32),
    ]


class NormDesc(ctypes.Structure):
    """glacier_norm_desc (include/glacier_norm.h)."""
    _fields_ = [
        ("rows", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("io_dtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


class LmHeadDesc(ctypes.Structure):
    """glacier_lmhead_desc (include/glacier_lmhead.h)."""
    _fields_ = [
        ("tokens", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("io_dtype", ctypes.c_int32),
    ]


class LoraHeader(ctypes.Structure):
    """glacier_lora_header (include/glacier_lora_file.h)."""
    _fields_ = [
        ("version", ctypes.c_uint32),
        ("layer_count", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("tensor_count", ctypes.c_int32),
    ]


class LoraProj(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("lora_a", ctypes.c_void_p),
        ("lora_b", ctypes.c_void_p),
        ("scaling", ctypes.c_float),
        ("out_features", ctypes.c_int32),
        ("y", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("grad_a", ctypes.c_void_p),
        ("grad_b", ctypes.c_void_p),
    ]


_lib = None


def header_functions() -> list[str]:
    """Names of every function the headers in include/ declare."""
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(glacier_(?:attn|proj|rmsnorm|lmhead|lora)_[a-z_]+)\s*\(", text))
    return sorted(names)


def load():
    """Loads the built library (raises if it is not built: no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python glacier.tune_amd/build.py`")
    L = ctypes.CDLL(LIB_PATH)
    c_int, c_float, vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
    fp = ctypes.POINTER(ctypes.c_float)
    L.glacier_attn_create.argtypes = [c_int, c_int, ctypes.POINTER(vp)]
    L.glacier_attn_destroy.argtypes = [vp]
    L.glacier_attn_destroy.restype = None
    L.glacier_attn_last_error.restype = ctypes.c_char_p
    L.glacier_attn_supports.argtypes = [c_int, c_int]
    L.glacier_attn_forward_host.argtypes = [vp, c_int, fp, fp, fp, fp, fp, c_int, c_int,
                                            c_int, c_int, c_float]
    L.glacier_attn_backward_host.argtypes = [vp, c_int, fp, fp, fp, fp, fp, fp, fp, fp, fp,
                                             c_int, c_int, c_int, c_int, c_float]
    L.glacier_attn_forward.argtypes = [vp, ctypes.POINTER(Desc), vp, vp, vp, vp, vp, vp, vp]
    L.glacier_attn_backward.argtypes = [vp, ctypes.POINTER(Desc), vp, vp, vp, vp, vp, vp, vp,
                                        vp, vp]
    L.glacier_attn_backward_noalloc.argtypes = [vp, ctypes.POINTER(Desc), vp, vp, vp, vp, vp, vp,
                                                vp, vp, vp]
    L.glacier_attn_set_stream.argtypes = [vp, vp]
    L.glacier_attn_use_own_stream.argtypes = [vp]
    L.glacier_attn_synchronize.argtypes = [vp]
    L.glacier_attn_set_kernel_timing.argtypes = [vp, c_int]
    L.glacier_attn_kernel_name.restype = ctypes.c_char_p
    L.glacier_attn_kernel_name.argtypes = [c_int]
    L.glacier_attn_kernel_time.argtypes = [vp, c_int, ctypes.POINTER(ctypes.c_double),
                                           ctypes.POINTER(ctypes.c_int64)]
    L.glacier_proj_forward.argtypes = [vp, ctypes.POINTER(ProjDesc), vp, ctypes.POINTER(LoraProj),
                                       c_int]
    i32p = ctypes.POINTER(ctypes.c_int32)
    L.glacier_lora_save.argtypes = [ctypes.c_char_p, c_int, c_int, c_float, c_int,
                                    ctypes.POINTER(ctypes.c_char_p), i32p, i32p,
                                    ctypes.POINTER(fp)]
    L.glacier_lora_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(LoraHeader),
                                    ctypes.POINTER(vp)]
    L.glacier_lora_next.argtypes = [vp, ctypes.c_char_p, c_int, i32p, i32p]
    L.glacier_lora_read.argtypes = [vp, vp, c_int]
    L.glacier_lora_close.argtypes = [vp]
    L.glacier_lora_close.restype = None
    L.glacier_lmhead_loss.argtypes = [vp, ctypes.POINTER(LmHeadDesc), vp, vp, vp,
                                      ctypes.POINTER(ctypes.c_float), i32p]
    L.glacier_lmhead_loss_and_grad.argtypes = [vp, ctypes.POINTER(LmHeadDesc), vp, vp, vp, vp,
                                               ctypes.POINTER(ctypes.c_float), i32p]
    L.glacier_rmsnorm_forward.argtypes = [vp, ctypes.POINTER(NormDesc), vp, vp, vp, vp, vp]
    L.glacier_rmsnorm_backward.argtypes = [vp, ctypes.POINTER(NormDesc), vp, vp, vp, vp, vp, vp]
    L.glacier_proj_backward.argtypes = [vp, ctypes.POINTER(ProjDesc), vp,
                                        ctypes.POINTER(LoraProj), c_int, vp]
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != OK:
        msg = load().glacier_attn_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, GlacierAttnError)(rc, msg)


def supports_attention(seq_len: int, head_dim: int) -> bool:
    return bool(load().glacier_attn_supports(int(seq_len), int(head_dim)))


def _fptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _host(a, name):
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    return a


def kernel_names() -> list[str]:
    L = load()
    return [L.glacier_attn_kernel_name(i).decode() for i in range(L.glacier_attn_kernel_count())]


def _need(t, name, shape, dtype=None, like=None):
    """Checks a device tensor against what the descriptor promises the kernels
    (shape, dtype, contiguity, device) before its pointer crosses the ABI: a
    mismatched tensor would otherwise become an out-of-bounds device access.
    `like` gives the dtype and device of a reference tensor."""
    if t is None:
        raise TypeError(f"{name} is required")
    if tuple(t.shape) != tuple(shape):
        raise TypeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    want = like.dtype if like is not None else dtype
    if want is not None and t.dtype != want:
        raise TypeError(f"{name} must be {want}, got {t.dtype}")
    if not t.is_contiguous():
        raise TypeError(f"{name} must be contiguous")


def _on_gpu(*named):
    """Every given (name, tensor) on the GPU, on the first one's device."""
    dev = None
    for name, t in named:
        if t is None:
            continue
        if not t.is_cuda:
            raise TypeError(f"{name} must be a GPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise TypeError(f"{name} must be on {dev}, got {t.device}")


def check_forward_args(q, k, v, out=None, lse=None, q_rot=None, k_rot=None):
    """The forward's tensors: q [T,Hq,D], k and v [T,Hkv,D] of q's dtype;
    out and q_rot like q, k_rot like k, lse float32 [Hq,T]."""
    import torch

    if q.dim() != 3 or k.dim() != 3:
        raise TypeError("q must be [T, Hq, D] and k [T, Hkv, D]")
    T, hq, d = q.shape
    hkv = k.shape[1]
    _need(q, "q", (T, hq, d), like=None, dtype=q.dtype)
    _need(k, "k", (T, hkv, d), like=q)
    _need(v, "v", (T, hkv, d), like=q)
    for t, name, shape in ((out, "out", (T, hq, d)), (q_rot, "q_rot", (T, hq, d)),
                           (k_rot, "k_rot", (T, hkv, d))):
        if t is not None:
            _need(t, name, shape, like=q)
    if lse is not None:
        _need(lse, "lse", (hq, T), dtype=torch.float32)
    _on_gpu(("q", q), ("k", k), ("v", v), ("out", out), ("lse", lse), ("q_rot", q_rot),
            ("k_rot", k_rot))


def check_backward_args(d_out, q_rot, k_rot, v, out, lse, dq=None, dk=None, dv=None):
    """The backward's tensors: d_out, q_rot, out, dq [T,Hq,D]; k_rot, v, dk,
    dv [T,Hkv,D], all of q_rot's dtype; lse float32 [Hq,T]."""
    import torch

    if q_rot.dim() != 3 or k_rot.dim() != 3:
        raise TypeError("q_rot must be [T, Hq, D] and k_rot [T, Hkv, D]")
    T, hq, d = q_rot.shape
    hkv = k_rot.shape[1]
    _need(q_rot, "q_rot", (T, hq, d), dtype=q_rot.dtype)
    for t, name, shape in ((d_out, "d_out", (T, hq, d)), (out, "out", (T, hq, d)),
                           (k_rot, "k_rot", (T, hkv, d)), (v, "v", (T, hkv, d)),
                           (dq, "dq", (T, hq, d)), (dk, "dk", (T, hkv, d)), (dv, "dv", (T, hkv, d))):
        if t is not None or name in ("d_out", "out", "k_rot", "v"):
            _need(t, name, shape, like=q_rot)
    _need(lse, "lse", (hq, T), dtype=torch.float32)
    _on_gpu(("q_rot", q_rot), ("d_out", d_out), ("out", out), ("k_rot", k_rot), ("v", v),
            ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv))


def check_proj_args(x, projs, rank, backward):
    """x [T, in]; per projection w [out, in] of x's dtype, float32 bias
    [out], lora a [in, rank], b [rank, out], grad_a/grad_b like a/b, and y
    (forward) or dy (backward) [T, out] of x's dtype."""
    import torch

    if x.dim() != 2:
        raise TypeError("x must be [T, in]")
    T, n_in = x.shape
    _need(x, "x", (T, n_in), dtype=x.dtype)
    for i, pr in enumerate(projs):
        w = pr.get("w")
        if w is None or w.dim() != 2:
            raise TypeError(f"proj[{i}].w must be a [out, in] tensor")
        n_out = w.shape[0]
        _need(w, f"proj[{i}].w", (n_out, n_in), like=x)
        f32 = {"bias": (n_out,), "a": (n_in, rank), "b": (rank, n_out),
               "grad_a": (n_in, rank), "grad_b": (rank, n_out)}
        for key, shape in f32.items():
            if pr.get(key) is not None:
                _need(pr[key], f"proj[{i}].{key}", shape, dtype=torch.float32)
        io = "dy" if backward else "y"
        if backward or pr.get(io) is not None:
            _need(pr.get(io), f"proj[{i}].{io}", (T, n_out), like=x)
    _on_gpu(("x", x), *[(f"proj[{i}].{key}", pr.get(key)) for i, pr in enumerate(projs)
                        for key in ("w", "bias", "a", "b", "grad_a", "grad_b", "y", "dy")])


def check_norm_args(x, weight, d_weight=None):
    """weight (and d_weight) float32 [n] for x [rows, n]."""
    import torch

    n = x.shape[1]
    _need(weight, "weight", (n,), dtype=torch.float32)
    if d_weight is not None:
        _need(d_weight, "d_weight", (n,), dtype=torch.float32)
    _on_gpu(("x", x), ("weight", weight), ("d_weight", d_weight))


class GpuAttentionEngine:
    """One library context: a device, a stream and grow-only scratch."""

    def __init__(self, device_ordinal: int = 0, precision: int = PREC_BF16):
        L = load()
        h = ctypes.c_void_p()
        _check(L.glacier_attn_create(int(device_ordinal), int(precision), ctypes.byref(h)))
        self._h = h
        self.precision = precision

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().glacier_attn_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def supports_attention(seq_len: int, head_dim: int) -> bool:
        return supports_attention(seq_len, head_dim)

    # ---- host (numpy float32) entry points -------------------------------
    def forward_attention(self, layer_index, q, k, v, attn_out, attn_lse, seq_len,
                          n_heads_q, n_heads_kv, head_dim, rope_freq_base):
        """In place like the C# engine: attn_out written; with attn_lse given,
        q/k become post-RoPE and attn_lse [Hq, S] is written."""
        for a, n in ((q, "q"), (k, "k"), (v, "v"), (attn_out, "attn_out")):
            _host(a, n)
        if attn_lse is not None:
            _host(attn_lse, "attn_lse")
        _check(load().glacier_attn_forward_host(
            self._h, int(layer_index), _fptr(q), _fptr(k), _fptr(v), _fptr(attn_out),
            _fptr(attn_lse), int(seq_len), int(n_heads_q), int(n_heads_kv), int(head_dim),
            float(rope_freq_base)))

    def backward_attention(self, layer_index, d_attn_out, q, k, v, attn_out, attn_lse, dq, dk,
                           dv, seq_len, n_heads_q, n_heads_kv, head_dim, rope_freq_base):
        for a, n in ((d_attn_out, "d_attn_out"), (q, "q"), (k, "k"), (v, "v"),
                     (attn_out, "attn_out"), (attn_lse, "attn_lse"), (dq, "dq"), (dk, "dk"),
                     (dv, "dv")):
            _host(a, n)
        _check(load().glacier_attn_backward_host(
            self._h, int(layer_index), _fptr(d_attn_out), _fptr(q), _fptr(k), _fptr(v),
            _fptr(attn_out), _fptr(attn_lse), _fptr(dq), _fptr(dk), _fptr(dv), int(seq_len),
            int(n_heads_q), int(n_heads_kv), int(head_dim), float(rope_freq_base)))

    # ---- device (torch tensor) entry points -------------------------------
    @staticmethod
    def _desc(T, hq, hkv, d, base, precision, io, cu):
        desc = Desc()
        desc.total_tokens = int(T)
        desc.n_heads_q, desc.n_heads_kv, desc.head_dim = int(hq), int(hkv), int(d)
        desc.rope_freq_base = float(base)
        desc.precision, desc.io_dtype = int(precision), int(io)
        keep = None
        if cu is None:
            desc.n_seqs = 1
            desc.cu_seqlens = None
        else:
            keep = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
            desc.n_seqs = len(keep) - 1
            desc.cu_seqlens = keep.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        return desc, keep

    def _bind_stream(self):
        import torch

        _check(load().glacier_attn_set_stream(self._h, ctypes.c_void_p(
            torch.cuda.current_stream().cuda_stream)))

    @staticmethod
    def _ptr(t):
        return None if t is None else ctypes.c_void_p(t.data_ptr())

    @staticmethod
    def _io_of(t):
        import torch

        if t.dtype == torch.float32:
            return IO_F32
        if t.dtype == torch.bfloat16:
            return IO_BF16
        raise TypeError(f"unsupported tensor dtype {t.dtype}")

    def forward(self, q, k, v, rope_freq_base, precision=None, cu_seqlens=None, save=True,
                out=None, lse=None, q_rot=None, k_rot=None):
        """q [T,Hq,D], k/v [T,Hkv,D] (pre-RoPE, on the GPU, float32 or bfloat16).
        Returns (out, lse, q_rot, k_rot); the last three are None unless save."""
        import torch

        prec = self.precision if precision is None else precision
        check_forward_args(q, k, v, out, lse if save else None, q_rot if save else None,
                           k_rot if save else None)
        T, hq, d = q.shape
        hkv = k.shape[1]
        io = self._io_of(q)
        out = torch.empty_like(q) if out is None else out
        if save:
            lse = torch.empty((hq, T), dtype=torch.float32, device=q.device) if lse is None else lse
            q_rot = torch.empty_like(q) if q_rot is None else q_rot
            k_rot = torch.empty_like(k) if k_rot is None else k_rot
        else:
            lse = q_rot = k_rot = None
        desc, _keep = self._desc(T, hq, hkv, d, rope_freq_base, prec, io, cu_seqlens)
        self._bind_stream()
        _check(load().glacier_attn_forward(self._h, ctypes.byref(desc), self._ptr(q),
                                           self._ptr(k), self._ptr(v), self._ptr(out),
                                           self._ptr(lse), self._ptr(q_rot), self._ptr(k_rot)))
        return out, lse, q_rot, k_rot

    def backward(self, d_out, q_rot, k_rot, v, out, lse, rope_freq_base, precision=None,
                 cu_seqlens=None, dq=None, dk=None, dv=None):
        """Returns (dq, dk, dv); dq/dk w.r.t. the pre-RoPE q/k."""
        import torch

        prec = self.precision if precision is None else precision
        check_backward_args(d_out, q_rot, k_rot, v, out, lse, dq, dk, dv)
        T, hq, d = q_rot.shape
        hkv = k_rot.shape[1]
        io = self._io_of(q_rot)
        dq = torch.empty_like(q_rot) if dq is None else dq
        dk = torch.empty_like(k_rot) if dk is None else dk
        dv = torch.empty_like(v) if dv is None else dv
        desc, _keep = self._desc(T, hq, hkv, d, rope_freq_base, prec, io, cu_seqlens)
        self._bind_stream()
        _check(load().glacier_attn_backward(self._h, ctypes.byref(desc), self._ptr(d_out),
                                            self._ptr(q_rot), self._ptr(k_rot), self._ptr(v),
                                            self._ptr(out), self._ptr(lse), self._ptr(dq),
                                            self._ptr(dk), self._ptr(dv)))
        return dq, dk, dv

    def _bound(self, fn, args, desc, keep):
        """A callable that enqueues fn(*args) on the stream bound last."""
        def call():
            rc = fn(*args)
            if rc != OK:
                _check(rc)

        call._keep = (desc, keep)  # the descriptor and cu_seqlens outlive the calls
        call.rebind = self._bind_stream
        return call

    def bind_forward(self, q, k, v, out, rope_freq_base, precision=None, cu_seqlens=None,
                     lse=None, q_rot=None, k_rot=None):
        """forward() on fixed tensors with every argument checked and
        converted once: returns call(), which enqueues glacier_attn_forward on
        torch's current stream (bound now; call.rebind() binds it again).
        Saves lse/q_rot/k_rot when all three are given, none of them
        otherwise.  The tensors must stay alive and in place while it is used."""
        save = lse is not None or q_rot is not None or k_rot is not None
        if save and (lse is None or q_rot is None or k_rot is None):
            raise ValueError("bind_forward saves lse, q_rot and k_rot together")
        check_forward_args(q, k, v, out, lse, q_rot, k_rot)
        prec = self.precision if precision is None else precision
        T, hq, d = q.shape
        desc, keep = self._desc(T, hq, k.shape[1], d, rope_freq_base, prec, self._io_of(q),
                                cu_seqlens)
        self._bind_stream()
        p = self._ptr
        args = (self._h, ctypes.byref(desc), p(q), p(k), p(v), p(out), p(lse), p(q_rot), p(k_rot))
        return self._bound(load().glacier_attn_forward, args, desc, keep)

    def bind_backward(self, d_out, q_rot, k_rot, v, out, lse, dq, dk, dv, rope_freq_base,
                      precision=None, cu_seqlens=None):
        """backward() on fixed tensors with every argument checked and
        converted once (see bind_forward)."""
        check_backward_args(d_out, q_rot, k_rot, v, out, lse, dq, dk, dv)
        prec = self.precision if precision is None else precision
        T, hq, d = q_rot.shape
        desc, keep = self._desc(T, hq, k_rot.shape[1], d, rope_freq_base, prec,
                                self._io_of(q_rot), cu_seqlens)
        self._bind_stream()
        p = self._ptr
        args = (self._h, ctypes.byref(desc), p(d_out), p(q_rot), p(k_rot), p(v), p(out), p(lse),
                p(dq), p(dk), p(dv))
        return self._bound(load().glacier_attn_backward, args, desc, keep)

    def bind_step(self, fwd, bwd, rope_freq_base, precision=None, cu_seqlens=None):
        """A forward + backward on fixed tensors with every argument checked
        and converted once: returns step(), which enqueues glacier_attn_forward
        then glacier_attn_backward on torch's current stream (bound now) with
        the prepared arguments.  fwd = dict(q, k, v, out, lse, q_rot, k_rot),
        bwd = dict(d_out, dq, dk, dv) (q_rot, k_rot, v, out, lse from fwd).
        The tensors must stay alive and in place while step() is used."""
        prec = self.precision if precision is None else precision
        q, k, v = fwd["q"], fwd["k"], fwd["v"]
        check_forward_args(q, k, v, fwd["out"], fwd["lse"], fwd["q_rot"], fwd["k_rot"])
        check_backward_args(bwd["d_out"], fwd["q_rot"], fwd["k_rot"], v, fwd["out"], fwd["lse"],
                            bwd["dq"], bwd["dk"], bwd["dv"])
        T, hq, d = q.shape
        desc, keep = self._desc(T, hq, k.shape[1], d, rope_freq_base, prec, self._io_of(q),
                                cu_seqlens)
        self._bind_stream()
        L, p, h, dp = load(), self._ptr, self._h, ctypes.byref(desc)
        fa = (h, dp, p(q), p(k), p(v), p(fwd["out"]), p(fwd["lse"]), p(fwd["q_rot"]),
              p(fwd["k_rot"]))
        ba = (h, dp, p(bwd["d_out"]), p(fwd["q_rot"]), p(fwd["k_rot"]), p(v), p(fwd["out"]),
              p(fwd["lse"]), p(bwd["dq"]), p(bwd["dk"]), p(bwd["dv"]))
        f, b = L.glacier_attn_forward, L.glacier_attn_backward

        def step():
            """Enqueues on the stream bound last (bind_step binds torch's
            current stream; rebind() binds it again, e.g. under capture)."""
            rc = f(*fa)
            if rc != OK:
                _check(rc)
            rc = b(*ba)
            if rc != OK:
                _check(rc)

        step._keep = (desc, keep)  # the descriptor and cu_seqlens outlive the calls
        step.rebind = self._bind_stream
        return step

    # ---- projections with LoRA adapters (device tensors) ------------------
    @staticmethod
    def _proj_array(projs, x, rank, backward):
        check_proj_args(x, projs, rank, backward)
        arr = (LoraProj * len(projs))()
        p = GpuAttentionEngine._ptr
        for i, pr in enumerate(projs):
            w = pr["w"]
            if not (w.is_cuda and w.is_contiguous() and w.dtype == x.dtype and w.dim() == 2
                    and w.shape[1] == x.shape[1]):
                raise TypeError("w must be a contiguous [out, in] GPU tensor of x's dtype")
            for key in ("bias", "a", "b", "grad_a", "grad_b"):
                t = pr.get(key)
                if t is not None and not (t.is_cuda and t.is_contiguous() and t.dtype.is_floating_point
                                          and t.element_size() == 4):
                    raise TypeError(f"{key} must be a contiguous float32 GPU tensor")
            e = arr[i]
            e.w = p(w).value
            e.bias = None if pr.get("bias") is None else p(pr["bias"]).value
            e.lora_a = None if pr.get("a") is None else p(pr["a"]).value
            e.lora_b = None if pr.get("b") is None else p(pr["b"]).value
            e.scaling = float(pr.get("scaling", 0.0))
            e.out_features = int(w.shape[0])
            e.y = None if pr.get("y") is None else p(pr["y"]).value
            e.dy = None if pr.get("dy") is None else p(pr["dy"]).value
            e.grad_a = None if pr.get("grad_a") is None else p(pr["grad_a"]).value
            e.grad_b = None if pr.get("grad_b") is None else p(pr["grad_b"]).value
        return arr

    def _proj_desc(self, x, rank, precision):
        desc = ProjDesc()
        desc.total_tokens, desc.in_features = int(x.shape[0]), int(x.shape[1])
        desc.rank = int(rank)
        desc.precision = int(self.precision if precision is None else precision)
        desc.io_dtype = self._io_of(x)
        return desc

    def proj_forward(self, x, projs, rank=0, precision=None):
        """x [T, in] (GPU, float32 or bfloat16).  projs: dicts with w [out, in]
        (x's dtype), optional bias [out], a [in, rank], b [rank, out] (float32),
        scaling, and optionally y [T, out] to write.  Returns the list of y."""
        import torch

        if not (x.is_cuda and x.is_contiguous() and x.dim() == 2):
            raise TypeError("x must be a contiguous [T, in] GPU tensor")
        for pr in projs:
            if pr.get("y") is None:
                pr["y"] = torch.empty((x.shape[0], pr["w"].shape[0]), dtype=x.dtype, device=x.device)
        arr = self._proj_array(projs, x, rank, False)
        desc = self._proj_desc(x, rank, precision)
        self._bind_stream()
        _check(load().glacier_proj_forward(self._h, ctypes.byref(desc), self._ptr(x), arr,
                                           len(projs)))
        return [pr["y"] for pr in projs]

    def proj_backward(self, x, projs, rank=0, precision=None, dx=None):
        """projs as for proj_forward with dy [T, out] (x's dtype) and optional
        float32 grad_a [in, rank] / grad_b [rank, out] accumulators (added to).
        Returns dx [T, in] (overwritten)."""
        import torch

        if not (x.is_cuda and x.is_contiguous() and x.dim() == 2):
            raise TypeError("x must be a contiguous [T, in] GPU tensor")
        for pr in projs:
            dy = pr.get("dy")
            if dy is None or not (dy.is_cuda and dy.is_contiguous() and dy.dtype == x.dtype):
                raise TypeError("dy must be a contiguous GPU tensor of x's dtype")
        dx = torch.empty_like(x) if dx is None else dx
        arr = self._proj_array(projs, x, rank, True)
        desc = self._proj_desc(x, rank, precision)
        self._bind_stream()
        _check(load().glacier_proj_backward(self._h, ctypes.byref(desc), self._ptr(x), arr,
                                            len(projs), self._ptr(dx)))
        return dx

    # ---- residual add and RMSNorm (glacier_norm.h) -----------------------
    def _norm_desc(self, x, eps):
        if not (x.is_cuda and x.is_contiguous() and x.dim() == 2):
            raise TypeError("x must be a contiguous [rows, n] GPU tensor")
        desc = NormDesc()
        desc.rows, desc.n = int(x.shape[0]), int(x.shape[1])
        desc.io_dtype = self._io_of(x)
        desc.eps = float(eps)
        return desc

    @staticmethod
    def _like(t, ref, name):
        if t is not None and not (t.is_cuda and t.is_contiguous() and t.shape == ref.shape
                                  and t.dtype == ref.dtype):
            raise TypeError(f"{name} must be a contiguous GPU tensor like x")

    def rmsnorm_forward(self, x, weight, eps, delta=None, x1=None, y=None):
        """x1 = x + delta, y = RMSNorm(x1) weight (delta None: y = RMSNorm(x)
        weight and x1 is None).  x, delta [rows, n] float32 or bfloat16, weight
        [n] float32.  Returns (x1, y)."""
        import torch

        desc = self._norm_desc(x, eps)
        check_norm_args(x, weight)
        for t, name in ((delta, "delta"), (x1, "x1"), (y, "y")):
            self._like(t, x, name)
        y = torch.empty_like(x) if y is None else y
        if delta is not None and x1 is None:
            x1 = torch.empty_like(x)
        self._bind_stream()
        _check(load().glacier_rmsnorm_forward(self._h, ctypes.byref(desc), self._ptr(x),
                                              self._ptr(delta), self._ptr(weight),
                                              self._ptr(x1 if delta is not None else None),
                                              self._ptr(y)))
        return (x1 if delta is not None else None), y

    def rmsnorm_backward(self, dy, x, weight, eps, d_residual=None, dx=None, d_weight=None):
        """dx = RMSNormBackward(dy; x, weight) + d_residual; d_weight (float32
        [n], optional) is accumulated.  Returns dx."""
        import torch

        desc = self._norm_desc(x, eps)
        check_norm_args(x, weight, d_weight)
        if dy is None:
            raise TypeError("dy is required")
        for t, name in ((dy, "dy"), (d_residual, "d_residual"), (dx, "dx")):
            self._like(t, x, name)
        dx = torch.empty_like(x) if dx is None else dx
        self._bind_stream()
        _check(load().glacier_rmsnorm_backward(self._h, ctypes.byref(desc), self._ptr(dy),
                                               self._ptr(x), self._ptr(weight),
                                               self._ptr(d_residual), self._ptr(dx),
                                               self._ptr(d_weight)))
        return dx

    # ---- LM-head cross-entropy (glacier_lmhead.h) -------------------------
    def _lmhead(self, hidden, targets, weight, d_hidden, grad, precision):
        import numpy as np

        for t, name in ((hidden, "hidden"), (weight, "weight")):
            if not (t.is_cuda and t.is_contiguous() and t.dim() == 2):
                raise TypeError(f"{name} must be a contiguous 2-D GPU tensor")
        if weight.dtype != hidden.dtype or weight.shape[1] != hidden.shape[1]:
            raise TypeError("weight must be [vocab, hidden] of hidden's dtype")
        tg = np.ascontiguousarray(np.asarray(targets), np.int32)
        if tg.shape != (hidden.shape[0],):
            raise TypeError("targets must have one entry per row of hidden")
        desc = LmHeadDesc()
        desc.tokens, desc.hidden = int(hidden.shape[0]), int(hidden.shape[1])
        desc.vocab = int(weight.shape[0])
        desc.io_dtype = self._io_of(hidden)
        desc.precision = int(self.precision if precision is None else precision)
        loss = ctypes.c_float()
        nv = ctypes.c_int32()
        tp = tg.ctypes.data_as(ctypes.c_void_p)
        self._bind_stream()
        if grad:
            _check(load().glacier_lmhead_loss_and_grad(self._h, ctypes.byref(desc), self._ptr(hidden),
                                                       tp, self._ptr(weight), self._ptr(d_hidden),
                                                       ctypes.byref(loss), ctypes.byref(nv)))
        else:
            _check(load().glacier_lmhead_loss(self._h, ctypes.byref(desc), self._ptr(hidden), tp,
                                              self._ptr(weight), ctypes.byref(loss), ctypes.byref(nv)))
        return loss.value, nv.value

    def lmhead_loss(self, hidden, targets, weight, precision=None):
        """Mean cross-entropy of softmax(hidden weight^T) against targets (host
        ints; rows outside [0, vocab) dropped).  Returns (loss, n_valid)."""
        return self._lmhead(hidden, targets, weight, None, False, precision)

    def lmhead_loss_and_grad(self, hidden, targets, weight, d_hidden=None, precision=None):
        """As lmhead_loss, plus d_hidden [T, hidden] (overwritten).  Returns
        (loss, n_valid, d_hidden)."""
        import torch

        d_hidden = torch.empty_like(hidden) if d_hidden is None else d_hidden
        loss, nv = self._lmhead(hidden, targets, weight, d_hidden, True, precision)
        return loss, nv, d_hidden

    # ---- instrumentation ---------------------------------------------------
    def set_kernel_timing(self, enable: bool) -> None:
        _check(load().glacier_attn_set_kernel_timing(self._h, 1 if enable else 0))

    def kernel_times(self) -> dict:
        """{kernel name: (total ms, launches)} since timing was enabled."""
        L = load()
        res = {}
        for i, name in enumerate(kernel_names()):
            ms = ctypes.c_double()
            n = ctypes.c_int64()
            _check(L.glacier_attn_kernel_time(self._h, i, ctypes.byref(ms), ctypes.byref(n)))
            res[name] = (ms.value, n.value)
        return res

    def synchronize(self) -> None:
        _check(load().glacier_attn_synchronize(self._h))


# ---- the 'LORA' v1 adapter file (include/glacier_lora_file.h) -------------
ERR_DATA = 5  # GLACIER_LORA_ERR_DATA


def lora_save(path, layer_count, rank, alpha, tensors):
    """Writes adapter_model.bin: tensors is a list of (name, 2-D float32 array)."""
    import numpy as np

    L = load()
    arrs = [np.ascontiguousarray(a, np.float32) for _, a in tensors]
    n = len(arrs)
    names = (ctypes.c_char_p * max(n, 1))(*[nm.encode() for nm, _ in tensors])
    d0 = (ctypes.c_int32 * max(n, 1))(*[a.shape[0] for a in arrs])
    d1 = (ctypes.c_int32 * max(n, 1))(*[a.shape[1] for a in arrs])
    fp = ctypes.POINTER(ctypes.c_float)
    data = (fp * max(n, 1))(*[a.ctypes.data_as(fp) for a in arrs])
    _check(L.glacier_lora_save(os.fsencode(path), int(layer_count), int(rank), float(alpha), n,
                               names, d0, d1, data))


def lora_load(path, transpose=None):
    """Reads an adapter file: returns (header dict, list of (name, array)).
    transpose(name, dim0, dim1) -> bool, if given, picks records to read in the
    other layout ([dim1][dim0])."""
    import numpy as np

    L = load()
    hdr = LoraHeader()
    r = ctypes.c_void_p()
    _check(L.glacier_lora_open(os.fsencode(path), ctypes.byref(hdr), ctypes.byref(r)))
    out = []
    try:
        buf = ctypes.create_string_buffer(4096)
        d0, d1 = ctypes.c_int32(), ctypes.c_int32()
        for _ in range(hdr.tensor_count):
            _check(L.glacier_lora_next(r, buf, len(buf), ctypes.byref(d0), ctypes.byref(d1)))
            name = buf.value.decode()
            tr = bool(transpose and transpose(name, d0.value, d1.value))
            a = np.empty((d1.value, d0.value) if tr else (d0.value, d1.value), np.float32)
            _check(L.glacier_lora_read(r, a.ctypes.data_as(ctypes.c_void_p), 1 if tr else 0))
            out.append((name, a))
    finally:
        L.glacier_lora_close(r)
    header = {"version": hdr.version, "layer_count": hdr.layer_count, "rank": hdr.rank,
              "alpha": hdr.alpha, "tensor_count": hdr.tensor_count}
    return header, out
