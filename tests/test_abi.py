"""C-ABI checks that need no GPU: the library loads, exports every function
include/glacier_attn.h and include/glacier_qkv.h declare, and rejects bad arguments before it touches
a device (so these run on any CPU host).  No compute call is made here."""
import ctypes
import subprocess

import numpy as np
import pytest

import glacier_attn as ga


def test_library_exports_every_header_function():
    lib = ga.load()
    declared = ga.header_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", ga.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared) <= exported
    # nothing else leaks into the ABI under the library's prefixes
    assert {e for e in exported
            if e.startswith(("glacier_attn_", "glacier_proj_", "glacier_rmsnorm_",
                             "glacier_lmhead_", "glacier_lora_"))} == set(declared)
    assert {"glacier_proj_forward", "glacier_proj_backward"} <= set(declared)


def test_supports_attention_gate():
    # GpuLoraEngine.SupportsAttention (GpuLoraEngine.cs:111-112) equivalent
    assert ga.supports_attention(512, 128)
    assert ga.supports_attention(4096, 64)
    assert ga.supports_attention(1, 128)
    for d in (32, 96, 256):
        assert ga.supports_attention(512, d)
    # other sizes up to 256 run the kernels on padded rows
    for d in (1, 7, 80, 127, 160, 255):
        assert ga.supports_attention(512, d)
    for d in (0, 257, 512, 1024):
        assert not ga.supports_attention(512, d)
    assert not ga.supports_attention(0, 128)
    assert not ga.supports_attention(65537, 128)


def _fwd_host_rc(n, hq, hkv, d, base=1.0e4, ctx=None):
    L = ga.load()
    q = np.zeros((max(n, 1), hq, max(d, 1)), np.float32)
    k = np.zeros((max(n, 1), hkv, max(d, 1)), np.float32)
    p = ga._fptr
    rc = L.glacier_attn_forward_host(ctx, 0, p(q), p(k), p(k), p(q), None, n, hq, hkv, d, base)
    return rc, L.glacier_attn_last_error().decode()


def test_argument_errors_come_before_any_device_work():
    rc, msg = _fwd_host_rc(8, 3, 2, 64)
    assert rc == ga.ERR_INVALID_ARGUMENT and "multiple" in msg
    rc, msg = _fwd_host_rc(8, 2, 2, 2000)
    assert rc == ga.ERR_INVALID_ARGUMENT and "headDim" in msg
    rc, msg = _fwd_host_rc(8, 2, 2, 300)
    assert rc == ga.ERR_UNSUPPORTED and "300" in msg
    rc, msg = _fwd_host_rc(8, 2, 2, 256)  # fp32 operands: 256 is bf16-only
    assert rc == ga.ERR_UNSUPPORTED and "BF16" in msg
    rc, msg = _fwd_host_rc(8, 2, 2, 200)  # padded to 256: bf16-only too
    assert rc == ga.ERR_UNSUPPORTED and "BF16" in msg
    rc, msg = _fwd_host_rc(8, 2, 2, 80)  # runs on padded rows: only the context is missing
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg
    rc, msg = _fwd_host_rc(8, 0, 2, 64)
    assert rc == ga.ERR_INVALID_ARGUMENT
    rc, msg = _fwd_host_rc(8, 2, 2, 64, base=-1.0)
    assert rc == ga.ERR_INVALID_ARGUMENT
    rc, msg = _fwd_host_rc(8, 2, 2, 64)  # a valid shape: only the context is missing
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg


def test_device_descriptor_validation():
    L = ga.load()
    cu = np.array([0, 5, 3, 9], np.int32)
    desc, _keep = ga.GpuAttentionEngine._desc(9, 4, 2, 64, 1e4, ga.PREC_BF16, ga.IO_BF16, cu)
    rc = L.glacier_attn_forward(None, ctypes.byref(desc), None, None, None, None, None, None, None)
    assert rc == ga.ERR_INVALID_ARGUMENT and b"non-decreasing" in L.glacier_attn_last_error()
    desc, _keep = ga.GpuAttentionEngine._desc(10, 4, 2, 64, 1e4, ga.PREC_BF16, ga.IO_BF16,
                                              np.array([0, 4, 9], np.int32))
    rc = L.glacier_attn_forward(None, ctypes.byref(desc), None, None, None, None, None, None, None)
    assert rc == ga.ERR_INVALID_ARGUMENT and b"total_tokens" in L.glacier_attn_last_error()
    desc, _keep = ga.GpuAttentionEngine._desc(10, 4, 2, 64, 1e4, ga.PREC_FP32, ga.IO_BF16, None)
    rc = L.glacier_attn_backward(None, ctypes.byref(desc), *([None] * 9))
    assert rc == ga.ERR_INVALID_ARGUMENT and b"bf16" in L.glacier_attn_last_error()
    desc, _keep = ga.GpuAttentionEngine._desc(70000, 4, 2, 64, 1e4, ga.PREC_BF16, ga.IO_BF16, None)
    rc = L.glacier_attn_forward(None, ctypes.byref(desc), *([None] * 7))
    assert rc == ga.ERR_UNSUPPORTED


def test_noalloc_backward_argument_errors_come_before_any_device_work():
    L = ga.load()
    rc = L.glacier_attn_backward_noalloc(None, None, *([None] * 9))
    assert rc == ga.ERR_INVALID_ARGUMENT and b"desc" in L.glacier_attn_last_error()
    cu = np.array([0, 5, 3, 9], np.int32)
    desc, _keep = ga.GpuAttentionEngine._desc(9, 4, 2, 64, 1e4, ga.PREC_BF16, ga.IO_BF16, cu)
    rc = L.glacier_attn_backward_noalloc(None, ctypes.byref(desc), *([None] * 9))
    assert rc == ga.ERR_INVALID_ARGUMENT and b"non-decreasing" in L.glacier_attn_last_error()
    desc, _keep = ga.GpuAttentionEngine._desc(9, 4, 2, 80, 1e4, ga.PREC_BF16, ga.IO_BF16, None)
    rc = L.glacier_attn_backward_noalloc(None, ctypes.byref(desc), *([None] * 9))
    assert rc == ga.ERR_UNSUPPORTED
    desc, _keep = ga.GpuAttentionEngine._desc(9, 4, 2, 64, 1e4, ga.PREC_BF16, ga.IO_BF16, None)
    rc = L.glacier_attn_backward_noalloc(None, ctypes.byref(desc), *([None] * 9))
    assert rc == ga.ERR_INVALID_ARGUMENT and b"ctx" in L.glacier_attn_last_error()


def test_kernel_names_and_last_error_reset():
    names = ga.kernel_names()
    assert names == ["rope_k", "attn_fwd", "attn_bwd", "attn_bwd_reduce", "rmsnorm_fwd",
                     "rmsnorm_bwd", "attn_bwd_stats"]
    L = ga.load()
    assert L.glacier_attn_kernel_name(99) is None
    _fwd_host_rc(8, 3, 2, 64)
    assert L.glacier_attn_last_error() != b""
    assert L.glacier_attn_supports(8, 64) == 1


def test_no_gpu_context_creation_reports_an_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(ga.GlacierAttnError):
        ga.GpuAttentionEngine(0, ga.PREC_BF16)


def test_python_front_end_rejects_wrong_host_arrays():
    with pytest.raises(TypeError):
        ga._host(np.zeros((2, 2), np.float64), "q")
    with pytest.raises(TypeError):
        ga._host(np.zeros((4, 4), np.float32)[:, ::2], "q")


def _proj_rc(T=8, n_in=16, outs=(8,), rank=4, prec=ga.PREC_BF16, io=ga.IO_BF16, lora=True,
             n_proj=None, backward=False, misaligned=()):
    L = ga.load()
    desc = ga.ProjDesc(T, n_in, rank, prec, io)
    arr = (ga.LoraProj * max(len(outs), 1))()
    # any non-null address: validation fails before it is used (8 for the
    # tensors named in misaligned)
    addr = lambda name: 8 if name in misaligned else 16
    for i, o in enumerate(outs):
        arr[i].w = addr("w")
        arr[i].out_features = o
        arr[i].y = addr("y")
        arr[i].dy = addr("dy")
        arr[i].scaling = 2.0
        if lora:
            arr[i].lora_a = addr("lora_a")
            arr[i].lora_b = addr("lora_b")
    n = len(outs) if n_proj is None else n_proj
    if backward:
        rc = L.glacier_proj_backward(None, ctypes.byref(desc), addr("x"), arr, n, addr("dx"))
    else:
        rc = L.glacier_proj_forward(None, ctypes.byref(desc), addr("x"), arr, n)
    return rc, L.glacier_attn_last_error().decode()


def test_projection_argument_errors_come_before_any_device_work():
    rc, msg = _proj_rc(rank=0)
    assert rc == ga.ERR_INVALID_ARGUMENT and "rank" in msg
    rc, msg = _proj_rc(rank=65)
    assert rc == ga.ERR_INVALID_ARGUMENT and "rank" in msg
    rc, msg = _proj_rc(prec=ga.PREC_FP32, io=ga.IO_BF16)
    assert rc == ga.ERR_INVALID_ARGUMENT and "bf16" in msg
    rc, msg = _proj_rc(outs=(8, 8, 8, 8, 8))
    assert rc == ga.ERR_INVALID_ARGUMENT and "n_proj" in msg
    rc, msg = _proj_rc(n_proj=0)
    assert rc == ga.ERR_INVALID_ARGUMENT and "n_proj" in msg
    rc, msg = _proj_rc(outs=(0,))
    assert rc == ga.ERR_INVALID_ARGUMENT and "out_features" in msg
    rc, msg = _proj_rc(outs=(10,))
    assert rc == ga.ERR_UNSUPPORTED and "multiple of 4" in msg
    rc, msg = _proj_rc(n_in=18)
    assert rc == ga.ERR_UNSUPPORTED and "multiple of 4" in msg
    rc, msg = _proj_rc(T=-1)
    assert rc == ga.ERR_INVALID_ARGUMENT and "total_tokens" in msg
    for name, backward in (("x", False), ("y", False), ("lora_a", False), ("lora_b", False),
                           ("dy", True)):
        rc, msg = _proj_rc(misaligned=(name,), backward=backward)
        assert rc == ga.ERR_UNSUPPORTED and "16-byte aligned" in msg and name in msg, name
    # unused by the call: not checked
    rc, msg = _proj_rc(misaligned=("dy",))
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg
    # no adapter: the rank is not checked; a valid call then needs the context
    rc, msg = _proj_rc(rank=0, lora=False)
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg
    rc, msg = _proj_rc(backward=True)
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg


def _norm_rc(rows=8, n=64, io=ga.IO_BF16, eps=1e-6, backward=False, delta=True, x1=True,
             misaligned=()):
    L = ga.load()
    desc = ga.NormDesc(rows, n, io, eps)
    addr = lambda name: 8 if name in misaligned else 16  # validation fails before use
    if backward:
        rc = L.glacier_rmsnorm_backward(None, ctypes.byref(desc), addr("dy"), addr("x"),
                                        addr("weight"), addr("d_residual"), addr("dx"), None)
    else:
        rc = L.glacier_rmsnorm_forward(None, ctypes.byref(desc), addr("x"),
                                       addr("delta") if delta else None, addr("weight"),
                                       addr("x1") if x1 else None, addr("y"))
    return rc, L.glacier_attn_last_error().decode()


def test_rmsnorm_argument_errors_come_before_any_device_work():
    rc, msg = _norm_rc(rows=-1)
    assert rc == ga.ERR_INVALID_ARGUMENT and "rows" in msg
    rc, msg = _norm_rc(n=0)
    assert rc == ga.ERR_INVALID_ARGUMENT and "n must" in msg
    rc, msg = _norm_rc(io=7)
    assert rc == ga.ERR_INVALID_ARGUMENT and "io dtype" in msg
    for eps in (-1.0, float("nan"), float("inf")):
        rc, msg = _norm_rc(eps=eps)
        assert rc == ga.ERR_INVALID_ARGUMENT and "eps" in msg
    rc, msg = _norm_rc(n=66)
    assert rc == ga.ERR_UNSUPPORTED and "multiple of 4" in msg
    rc, msg = _norm_rc(n=8196)
    assert rc == ga.ERR_UNSUPPORTED and "at most" in msg
    rc, msg = _norm_rc(x1=False)
    assert rc == ga.ERR_INVALID_ARGUMENT and "x1" in msg
    for name in ("x", "delta", "weight", "x1", "y"):
        rc, msg = _norm_rc(misaligned=(name,))
        assert rc == ga.ERR_UNSUPPORTED and "16-byte aligned" in msg and name in msg, name
    for name in ("dy", "x", "weight", "d_residual", "dx"):
        rc, msg = _norm_rc(misaligned=(name,), backward=True)
        assert rc == ga.ERR_UNSUPPORTED and "16-byte aligned" in msg and name in msg, name
    # valid calls then need the context; without delta x1 may be NULL
    rc, msg = _norm_rc(delta=False, x1=False)
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg
    rc, msg = _norm_rc(backward=True)
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg


def _lmhead_rc(T=8, H=64, V=100, prec=ga.PREC_BF16, io=ga.IO_BF16, grad=True, targets=True,
               misaligned=()):
    L = ga.load()
    desc = ga.LmHeadDesc(T, H, V, prec, io)
    addr = lambda name: 8 if name in misaligned else 16  # validation fails before use
    tg = (ctypes.c_int32 * max(T, 1))() if targets else None
    loss = ctypes.c_float(-1.0)
    nv = ctypes.c_int32(-1)
    if grad:
        rc = L.glacier_lmhead_loss_and_grad(None, ctypes.byref(desc), addr("hidden"), tg,
                                            addr("weight"), addr("d_hidden"), ctypes.byref(loss),
                                            ctypes.byref(nv))
    else:
        rc = L.glacier_lmhead_loss(None, ctypes.byref(desc), addr("hidden"), tg, addr("weight"),
                                   ctypes.byref(loss), ctypes.byref(nv))
    return rc, L.glacier_attn_last_error().decode()


def test_lmhead_argument_errors_come_before_any_device_work():
    rc, msg = _lmhead_rc(T=-1)
    assert rc == ga.ERR_INVALID_ARGUMENT and "tokens" in msg
    rc, msg = _lmhead_rc(H=0)
    assert rc == ga.ERR_INVALID_ARGUMENT and "hidden" in msg
    rc, msg = _lmhead_rc(V=0)
    assert rc == ga.ERR_INVALID_ARGUMENT and "vocab" in msg
    rc, msg = _lmhead_rc(prec=ga.PREC_FP32, io=ga.IO_BF16)
    assert rc == ga.ERR_INVALID_ARGUMENT and "bf16" in msg
    rc, msg = _lmhead_rc(targets=False)
    assert rc == ga.ERR_INVALID_ARGUMENT and "targets" in msg
    rc, msg = _lmhead_rc(H=60)
    assert rc == ga.ERR_UNSUPPORTED and "multiple of 8" in msg
    for name in ("hidden", "weight", "d_hidden"):
        rc, msg = _lmhead_rc(misaligned=(name,))
        assert rc == ga.ERR_UNSUPPORTED and "16-byte aligned" in msg and name in msg, name
    rc, msg = _lmhead_rc(grad=False, misaligned=("d_hidden",))  # unused without the gradient
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg
    rc, msg = _lmhead_rc()
    assert rc == ga.ERR_INVALID_ARGUMENT and "ctx" in msg


def test_python_front_end_checks_device_tensors_before_the_abi():
    """Every tensor whose pointer the front end passes is checked against the
    shapes the descriptor promises (shape, dtype, contiguity before device), so
    a mismatched tensor raises TypeError instead of reaching a kernel as an
    out-of-bounds access.  CPU tensors with the wrong shape or dtype show the
    shape/dtype checks; the device check comes last."""
    import torch

    T, hq, hkv, d = 8, 4, 2, 64
    q = torch.zeros(T, hq, d, dtype=torch.bfloat16)
    k = torch.zeros(T, hkv, d, dtype=torch.bfloat16)
    lse = torch.zeros(hq, T)

    def raises(fn, text):
        with pytest.raises(TypeError, match=text):
            fn()

    raises(lambda: ga.check_forward_args(q, k, k[:, :1]), "v must have shape")
    raises(lambda: ga.check_forward_args(q, k, k.float()), "v must be torch.bfloat16")
    raises(lambda: ga.check_forward_args(q, k, k, out=q[:4]), "out must have shape")
    raises(lambda: ga.check_forward_args(q, k, k, lse=lse.T.contiguous()), "lse must have shape")
    raises(lambda: ga.check_forward_args(q, k, k, lse=lse.bfloat16()), "lse must be torch.float32")
    raises(lambda: ga.check_forward_args(q, k, k, k_rot=q), "k_rot must have shape")
    raises(lambda: ga.check_forward_args(q, k, k, q_rot=q.transpose(0, 1).contiguous().transpose(0, 1)),
           "q_rot must be contiguous")
    raises(lambda: ga.check_forward_args(q, k, k), "must be a GPU tensor")  # all shapes fine
    raises(lambda: ga.check_backward_args(q, q, k, k, q, lse[:, :4]), "lse must have shape")
    raises(lambda: ga.check_backward_args(q, q, k, k, q, lse.double()), "lse must be torch.float32")
    raises(lambda: ga.check_backward_args(q, q, k, k, q[:, :2], lse), "out must have shape")
    raises(lambda: ga.check_backward_args(q, q, k, k, q, lse, dk=q), "dk must have shape")
    raises(lambda: ga.check_backward_args(q.float(), q, k, k, q, lse), "d_out must be torch.bfloat16")

    x = torch.zeros(T, 32, dtype=torch.bfloat16)
    w = torch.zeros(16, 32, dtype=torch.bfloat16)
    good = {"w": w, "a": torch.zeros(32, 4), "b": torch.zeros(4, 16), "bias": torch.zeros(16),
            "dy": torch.zeros(T, 16, dtype=torch.bfloat16)}
    raises(lambda: ga.check_proj_args(x, [dict(good, a=torch.zeros(32, 8))], 4, True), r"proj\[0\].a must have shape")
    raises(lambda: ga.check_proj_args(x, [dict(good, b=torch.zeros(16, 4))], 4, True), r"proj\[0\].b must have shape")
    raises(lambda: ga.check_proj_args(x, [dict(good, bias=torch.zeros(15))], 4, True), r"proj\[0\].bias must have shape")
    raises(lambda: ga.check_proj_args(x, [dict(good, grad_a=torch.zeros(32, 4, dtype=torch.float64))], 4, True),
           r"proj\[0\].grad_a must be torch.float32")
    raises(lambda: ga.check_proj_args(x, [dict(good, w=torch.zeros(16, 31, dtype=torch.bfloat16))], 4, True),
           r"proj\[0\].w must have shape")
    raises(lambda: ga.check_proj_args(x, [dict(good, dy=torch.zeros(T, 17, dtype=torch.bfloat16))], 4, True),
           r"proj\[0\].dy must have shape")
    raises(lambda: ga.check_proj_args(x, [dict(good, dy=None)], 4, True), r"proj\[0\].dy is required")
    raises(lambda: ga.check_norm_args(x, torch.zeros(31)), "weight must have shape")
    raises(lambda: ga.check_norm_args(x, torch.zeros(32), torch.zeros(32, dtype=torch.bfloat16)),
           "d_weight must be torch.float32")
