"""C-ABI checks that need no GPU: the library loads, exports every function
include/glacier_attn.h declares, and rejects bad arguments before it touches
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
    # nothing else leaks into the ABI under the glacier_attn_ prefix
    assert {e for e in exported if e.startswith("glacier_attn_")} == set(declared)


def test_supports_attention_gate():
    # GpuLoraEngine.SupportsAttention (GpuLoraEngine.cs:111-112) equivalent
    assert ga.supports_attention(512, 128)
    assert ga.supports_attention(4096, 64)
    assert ga.supports_attention(1, 128)
    assert not ga.supports_attention(512, 96)
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
    rc, msg = _fwd_host_rc(8, 2, 2, 96)
    assert rc == ga.ERR_UNSUPPORTED and "96" in msg
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


def test_kernel_names_and_last_error_reset():
    names = ga.kernel_names()
    assert names == ["rope_k", "attn_fwd", "attn_bwd", "attn_bwd_reduce"]
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
