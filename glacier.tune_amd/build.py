"""Builds libglacier_attn.so (gfx950) in place with hipcc.

    python glacier.tune_amd/build.py
    python glacier.tune_amd/build.py --stamps OUT.so   # profiling build

The profiling build defines GLACIER_PHASE_STAMPS: every workgroup records
wall-clock stamps at the phases of its kernel (GL_STAMP in attn_common.hpp),
readable with glacier_attn_debug_stamps().  It is written to OUT.so, never
over the product library.

Every HIP translation unit is compiled with the packed-fp32 target feature
disabled (-Xclang -target-feature -Xclang -packed-fp32-ops): the compiler
then never forms v_pk_{add,mul,fma}_f32 from plain float code.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libglacier_attn.so")
OBJDIR = os.path.join(HERE, "_build")

# source -> extra hipcc flags.  -amdgpu-mfma-vgpr-form: the MFMAs the
# compiler emits write VGPRs (their results feed VALU code); in attn_fwd.hip,
# attn_bwd.hip and attn_bwd3.hip the long-lived accumulators are pinned to
# AGPRs by inline assembly.  In attn_kernels.hip (the 16-row kernels) it
# leaves the bf16 head_dim 64/128 instances instruction-for-instruction
# unchanged and made steady-state steps faster at 256
# (66.3 -> 63.4 us, 8/2 heads S=512), 96 (52.5 -> 51.0 us) and in the fp32
# mode (161.3 -> 158.5 us at the Qwen2.5-7B S=512 shape).  Preload count N: the
# first N arguments of each kernel of the file (as many as fit in 14 dwords)
# arrive preloaded in SGPRs, so its first loads need no kernarg-segment round
# trip; the kernels take the arguments they need first in front.
# attn_kernels.hip: the head_dim 256 backward asks for more full unrolling
# than the compiler grants (it runs those loops rolled), which it reports as
# a failed pass.
PRELOAD = ("-mllvm", "-amdgpu-kernarg-preload-count=9")
SOURCES = {
    "attn_kernels.hip": ("-Wno-pass-failed", "-mllvm", "-amdgpu-mfma-vgpr-form", *PRELOAD),
    "attn_fwd.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form", *PRELOAD),
    "attn_bwd.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "attn_bwd3.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-kernarg-preload-count=10"),
    "attn_noalloc.hip": (),
    "attn_pad.hip": (),
    "blas_lt.cpp": (),
    "proj_lora.hip": (),
    "proj_gemm.hip": (),
    "rmsnorm.hip": (),
    "lmhead.hip": (),
    "lora_file.cpp": (),
    "engine.cpp": (),
}
COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libglacier_attn.so)")


def _compile(src: str, objdir: str = OBJDIR, extra: tuple = ()) -> str:
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = False, out: str = OUT, stamps: bool = False) -> str:
    objdir = OBJDIR + ("_stamps" if stamps else "")
    extra = ("-DGLACIER_PHASE_STAMPS",) if stamps else ()
    os.makedirs(objdir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda src: _compile(src, objdir, extra + SOURCES[src]), SOURCES))
    tmp = out + ".tmp"
    # hipBLASLt runs the LM head's logits GEMMs (lmhead.hip)
    rocm_lib = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(hipcc()))), "lib")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp,
           "-L" + rocm_lib, "-Wl,-rpath," + rocm_lib, "-lhipblaslt"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stderr)
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--stamps":
        target = os.path.abspath(sys.argv[2])
        if target == OUT:
            sys.exit("--stamps must not overwrite the product library")
        build(verbose=True, out=target, stamps=True)
    else:
        build(verbose=True)
