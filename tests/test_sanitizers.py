"""CPU sanitizer builds (no GPU): AddressSanitizer + UndefinedBehaviorSanitizer.

- oracle/*.c, driven by tests/sanitize/oracle_asan_driver.c over edge shapes
  with exactly-sized heap buffers;
- the 'LORA' v1 writer/reader (glacier.tune_amd/csrc/lora_file.cpp), driven
  by tests/sanitize/lora_fuzz.cpp over every truncation, boundary-byte
  changes, hand-made hostile records and random corruptions of a valid file
  (the reference's LoadAdapter reads untrusted files, GgufLoraModel.cs:697-796);
- the library's host code (every source of glacier.tune_amd/csrc, built with
  the sanitizers on hipcc's host pass only), driven by
  tests/sanitize/abi_asan_driver.cpp through the C ABI's argument checks,
  which run before any device work and so need no GPU, and by
  tests/sanitize/lmhead_bounds_driver.cpp, which walks every access of the
  LM-head launch plan (each kernel thread's indices, each GEMM operand's
  stored extent) against its buffers at the shape whose first GPU run
  faulted and four more.

They are built into a temporary directory and run as child processes; any
sanitizer report aborts the child (-fno-sanitize-recover) and fails the test.
"""
import concurrent.futures as cf
import importlib.util
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# the runtimes are linked statically, so the executables need no preloaded
# sanitizer library
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1", "-static-libasan", "-static-libubsan"]


def _have(cc):
    return shutil.which(cc) is not None


def _build(cmd, cwd):
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if res.returncode != 0 and "asan" in (res.stderr + res.stdout).lower():
        pytest.skip("the sanitizer runtime is not installed: " + res.stderr[-300:])
    assert res.returncode == 0, res.stderr


def _run(cmd, env_extra, timeout):
    env = dict(os.environ)
    env.update(env_extra)
    res = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=timeout)
    return res


@pytest.mark.skipif(not _have("gcc"), reason="gcc not found")
def test_oracle_under_asan_and_ubsan(tmp_path):
    src = [os.path.join(ROOT, "oracle", f) for f in
           ("attn_oracle.c", "lora_oracle.c", "norm_oracle.c", "ce_oracle.c")]
    exe = str(tmp_path / "oracle_asan")
    _build(["gcc", *SAN, "-std=gnu11", "-ffp-contract=off", "-fopenmp", *src,
            os.path.join(ROOT, "tests", "sanitize", "oracle_asan_driver.c"), "-lm", "-o", exe],
           str(tmp_path))
    res = _run([exe], {"OMP_NUM_THREADS": "2",
                       "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
                       "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}, 240)
    assert res.returncode == 0, res.stderr[-4000:]
    assert "ORACLE_SANITIZE_OK" in res.stdout
    assert "runtime error" not in res.stderr, res.stderr[-4000:]


@pytest.mark.skipif(not _have("g++"), reason="g++ not found")
def test_adapter_reader_fuzz_under_asan_and_ubsan(tmp_path):
    exe = str(tmp_path / "lora_fuzz")
    _build(["g++", *SAN, "-std=c++17",
            os.path.join(ROOT, "glacier.tune_amd", "csrc", "lora_file.cpp"),
            os.path.join(ROOT, "tests", "sanitize", "lora_fuzz.cpp"), "-o", exe], str(tmp_path))
    work = tmp_path / "work"
    work.mkdir()
    res = _run([exe, str(work), "3000"],
               {"ASAN_OPTIONS": "detect_leaks=1:halt_on_error=1",
                "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}, 240)
    assert res.returncode == 0, (res.stdout[-2000:], res.stderr[-4000:])
    assert "LORA_FUZZ_OK" in res.stdout
    assert "runtime error" not in res.stderr, res.stderr[-4000:]


def _library_build_module():
    spec = importlib.util.spec_from_file_location(
        "glacier_build", os.path.join(ROOT, "glacier.tune_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_library_host_code_under_asan_and_ubsan(tmp_path):
    try:
        build = _library_build_module()
        hipcc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not found")
    # sanitizers on the host pass only (the device code is built as usual)
    host_san = ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]
    csrc = os.path.join(ROOT, "glacier.tune_amd", "csrc")

    def compile_one(src, path, extra):
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        cmd = [hipcc, "-x", "hip", *build.COMMON, *extra, *host_san, "-c", path, "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        return obj

    drivers = ("abi_asan_driver.cpp", "lmhead_bounds_driver.cpp")
    jobs = [(s, os.path.join(csrc, s), build.SOURCES[s]) for s in build.SOURCES]
    jobs += [(d, os.path.join(ROOT, "tests", "sanitize", d), ()) for d in drivers]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        objs = dict(zip([j[0] for j in jobs], ex.map(lambda j: compile_one(*j), jobs)))
    lib_objs = [objs[s] for s in build.SOURCES]
    rocm_lib = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(hipcc))), "lib")
    env = {"ASAN_OPTIONS": "detect_leaks=1:halt_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}
    for driver, ok in zip(drivers, ("ABI_SANITIZE_OK", "LMHEAD_BOUNDS_OK")):
        exe = str(tmp_path / driver.replace(".cpp", ""))
        res = subprocess.run([hipcc, "--offload-arch=gfx950", "-Xarch_host", "-fsanitize=address",
                              "-Xarch_host", "-fsanitize=undefined", objs[driver], *lib_objs,
                              "-o", exe, "-L" + rocm_lib, "-Wl,-rpath," + rocm_lib, "-lhipblaslt"],
                             capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        res = _run([exe], env, 400)
        print(res.stdout)
        assert res.returncode == 0, (res.stdout[-3000:], res.stderr[-4000:])
        assert ok in res.stdout
        assert "runtime error" not in res.stderr, res.stderr[-4000:]
