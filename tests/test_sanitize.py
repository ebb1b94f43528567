"""Sanitizer tier: the C ABI's host-side layer and the C oracle under
AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

Builds, in a temporary directory, avelang_amd/csrc/*.hip with the
sanitizers on host code only (-Xarch_host; the gfx950 device code is built
as usual and never launched) and oracle/gdn_cpu.c with clang, links
tests/sanitize/gdn_host_driver.cpp against them and runs it, on the CPU.  The driver exercises argument validation of every
entry point, empty problems, the cu_seqlens contract check, the workspace
sizes, the thread-local error channel and the oracle's chunked form against
its recurrence (see the driver's header).  Leak detection is off: the HIP
runtime the library links keeps allocations until exit.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
CLANG = os.path.join(ROCM, "llvm", "bin", "clang")
CLANGXX = os.path.join(ROCM, "llvm", "bin", "clang++")
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=undefined"]
DBG = ["-O1", "-g", "-fno-omit-frame-pointer"]


def _run(cmd, **kw):
    p = subprocess.run(cmd, capture_output=True, text=True, **kw)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in p.stderr.splitlines() if noise not in l)
    return p.returncode, p.stdout, err


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not (os.path.exists(HIPCC) and os.path.exists(CLANG)):
        pytest.skip("ROCm hipcc / clang not found")
    out = tmp_path_factory.mktemp("san")
    csrc = os.path.join(ROOT, "avelang_amd", "csrc")
    srcs = sorted(f for f in os.listdir(csrc) if f.endswith(".hip"))

    def compile_hip(f):
        obj = os.path.join(out, f + ".o")
        rc, _, err = _run([HIPCC, "-std=c++17", "--offload-arch=gfx950", *DBG, *SAN,
                           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                           "-fPIC", "-c", os.path.join(csrc, f), "-o", obj])
        assert rc == 0, f"{f}:\n{err}"
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_hip, srcs))
    oracle_obj = os.path.join(out, "gdn_cpu.o")
    rc, _, err = _run([CLANG, "-std=c11", *DBG, "-fsanitize=address,undefined",
                       "-fno-sanitize-recover=undefined", "-Wno-unknown-pragmas", "-c",
                       os.path.join(ROOT, "oracle", "gdn_cpu.c"), "-o", oracle_obj])
    assert rc == 0, err
    exe = os.path.join(out, "gdn_host_driver")
    rc, _, err = _run([CLANGXX, "-std=c++17", *DBG, "-fsanitize=address,undefined",
                       "-fno-sanitize-recover=undefined",
                       os.path.join(ROOT, "tests", "sanitize", "gdn_host_driver.cpp"),
                       *objs, oracle_obj, "-o", exe, "-L" + os.path.join(ROCM, "lib"),
                       "-Wl,-rpath," + os.path.join(ROCM, "lib"), "-lamdhip64", "-lm",
                       "-lpthread"])
    assert rc == 0, err
    yield exe
    shutil.rmtree(out, ignore_errors=True)


def test_host_layer_and_oracle_clean_under_asan_ubsan(driver):
    env = dict(os.environ,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               HIP_VISIBLE_DEVICES=os.environ.get("HIP_VISIBLE_DEVICES", ""))
    rc, out, err = _run([driver], env=env, timeout=300)
    assert rc == 0 and out.strip().endswith("OK"), f"rc={rc}\n{out}\n{err[-4000:]}"
    assert "runtime error" not in err and "AddressSanitizer" not in err, err[-4000:]
