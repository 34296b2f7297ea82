"""The C-ABI host code under AddressSanitizer and UndefinedBehaviorSanitizer,
on the CPU (no GPU needed).

api.hip is compiled with the sanitizers on its host pass only (-Xarch_host
before each -fsanitize=), linked with the other librq objects into a separate
library under a temporary directory, and driven by tests/asan/driver.cpp
through every entry point's GPU-free paths: argument checks, NULL / unknown /
dangling handles (the registries must reject them without dereferencing),
the thread-local error message under concurrent failures, the status strings
and the pure helpers. The run must exit 0 with no sanitizer report. Leak
detection is off: the HIP runtime keeps process-lifetime allocations."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.fixture(scope="module")
def asan_build(tmp_path_factory):
    from raster_amd import build as rqb

    if not os.path.exists(CLANG):
        pytest.skip("ROCm clang++ not found")
    rqb.build()  # the other objects, unsanitized
    d = tmp_path_factory.mktemp("asan")
    api_o = str(d / "api.o")
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-omit-frame-pointer"]
    r = subprocess.run([rqb.hipcc(), f"--offload-arch={rqb.ARCH}", "-O1", "-g", "-std=c++17", "-fPIC",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *san, "-c", "-o", api_o,
                        os.path.join(rqb.CSRC, "api.hip")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    objs = [o for o in sorted(os.listdir(rqb.OBJ)) if o.endswith(".o") and o != "api.o"]
    lib = str(d / "librq_asan.so")
    r = subprocess.run([rqb.hipcc(), f"--offload-arch={rqb.ARCH}", "-shared", "-fPIC", "-Xarch_host",
                        "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-shared-libasan", "-o", lib,
                        api_o, *[os.path.join(rqb.OBJ, o) for o in objs], *rqb.LINK_LIBS],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    drv = str(d / "driver")
    r = subprocess.run([CLANG, "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-shared-libasan",
                        "-fno-omit-frame-pointer", "-o", drv, os.path.join(ROOT, "tests", "asan", "driver.cpp"),
                        f"-L{d}", "-lrq_asan", f"-Wl,-rpath,{d}", "-lpthread"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    rt = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    yield drv, os.path.dirname(rt.stdout.strip())
    shutil.rmtree(d, ignore_errors=True)


def test_c_abi_host_code_is_sanitizer_clean(asan_build):
    drv, rtdir = asan_build
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               LD_LIBRARY_PATH=rtdir + ":" + os.environ.get("LD_LIBRARY_PATH", ""),
               HIP_VISIBLE_DEVICES="")
    r = subprocess.run([drv], capture_output=True, text=True, env=env, timeout=300)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert "all checks passed" in out


def test_sanitizer_reports_a_planted_overflow(asan_build, tmp_path):
    # the same toolchain and options catch a heap overflow planted in a CPU
    # program, so the clean run above is not clean by default
    _, rtdir = asan_build
    src = tmp_path / "planted.cpp"
    src.write_text("#include <vector>\nint main(){std::vector<int> v(4);int* p=v.data();"
                   "volatile int i=4;return p[i];}\n")
    exe = str(tmp_path / "planted")
    r = subprocess.run([CLANG, "-g", "-O0", "-fsanitize=address", "-shared-libasan", "-o", exe, str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", LD_LIBRARY_PATH=rtdir)
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=60)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr
