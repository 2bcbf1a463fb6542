"""The plan builder under AddressSanitizer (host code only; no device needed).

``tests/native/plan_builder_fuzz.cpp`` sends random segment tables, valid and not, through
``emrs_plan_create`` / ``emrs_plan_stats_get`` / ``emrs_plan_execute`` (which must refuse without a
device) / ``emrs_plan_destroy``, random launch shapes through ``emrs_set_tuning``, and malformed
hand-off records through ``emrs_ipc_open`` / ``emrs_ipc_close`` (refused before the driver).  The library
is rebuilt for the test with the host half sanitized (``-Xarch_host``); its device code is the
ordinary gfx950 build and is never launched here.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "elasticmegatron_amd", "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _tool(name, *candidates):
    for c in candidates:
        if c and os.path.exists(c):
            return c
    return shutil.which(name)


@pytest.mark.timeout(900)
def test_plan_builder_is_memory_safe_under_asan(tmp_path):
    hipcc = _tool("hipcc", os.path.join(ROCM, "bin", "hipcc"))
    clang = _tool("clang++", os.path.join(ROCM, "llvm", "bin", "clang++"))
    if not hipcc or not clang:
        pytest.skip("hipcc and ROCm's clang++ are needed to build the sanitized library")
    lib = tmp_path / "libemrs_asan.so"
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    host_asan = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-shared", *host_asan,
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-I", os.path.join(ROOT, "include"), "-I", CSRC, *srcs, "-o", str(lib)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    exe = tmp_path / "plan_builder_fuzz"
    r = subprocess.run([clang, "-O1", "-g", "-std=c++17", "-fsanitize=address", "-fno-omit-frame-pointer",
                        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"),
                        os.path.join(ROOT, "tests", "native", "plan_builder_fuzz.cpp"), "-L", str(tmp_path), "-lemrs_asan",
                        f"-Wl,-rpath,{tmp_path}", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
                        f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-o", str(exe)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([str(exe), "4000"], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "LeakSanitizer" not in r.stderr
    ok, rejected = (int(x) for x in r.stdout.split()[1::2])
    assert ok > 1000 and rejected > 1000  # both the valid and the refused paths ran
