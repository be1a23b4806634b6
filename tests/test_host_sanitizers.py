"""The library's host bookkeeping under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU.

pcl_hip.cpp (the C-ABI shim: per-stream scratch grow/retire/release, graph
pinning, the thread-local staging slots of the host-pointer drop-ins, the
realigned FP32 operands, pcl_head_ce's chunk buffers) and the bench harness
(drivers/bench_harness.c, whose decode sweep ended once with a heap-corruption
report under the profiler) are compiled for the host with the sanitizers and
linked against a mock HIP runtime (tests/host_asan/mock_hip.cpp: host memory
for device memory, launchers that write every byte of the buffers they are
handed). tests/host_asan/driver.c drives them: growth inside and outside graph
capture, release refused while a graph may use the scratch, six threads on
their own streams and the shared null stream, the realign and head paths, the
decode sweep eager, as graphs, INT8 and grouped. Any invalid access, double
free, undefined behaviour or leak fails the test.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HERE = os.path.join(ROOT, "tests", "host_asan")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.mark.skipif(not (shutil.which("g++") and os.path.isdir("/opt/rocm/include")),
                    reason="needs g++ and the ROCm headers")
def test_host_bookkeeping_under_asan_ubsan(tmp_path):
    hip = ["-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-w"]
    objs = []
    for src, cc, extra in [
        (os.path.join(ROOT, "pure-c-llm_amd", "csrc", "pcl_hip.cpp"), "g++", ["-std=c++17"] + hip),
        (os.path.join(HERE, "mock_hip.cpp"), "g++", ["-std=c++17"] + hip),
        (os.path.join(ROOT, "pure-c-llm_amd", "drivers", "bench_harness.c"), "gcc",
         ["-std=c11", "-D_GNU_SOURCE", "-w", "-I" + os.path.join(ROOT, "include")]),
        (os.path.join(HERE, "driver.c"), "gcc", ["-std=c11", "-w", "-I" + os.path.join(ROOT, "include")]),
    ]:
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        subprocess.run([cc] + extra + SAN + ["-c", src, "-o", obj], check=True, timeout=300)
        objs.append(obj)
    exe = str(tmp_path / "host_asan")
    subprocess.run(["g++"] + SAN + objs + ["-o", exe, "-lpthread", "-lm"], check=True, timeout=120)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-6000:]
    assert "host bookkeeping ok" in r.stdout
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
