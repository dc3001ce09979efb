"""CPU: the profiler's arithmetic (host markers, device spans, floors, detail
levels, warmup, writers) and the residency pass-through, compiled from
tests/cpp/test_profiler.cpp with g++ and the host sources they test."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_profiler_and_residency(tmp_path):
    exe = str(tmp_path / "test_profiler")
    srcs = [os.path.join(ROOT, "tests", "cpp", "test_profiler.cpp"),
            os.path.join(ROOT, "kanjoos_amd", "host", "knj_profiler.cpp"),
            os.path.join(ROOT, "kanjoos_amd", "host", "knj_residency.cpp")]
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", *srcs, "-o", exe],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
