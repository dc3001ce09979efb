"""CPU: the profiler's arithmetic (host markers, device spans, floors, detail
levels, warmup, writers) and the residency pass-through, compiled from
tests/cpp/test_profiler.cpp with g++ and the host sources they test."""
import json
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
    out = tmp_path / "prof" / "nested"
    r = subprocess.run([exe, str(out)], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    # the files parse, with the reference's JSON keys and CSV columns
    data = json.load(open(out / "profile.json"))
    for key in ("clock_domain", "detail", "subtract_floor", "warmup_steps", "steps_kept",
                "steps_discarded", "max_depth", "nested_scopes_self_time", "ops", "floor",
                "device_backend", "device_spans", "device_spans_dropped",
                "device_floor_measured", "components", "residency_measured", "residency",
                "transfer_measured"):
        assert key in data, key
    comps = {c["component"]: c for c in data["components"]}
    assert comps["head"]["dev_ns"] == 1000 and comps["head"]["dev_ns_self"] == 900.0
    assert comps["qkv"]["idle_ns"] == 500 and comps["decode"]["dev_ns"] == 0
    assert data["floor"]["dev_ns"] == 100 and data["residency"]["vram_pct"] == 100.0
    lines = open(out / "profile.csv").read().splitlines()
    assert lines[0] == "component,ops,dev_ns,idle_ns,host_ns,clock_domain,detail,floor_dev_ns"
    assert any(l.startswith("qkv,0,500,500,0,device,class,100") for l in lines)
    assert "component" in open(out / "profile.txt").read()
