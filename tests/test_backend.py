"""CPU: a caller written against the reference's device interface
(/root/reference/src/device/backend.h:37-76) compiles against include/knj/backend.h,
links the host classes and the C-ABI library, and sees the reference's gating
behaviour through from_caps() (tests/cpp/test_backend_caller.cpp)."""
import os
import subprocess

import pytest

import kanjoos_amd as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def build_caller(tmp_path):
    exe = str(tmp_path / "test_backend_caller")
    srcs = [os.path.join(ROOT, "tests", "cpp", "test_backend_caller.cpp"),
            os.path.join(ROOT, "kanjoos_amd", "host", "knj_host.cpp")]
    libdir = os.path.dirname(K.LIB_PATH)
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror",
                        "-I", os.path.join(ROOT, "include"), *srcs, "-o", exe, "-L", libdir,
                        "-lkanjoos_amd", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr
    return exe


def test_reference_style_caller(tmp_path):
    exe = build_caller(tmp_path)
    env = dict(os.environ)
    if not os.path.exists("/dev/kfd"):
        env["KNJ_EXPECT_NO_DEVICE"] = "1"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.gpu
def test_reference_style_caller_on_device(tmp_path):
    """The same caller on the GPU: additionally, launch_kv_write with the
    reference's plan (no output buffer) writes the cache slot, bit-identical to
    launch_attention with an explicit output, and a refused plan leaves a
    reason in knj_last_refusal()."""
    exe = build_caller(tmp_path)
    env = dict(os.environ, KNJ_DEVICE_CHECKS="1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "device KV write" in r.stdout
