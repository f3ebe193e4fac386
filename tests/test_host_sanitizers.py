"""The host repack (mashbox_amd/csrc/mbq_host_repack.h: raw pointer arithmetic on C++ threads) built alone with g++
under AddressSanitizer + UndefinedBehaviorSanitizer, and under ThreadSanitizer, running tests/host_repack_check.cpp's
round trips (every GGUF type and the tiled int8 planes, on one host thread and on several). CPU only."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "mashbox_amd", "csrc")
SRC = os.path.join(HERE, "host_repack_check.cpp")


def _build_and_run(tmp_path, flags, env_extra):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = str(tmp_path / "host_repack_check")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", *flags, "-I", CSRC, SRC, "-o", exe, "-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ, **env_extra)
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "round trips ok" in r.stdout
    assert "ERROR" not in r.stderr and "runtime error" not in r.stderr, r.stderr


def test_host_repack_under_address_and_undefined_behavior_sanitizers(tmp_path):
    _build_and_run(tmp_path, ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"],
                   {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"})


def test_host_repack_under_thread_sanitizer(tmp_path):
    _build_and_run(tmp_path, ["-fsanitize=thread"], {"TSAN_OPTIONS": "halt_on_error=1"})
