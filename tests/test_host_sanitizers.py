"""The host repacker (qwenny_amd/csrc/host.cpp) under AddressSanitizer and UndefinedBehaviorSanitizer: a C++ driver
(tests/host_sanitizer_driver.cpp) packs and unpacks every storage at several shapes, row orders and group sizes
through the C ABI; any out-of-bounds access or undefined behaviour aborts it. Host code only (no GPU, no hipcc)."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_repacker_under_sanitizers(tmp_path):
    exe = str(tmp_path / "driver")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-fno-omit-frame-pointer", "-pthread", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "qwenny_amd", "csrc", "host.cpp"),
                    os.path.join(HERE, "host_sanitizer_driver.cpp"), "-o", exe], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "asan driver ok" in r.stdout
