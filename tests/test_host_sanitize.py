"""Host-only AddressSanitizer / UndefinedBehaviorSanitizer build of the C ABI's
validation, planning and launch sequencing (fa_api.cpp), with the kernel
launchers and HIP runtime calls replaced by the recording stubs of
tests/host/fa_host_harness.cpp. Runs on the CPU: every batch size around the
2048-sequence chunk boundary, every layout kind, and invalid / extreme inputs."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "flash-attention-npu_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_c_abi_host_code_under_asan_ubsan(tmp_path):
    exe = tmp_path / "harness"
    # host code only (g++, no HIP device code): the sanitizers instrument fa_api.cpp
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-D__HIP_PLATFORM_AMD__=1", "-I", "/opt/rocm/include",
           "-I", os.path.join(REPO, "include"), "-I", CSRC,
           os.path.join(CSRC, "fa_api.cpp"), os.path.join(REPO, "tests", "host", "fa_host_harness.cpp"),
           "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "0 failures" in r.stdout, r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_decode_split_against_brute_force(tmp_path):
    """The decode kernel's tile split and the merge's owner / slot lookups
    (csrc/fa_decode_split.h, host and device code alike) against brute force,
    under ASan / UBSan."""
    exe = tmp_path / "split_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", CSRC, os.path.join(REPO, "tests", "host", "fa_decode_split_check.cpp"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert " 0 failures" in r.stdout, r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_invariant_division_against_plain_division(tmp_path):
    """The multiply-high division by a run-time invariant divisor that the
    backward's tile loop uses for packed row -> query position
    (csrc/fa_udiv.h, host and device code alike) against n / d, under
    ASan / UBSan."""
    exe = tmp_path / "udiv_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", CSRC, os.path.join(REPO, "tests", "host", "fa_udiv_check.cpp"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert " 0 failures" in r.stdout, r.stdout
