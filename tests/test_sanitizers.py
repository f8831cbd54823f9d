"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

Builds tests/sanitize/host_checks.cpp with the library's host types
(grokking_abmod_amd/csrc/meshgpt_types.cpp, geometry.cpp) and the CPU oracle,
all with -fsanitize=address,undefined, and runs it: configuration checks,
layouts and seeded initialisation, every token-code geometry, the tokenizer,
checkpoint parsing of intact, truncated and corrupted files, and the oracle's
entry points on small models.  Any sanitizer report fails the test.
"""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
         "-ffp-contract=off"]


def _build(tmp_path):
    csrc = os.path.join(ROOT, "grokking_abmod_amd", "csrc")
    oracle = os.path.join(ROOT, "oracle")
    obj = str(tmp_path / "oracle.o")
    exe = str(tmp_path / "host_checks")
    cc = subprocess.run(["gcc", "-std=c11", *FLAGS, "-I", oracle, "-c", os.path.join(oracle, "meshgpt_oracle.c"),
                         "-o", obj], capture_output=True, text=True)
    if cc.returncode != 0 and "asan" in cc.stderr.lower():
        pytest.skip("the C compiler has no sanitizer runtime")
    assert cc.returncode == 0, cc.stderr
    cxx = subprocess.run(["g++", "-std=c++17", *FLAGS, "-I", oracle, "-I", csrc,
                          os.path.join(ROOT, "tests", "sanitize", "host_checks.cpp"),
                          os.path.join(csrc, "meshgpt_types.cpp"), os.path.join(csrc, "geometry.cpp"), obj,
                          "-o", exe], capture_output=True, text=True)
    assert cxx.returncode == 0, cxx.stderr
    return exe


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="no host compiler")
def test_host_code_is_clean_under_address_and_undefined_sanitizers(tmp_path):
    exe = _build(tmp_path)
    env = dict(os.environ)
    # The sanitizer runtime need not be first in the preload list (a harness
    # may preload its own library); leaks are reported.
    env["ASAN_OPTIONS"] = "verify_asan_link_order=0:detect_leaks=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    run = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    report = run.stdout + run.stderr
    assert run.returncode == 0, report[-4000:]
    assert "host checks ok" in run.stdout
    assert "runtime error" not in report and "AddressSanitizer" not in report, report[-4000:]
