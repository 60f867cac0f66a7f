"""The host code of this repository under the address and undefined-
behaviour sanitizers (CPU only): tests/native/sanitize_check.cpp, built here
with gcc/g++ -fsanitize=address,undefined, exercises libndattn's session
bookkeeping (esp32-needle-3_amd/csrc/nda_state.h: slot arithmetic against the
oracle's kv_slot, randomized page-table operations with their invariants and
transaction rollbacks) and the oracle (sessions with snapshot / rewind /
prefix restore, the front, the threaded fp16 batch decode). Any sanitizer
report or failed check fails the test. The C engine shim needs a GPU context
for every call past its argument checks, so it is not run here."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-O1", "-g"]


@pytest.mark.skipif(not shutil.which("gcc") or not shutil.which("g++"), reason="no host compiler")
def test_host_code_under_sanitizers(tmp_path):
    obj = tmp_path / "nd_oracle.o"
    exe = tmp_path / "sanitize_check"
    subprocess.run(["gcc", "-std=gnu99", "-ffp-contract=off", *SAN, "-c", os.path.join(REPO, "oracle", "nd_oracle.c"),
                    "-o", str(obj)], check=True)
    subprocess.run(["g++", "-std=c++17", *SAN, "-I" + os.path.join(REPO, "oracle"),
                    "-I" + os.path.join(REPO, "esp32-needle-3_amd", "csrc"),
                    os.path.join(REPO, "tests", "native", "sanitize_check.cpp"), str(obj), "-o", str(exe),
                    "-lpthread", "-lm"], check=True)
    # the environment is passed on as it is; should a library be preloaded
    # ahead of the sanitizer runtime, ASan is told not to insist on coming
    # first
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "sanitize_check: ok" in r.stdout
