"""The repository's host C under AddressSanitizer and UndefinedBehaviorSanitizer:
the .dpuf packer, container writer and reader (JSON header parser, tile CRC
verify and heal), the CRC helpers and the oracle, built with gcc and
-fsanitize=address,undefined from their sources into one driver
(tests/sanitize/drive.c), which round-trips models, runs the oracle on both
KV cache types and opens ~400 damaged containers.  Any sanitizer report
fails the run."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = [os.path.join(ROOT, "tests", "sanitize", "drive.c"),
       os.path.join(ROOT, "dpuf_amd", "csrc", "dpuf_tools.c"),
       os.path.join(ROOT, "dpuf_amd", "csrc", "dpuf_crc.c"),
       os.path.join(ROOT, "oracle", "oracle.c")]


@pytest.mark.timeout(600)
def test_host_c_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "drive")
    cmd = ["gcc", "-O1", "-g", "-std=gnu11", "-fopenmp", "-march=x86-64-v3", "-ffp-contract=off",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
           "-I" + os.path.join(ROOT, "include"), *SRC, "-o", exe, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "libasan" in r.stderr:
        pytest.skip("gcc has no AddressSanitizer runtime here")
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", OMP_NUM_THREADS="4")
    run = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, env=env, timeout=540)
    out = run.stdout + run.stderr
    assert run.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert "damaged containers" in out, out[-2000:]
