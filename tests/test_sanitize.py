"""The host C under AddressSanitizer + UndefinedBehaviorSanitizer (no GPU):
the long-audio splitter (csrc/chunk.c) and the synthetic-workload generator
(host/synth.c) are built with -fsanitize=address,undefined
-fno-sanitize-recover=all (`make -C cohere-transcribe_amd sanitize`) and
loaded in place of the normal builds by a child pytest run with the ASan
runtime preloaded: tests/test_chunking.py (the splitter against the
oracle's, bit for bit, and the oracle against closed forms) and
tests/asan_cases.py (the generator's output identical to the normal
build's).  Any sanitizer report aborts the child."""
import json
import os
import subprocess
import sys

import pytest

import ctbind as cb

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "cohere-transcribe_amd")


def runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.mark.skipif(runtime("libasan.so") is None, reason="gcc's ASan runtime is not installed")
def test_host_code_under_asan_ubsan():
    subprocess.run(["make", "-s", "-C", PKG, "sanitize"], check=True)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import asan_cases
    expect = asan_cases.digests()          # the normal builds, in this process
    env = dict(os.environ,
               LD_PRELOAD=runtime("libasan.so"),
               CT_HOST_LIB=os.path.join(PKG, "_build", "asan", "libct_host.so"),
               CT_CHUNK_LIB=os.path.join(PKG, "_build", "asan", "libct_chunk.so"),
               CT_ASAN_EXPECT=json.dumps(expect),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(REPO, "tests", "test_chunking.py"),
                        os.path.join(REPO, "tests", "asan_cases.py")],
                       cwd=REPO, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in r.stdout
