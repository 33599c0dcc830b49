"""The host code that parses untrusted input, under AddressSanitizer and
UndefinedBehaviorSanitizer: the safetensors reader and the C-ABI around it
(tests/test_abi.py: round trips, read-back, crafted and malformed headers,
overflowing shapes, bad weights) and the decision front end
(tests/test_frontend.py, tests/test_native_frontend.py: tokenizer.json,
charsmap, Unigram Viterbi, word split, schema).  The sanitized libraries are
built by build() into gliner-decide-metal_amd/lib/sanitize/ (device code
unchanged); the tests run in a child interpreter with the clang ASan runtime
preloaded, and any sanitizer report fails the test."""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "gliner-decide-metal_amd"
SAN = PKG / "lib" / "sanitize"


def _runtime():
    sys.path.insert(0, str(PKG))
    import importlib.util
    spec = importlib.util.spec_from_file_location("gd_build_san", PKG / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.asan_runtime()


@pytest.mark.skipif(not (SAN / "libgliner_decide_hip.so").exists() or
                    not (SAN / "libgliner_decide_frontend.so").exists(),
                    reason="sanitized libraries not built (build() makes them)")
def test_host_parsers_under_asan_ubsan():
    env = dict(os.environ,
               LD_PRELOAD=str(_runtime()),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               GLINER_DECIDE_LIB=str(SAN / "libgliner_decide_hip.so"),
               GLINER_DECIDE_FRONTEND_LIB=str(SAN / "libgliner_decide_frontend.so"))
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
           "tests/test_abi.py", "tests/test_frontend.py", "tests/test_native_frontend.py"]
    p = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    out = p.stdout + p.stderr
    assert "ERROR: AddressSanitizer" not in out, out[-4000:]
    assert "runtime error:" not in out, out[-4000:]
    assert p.returncode == 0, out[-4000:]
    assert " passed" in out
