"""The C host of libcmol (GGUF parser, tokenizer, sampler and its worker pool,
cross-session scheduler, load error paths) and the oracle, built with
AddressSanitizer + UndefinedBehaviorSanitizer and with ThreadSanitizer
(tests/native/Makefile, gcc, no device: tests/native/no_device.c answers the
device calls) and driven by tests/native/host_check.c.  The reference builds
its own tests with the same sanitizers (its Makefile's debug flags)."""
import os
import shutil
import subprocess

import pytest

from tests.test_text import NAMES, tokenizer_model

HERE = os.path.dirname(os.path.abspath(__file__))
NATIVE = os.path.join(HERE, "native")


@pytest.fixture(scope="module")
def built():
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    subprocess.run(["make", "-s", "-C", NATIVE, "asan", "tsan"], check=True, timeout=600)
    return NATIVE


@pytest.mark.parametrize("kind", ["asan", "tsan"])
def test_host_under_sanitizers(built, tmp_path, kind):
    gguf = tokenizer_model(NAMES[0], str(tmp_path))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", TSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([os.path.join(built, "_build", f"host_check_{kind}"), gguf], capture_output=True,
                       text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ok: 0 failures" in out
    for bad in ("ERROR: AddressSanitizer", "runtime error:", "WARNING: ThreadSanitizer", "LeakSanitizer"):
        assert bad not in out, out[-4000:]
