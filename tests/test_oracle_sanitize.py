"""The oracle under AddressSanitizer and UndefinedBehaviorSanitizer: `make
-C oracle sanitize` builds oracle/sanitize_driver.c with llm_oracle.c
(host code, -fno-sanitize-recover) into a temporary directory, and the
driver runs the whole oracle API on small shapes; any sanitizer report
ends it with a non-zero status."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_asan_ubsan_clean():
    with tempfile.TemporaryDirectory() as d:
        mk = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "sanitize",
                             f"OUT={d}"], capture_output=True, text=True)
        if mk.returncode != 0 and "asan" in (mk.stderr + mk.stdout).lower():
            pytest.skip("this gcc has no sanitizer runtime")
        assert mk.returncode == 0, mk.stderr[-2000:]
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
                   UBSAN_OPTIONS="print_stacktrace=1", OMP_NUM_THREADS="2")
        run = subprocess.run([os.path.join(d, "orc_sanitize")], capture_output=True,
                             text=True, env=env, timeout=600)
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-4000:])
    assert "sanitize OK" in run.stdout
    assert "runtime error" not in run.stderr and "ERROR: AddressSanitizer" not in run.stderr
