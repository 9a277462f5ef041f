"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer: `make -C oracle sanitize`
builds oracle/sanitize_check.c with vdsl_oracle.c, which runs every oracle routine on small, empty
and ragged shapes with buffers of exactly their contract's size; any out-of-bounds access, leak or
undefined operation aborts it with a report."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("make") is None or shutil.which("cc") is None, reason="needs make and a C compiler")
def test_oracle_is_clean_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True)
    # verify_asan_link_order=0: the process may start with other libraries preloaded
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(ROOT, "oracle", "_san", "sanitize_check")], capture_output=True, text=True,
                       env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "sanitize_check: ok" in r.stdout
