"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer, driven through
its C ABI on the GPU: vernondsl_amd/csrc/abi_check.c (built by `make -C vernondsl_amd/csrc
sanitize`, which __graft_entry__.build() runs) calls every entry point with handles, shapes and
buffers it must refuse and with a small valid workload, then releases everything.  Any
out-of-bounds access, use after free, undefined operation or leak of the library's own memory in
host code aborts the driver with a report.  Leaks inside the HIP runtime's own libraries are
suppressed (they are not this library's code)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "vernondsl_amd", "csrc", "_san", "abi_check")
RUNTIME_LIBS = ("libamdhip64", "libhsa-runtime64", "libhiprtc", "libamd_comgr", "libdrm", "libelf", "libnuma",
                "librocprofiler", "libroctracer", "libstdc++")


def test_c_abi_host_code_clean_under_asan_and_ubsan(tmp_path):
    if not os.path.exists(DRIVER):
        pytest.fail("the sanitizer driver is not built: run `make -C vernondsl_amd/csrc sanitize`")
    supp = tmp_path / "lsan.supp"
    supp.write_text("".join(f"leak:{lib}\n" for lib in RUNTIME_LIBS))
    env = dict(os.environ,
               ASAN_OPTIONS="detect_leaks=1:verify_asan_link_order=0:abort_on_error=0:halt_on_error=1",
               LSAN_OPTIONS=f"suppressions={supp}:print_suppressions=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([DRIVER], capture_output=True, text=True, env=env, timeout=240)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-6000:])
    assert "abi_check: ok" in r.stdout
