"""Sanitizer runs of host code (AddressSanitizer + UndefinedBehaviorSanitizer,
first report fatal).

- The CPU oracle: `make -C oracle sanitize` builds oracle/sanitize_check.c
  with rk_oracle.c under both sanitizers and runs it (no GPU).
- The library's host code behind the C ABI: tests/sanitize/abi_driver.cpp,
  built by `make -C tests/sanitize` from the library's sources with the
  sanitizers on the host side only (the GPU code objects are the product's),
  drives the ABI as the reference's Rust backend does and checks every result
  bit-exact against the oracle. It needs a GPU; the test is skipped when the
  sanitizer build is absent from the tree.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_oracle_under_asan_ubsan():
    if shutil.which("gcc") is None or shutil.which("make") is None:
        pytest.skip("gcc and make are needed to build the sanitizer run of the oracle")
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "oracle sanitizer run: 0 failed checks" in r.stdout


@pytest.mark.gpu
def test_library_host_code_under_asan_ubsan():
    exe = os.path.join(ROOT, "tests", "sanitize", "_build", "abi_driver")
    if not os.path.exists(exe):
        pytest.skip("sanitizer build absent: make -C tests/sanitize -j4")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    print("running", exe, flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env,
                       cwd=os.path.dirname(exe))
    assert r.returncode == 0, (r.stdout + r.stderr)[-6000:]
    assert "abi sanitizer run: 0 failed checks" in r.stdout
