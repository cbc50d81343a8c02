"""Host sanitizer runs (CPU, no GPU): the oracle's self-test under
AddressSanitizer + UndefinedBehaviorSanitizer and its threaded multi-head paths
under ThreadSanitizer (oracle/Makefile targets `sanitize` / `tsan`), and the C
ABI's host-side argument checks under AddressSanitizer +
UndefinedBehaviorSanitizer (tests/sanitize/Makefile; nothing is launched), and
the kernels' shared work orders (tests/sanitize/order_selftest.cpp)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(cmd, env=None):
    r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, f"{cmd}: rc {r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
    return r.stdout


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is not installed")
def test_oracle_asan_ubsan():
    _run(["make", "-s", "-f", os.path.join(ROOT, "oracle", "Makefile"), "sanitize"])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    assert "all checks passed" in _run([os.path.join(ROOT, "oracle", "_san", "selftest_asan")], env)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is not installed")
def test_oracle_tsan_threads():
    _run(["make", "-s", "-f", os.path.join(ROOT, "oracle", "Makefile"), "tsan"])
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1")
    assert "all checks passed" in _run([os.path.join(ROOT, "oracle", "_san", "selftest_tsan"), "threads"], env)


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc is not installed")
def test_abi_host_asan_ubsan():
    _run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "tests", "sanitize")])
    # the HIP runtime's own allocations are not the library's: no leak check
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    assert "all checks passed" in _run([os.path.join(ROOT, "tests", "sanitize", "_build", "abi_selftest")], env)


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc is not installed")
def test_work_orders_asan_ubsan():
    """The work order of resident causal grids (cu_order_wg) and the GQA
    split's share indices (dkv_first_work against dkv_work), host side."""
    _run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "tests", "sanitize")])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    assert "all checks passed" in _run([os.path.join(ROOT, "tests", "sanitize", "_build", "order_selftest")], env)
