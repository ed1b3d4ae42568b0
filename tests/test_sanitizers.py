"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer.

* The CPU restatement (oracle/oracle.c) built with -fsanitize=address,undefined
  (oracle/_san/liboracle.so, `make -C oracle san`) runs the whole oracle test module.
* The jasmine-compatible C++ headers, compiled into the user-code driver
  (tests/cpp/libjasapi_san.so, `make -C tests/cpp san`), run the C++ API module on the GPU;
  the headers hold no device code, so all of their host code is instrumented.
Each run is a child process with libasan preloaded (the Python interpreter itself is not
instrumented); any sanitizer report aborts the child and fails the test.
"""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _libasan():
    try:
        p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True, check=True)
    except (OSError, subprocess.CalledProcessError):
        return None
    path = p.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def _run_under_asan(extra_env, args, timeout):
    asan = _libasan()
    if asan is None:
        pytest.skip("gcc's libasan is not available")
    env = dict(os.environ)
    env.update(extra_env)
    env["LD_PRELOAD"] = asan
    # leaks: the interpreter's own allocations are reported at exit, not ours
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider"] + args, cwd=ROOT,
                       env=env, capture_output=True, text=True, timeout=timeout)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error:" not in tail, tail


def test_oracle_under_asan_ubsan():
    so = os.path.join(ROOT, "oracle", "_san", "liboracle.so")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "san"], check=True)
    _run_under_asan({"JAS_ORACLE_SO": so}, ["tests/test_oracle.py", "-m", "not gpu"], timeout=900)


@pytest.mark.gpu
def test_cpp_api_under_asan_ubsan():
    so = os.path.join(HERE, "cpp", "libjasapi_san.so")
    if not os.path.exists(so):
        pytest.skip("tests/cpp/libjasapi_san.so is not built (make -C tests/cpp san)")
    _run_under_asan({"JAS_API_SO": so}, ["tests/test_cpp_api.py", "-m", "gpu"], timeout=600)
