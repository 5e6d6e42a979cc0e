"""The C-ABI checks of tests/test_abi.py again, against a host-side ASan + UBSan build of the
library (``make -C ds-flashdmla-moe_amd/csrc sanitize``): argument validation, plan and
workspace arithmetic and error reporting must run without a memory error or undefined
behaviour (signed overflow, shifts, misaligned or out-of-range accesses).  No GPU: those checks
all return before a launch.  The sanitizer runtime is preloaded into a child interpreter."""
import os
import subprocess
import sys

import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "ds-flashdmla-moe_amd", "csrc")
SAN_LIB = os.path.join(CSRC, "_build", "san", "libflashdmla_san.so")
HIPCC = "/opt/rocm/bin/hipcc"


def _asan_runtime():
    out = subprocess.run([HIPCC, "--print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if out.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is needed to build the sanitizer variant")
def test_c_abi_checks_under_asan_and_ubsan():
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("the clang AddressSanitizer runtime is not installed")
    build = subprocess.run(["make", "-C", CSRC, "-j8", "sanitize"], capture_output=True, text=True, timeout=900)
    assert build.returncode == 0, build.stdout[-2000:] + build.stderr[-2000:]
    env = dict(os.environ)
    env.update(
        LD_PRELOAD=rt,
        DMLA_LIBRARY=SAN_LIB,
        # uninstrumented libraries (python, torch, the HIP runtime) keep their own allocations
        ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:alloc_dealloc_mismatch=0:detect_odr_violation=0",
        UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
    )
    # the child really maps the sanitizer runtime and the sanitized library
    probe = subprocess.run(
        [sys.executable, "-c", "import sys; sys.path.insert(0, sys.argv[1]); from python import _lib; _lib.lib(); "
         "print(open('/proc/self/maps').read())", os.path.join(ROOT, "ds-flashdmla-moe_amd")],
        env=env, capture_output=True, text=True, timeout=300,
    )
    assert probe.returncode == 0, probe.stderr[-2000:]
    assert SAN_LIB in probe.stdout and os.path.basename(rt) in probe.stdout
    run = subprocess.run(
        [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests", "test_abi.py"), "-q", "-x", "-m", "not gpu",
         "-p", "no:cacheprovider"],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=900,
    )
    log = run.stdout[-4000:] + run.stderr[-4000:]
    assert run.returncode == 0, log
    assert "AddressSanitizer" not in run.stderr and "runtime error" not in run.stderr, log
    assert " passed" in run.stdout, log
