"""The CPU suite under host AddressSanitizer + UndefinedBehaviorSanitizer.

`make -C gfxinfer_amd sanitize` builds the library with every host translation unit
(artifact parser, tiler, decode policy, launch validation) instrumented and the
oracle with the same clang runtime; this test runs the other CPU tests against
those builds in a child process with the runtime preloaded, as the reference's
GFXINFER_SANITIZE build does for its own tests (CMakeLists.txt:17,62-65).  Any
sanitizer report aborts the child (halt_on_error, no UB recovery).
"""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUNTIME = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))


@pytest.mark.skipif(not RUNTIME, reason="clang ASan runtime not installed")
def test_cpu_suite_under_address_and_undefined_sanitizers():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "gfxinfer_amd"), "-j8", "sanitize"], check=True)
    env = dict(os.environ)
    env.update(
        GFXINFER_AMD_LIBRARY=os.path.join(ROOT, "gfxinfer_amd", "_build_san", "libgfxinfer_amd.so"),
        GFXINFER_ORACLE_LIBRARY=os.path.join(ROOT, "oracle", "_san", "liboracle.so"),
        ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
        UBSAN_OPTIONS="print_stacktrace=1",
        LD_PRELOAD=RUNTIME[-1],
    )
    child = subprocess.run(
        [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-q", "-m", "not gpu",
         "-p", "no:cacheprovider", "--ignore", os.path.abspath(__file__)],
        cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    assert child.returncode == 0, child.stdout[-4000:] + child.stderr[-4000:]
    assert "runtime error" not in child.stderr and "ERROR: AddressSanitizer" not in child.stderr
