"""The C-ABI's CPU tests under AddressSanitizer.

nanopd_amd.build.build_asan() compiles every C-ABI source with
-fsanitize=address on the host pass into _build/asan/libnanopd_hip_asan.so. Here a
child Python process loads that library (NPD_LIB) with clang's sanitizer
runtime preloaded and runs tests/test_capi.py: every validation path of every
entry point (bad dtypes, shapes, alignment, null pointers, int32 ranges, the
error-message buffer), the workspace-size functions and the Python mirror's
checks. Any heap, stack or global overflow or use-after-free in the host
code those tests reach stops the child with a report. A planted
out-of-bounds copy in a child shows that the runtime is live there.

Skipped where a GPU is visible (the validation tests use fake pointers and
skip themselves there) and where the environment already preloads a library
(this test adds none beside it)."""
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from nanopd_amd import build

ROOT = Path(__file__).resolve().parents[1]

pytestmark = [
    pytest.mark.skipif(torch.cuda.is_available(), reason="CPU-only: fake pointers"),
    pytest.mark.skipif(bool(os.environ.get("LD_PRELOAD")),
                       reason="the environment already preloads a library"),
]


@pytest.fixture(scope="module")
def asan_env():
    rt = build.asan_runtime()
    if rt is None:
        pytest.skip("no AddressSanitizer runtime next to hipcc's clang")
    lib = build.ASAN_LIB_PATH
    srcs = build.sources()
    if not lib.exists() or lib.stat().st_mtime < max(s.stat().st_mtime for s in srcs):
        build.build_asan()
    env = dict(os.environ, NPD_LIB=str(lib), LD_PRELOAD=str(rt),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1")
    return lib, env


def test_asan_library_is_instrumented(asan_env):
    lib, _ = asan_env
    out = subprocess.run(["nm", "-D", str(lib)], capture_output=True, text=True, check=True).stdout
    assert "__asan_report_load" in out or "__asan_report_store" in out
    assert " T npd_paged_attention" in out


def test_asan_runtime_catches_a_planted_overflow(asan_env):
    _, env = asan_env
    code = ("import ctypes\n"
            "a = ctypes.create_string_buffer(16)\n"
            "ctypes.memmove(ctypes.addressof(a), b'x' * 64, 64)\n")
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=120)
    assert res.returncode != 0 and "AddressSanitizer" in res.stderr


def test_capi_tests_pass_under_asan(asan_env):
    _, env = asan_env
    res = subprocess.run([sys.executable, "-m", "pytest", "tests/test_capi.py", "-q",
                          "-p", "no:cacheprovider"], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=600)
    out = res.stdout + res.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert res.returncode == 0 and " passed" in out, out[-4000:]
