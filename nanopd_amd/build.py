"""Builds libnanopd_hip.so (the C-ABI library) for gfx950, in-tree.

hipcc compiles every source under nanopd_amd/csrc/ to an object in
nanopd_amd/_build/ (in parallel) and links them into nanopd_amd/lib/. Run as
``python -m nanopd_amd.build`` or call :func:`build`.

:func:`build_asan` builds the same sources with AddressSanitizer on the host
pass into libnanopd_hip_asan.so, for the CPU tests of the C-ABI's
argument validation (tests/test_asan_capi.py), under _build/asan/. The
product path never loads it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB_PATH = LIB_DIR / "libnanopd_hip.so"
ARCH = os.environ.get("NPD_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU ops (v_pk_fma_f32 and kin) are kept out of the generated
# code: some of their forms have given wrong results on this hardware pool.
# The host pass warns that it does not know the feature.
COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-file additions. prefill_attention: attention scores are finite or -inf
# (masked keys), so the row maxima need no NaN quieting (v_max_f32 x, x, x
# before every max).
FILE_FLAGS = {
    "prefill_attention.hip": ["-fno-honor-nans"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(hipcc: str, src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, f"--offload-arch={ARCH}", *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c",
           str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{out}")
    if verbose and out.strip():
        print(out, flush=True)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles and links the library; always rebuilds. Returns the .so path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


ASAN_DIR = BUILD_DIR / "asan"
ASAN_LIB_PATH = ASAN_DIR / "libnanopd_hip_asan.so"   # a test artefact: stays out of lib/
# The sanitizer applies to the host pass only; the device code is compiled
# (the host objects register it) but never launched from this library.
ASAN_FLAGS = ["-std=c++17", "-fPIC", "-O1", "-gline-tables-only", "-fno-omit-frame-pointer",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Xarch_host", "-fsanitize=address"]


def build_asan(verbose: bool = False) -> Path:
    """AddressSanitizer build (host pass) of every C-ABI source; always rebuilds.
    The library leaves the sanitizer runtime to the process that loads it
    (asan_runtime() names the one matching hipcc's compiler)."""
    hipcc = _hipcc()
    ASAN_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)

    def one(src: Path) -> Path:
        obj = ASAN_DIR / (src.stem + ".o")
        cmd = [hipcc, f"--offload-arch={ARCH}", *ASAN_FLAGS, *FILE_FLAGS.get(src.name, []),
               "-c", str(src), "-o", str(obj)]
        if src.suffix == ".cpp":
            cmd[1:1] = ["-x", "hip"]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc (asan) failed on {src.name}:\n{res.stdout}{res.stderr}")
        return obj

    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(one, srcs))
    tmp = ASAN_LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
           "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link (asan) failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, ASAN_LIB_PATH)
    return ASAN_LIB_PATH


def asan_runtime() -> Path | None:
    """The AddressSanitizer runtime of hipcc's clang, or None."""
    clang = Path(_hipcc()).resolve().parent.parent / "lib" / "llvm" / "bin" / "clang++"
    for cand in (clang, Path("/opt/rocm/llvm/bin/clang++")):
        if cand.exists():
            res = subprocess.run([str(cand), "-print-file-name=libclang_rt.asan-x86_64.so"],
                                 capture_output=True, text=True)
            p = Path(res.stdout.strip())
            if res.returncode == 0 and p.is_absolute() and p.exists():
                return p
    return None


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
    if "--asan" in sys.argv:
        print(build_asan(verbose="-v" in sys.argv))
