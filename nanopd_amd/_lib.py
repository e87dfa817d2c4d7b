"""ctypes binding of libnanopd_hip.so (declarations in include/nanopd.h).

The library is loaded once per process. There is no fallback: if the built
library is missing, every op raises instead of computing anything elsewhere.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libnanopd_hip.so"

NPD_DTYPE_F16 = 0
NPD_DTYPE_BF16 = 1
# size of the static scratch of npd_paged_attention_noalloc (NPD_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 64 << 20

# name -> (restype, argtypes)
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
SIGNATURES = {
    "npd_last_error": (ctypes.c_char_p, []),
    "npd_version": (ctypes.c_int, []),
    "npd_paged_kv_store": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                          _I64, _I64, _I64, _I32, _P]),
    "npd_paged_kv_store_slots": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                                _I64, _I64, _I32, _P]),
    "npd_paged_kv_store_slots_fp8": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                                    _I64, _I64, _I64, _I64, _I32, _P]),
    "npd_paged_attention_workspace_size": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "npd_paged_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                           _I64, _I64, _F, _I64, _I64, _I64, _I64, _P, _I64, _I32,
                                           _P]),
    "npd_paged_attention_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                                   _I64, _I64, _I64, _F, _I64, _I64, _I64, _I64,
                                                   _I32, _P]),
    "npd_paged_attention_fp8": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                               _I64, _I64, _I64, _I64, _F, _I64, _I64, _I64, _I64,
                                               _P, _I64, _I32, _P]),
    "npd_paged_prefill_workspace_size": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "npd_paged_prefill_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                                   _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F,
                                                   _I64, _I64, _I64, _I64, _P, _I64, _I32, _P]),
    "npd_paged_prefill_attention_fp8": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                                       _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                                       _I64, _I64, _F, _I64, _I64, _I64, _I64, _P,
                                                       _I64, _I32, _P]),
    "npd_copy_blocks": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _I32, _P]),
    "npd_kv_gather_blocks": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P]),
    "npd_kv_scatter_blocks": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P]),
    "npd_qk_norm_rope_store": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                              _I64, _I64, _I64, _I64, _I64, _I64, _F, _I32, _P]),
    "npd_qk_norm_rope_store_fp8": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                  _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                                  _F, _I32, _P]),
    "npd_pack_metadata": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P,
                                         _P, _P]),
}

_lock = threading.Lock()
_lib = None


class NpdError(RuntimeError):
    """A call into libnanopd_hip.so returned an error code."""


def load() -> ctypes.CDLL:
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = Path(os.environ.get("NPD_LIB", LIB_PATH))
            if not path.exists():
                raise RuntimeError(
                    f"{path} is not built; run `python -m nanopd_amd.build` (or "
                    "__graft_entry__.build()) first")
            lib = ctypes.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().npd_last_error().decode(errors="replace")
        raise NpdError(f"nanopd error {rc}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
