"""ctypes binding of ``libgguf_hip.so`` (the C ABI in ``include/gguf_hip.h``).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7``
dependency resolves (by SONAME) to the HIP runtime torch already loaded:
one runtime per process, so torch's device pointers and ``hipStream_t``
handles are valid in the library.  Loading refuses to continue if two HIP
runtimes end up mapped, and raises if the library has not been built — there
is no fallback path.
"""

from __future__ import annotations

import ctypes
import os

from .ggml import GGMLTypeError

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgguf_hip.so")
ABI_VERSION = 18

ERR_TYPE, ERR_SHAPE, ERR_NULL, ERR_ALIGN, ERR_DTYPE, ERR_BYTES, ERR_HIP = -1, -2, -3, -4, -5, -6, -7
VARIANT_AUTO, VARIANT_DECODE, VARIANT_GEMM = 0, 1, 2
PROLOGUE_NONE, PROLOGUE_RMSNORM, PROLOGUE_SWIGLU = 0, 1, 2
EPILOGUE_STORE, EPILOGUE_ACCUMULATE, EPILOGUE_SWIGLU = 0, 1, 2
DECODE_MAX_M = 32
NOALLOC_ATTENTION_BYTES = 8 << 20

# Every symbol include/gguf_hip.h declares: name -> (restype, argtypes)
_vp, _i32, _i64, _fp = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
SIGNATURES = {
    "gguf_hip_abi_version": (_i32, []),
    "gguf_hip_last_error": (ctypes.c_char_p, []),
    "gguf_hip_type_traits": (_i32, [_i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "gguf_hip_raw_bytes": (_i64, [_i32, _i64, _i64]),
    "gguf_hip_tile_bytes": (_i64, [_i32, _i64, _i64]),
    "gguf_hip_repack": (_i32, [_vp, _i64, _i32, _i64, _i64, _vp, _i64, _vp]),
    "gguf_hip_dequant": (_i32, [_vp, _i32, _i64, _i64, _fp, _i64, _vp]),
    "gguf_hip_dequant_raw": (_i32, [_vp, _i32, _i64, _fp, _vp]),
    "gguf_hip_get_rows": (_i32, [_vp, _i32, _i64, _i64, _vp, _i64, _fp, _i64, _vp]),
    "gguf_hip_matmul": (_i32, [_vp, _i32, _i64, _vp, _i32, _i64, _i64, _fp, _i64, _i64, _vp]),
    "gguf_hip_matmul_variant": (_i32, [_vp, _i32, _i64, _vp, _i32, _i64, _i64, _fp, _i64, _i64,
                                       _i32, _vp]),
    "gguf_hip_matmul_ws": (_i32, [_vp, _i32, _i64, _vp, _i32, _i64, _i64, _fp, _i64, _i64, _i32,
                                  _vp, _i64, _vp]),
    "gguf_hip_matmul_workspace": (_i64, [_i32, _i32, _i64, _i64, _i64]),
    "gguf_hip_matmul_fused": (_i32, [_fp, _vp, _i32, _i64, _i64, _fp, _i32, _fp, ctypes.c_float,
                                     _i32, _vp]),
    "gguf_hip_rmsnorm": (_i32, [_fp, _fp, ctypes.c_float, _fp, _i64, _i64, _vp]),
    "gguf_hip_add_rmsnorm": (_i32, [_fp, _fp, _fp, ctypes.c_float, _fp, _i64, _i64, _vp]),
    "gguf_hip_swiglu": (_i32, [_fp, _fp, _i64, _i64, _vp]),
    "gguf_hip_attention_decode": (_i32, [_fp, _vp, _fp, _fp, _fp, _fp, _fp, _i32, _i32, _i32,
                                         _i64, _vp, _vp]),
    "gguf_hip_attention_workspace": (_i64, [_i32, _i32, _i32, _i64]),
    "gguf_hip_attention_decode_noalloc": (_i32, [_fp, _vp, _fp, _fp, _fp, _fp, _fp, _i32, _i32,
                                                 _i32, _i64, _vp]),
    "gguf_hip_attention_prefill": (_i32, [_fp, _i64, _vp, _i64, _fp, _fp, _fp, _fp, _fp, _i64,
                                          _i32, _i32, _i32, _i64, _vp]),
    "gguf_hip_matmul_attn_merge": (_i32, [_vp, _vp, _i32, _i32, _i32, _i64, _vp, _i32, _i64, _fp,
                                          _i32, _vp]),
    "gguf_hip_argmax": (_i32, [_fp, _i64, _vp, _vp, _vp]),
    "gguf_hip_argmax_workspace": (_i64, []),
}


class GGUFHipError(RuntimeError):
    """A HIP runtime or launch failure reported by the library."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


_lib = None


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    try:
        with open("/proc/self/maps", encoding="utf-8") as f:
            for line in f:
                p = line.split()[-1] if line.strip() else ""
                if os.path.basename(p).startswith("libamdhip64.so"):
                    paths.add(os.path.realpath(p))
    except OSError:
        pass
    return paths


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    import torch  # noqa: F401  — bind to torch's HIP runtime first

    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"{p} is not built; run `python artifex-assistantv5_amd/build.py` "
            "(the GGUF HIP path has no CPU fallback)")
    lib = ctypes.CDLL(p, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.gguf_hip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libgguf_hip ABI {lib.gguf_hip_abi_version()} != {ABI_VERSION}")
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(f"two HIP runtimes mapped in this process: {sorted(runtimes)}")
    if path is None:
        _lib = lib
    return lib


def last_error(lib=None) -> str:
    lib = lib or load_library()
    msg = lib.gguf_hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int, lib=None) -> int:
    """Map a negative return code onto the exception the reference would throw."""
    if rc >= 0:
        return rc
    msg = last_error(lib) or f"libgguf_hip error {rc}"
    if rc == ERR_TYPE:
        raise GGMLTypeError(msg)
    if rc in (ERR_SHAPE, ERR_NULL, ERR_ALIGN, ERR_DTYPE, ERR_BYTES):
        raise ValueError(msg)
    raise GGUFHipError(rc, msg)
