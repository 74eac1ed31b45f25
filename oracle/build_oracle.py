"""Compile the C restatement of the oracle (oracle/gguf_ref_c.c) into
oracle/liboracle.so for the host it runs on: x86-64-v3 (AVX2, FMA) with OpenMP.

Test infrastructure, like the rest of oracle/: the library is loaded only by
tests/ and by the cpu_baseline leg of bench.py.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "gguf_ref_c.c")
LIB = os.path.join(HERE, "liboracle.so")


def build() -> str:
    tmp = LIB + ".tmp"
    subprocess.run(["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-shared", "-fPIC", "-Wall",
                    SRC, "-o", tmp, "-lm"], check=True)
    os.replace(tmp, LIB)
    return LIB


def load():
    """The built library through ctypes, with argument types set; None if it is
    not built."""
    import ctypes

    if not os.path.exists(LIB):
        return None
    lib = ctypes.CDLL(LIB)
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.oracle_dequant_rows_q4_k.argtypes = [p, i64, i64, p, i32]
    lib.oracle_dequant_rows_q4_k.restype = i32
    lib.oracle_matmul_q4_k.argtypes = [p, i64, i64, p, i64, p, i32]
    lib.oracle_matmul_q4_k.restype = i32
    return lib


if __name__ == "__main__":
    print(build())
