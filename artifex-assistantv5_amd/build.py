"""Build ``libgguf_hip.so`` in-tree with hipcc for gfx950.

``python -m`` is awkward for a hyphenated package, so run it as a script:
``python artifex-assistantv5_amd/build.py`` (or call ``build()``).
Objects go to ``_build/`` next to this file; the shared library is written
next to this file, where ``_native.py`` loads it from.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgguf_hip.so")
# every .hip file of csrc/ (the decode kernels are one translation unit per
# ggml type, decode_<type>.hip, so that they compile in parallel)
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    # no packed-fp32 (v_pk_*_f32) instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm install required to build libgguf_hip)")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or res.returncode:
        out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                        if "packed-fp32-ops" not in l)
        if out.strip():
            print(out, file=sys.stderr)
    if res.returncode:
        raise RuntimeError(f"hipcc failed for {src} (exit {res.returncode})")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link ``libgguf_hip.so``; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    workers = max(1, min(len(SOURCES), len(os.sched_getaffinity(0))))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    # Export the C ABI only: kernel stubs and helpers bind locally, so two
    # builds of the library in one process cannot interpose each other.
    vers = os.path.join(BUILD, "exports.map")
    with open(vers, "w", encoding="utf-8") as f:
        f.write("{ global: gguf_hip_*; local: *; };\n")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={vers}",
           *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        print(res.stdout + res.stderr, file=sys.stderr)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
