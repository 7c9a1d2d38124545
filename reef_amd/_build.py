"""Builds reef_amd/libreef_hip.so: every HIP kernel and the C ABI, for gfx950 only.

Run ``python -m reef_amd._build``; ``__graft_entry__.build()`` calls build().
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
SOURCES = ["quant.hip", "prefill.hip", "prefill_packed.hip", "prefill_cache.hip", "decode.hip",
           "kv_append.hip", "int_head.hip", "linear.hip"]
LIB = os.path.join(PKG, "libreef_hip.so")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # No packed fp32 instructions (v_pk_{add,mul,fma}_f32) in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"),
]


def command(extra=None):
    srcs = [os.path.join(PKG, "csrc", s) for s in SOURCES]
    return ["hipcc", *FLAGS, *(extra or []), "-o", LIB + ".tmp", *srcs]


def build(verbose: bool = False) -> str:
    cmd = command()
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature name; that warning is noise.
    noise = "is not a recognized feature for this target"
    msgs = [l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if msgs and verbose:
        print("\n".join(msgs))
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
