"""Build the gfx950 C-ABI library in-tree: megaqwen_amd/libmegaqwen_amd.so.

One explicit hipcc invocation (no JIT, no torch extension): the shared
library exports exactly the entry points declared in include/megaqwen_amd.h.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmegaqwen_amd.so")
SOURCES = ["mq_decode.hip", "mq_prefill.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=fast",
    # packed-fp32 (v_pk_*_f32) forms are disabled on this fleet
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: attn_prefill_fa3 parks its block of scores in the AGPRs
    # and needs every MFMA to accumulate in VGPRs; no other kernel's code changes with it
    # (checked instruction for instruction)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I" + os.path.join(ROOT, "include"),
    "-Wno-unused-command-line-argument",
]


def sources() -> list[str]:
    return [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]


def build(verbose: bool = False) -> str:
    """Compile every HIP source into the in-tree shared library; returns its path."""
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, *sources(), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    os.replace(tmp, LIB)
    return LIB


TRACE_SRC = os.path.join(CSRC, "trace", "mq_decode_trace.cpp")
TRACE_BIN = os.path.join(CSRC, "trace", "mq_decode_trace")
PROBE_SRC = os.path.join(CSRC, "trace", "stream_order_probe.hip")
PROBE_BIN = os.path.join(CSRC, "trace", "stream_order_probe")


def build_trace(verbose: bool = False) -> str:
    """Compile the profiling tools: the tracing build of the decode kernel (a stand-alone
    executable that prints the per-stage critical path of a layer) and the stream-order
    probe; returns the tracing build's path."""
    flags = [f for f in FLAGS if f not in ("-fPIC", "-shared")]
    for src, out in ((TRACE_SRC, TRACE_BIN), (PROBE_SRC, PROBE_BIN)):
        cmd = [HIPCC, *flags, src, "-o", out]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    return TRACE_BIN


if __name__ == "__main__":
    if "--trace" in sys.argv[1:]:
        print(build_trace(verbose=True))
    else:
        print(build(verbose=True))
