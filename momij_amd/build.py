"""Build libmomij_hip.so in-tree with hipcc for gfx950.

Each source compiles to an object under momij_amd/_build/ (in parallel), then one link.
Compiled every time build() is called; importers only load what is already built.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmomij_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    # no packed fp32 ops are generated (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result", "-Wno-unused-value",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]
# Measurement variants: MJ_BUILD_DEFINES="NAME=VALUE ..." adds -DNAME=VALUE to every compile
# (e.g. MJ_TILE_MIN_ROWS=2 builds the one-row MoE through the VALU GEMV path).
FLAGS += ["-D" + d for d in os.environ.get("MJ_BUILD_DEFINES", "").split()]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


# Kernels whose waits count their own outstanding vector-memory requests (s_waitcnt vmcnt(N)
# with N > 0): a register spill to scratch memory would add requests to that count, so none
# may use scratch (SGPR spills into VGPR lanes, which issue no memory requests, are allowed).
COUNTED_WAIT_KERNELS = ("k_gather5", "k_moe_fused", "k_lm_head")


def _spills(stderr: str) -> list:
    """(kernel, what) of the counted-wait kernels that spill VGPRs or use scratch memory, from
    the resource remarks of one compile."""
    out, cur = [], None
    for line in stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            continue
        if not cur or not any(k in cur for k in COUNTED_WAIT_KERNELS):
            continue
        m = re.search(r"VGPRs Spill: (\d+)", line)
        if m and int(m.group(1)) > 0:
            out.append((cur, f"{m.group(1)} VGPR spills"))
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            out.append((cur, f"{m.group(1)} scratch bytes a lane"))
    return out


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-x", "hip", *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    bad = _spills(r.stderr)
    if bad:
        raise RuntimeError(f"{src}: kernels with counted waits spill registers: {bad}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
