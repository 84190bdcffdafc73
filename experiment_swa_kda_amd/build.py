"""Builds libkda_mi355x.so (gfx950) in-tree with hipcc.

Usage: python -m experiment_swa_kda_amd.build   (or build() from Python).

Every HIP source is compiled for gfx950 only, with packed-f32 instruction selection
disabled (-Xclang -target-feature -Xclang -packed-fp32-ops), and linked into one shared
library next to this file.  Objects go to ``_build/`` at the repository root.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import re
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_NAME = "libkda_mi355x.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

SOURCES = ["capi.cpp", "decode.hip", "conv.hip", "norm_gate.hip", "chunk_fwd.hip", "chunk_bwd.hip", "softcap_ce.hip",
           "weight_grad.hip", "trainer_ops.hip", "mfma_probe.hip", "generic.hip"]
# Per-source extra flags.  The chunk kernels keep MFMA accumulators in VGPRs: their
# accumulators feed VALU work every step, and the AGPR form costs a copy per element.
EXTRA_FLAGS = {
    "chunk_fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "chunk_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the MI355X KDA library needs ROCm's hipcc")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-fPIC",
        "-std=c++17",
        "-Wall",
        "-Wno-unused-function",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{os.path.join(ROOT, 'include')}",
    ]


def vgpr_spills(remarks: str) -> dict[str, int]:
    """Kernels with spilled VGPRs, from hipcc's kernel-resource-usage remarks."""
    out, name = {}, None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"VGPRs Spill: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            out[name] = int(m.group(1))
    return out


def _compile(src: str) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    remarks = ["-Rpass-analysis=kernel-resource-usage"] if src.endswith(".hip") else []
    cmd = [_hipcc(), *_flags(), *EXTRA_FLAGS.get(src, []), *remarks, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    # A VGPR spill is refused: this compiler has placed a spill store in a join block
    # before the instruction that restores the full exec mask, so only some lanes saved
    # the value and the reload gave the others garbage (wrong dq / dk, no error).
    spills = vgpr_spills(proc.stderr)
    if spills:
        os.remove(obj)
        raise RuntimeError(f"{src}: kernels spill VGPRs (refused): {spills}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile all sources and link the shared library; returns its path."""
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
