"""Compile the HIP sources in ../csrc into dsmoe/libdsmoe.so for gfx950.

Run as ``python -m dsmoe.build`` (from deepseek-v3-lite_amd/) or through
``__graft_entry__.build()``.  hipcc cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent                      # deepseek-v3-lite_amd/
REPO = ROOT.parent
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
BUILD = ROOT / "_build"
LIB = PKG / "libdsmoe.so"
PROBE_LIB = PKG / "libdsmoe_probe.so"     # measurement tooling (bench.py --dma-mb), not the layer

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # No packed-FP32 instructions in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
# Per-source flags: the attention kernels keep MFMA accumulators in VGPRs (their
# online-softmax rescaling reads and writes them every key block).
EXTRA_FLAGS = {"mla.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
SOURCES = ["api.hip", "gate.hip", "permute.hip", "gemm.hip", "gemm_qp.hip", "gemm_sk.hip", "gemm_x.hip", "gemm_xm.hip", "gemm_xq.hip", "bwd.hip", "combine.hip", "mla.hip"]
PROBE_SOURCES = ["probe.hip"]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if warn:
        print(f"[dsmoe.build] {src.name}:\n{warn}", file=sys.stderr)
    return obj


def _link(objs, out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{r.stdout}\n{r.stderr}")
    tmp.replace(out)


def build(verbose: bool = True) -> Path:
    """Compile every source and link libdsmoe.so and the measurement probe
    library libdsmoe_probe.so (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES + PROBE_SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs[:len(SOURCES)], LIB)
    _link(objs[len(SOURCES):], PROBE_LIB)
    if verbose:
        print(f"[dsmoe.build] built {LIB} ({LIB.stat().st_size} bytes) and {PROBE_LIB.name}")
    return LIB


if __name__ == "__main__":
    build()
