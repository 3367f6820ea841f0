"""Builds ``libsparsefold_hip.so`` from ``csrc/*.hip`` for gfx950 with hipcc.

Objects are compiled in parallel into ``sparsefold_amd/_build/`` and linked in-tree, so the
library travels with the source tree.  Every HIP translation unit is compiled with the
packed-fp32 feature disabled and with MFMA accumulators in VGPRs.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsparsefold_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    # MFMA accumulators in VGPRs: left to its heuristics the compiler put the attention
    # kernels' accumulators in AGPRs and copied them to VGPRs and back around every tile
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
  for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
    if cand and Path(cand).exists():
      return cand
  raise RuntimeError("hipcc not found; the HIP library cannot be built")


def _compile(src: Path) -> Path:
  obj = BUILD / (src.stem + ".o")
  cmd = [hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
  res = subprocess.run(cmd, capture_output=True, text=True)
  if res.returncode != 0:
    raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
  return obj


def build(verbose: bool = False) -> Path:
  """Compiles every ``csrc/*.hip`` and links ``libsparsefold_hip.so``; returns its path."""
  BUILD.mkdir(exist_ok=True)
  srcs = sorted(CSRC.glob("*.hip"))
  with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
    objs = list(ex.map(_compile, srcs))
  tmp = LIB.with_suffix(".so.tmp")
  cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
  res = subprocess.run(cmd, capture_output=True, text=True)
  if res.returncode != 0:
    raise RuntimeError(f"link failed:\n{res.stderr}")
  os.replace(tmp, LIB)
  if verbose:
    print(f"built {LIB}")
  return LIB


if __name__ == "__main__":
  build(verbose=True)
