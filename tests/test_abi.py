"""The C ABI: library loads, exports every declared entry point, and the ctypes mirrors
have the header's exact struct layouts (checked by compiling the header with gcc)."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from sparsefold_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sparsefold_hip.h"


def declared_functions():
  text = HEADER.read_text()
  return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(sf_hip_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
  lib = _lib.load()
  names = declared_functions()
  assert len(names) >= 9
  for name in names:
    assert hasattr(lib, name), name
  assert {n for n, _, _ in _lib.SIGNATURES} == set(names)
  assert lib.sf_hip_abi_version() == _lib.ABI_VERSION


def test_error_reporting_without_gpu_work():
  lib = _lib.load()
  a = _lib.AttentionArgs()           # all-zero: rejected before any launch
  rc = lib.sf_hip_attention_fwd(ctypes.byref(a), None)
  assert rc != 0
  assert "non-null" in _lib.last_error()
  with pytest.raises(RuntimeError, match="sf_hip_attention_fwd failed"):
    _lib.check(rc, "sf_hip_attention_fwd")
  d = _lib.DiffusionConditioningArgs()
  assert lib.sf_hip_diffusion_conditioning_fwd(ctypes.byref(d), None, 0, None) != 0
  assert "non-null" in _lib.last_error()
  t = _lib.TriangleMultArgs(N=8, C=128)          # refused before any launch: no workspace given
  assert lib.sf_hip_triangle_mult_fwd(ctypes.byref(t), None, 0, None) != 0
  assert "non-null" in _lib.last_error()
  nbytes = lib.sf_hip_triangle_mult_workspace_bytes(8, 128)
  assert nbytes > 0 and lib.sf_hip_triangle_mult_workspace_bytes(8, 64) == 0
  assert lib.sf_hip_triangle_workspace_bytes(0, 128, 4, 32) == 0
  assert lib.sf_hip_triangle_workspace_bytes(768, 128, 4, 32) > 768 * 768 * 128 * 2


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layouts_match_header(tmp_path):
  lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
  for cname, py in _lib.STRUCTS.items():
    lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
    for fname, _ in py._fields_:
      lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
  lines.append("return 0;}")
  src = tmp_path / "layout.c"
  src.write_text("\n".join(lines))
  exe = tmp_path / "layout"
  subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
  out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
  seen = 0
  for line in filter(None, out):
    cname, field, val = line.split()
    py = _lib.STRUCTS[cname]
    expect = ctypes.sizeof(py) if field == "size" else getattr(py, field).offset
    assert int(val) == expect, (cname, field, val, expect)
    seen += 1
  assert seen == sum(len(p._fields_) + 1 for p in _lib.STRUCTS.values())
