"""Committed fixtures: the reference's convert() known answers, and oracle regression cases."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import modules as OM
from oracle.sdpa import dot_product_attention

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _convert_args(case):
  idx = torch.tensor(case["gather_idxs"], dtype=torch.int32)
  mask = torch.tensor(case["gather_mask"], dtype=torch.bool)
  n = int(np.prod(case["arr_shape"]))
  arr = torch.arange(n, dtype=torch.float32).reshape(case["arr_shape"])
  return idx, mask, tuple(case["input_shape"]), arr, tuple(case["layout_axes"])


def test_convert_known_answers_from_reference_tests():
  data = json.load(open(os.path.join(HERE, "convert_known_answers.json")))
  for case in data["cases"]:
    idx, mask, ishape, arr, axes = _convert_args(case)
    out = OM.atom_layout_convert(idx, mask, ishape, arr, layout_axes=axes)
    torch.testing.assert_close(out, torch.tensor(case["expected"], dtype=torch.float32))
  for case in data["rejected"]:
    idx, mask, ishape, arr, axes = _convert_args(case)
    with pytest.raises(ValueError):
      OM.atom_layout_convert(idx, mask, ishape, arr, layout_axes=axes)


def test_oracle_reproduces_committed_regression_fixtures():
  f = np.load(os.path.join(HERE, "oracle_small.npz"))
  for tag in ("scalar", "2", "2x3"):
    g = lambda n: torch.from_numpy(f[f"sdpa808_{tag}_{n}"])
    q = g("q")
    bs = tuple(q.shape[:-3])
    mq = torch.tensor([True, False, True]).expand(*bs, 3)
    mk = torch.tensor([True, False, True, True, False]).expand(*bs, 5)
    out = dot_product_attention(q, g("k"), g("v"), scale=0.4, mask_q=mq, mask_k=mk, bias=g("bias"))
    torch.testing.assert_close(out, g("out"))
  for tr, tag in ((False, "start"), (True, "end")):
    pre = f"tri20_{tag}_param_"
    p = {k[len(pre):]: torch.from_numpy(f[k]) for k in f.files if k.startswith(pre)}
    upd = OM.grid_self_attention(torch.from_numpy(f[f"tri20_{tag}_z"]), torch.from_numpy(f[f"tri20_{tag}_seq"]),
                                 p, transpose=tr, return_update=True)
    torch.testing.assert_close(upd, torch.from_numpy(f[f"tri20_{tag}_update"]), rtol=1e-5, atol=1e-6)
