"""Writes the committed fixtures under tests/golden/.

1. convert_known_answers.json -- the known-answer vectors of the reference's own tests for
   atom_layout.convert (tests/test_schema.py:76-86 and :187-196), restated as data: inputs,
   expected outputs, and the shapes that must be rejected.
2. oracle_small.npz -- small seeded cases produced by this repository's oracle (float32),
   used as regression fixtures: the seed-808 attention spec of
   tests/test_runtime_reference.py:117-138 and a sharp-weight triangle attention at N=20.

Run from the repository root: python tests/golden/make_fixtures.py
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import modules as OM  # noqa: E402
from oracle.sdpa import dot_product_attention  # noqa: E402
from sparsefold_amd import workloads as W  # noqa: E402


def convert_cases():
  return {
      "source": "tests/test_schema.py:76-86,187-196 of the reference",
      "cases": [
          {"gather_idxs": [[2, 0], [1, 0]], "gather_mask": [[1, 1], [1, 0]], "input_shape": [3],
           "arr_shape": [3, 3], "arr": "arange", "layout_axes": [0],
           "expected": [[[6, 7, 8], [0, 1, 2]], [[3, 4, 5], [0, 0, 0]]]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [3, 2], "arr": "arange", "layout_axes": [0, 1], "expected": [[0, 4], [5, 1]]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [2, 3], "arr": "arange", "layout_axes": [0, 1], "expected": [[0, 4], [5, 1]]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [6], "arr": "arange", "layout_axes": [0], "expected": [[0, 4], [5, 1]]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [4, 2], "arr": "arange", "layout_axes": [0, 1], "expected": [[0, 4], [5, 1]]},
      ],
      "rejected": [
          {"gather_idxs": [[2, 0], [1, 0]], "gather_mask": [[1, 1], [1, 0]], "input_shape": [3],
           "arr_shape": [2, 3], "layout_axes": [0]},
          {"gather_idxs": [[2, 0], [1, 0]], "gather_mask": [[1, 1], [1, 0]], "input_shape": [3],
           "arr_shape": [3, 3], "layout_axes": []},
          {"gather_idxs": [[2, 0], [1, 0]], "gather_mask": [[1, 1], [1, 0]], "input_shape": [3],
           "arr_shape": [3, 3], "layout_axes": [1, 0]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [3, 3], "layout_axes": [0, 1]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [4, 3], "layout_axes": [0, 1]},
          {"gather_idxs": [[0, 4], [5, 1]], "gather_mask": [[1, 1], [1, 1]], "input_shape": [3, 2],
           "arr_shape": [2, 2], "layout_axes": [0, 1]},
      ],
  }


def oracle_cases():
  out = {}
  for bs in [(), (2,), (2, 3)]:
    g = torch.Generator().manual_seed(808)
    q = torch.randn(*bs, 3, 2, 4, generator=g)
    k = torch.randn(*bs, 5, 2, 4, generator=g)
    v = torch.randn(*bs, 5, 2, 6, generator=g)
    bias = torch.randn(*bs, 2, 3, 5, generator=g)
    mq = torch.tensor([True, False, True]).expand(*bs, 3)
    mk = torch.tensor([True, False, True, True, False]).expand(*bs, 5)
    tag = "x".join(map(str, bs)) or "scalar"
    o = dot_product_attention(q, k, v, scale=0.4, mask_q=mq, mask_k=mk, bias=bias)
    for name, t in (("q", q), ("k", k), ("v", v), ("bias", bias), ("out", o)):
      out[f"sdpa808_{tag}_{name}"] = t.numpy()
  for tr in (False, True):
    mod, z, seq = W.make_triangle(20, seed=21, sharp=True, padded=True, transpose=tr, dtype=torch.float32,
                                   act_norm_bias=True)
    p = W.state_dict_f32(mod)
    upd = OM.grid_self_attention(z, seq, p, transpose=tr, return_update=True)
    tag = "end" if tr else "start"
    out[f"tri20_{tag}_z"] = z.numpy()
    out[f"tri20_{tag}_seq"] = seq.numpy()
    out[f"tri20_{tag}_update"] = upd.numpy()
    for k_, v_ in p.items():
      out[f"tri20_{tag}_param_{k_}"] = v_.numpy()
  return out


if __name__ == "__main__":
  with open(os.path.join(HERE, "convert_known_answers.json"), "w") as f:
    json.dump(convert_cases(), f, indent=1)
  np.savez_compressed(os.path.join(HERE, "oracle_small.npz"), **oracle_cases())
  print("wrote convert_known_answers.json, oracle_small.npz")
