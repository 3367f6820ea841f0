"""Oracle restatement of SparseFold's projection / norm / gate primitives.

TEST INFRASTRUCTURE: imported only by tests, smoke() and bench's CPU baseline.

Follows ``src/sparsefold/model/layers/primitives.py``:
* ``linear``               -- ``Linear.forward`` (:328-372): einsum over the
  trailing input dims, input cast to the weight dtype, bias add, optional
  post-op, output cast back to the input dtype.  Weight layout is the
  reference's: ``[*in, *out]`` by default, ``[*out, *in]`` with
  ``transpose_weights=True`` (:231-253).
* ``cpu_bounded_sigmoid``  -- ``_cpu_bounded_sigmoid`` (:163-175).
* ``sigmoid_post_op``      -- ``apply_linear_post_op`` (:144-160): CPU uses the
  bounded sigmoid, other devices ``torch.sigmoid``.
* ``layer_norm``           -- ``LayerNorm.forward`` (:471-497): normalise in
  ``compute_dtype`` (input dtype when None), eps 1e-5, cast back.
* ``swish`` / ``gated_linear_unit`` -- ``swish`` (:688-699, CPU form: bounded sigmoid, zero
  below -20) and ``gated_linear_unit`` (:645-685): ``x @ W`` with ``W`` ``[K, 2, N]``
  collapsed to ``[K, 2N]``, ``swish(first half) * second half``, cast to the input dtype.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

LN_EPS = 1e-5


def cpu_bounded_sigmoid(x: torch.Tensor) -> torch.Tensor:
  """primitives.py:163-175: clamp to +-20, exp(-|x|) as Taylor5(-|x|/256)^(2^8)."""
  bounded = x.to(torch.float32).clamp(-20, 20)
  z = -bounded.abs() / 256.0
  e = 1.0 + z * (1.0 + z * (0.5 + z * (1.0 / 6.0 + z * (1.0 / 24.0 + z / 120.0))))
  for _ in range(8):
    e = e * e
  den = 1.0 + e
  return torch.where(bounded >= 0, 1.0 / den, e / den).to(x.dtype)


def sigmoid_post_op(x: torch.Tensor) -> torch.Tensor:
  """primitives.py:157-159: bounded sigmoid on CPU, torch.sigmoid elsewhere."""
  if x.device.type == "cpu":
    return cpu_bounded_sigmoid(x)
  return torch.sigmoid(x)


def _equation(n_in: int, n_out: int, transpose_weights: bool) -> str:
  """primitives.py:241-253 einsum equation for arbitrary-rank in/out dims."""
  ins = "abcde"[:n_in]
  outs = "hijkl"[:n_out]
  if transpose_weights:
    return f"...{ins},{outs}{ins}->...{outs}"
  return f"...{ins},{ins}{outs}->...{outs}"


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
           n_in: int = 1, transpose_weights: bool = False, post_op: str | None = None,
           residual: torch.Tensor | None = None) -> torch.Tensor:
  """primitives.py:328-372 (Linear.forward)."""
  in_dtype = x.dtype
  if in_dtype != weight.dtype:
    x = x.to(weight.dtype)
  n_out = weight.ndim - n_in
  out = torch.einsum(_equation(n_in, n_out, transpose_weights), x, weight)
  if bias is not None:
    out = out + bias
  if residual is not None:
    out = out + residual.to(out.dtype)
  if post_op == "sigmoid":
    out = sigmoid_post_op(out)
  elif post_op is not None:
    raise ValueError(f"unsupported post_op {post_op!r}")
  return out.to(in_dtype)


def layer_norm(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
               compute_dtype: torch.dtype | None = None, eps: float = LN_EPS) -> torch.Tensor:
  """primitives.py:471-497 (LayerNorm.forward over the last dim)."""
  dtype = x.dtype
  y = x.to(compute_dtype) if compute_dtype is not None else x
  if weight is not None and weight.dtype != y.dtype:
    weight = weight.to(y.dtype)
  if bias is not None and bias.dtype != y.dtype:
    bias = bias.to(y.dtype)
  out = F.layer_norm(y, (y.shape[-1],), weight, bias, eps)
  return out.to(dtype)


def swish(x: torch.Tensor) -> torch.Tensor:
  """primitives.py:688-699 on the CPU: x * bounded sigmoid(x), exactly 0 below -20."""
  if x.device.type == "cpu":
    return torch.where(x < -20, torch.zeros_like(x), x * cpu_bounded_sigmoid(x))
  return x * torch.sigmoid(x)


def gated_linear_unit(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
  """primitives.py:645-685 with the swish activation: weight ``[K, 2, N]`` (or ``[K, 2N]``)."""
  w = weight.reshape(weight.shape[0], -1)
  if x.dtype != w.dtype:
    w = w.to(x.dtype)
  y = torch.matmul(x, w)
  a, b = torch.tensor_split(y, 2, dim=-1)
  return (swish(a) * b).to(x.dtype)
