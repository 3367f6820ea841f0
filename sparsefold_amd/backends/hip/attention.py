"""HIP ``dot_product_attention``: drop-in for the reference op.

Same signature, argument meaning and output layout as
``src/sparsefold/backends/torch/attention/sdpa.py:22-121``:
q ``(..., Q, H, D)``, k ``(..., K, H, D)``, v ``(..., K, H, Dv)``, optional bool masks
``(..., Q)`` / ``(..., K)`` and an additive bias ``(..., H, Q, K)`` that broadcasts against
the batch dims.  Returns ``(..., Q, H, Dv)`` in ``q.dtype``.

Differences by design: the arithmetic is bf16 MFMA with fp32 softmax/accumulation (float32
inputs are rounded to bf16 on entry and the result cast back), and the bias / masks are never
materialised as a ``[B, H, Q, K]`` tensor -- broadcast dims reach the kernel as zero strides.
A keyword-only ``gate`` fuses the ``* sigmoid(gate)`` that every caller applies next.
"""
from __future__ import annotations

import math

import torch

from sparsefold_amd.backends.hip import ops


def _split_batch(shape: tuple[int, ...]) -> tuple[int, int]:
  if len(shape) == 0:
    return 1, 1
  if len(shape) == 1:
    return shape[0], 1
  return math.prod(shape[:-1]), shape[-1]


def _as5(t: torch.Tensor, batch: tuple[int, ...], b0: int, b1: int) -> torch.Tensor:
  """Broadcast ``t`` to ``batch + t.shape[-3:]`` and view it as ``[B0, B1, ...]``."""
  if t.stride(-1) != 1:
    t = t.contiguous()
  t = t.expand(*batch, *t.shape[-3:])
  return t.reshape(b0, b1, *t.shape[-3:])


def dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          scale: float | None = None,
                          mask_q: torch.Tensor | None = None,
                          mask_k: torch.Tensor | None = None,
                          bias: torch.Tensor | None = None,
                          *, gate: torch.Tensor | None = None, schedule: int = 0) -> torch.Tensor:
  if q.ndim < 3 or k.ndim < 3 or v.ndim < 3:
    raise ValueError("dot_product_attention: q, k, v need (..., L, H, D) layouts")
  dtype = q.dtype
  batch = tuple(q.shape[:-3])
  Q, H, D = q.shape[-3:]
  K = k.shape[-3]
  Dv = v.shape[-1]
  if tuple(k.shape[:-3]) != batch or tuple(v.shape[:-3]) != batch:
    raise ValueError("dot_product_attention: q, k, v batch dims differ")
  if k.shape[-2:] != (H, D) or v.shape[-3:-1] != (K, H):
    raise ValueError(f"dot_product_attention: shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
  if scale is None:
    scale = 1.0 / math.sqrt(D)
  b0, b1 = _split_batch(batch)
  bf = torch.bfloat16
  q5 = _as5(q.to(bf), batch, b0, b1)
  k5 = _as5(k.to(bf), batch, b0, b1)
  v5 = _as5(v.to(bf), batch, b0, b1)
  bias5 = None
  if bias is not None:
    bias5 = _as5(bias.to(bf), batch, b0, b1)
  mq5 = mk5 = None
  if mask_q is not None:
    mq = ops._u8(mask_q).expand(*batch, Q)
    mq5 = mq.reshape(b0, b1, Q)
  if mask_k is not None:
    mk = ops._u8(mask_k).expand(*batch, K)
    mk5 = mk.reshape(b0, b1, K)
  g5 = None
  if gate is not None:
    g5 = _as5(gate.to(bf).reshape(*batch, Q, H, Dv), batch, b0, b1)
  out = torch.empty((*batch, Q, H, Dv), dtype=bf, device=q.device)
  ops.attention(q5, k5, v5, scale=scale, bias=bias5, mask_q=mq5, mask_k=mk5, gate=g5,
                out=out.view(b0, b1, Q, H, Dv), schedule=schedule)
  return out if dtype == bf else out.to(dtype)
