"""Oracle restatement of ``dot_product_attention`` (the Torch math path).

TEST INFRASTRUCTURE: imported only by tests, smoke() and bench's CPU baseline.

Follows ``src/sparsefold/backends/torch/attention/sdpa.py:22-121``:
  1. additive ``attn_bias`` of shape ``(..., 1, Q, K)`` in ``q.dtype``, filled
     with ``-finfo(q.dtype).max`` where ``mask_q`` or ``mask_k`` is False
     (masked_fill, so a doubly masked logit is still exactly ``-max``), then
     ``+ bias.to(q.dtype)``                                     (:62-80)
  2. batch dims flattened, layout ``(B, H, L, D)``               (:85-95)
  3. ``F.scaled_dot_product_attention`` under the MATH backend   (:98-114)
  4. layout restored to ``(..., Q, H, Dv)``                      (:116-121)

Consequence used throughout the tests: a query row whose every key is masked
has all logits equal to ``-max`` and therefore returns the plain mean of V
over *all* keys (masked ones included).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          scale: float | None = None,
                          mask_q: torch.Tensor | None = None,
                          mask_k: torch.Tensor | None = None,
                          bias: torch.Tensor | None = None) -> torch.Tensor:
  """q ``(..., Q, H, D)``, k ``(..., K, H, D)``, v ``(..., K, H, Dv)``,
  masks ``(..., Q)`` / ``(..., K)`` bool, bias ``(..., H, Q, K)`` broadcastable.
  Returns ``(..., Q, H, Dv)`` in ``q.dtype``."""
  dtype = q.dtype
  batch_shape = q.shape[:-3]
  attn_bias = None
  if mask_q is not None or mask_k is not None or bias is not None:
    min_val = -float(torch.finfo(dtype).max)
    attn_bias = torch.zeros(batch_shape + (1, q.shape[-3], k.shape[-3]), dtype=dtype, device=q.device)
    if mask_q is not None:
      attn_bias.masked_fill_(~mask_q[..., None, :, None].bool(), min_val)
    if mask_k is not None:
      attn_bias.masked_fill_(~mask_k[..., None, None, :].bool(), min_val)
    if bias is not None:
      attn_bias = attn_bias + bias.to(dtype)
  qf = q.reshape((-1,) + q.shape[-3:]).transpose(-3, -2)
  kf = k.reshape((-1,) + k.shape[-3:]).transpose(-3, -2)
  vf = v.reshape((-1,) + v.shape[-3:]).transpose(-3, -2)
  if attn_bias is not None:
    if attn_bias.shape[:-3] != batch_shape:
      attn_bias = attn_bias.expand(*batch_shape, *attn_bias.shape[-3:])
    attn_bias = attn_bias.reshape((-1,) + attn_bias.shape[-3:])
  with torch.nn.attention.sdpa_kernel(backends=[torch.nn.attention.SDPBackend.MATH]):
    out = F.scaled_dot_product_attention(qf, kf, vf, attn_mask=attn_bias, scale=scale)
  out = out.transpose(-3, -2)
  return out.reshape(*batch_shape, *out.shape[-3:])
