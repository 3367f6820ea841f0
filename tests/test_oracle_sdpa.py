"""Pins oracle.sdpa.dot_product_attention (restating sdpa.py:22-121)."""
import numpy as np
import pytest
import torch

from oracle import brute
from oracle.sdpa import dot_product_attention


def _bcast(bias, batch, H, Q, K):
  return np.broadcast_to(bias.numpy(), batch + (H, Q, K)).reshape((-1, H, Q, K))


@pytest.mark.parametrize("batch_shape", [(), (2,), (2, 3)])
@pytest.mark.parametrize("with_masks", [False, True])
def test_reference_spec_matches_explicit_sdpa(batch_shape, with_masks):
  """The reference test tests/test_runtime_reference.py:117-138 (seed 808): explicit additive
  -finfo.max mask + bias into torch SDPA MATH."""
  gen = torch.Generator().manual_seed(808)
  q = torch.randn(*batch_shape, 3, 2, 4, generator=gen)
  k = torch.randn(*batch_shape, 5, 2, 4, generator=gen)
  v = torch.randn(*batch_shape, 5, 2, 6, generator=gen)
  bias = torch.randn(*batch_shape, 2, 3, 5, generator=gen)
  mask_q = torch.tensor([True, False, True]).expand(*batch_shape, 3) if with_masks else None
  mask_k = torch.tensor([True, False, True, True, False]).expand(*batch_shape, 5) if with_masks else None
  actual = dot_product_attention(q, k, v, scale=0.4, mask_q=mask_q, mask_k=mask_k, bias=bias)
  attn_bias = torch.zeros(*batch_shape, 1, 3, 5)
  if with_masks:
    attn_bias.masked_fill_(~mask_q[..., None, :, None], -float(torch.finfo(q.dtype).max))
    attn_bias.masked_fill_(~mask_k[..., None, None, :], -float(torch.finfo(q.dtype).max))
  attn_bias = attn_bias + bias
  with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
    expected = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(-3, -2), k.transpose(-3, -2), v.transpose(-3, -2), attn_mask=attn_bias, scale=0.4).transpose(-3, -2)
  torch.testing.assert_close(actual, expected)
  # and the float64 brute force (independent of torch SDPA)
  B = int(np.prod(batch_shape)) if batch_shape else 1
  mq = mask_q.reshape(B, 3).numpy() if with_masks else None
  mk = mask_k.reshape(B, 5).numpy() if with_masks else None
  ref = brute.attention(q.reshape(B, 3, 2, 4).numpy(), k.reshape(B, 5, 2, 4).numpy(), v.reshape(B, 5, 2, 6).numpy(),
                        0.4, mq, mk, _bcast(bias, batch_shape, 2, 3, 5))
  np.testing.assert_allclose(actual.reshape(B, 3, 2, 6).numpy(), ref, rtol=2e-5, atol=2e-6)


def test_fully_masked_row_is_mean_of_all_values():
  gen = torch.Generator().manual_seed(1)
  q, k = torch.randn(1, 4, 2, 8, generator=gen), torch.randn(1, 6, 2, 8, generator=gen)
  v, bias = torch.randn(1, 6, 2, 5, generator=gen), 3 * torch.randn(1, 2, 4, 6, generator=gen)
  mask_k = torch.zeros(1, 6, dtype=torch.bool)
  out = dot_product_attention(q, k, v, mask_k=mask_k, bias=bias)
  torch.testing.assert_close(out, v.mean(1, keepdim=True).expand(1, 4, 2, 5))
  mask_q = torch.tensor([[True, False, True, False]])
  out = dot_product_attention(q, k, v, mask_q=mask_q, bias=bias)
  torch.testing.assert_close(out[:, 1], v.mean(1))
  assert not torch.allclose(out[:, 0], v.mean(1))


def test_known_answers():
  q = torch.ones(2, 1, 3)                           # tests/test_runtime_reference.py:141-145
  torch.testing.assert_close(dot_product_attention(q, q, q), q)
  gen = torch.Generator().manual_seed(2)
  v = torch.randn(3, 1, 2, 4, generator=gen)       # single key -> v
  out = dot_product_attention(torch.randn(3, 5, 2, 4, generator=gen), torch.randn(3, 1, 2, 4, generator=gen), v)
  torch.testing.assert_close(out, v.expand(3, 5, 2, 4))
  k = torch.randn(1, 7, 2, 4, generator=gen)       # zero logits -> uniform mean
  v = torch.randn(1, 7, 2, 3, generator=gen)
  out = dot_product_attention(torch.zeros(1, 2, 2, 4), k, v)
  torch.testing.assert_close(out, v.mean(1, keepdim=True).expand(1, 2, 2, 3))
  bias = torch.randn(1, 2, 2, 7, generator=gen)    # bias-only logits -> softmax(bias) V
  out = dot_product_attention(torch.zeros(1, 2, 2, 4), k, v, bias=bias)
  exp = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(bias, -1), v)
  torch.testing.assert_close(out, exp)


def test_partially_masked_keys_get_zero_weight():
  gen = torch.Generator().manual_seed(3)
  q, k, v = (torch.randn(1, 3, 1, 4, generator=gen) for _ in range(3))
  mask_k = torch.tensor([[True, False, True]])
  out = dot_product_attention(q, k, v, mask_k=mask_k)
  sub = dot_product_attention(q, k[:, [0, 2]], v[:, [0, 2]])
  torch.testing.assert_close(out, sub)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_shapes_against_brute_force(seed):
  g = torch.Generator().manual_seed(100 + seed)
  B, Q, K, H, D, Dv = 2, 5 + seed, 7 + 2 * seed, 3, 4 + seed, 3 + seed
  q, k = torch.randn(B, Q, H, D, generator=g), torch.randn(B, K, H, D, generator=g)
  v, bias = torch.randn(B, K, H, Dv, generator=g), torch.randn(B, H, Q, K, generator=g)
  mq = torch.rand(B, Q, generator=g) > 0.3
  mk = torch.rand(B, K, generator=g) > 0.4
  mk[0] = False                                     # one fully masked batch
  out = dot_product_attention(q, k, v, scale=0.7, mask_q=mq, mask_k=mk, bias=bias)
  ref = brute.attention(q.numpy(), k.numpy(), v.numpy(), 0.7, mq.numpy(), mk.numpy(), bias.numpy())
  np.testing.assert_allclose(out.numpy(), ref, rtol=2e-5, atol=2e-6)
