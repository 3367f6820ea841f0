"""HIP dot_product_attention vs the oracle (float32 restatement of sdpa.py:22-121)."""
import pytest
import torch

from oracle.sdpa import dot_product_attention as oracle_dpa
from sparsefold_amd.backends.hip.attention import dot_product_attention as hip_dpa
from tests._metrics import assert_close_bf16, bf16_round

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(q, k, v, **kw):
  """HIP on bf16 inputs; oracle in float32 on the same (bf16-rounded) values."""
  cast = lambda t: None if t is None else t.to(DEV, torch.bfloat16)
  mq, mk = kw.pop("mask_q", None), kw.pop("mask_k", None)
  bias = kw.pop("bias", None)
  gate = kw.pop("gate", None)
  schedule = kw.pop("schedule", 0)
  out = hip_dpa(cast(q), cast(k), cast(v), mask_q=None if mq is None else mq.to(DEV),
                mask_k=None if mk is None else mk.to(DEV), bias=cast(bias), gate=cast(gate),
                schedule=schedule, **kw)
  torch.cuda.synchronize()
  ref = oracle_dpa(bf16_round(q), bf16_round(k), bf16_round(v), mask_q=mq, mask_k=mk,
                   bias=None if bias is None else bf16_round(bias), **kw)
  if gate is not None:
    ref = ref * torch.sigmoid(bf16_round(gate))
  return out.float().cpu(), ref


@pytest.mark.parametrize("batch_shape", [(), (2,), (2, 3)])
@pytest.mark.parametrize("with_masks", [False, True])
def test_reference_spec_seed808(batch_shape, with_masks):
  """Shapes / masks of tests/test_runtime_reference.py:117-138 (incl. a fully masked query, D=4, Dv=6)."""
  gen = torch.Generator().manual_seed(808)
  q = torch.randn(*batch_shape, 3, 2, 4, generator=gen)
  k = torch.randn(*batch_shape, 5, 2, 4, generator=gen)
  v = torch.randn(*batch_shape, 5, 2, 6, generator=gen)
  bias = torch.randn(*batch_shape, 2, 3, 5, generator=gen)
  mq = torch.tensor([True, False, True]).expand(*batch_shape, 3) if with_masks else None
  mk = torch.tensor([True, False, True, True, False]).expand(*batch_shape, 5) if with_masks else None
  out, ref = _run(q, k, v, scale=0.4, mask_q=mq, mask_k=mk, bias=bias)
  assert_close_bf16(out, ref, f"seed808 {batch_shape} masks={with_masks}")


def test_reference_gpu_spec_seed610():
  """tests/test_runtime_gpu.py:28-41 shapes (Dv=12 != D=16, bias per batch, key mask)."""
  gen = torch.Generator().manual_seed(610)
  q = torch.randn(2, 7, 3, 16, generator=gen)
  k = torch.randn(2, 9, 3, 16, generator=gen)
  v = torch.randn(2, 9, 3, 12, generator=gen)
  bias = torch.randn(2, 3, 7, 9, generator=gen)
  mk = torch.tensor([[True, False, True, True, True, False, True, False, True]]).expand(2, 9)
  out, ref = _run(q, k, v, mask_k=mk, bias=bias, scale=0.3)
  assert_close_bf16(out, ref, "seed610")


@pytest.mark.parametrize("D", [16, 24, 32, 48, 64])
@pytest.mark.parametrize("QK", [(77, 133), (128, 64), (200, 300)])
def test_head_dims_tails_masks_bias_gate(D, QK):
  Q, K = QK
  g = torch.Generator().manual_seed(1000 + D + Q)
  B, H = 2, 3
  q, k = torch.randn(B, Q, H, D, generator=g), torch.randn(B, K, H, D, generator=g)
  v = torch.randn(B, K, H, D, generator=g)
  bias = torch.randn(H, Q, K, generator=g)            # broadcast over the batch (stride 0)
  gate = torch.randn(B, Q, H, D, generator=g)
  mq = torch.rand(B, Q, generator=g) > 0.1
  mk = torch.rand(B, K, generator=g) > 0.3
  mk[1, :] = False                                    # batch 1: every query fully masked
  out, ref = _run(q, k, v, mask_q=mq, mask_k=mk, bias=bias, gate=gate)
  assert_close_bf16(out, ref, f"D={D} Q={Q} K={K}")


@pytest.mark.parametrize("D", [32, 48])
def test_shared_tile_workgroups(D):
  """Enough (batch, head) pairs that the kernel runs 4-wave workgroups sharing K/V tiles
  (at least 512 groups of 128 queries), with ragged query / key ranges, masks, bias, gate."""
  Q, K, B, H = 260, 257, 4, 48
  g = torch.Generator().manual_seed(2000 + D)
  q, k = torch.randn(B, Q, H, D, generator=g), torch.randn(B, K, H, D, generator=g)
  v = torch.randn(B, K, H, D, generator=g)
  bias = torch.randn(H, Q, K, generator=g)
  gate = torch.randn(B, Q, H, D, generator=g)
  mq = torch.rand(B, Q, generator=g) > 0.1
  mk = torch.rand(B, K, generator=g) > 0.3
  mk[2, :] = False
  out, ref = _run(q, k, v, mask_q=mq, mask_k=mk, bias=bias, gate=gate)
  assert_close_bf16(out, ref, f"shared D={D}")


def test_fully_masked_rows_are_exact_means():
  g = torch.Generator().manual_seed(5)
  q, k = torch.randn(1, 70, 2, 32, generator=g), torch.randn(1, 150, 2, 32, generator=g)
  v = torch.randn(1, 150, 2, 32, generator=g)
  bias = 5 * torch.randn(1, 2, 70, 150, generator=g)
  mq = torch.ones(1, 70, dtype=torch.bool)
  mq[0, ::3] = False
  out, _ = _run(q, k, v, mask_q=mq, bias=bias)
  mean = bf16_round(v).mean(1)                         # [1, 2, 32] over all 150 keys
  rows = out[0, ~mq[0]]                               # [n_masked, 2, 32]
  diff = (rows - mean).abs().max().item()
  print(f"[parity] fully masked rows: max |out - mean(v)| = {diff:.3e}")
  assert diff <= 2 ** -8 * mean.abs().max().item() + 1e-6


def test_no_mask_no_bias_and_known_answer():
  g = torch.Generator().manual_seed(6)
  q, k, v = (torch.randn(3, 40, 4, 32, generator=g) for _ in range(3))
  out, ref = _run(q, k, v)
  assert_close_bf16(out, ref, "plain")
  ones = torch.ones(2, 1, 3, device=DEV, dtype=torch.bfloat16)
  torch.testing.assert_close(hip_dpa(ones, ones, ones).float(), ones.float())


def test_fp32_inputs_round_trip_dtype():
  g = torch.Generator().manual_seed(7)
  q, k, v = (torch.randn(2, 33, 2, 32, generator=g).to(DEV) for _ in range(3))
  out = hip_dpa(q, k, v)
  assert out.dtype == torch.float32
  ref = oracle_dpa(bf16_round(q.cpu()), bf16_round(k.cpu()), bf16_round(v.cpu()))
  assert_close_bf16(out, ref, "fp32 in/out")


@pytest.mark.parametrize("mode", ["s", "p"])
def test_reference_point_moves_after_the_first_tile(mode):
  """The softmax keeps the first 64-key tile's maximum as its reference point and moves it only
  when a later tile's weight mass passes 2^60.  Three ways to get there, checked against the
  oracle: the first tile fully masked, logits 90 (log2 units) higher in a later tile, and both
  in one batch (shared-tile and per-wave task modes)."""
  gen = torch.Generator().manual_seed(99)
  B, Q, K, H, D = 3, 160, 320, 2, 32
  q = torch.randn(B, Q, H, D, generator=gen)
  k = torch.randn(B, K, H, D, generator=gen)
  v = torch.randn(B, K, H, D, generator=gen)
  bias = torch.randn(B, H, Q, K, generator=gen)
  mk = torch.ones(B, K, dtype=torch.bool)
  mk[0, :64] = False                                     # batch 0: the first tile is all masked
  bias[1, :, :, 200:] += 90.0 / 1.4426950408889634       # batch 1: +90 in log2 units after tile 3
  mk[2, :70] = False                                     # batch 2: both
  bias[2, :, :, 250:] += 70.0 / 1.4426950408889634
  out, ref = _run(q, k, v, mask_k=mk, bias=bias, schedule=1 if mode == "s" else 2)
  assert_close_bf16(out, ref, f"reference point moves ({mode})")


# ---- shared-bias kernel (schedule 3): 5 samples, head dim 48, one bias for every sample ----

def _sb_inputs(N, H, seed, *, mask_frac=0.0, gate=True):
  g = torch.Generator().manual_seed(seed)
  S, D = 5, 48
  q, k, v = (torch.randn(S, N, H, D, generator=g) for _ in range(3))
  bias = torch.randn(H, N, N, generator=g)                 # shared by the 5 samples (stride 0)
  mk = None
  if mask_frac:
    mk = torch.rand(N, generator=g) > mask_frac            # one key mask for every sample
  gt = torch.randn(S, N, H, D, generator=g) if gate else None
  return q, k, v, bias, mk, gt


@pytest.mark.parametrize("N,H,mask_frac,gate", [(256, 2, 0.0, True), (512, 3, 0.3, True), (768, 1, 0.0, False)])
def test_shared_bias_kernel_matches_oracle(N, H, mask_frac, gate):
  """Diffusion-transformer shape family (DiffusionSelfAttention.cpp:391,555: one pair bias for all
  samples): the shared-bias kernel against the float32 oracle, with and without a key mask / gate."""
  q, k, v, bias, mk, gt = _sb_inputs(N, H, 4000 + N + H, mask_frac=mask_frac, gate=gate)
  out, ref = _run(q, k, v, bias=bias, mask_k=mk, gate=gt, schedule=3)
  assert_close_bf16(out, ref, f"shared-bias N={N} H={H} mask={mask_frac} gate={gate}")


def test_shared_bias_kernel_agrees_with_tile_kernels_at_diffusion_size():
  """5 x 1024 tokens, 16 heads (the C4 block's attention): the shared-bias kernel against the
  shared-tile kernel on the same GPU inputs (same arithmetic up to fp32 summation order and the
  reference point of the softmax)."""
  g = torch.Generator(device=DEV).manual_seed(77)
  S, N, H, D = 5, 1024, 16, 48
  bf = torch.bfloat16
  q, k, v, gt = (torch.randn(S, N, H, D, device=DEV, generator=g).to(bf) for _ in range(4))
  bias = torch.randn(H, N, N, device=DEV, generator=g).to(bf)
  mk = torch.ones(N, dtype=torch.bool, device=DEV)
  mk[-N // 10:] = False
  outs = [hip_dpa(q, k, v, bias=bias, mask_k=mk, gate=gt, schedule=sch).float() for sch in (3, 1)]
  torch.cuda.synchronize()
  assert_close_bf16(outs[0].cpu(), outs[1].cpu(), "shared-bias vs shared-tile, 5x1024, H=16")


def test_shared_bias_kernel_exact_path_for_flagged_rows():
  """Rows the fast path cannot serve with its fixed reference point: every key masked (mean of V
  over all keys) and logits 200 above the rest (weight sum past 2^100), recomputed exactly."""
  N, H = 256, 2
  q, k, v, bias, _, gt = _sb_inputs(N, H, 4242, gate=True)
  bias[0, 5, 17] += 200.0                                  # one huge logit: row (h 0, q 5) overflows
  bias[1, 70:90, :] += 120.0                               # rows whose sum passes 2^100 on every key
  out, ref = _run(q, k, v, bias=bias, gate=gt, schedule=3)
  assert_close_bf16(out, ref, "shared-bias flagged rows (overflow)")
  mk = torch.zeros(N, dtype=torch.bool)                    # every key masked
  out, ref = _run(q, k, v, bias=bias, mask_k=mk, schedule=3)
  assert_close_bf16(out, ref, "shared-bias, every key masked")
  mean = bf16_round(v).mean(1)                             # [5, H, 48]
  diff = (out - mean[:, None]).abs().max().item()
  assert diff <= 2 ** -8 * mean.abs().max().item() + 1e-6, diff


def test_shared_bias_kernel_refuses_other_shapes():
  q, k, v, bias, _, _ = _sb_inputs(256, 2, 1)
  with pytest.raises(RuntimeError, match="schedule 3"):
    _run(q[..., :32], k[..., :32], v[..., :32], bias=bias, schedule=3)   # head dim 32
  with pytest.raises(RuntimeError, match="schedule 3"):
    _run(q[:4], k[:4], v[:4], bias=bias, schedule=3)                     # 4 samples
