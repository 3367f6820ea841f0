"""Tolerance checks shared by the GPU parity tests.

The bar (bf16 output vs float32 oracle): max-abs <= 2e-2 and rel-L2 <= 1e-2.  Outputs that
the reference itself stores in bf16 with magnitudes of several units (the pair-logit packs) may
also be given an elementwise relative allowance of one bf16 ulp (2^-7 |expected|), the storage
resolution of the reference's own result.
"""
import torch

MAX_ABS = 2e-2
REL_L2 = 1e-2


BF16_ULP = 2.0 ** -7


def errors(actual: torch.Tensor, expected: torch.Tensor, rtol: float = 0.0) -> tuple[float, float]:
  """(max over elements of |a - e| - rtol |e|, ||a - e|| / ||e||)."""
  a = actual.detach().float().cpu()
  e = expected.detach().float().cpu()
  diff = (a - e)
  max_abs = (diff.abs() - rtol * e.abs()).max().item() if diff.numel() else 0.0
  rel = (diff.norm() / e.norm().clamp_min(1e-30)).item()
  return max_abs, rel


def assert_close_bf16(actual, expected, what: str = "", max_abs: float = MAX_ABS, rel_l2: float = REL_L2,
                      rtol: float = 0.0):
  m, r = errors(actual, expected, rtol)
  print(f"[parity] {what}: max_abs={m:.3e}{f' (after {rtol:.2e}|e|)' if rtol else ''} rel_l2={r:.3e}", flush=True)
  assert m <= max_abs and r <= rel_l2, f"{what}: max_abs={m:.3e} (<= {max_abs}) rel_l2={r:.3e} (<= {rel_l2})"


def bf16_round(t: torch.Tensor) -> torch.Tensor:
  return t.to(torch.bfloat16).to(torch.float32)
