"""The allocation-free self-attention entry point (sf_hip_self_attention_fwd_noalloc) against
the workspace entry point (sf_hip_self_attention_fwd): the same kernels on the library's fixed
per-GPU scratch, so the outputs must be identical -- on two calls in a row, the second smaller
than the first (whatever the first left in the scratch must not leak into the second)."""
import pytest
import torch

from sparsefold_amd import _lib
from sparsefold_amd import backends
from sparsefold_amd import workloads as W
from sparsefold_amd.backends.hip import ops
from sparsefold_amd.runtime import config

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def hip_backend():
  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
  backends.init()
  yield
  config.configure_runtime(backend="torch")
  backends.init()
  config.reset()


def _diffusion_call(N, S, seed):
  mod, act, cond, bias, mask = W.make_diffusion(N, S=S, seed=seed, padded=True, sharp=True)
  mod = mod.to(DEV)
  backends.prepare(mod)
  args = (act.to(DEV), mask.to(DEV), bias.to(DEV), cond.to(DEV), mod._native_weights())
  return args, dict(num_head=mod.num_head, head_dim=mod.key_dim)


def _single_call(N, seed):
  mod, z, s, seq = W.make_single(N, seed=seed, padded=True, sharp=True)
  mod = mod.to(DEV)
  backends.prepare(mod)
  att = mod.single_attention
  pl = ops.pair_logits(z.to(DEV), mod._hip_pl_ln_w, mod._hip_pl_ln_b, mod._hip_pl_w).view(att.num_head, N, N)
  args = (s.to(DEV), seq.to(DEV), pl, None, att._native_weights())
  return args, dict(num_head=att.num_head, head_dim=att.key_dim)


def test_noalloc_entry_matches_workspace_entry_on_two_calls():
  big, kw_big = _diffusion_call(1024, 5, 41)          # ~53 MB of scratch
  small, kw_small = _single_call(300, 42)              # a smaller second call
  for args, kw in ((big, kw_big), (small, kw_small)):
    want = ops.self_attention_module(*args, **kw)
    got = ops.self_attention_module(*args, **kw, noalloc=True)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want), f"max diff {(got.float() - want.float()).abs().max().item()}"
  # and the big one again after the small one
  want = ops.self_attention_module(*big, **kw_big)
  got = ops.self_attention_module(*big, **kw_big, noalloc=True)
  assert torch.equal(got, want)


def test_noalloc_entry_refuses_sizes_beyond_its_scratch():
  x = torch.zeros(8, 4096, 768, dtype=torch.bfloat16, device=DEV)     # needs more than 64 MiB
  mod, *_ = W.make_diffusion(8, S=1, seed=43)
  mod = mod.to(DEV)
  backends.prepare(mod)
  with pytest.raises(RuntimeError, match="fixed scratch holds"):
    ops.self_attention_module(x, None, None, None, mod._native_weights(), num_head=mod.num_head,
                              head_dim=mod.key_dim, noalloc=True)
