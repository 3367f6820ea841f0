"""Seeded synthetic workloads for the five attention configurations.

All tensors are drawn on the CPU from a seeded ``torch.Generator`` in float32 and then cast,
so every consumer (parity tests, benchmark, CPU baseline) sees identical values.
Weights: Linear ~ N(0, std^2) (std 0.02 by default; ``sharp=True`` uses std = 1/sqrt(fan_in)
so the softmax is far from uniform); LayerNorm gamma = 1 + N(0, 0.02^2), beta ~ N(0, 0.02^2).

Configurations (sizes as used by the benchmark):
  triangle   z [N, N, 128], H=4, D=32; padded variant masks the last N//10 tokens
  single     s [N, 384], z [N, N, 128] -> bias [16, N, N]; H=16, D=24
  diffusion  act [S, N, 768], single_cond [N, 384], bias [16, N, N] shared by the S samples;
             H=16, D=48
  window     act [S, U, 32, 128] (U = atoms/32 windows), keys = 128 atoms starting at 32u-48,
             indices outside [0, atoms) masked, last `pad` atoms padded; bias [U, 4, 32, 128];
             H=4, D=32
  packs      Transformer pair-logit pack: pair_cond [N, N, 128] -> [6, 4, 16, N, N];
             CrossAttTransformer pack: pair_cond [U, 32, 128, 16] -> [3, U, 4, 32, 128]
"""
from __future__ import annotations

import dataclasses

import torch

from sparsefold_amd import modules as M


def _gen(seed: int) -> torch.Generator:
  return torch.Generator().manual_seed(int(seed))


def fill_parameters(module: torch.nn.Module, seed: int, std: float = 0.02, sharp: bool = False) -> torch.nn.Module:
  """Deterministically fills every parameter (sorted by name) of ``module`` in place."""
  g = _gen(seed)
  linears = {id(m.weight): m for m in module.modules() if isinstance(m, M.Linear)}
  norms = {id(m.weight): m for m in module.modules() if isinstance(m, M.LayerNorm) and m.weight is not None}
  norm_biases = {id(m.bias) for m in module.modules() if isinstance(m, M.LayerNorm) and m.bias is not None}
  with torch.no_grad():
    for name, p in sorted(module.named_parameters(), key=lambda kv: kv[0]):
      r = torch.randn(p.shape, generator=g, dtype=torch.float32)
      if id(p) in norms:
        val = 1.0 + 0.02 * r
      elif id(p) in norm_biases:
        val = 0.02 * r
      elif id(p) in linears and sharp:
        fan_in = 1
        for s in linears[id(p)].input_shape:
          fan_in *= s
        val = r / fan_in ** 0.5
      else:
        val = std * r
      p.copy_(val.to(p.dtype))
  return module


def state_dict_f32(module: torch.nn.Module) -> dict[str, torch.Tensor]:
  return {k: v.detach().to("cpu", torch.float32) for k, v in module.state_dict().items()}


# ---------------------------------------------------------------------------------------

def make_triangle(N: int, *, C: int = 128, H: int = 4, transpose: bool = False, padded: bool = False,
                  seed: int = 1, sharp: bool = False, dtype=torch.bfloat16, act_norm_bias: bool = False):
  """GridSelfAttention (blocks.py:188-366) and its z [N, N, C], mask [N].  ``act_norm_bias`` adds
  the LayerNorm offset the reference module does not have (a checkpoint may still carry one)."""
  g = _gen(seed)
  z = torch.randn(N, N, C, generator=g).to(dtype)
  seq = torch.ones(N, dtype=torch.bool)
  if padded:
    seq[N - N // 10:] = False
  mod = M.GridSelfAttention(M.GridSelfAttention.Config(num_head=H), M.GlobalConfig(), transpose,
                            num_channels=C, name="pair_attention", act_norm_bias=act_norm_bias)
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, z, seq


def make_trimul(N: int, *, C: int = 128, incoming: bool = False, padded: bool = False, seed: int = 7,
                sharp: bool = True, dtype=torch.bfloat16):
  """Triangle multiplicative update (blocks.py:425-566) and its z [N, N, C], mask [N]."""
  g = _gen(seed)
  z = torch.randn(N, N, C, generator=g).to(dtype)
  mask = torch.ones(N, dtype=torch.bool)
  if padded:
    mask[N - N // 10:] = False
  eq = M.TriangleMultiplication.EQUATIONS[int(incoming)]
  mod = M.TriangleMultiplication(M.TriangleMultiplication.Config(equation=eq), M.GlobalConfig(), num_channels=C,
                                 name="triangle_multiplication")
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, z, mask


def make_single(N: int, *, C_s: int = 384, C_z: int = 128, H: int = 16, seed: int = 3, sharp: bool = False,
                padded: bool = False, transition: bool = False, dtype=torch.bfloat16):
  g = _gen(seed)
  s = torch.randn(N, C_s, generator=g).to(dtype)
  z = torch.randn(N, N, C_z, generator=g).to(dtype)
  seq = torch.ones(N, dtype=torch.bool)
  if padded:
    seq[N - N // 10:] = False
  mod = M.SingleActUpdate(M.GlobalConfig(), C_z, C_s, M.SelfAttention.Config(num_head=H),
                          M.TransitionBlock.Config() if transition else None)
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, z, s, seq


def make_diffusion(N: int, *, S: int = 5, C: int = 768, C_cond: int = 384, H: int = 16, seed: int = 4,
                   sharp: bool = False, padded: bool = False, dtype=torch.bfloat16):
  g = _gen(seed)
  act = torch.randn(S, N, C, generator=g).to(dtype)
  cond = torch.randn(N, C_cond, generator=g).to(dtype)
  bias = torch.randn(H, N, N, generator=g).to(dtype)
  mask = torch.ones(N, dtype=torch.bool)
  if padded:
    mask[N - N // 10:] = False
  mod = M.SelfAttention(M.SelfAttention.Config(num_head=H), M.GlobalConfig(), num_channels=C,
                        single_cond_size=C_cond, name="diffusion_transformer")
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, act, cond, bias, mask


def make_diffusion_stack(N: int, *, S: int = 5, L: int = 24, C: int = 768, C_cond: int = 384, H: int = 16,
                         seed: int = 4, dtype=torch.bfloat16):
  """L diffusion-transformer attention blocks, each with its own seeded weights (block l from
  seed + 1000 + l), and the inputs of make_diffusion(N, seed=seed)."""
  mod0, act, cond, bias, mask = make_diffusion(N, S=S, C=C, C_cond=C_cond, H=H, seed=seed, dtype=dtype)
  mods = [mod0]
  for layer in range(1, L):
    m = M.SelfAttention(M.SelfAttention.Config(num_head=H), M.GlobalConfig(), num_channels=C,
                        single_cond_size=C_cond, name="diffusion_transformer")
    mods.append(fill_parameters(m, seed + 1000 + layer))
  return mods, act, cond, bias, mask


def make_transition(rows: int, *, C: int = 384, factor: int = 4, lead=(), seed: int = 9, sharp: bool = True,
                    dtype=torch.bfloat16):
  """Trunk transition (blocks.py:38-96) and its input ``[*lead, rows, C]``: the single transition of
  SingleActUpdate (C = 384, factor 4) or the pair transition (C = 128, lead = (N,))."""
  act = torch.randn(*lead, rows, C, generator=_gen(seed)).to(dtype)
  mod = M.TransitionBlock(M.TransitionBlock.Config(num_intermediate_factor=factor), M.GlobalConfig(),
                          num_channels=C, name="transition")
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, act


def make_diffusion_transition(N: int, *, S: int = 5, C: int = 768, C_cond: int | None = 384, factor: int = 2,
                              seed: int = 10, sharp: bool = True, dtype=torch.bfloat16):
  """Diffusion-transformer transition (transformer.py:157-231), its act ``[S, N, C]`` and condition
  ``[N, C_cond]`` (None: the unconditioned form)."""
  g = _gen(seed)
  act = torch.randn(S, N, C, generator=g).to(dtype)
  cond = None if C_cond is None else torch.randn(N, C_cond, generator=g).to(dtype)
  mod = M.DiffusionTransitionBlock(M.GlobalConfig(), num_channels=C, num_intermediate_factor=factor,
                                   single_cond_size=C_cond, name="diffusion_transition")
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, act, cond


@dataclasses.dataclass
class WindowLayout:
  """Key windows for 32-atom query blocks: window u covers atoms [32u - 48, 32u + 80)."""
  gather_idxs: torch.Tensor   # [U, Kw] int32, flat index into [U, Qw]
  gather_mask: torch.Tensor   # [U, Kw] bool, index inside [0, atoms)
  queries_mask: torch.Tensor  # [U, Qw] bool, atom present
  keys_mask: torch.Tensor     # [U, Kw] bool, key present


def window_layout(atoms: int, *, Qw: int = 32, Kw: int = 128, pad: int = 0) -> WindowLayout:
  U = atoms // Qw
  present = torch.ones(atoms, dtype=torch.bool)
  if pad:
    present[atoms - pad:] = False
  start = torch.arange(U) * Qw + Qw // 2 - Kw // 2
  idx = start[:, None] + torch.arange(Kw)[None, :]
  inside = (idx >= 0) & (idx < atoms)
  idx_c = idx.clamp(0, atoms - 1)
  return WindowLayout(gather_idxs=idx_c.to(torch.int32), gather_mask=inside,
                      queries_mask=present.view(U, Qw).clone(), keys_mask=inside & present[idx_c])


def make_window(atoms: int, *, S: int = 5, C: int = 128, H: int = 4, pad: int = 192, seed: int = 5,
                sharp: bool = False, dtype=torch.bfloat16):
  g = _gen(seed)
  lay = window_layout(atoms, pad=pad)
  U = atoms // 32
  act = torch.randn(S, U, 32, C, generator=g).to(dtype)
  qcond = torch.randn(U, 32, C, generator=g).to(dtype)
  torch.randn(U, 128, C, generator=g)              # (keeps the later draws of the seeded stream)
  # the keys' condition is the queries' gathered into the windows, zero outside
  # (keys_single_cond = convert(queries_to_keys, queries_single_cond), atom.py:279-281)
  kcond = torch.where(lay.gather_mask[..., None], qcond.reshape(U * 32, C)[lay.gather_idxs.long()],
                      torch.zeros((), dtype=dtype))
  bias = torch.randn(U, H, 32, 128, generator=g).to(dtype)
  mod = M.CrossAttention(M.CrossAttention.Config(num_head=H, key_dim=C, value_dim=C), M.GlobalConfig(),
                         num_channels=C, name="atom_transformer")
  fill_parameters(mod, seed + 1000, sharp=sharp)
  return mod, act, lay, qcond, kcond, bias


def make_transformer_pack(N: int, *, P: int = 128, num_blocks: int = 24, super_block_size: int = 4, H: int = 16,
                          seed: int = 6, dtype=torch.bfloat16):
  """Pair-conditioning half of the diffusion Transformer and its pair_cond [N, N, P]."""
  pair_cond = torch.randn(N, N, P, generator=_gen(seed)).to(dtype)
  mod = M.TransformerPairLogits(num_blocks=num_blocks, super_block_size=super_block_size, num_head=H,
                                pair_cond_size=P, dtype=dtype)
  fill_parameters(mod, seed + 1000, sharp=True)
  return mod, pair_cond


def make_cross_pack(U: int, *, Qw: int = 32, Kw: int = 128, P: int = 16, num_blocks: int = 3, H: int = 4,
                    seed: int = 8, dtype=torch.bfloat16):
  """Pair-conditioning half of the atom CrossAttTransformer and its pair_cond [U, Qw, Kw, P]."""
  pair_cond = torch.randn(U, Qw, Kw, P, generator=_gen(seed)).to(dtype)
  mod = M.CrossAttTransformerPairLogits(num_blocks=num_blocks, num_head=H, pair_cond_size=P)
  fill_parameters(mod, seed + 1000, sharp=True)
  return mod, pair_cond
