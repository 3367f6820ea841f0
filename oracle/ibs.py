"""Index-based block-sparse (IBS) triangle attention: the sampler and the sparse attention,
restated on the CPU.

TEST INFRASTRUCTURE: imported only by tests.

The reference selects this mode with its native backend (``GridSelfAttentionVecops``,
``src/sparsefold/backends/vecops/modules.py:1399-1640``; kernel
``backends/vecops/kernels/resources/GridSelfAttention.cpp:134-142,290-306``; parameters
``src/sparsefold/config.py:65-73`` and ``IBSAParameters``, ``model/trunk/blocks.py:405-418``).  Its
sampler and sparse attention live in the un-vendored vecops dependency (``ops::ibs_attention_indexer``
/ ``ops::ibs_attention`` of vecops@f8500b9c07dec26342ac980693c53f48c2b31906, absent here), so
what follows is this package's own sampler on the reference's interface:

* blocks of 32 queries x 32 keys; per (batch, attention row, head, query tile) ``num_samples``
  slots of ``index_map`` (int32 key-block index, -1 = unused) and ``weight_map`` (float32) --
  the reference's map shape ``[B, N, H, ceil(N/32), num_samples]`` (``registry.py:2982-2992``);
* block mass: the tile's mean query against every valid key plus the tile's mean bias,
  ``m_b = sum_{j in b} 2^(qbar . k_j + bbar_j)`` (logits in log2 units), ``p_b = m_b / sum m``;
  a block is valid when it holds at least one valid key (whatever its mass);
* every valid block selected, weight 1, when there are at most ``num_samples`` of them: the
  attention is then exactly the dense one;
* otherwise static blocks -- the heaviest in descending mass (ties: lower index first) until their
  mass reaches ``t_prob``, at most ``num_samples - num_rand_blocks`` -- with weight 1, then
  ``num_rand_blocks`` draws with replacement from the candidates (the next blocks in that order
  until the mass reaches ``tr_prob``) with proposal ``q_b`` proportional to
  ``max(p_b / M_cand, u_prob)`` (uniform when ``M_cand`` is 0); a block drawn ``c`` times gets
  weight ``c / (R q_b)`` (the
  importance-sampling estimate of the candidates' sum, ``sum_draws w q = 1``); blocks past
  ``tr_prob`` are dropped;
* draws come from a counter-based hash of (seed, batch, row, head, tile, draw), so the maps are a
  deterministic function of the seed and the inputs, identical on every device;
* attention over the selected blocks: ``o_i = sum_s w_s sum_{j in b_s} e_ij v_j / sum_s w_s
  sum_{j in b_s} e_ij``, ``e_ij = 2^(s_ij)``; a masked attention row keeps the dense rule (the
  mean of V over all keys).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

from oracle.primitives import layer_norm, linear

LOG2E = 1.4426950408889634
BLOCK = 32
MASK64 = (1 << 64) - 1


@dataclasses.dataclass(frozen=True)
class IBSParams:
  """``IBSAParameters`` (blocks.py:405-418) / ``[native.sparse_attention]`` (config.py:65-73)."""
  num_samples: int = 16
  num_rand_blocks: int = 5
  t_prob: float = 0.90
  tr_prob: float = 0.95
  u_prob: float = 0.02


def mix64(x: int) -> int:
  """SplitMix64 finaliser (a published 64-bit mixing function)."""
  x = (x + 0x9E3779B97F4A7C15) & MASK64
  x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
  x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & MASK64
  return x ^ (x >> 31)


def uniform(seed: int, batch: int, row: int, head: int, tile: int, draw: int) -> float:
  """A uniform number in [0, 1) from 24 bits of the hash of the draw's coordinates."""
  x = mix64(seed & MASK64)
  for v in (batch, row, head, tile, draw):
    x = mix64(x ^ (v & 0xFFFFFFFF))
  return (x >> 40) * (1.0 / (1 << 24))


def block_masses(q: torch.Tensor, k: torch.Tensor, bias: torch.Tensor, key_valid: torch.Tensor) -> torch.Tensor:
  """Per query tile and key block: the tile-mean query against each valid key plus the tile-mean
  bias (log2-domain logits, q already scaled), summed over the block as 2^x.  q, k ``[N, D]``
  (log2 units: q carries scale * log2 e), bias ``[N, N]`` (log2 units), key_valid ``[N]`` bool.
  Returns ``[T, KB]`` float64 block masses relative to each tile's largest block (max 1); -1 marks
  a block without a valid key."""
  N = q.shape[0]
  T = (N + BLOCK - 1) // BLOCK
  out = torch.zeros(T, T, dtype=torch.float64)
  qd, kd, bd = q.double(), k.double(), bias.double()
  for t in range(T):
    rows = slice(BLOCK * t, min(N, BLOCK * t + BLOCK))
    qbar = qd[rows].mean(0)
    bbar = bd[rows].mean(0)
    x = kd @ qbar + bbar
    x = torch.where(key_valid, x, torch.full_like(x, -math.inf))
    xmax = x.max()
    e = torch.exp2(x - xmax) if torch.isfinite(xmax) else torch.zeros_like(x)
    for b in range(T):
      out[t, b] = e[BLOCK * b:BLOCK * b + BLOCK].sum()
    mx = out[t].max()
    if mx > 0:
      out[t] /= mx
  for b in range(T):
    if not bool(key_valid[BLOCK * b:BLOCK * b + BLOCK].any()):
      out[:, b] = -1.0
  return out


def select_blocks(masses: torch.Tensor, params: IBSParams, seed: int, batch: int, row: int, head: int):
  """``[T, KB]`` block masses -> (index ``[T, S]`` int32, weight ``[T, S]`` float32)."""
  T, KB = masses.shape
  S, R = params.num_samples, params.num_rand_blocks
  index = np.full((T, S), -1, np.int32)
  weight = np.zeros((T, S), np.float32)
  for t in range(T):
    m = masses[t].tolist()
    valid = [b for b in range(KB) if m[b] >= 0]
    if not valid:
      continue
    if len(valid) <= S:
      for s, b in enumerate(valid):
        index[t, s], weight[t, s] = b, 1.0
      continue
    total = sum(m[b] for b in valid)
    order = sorted(valid, key=lambda b: (-m[b], b))
    p = {b: m[b] / total for b in valid}
    static, cum = [], 0.0
    for b in order:
      if cum >= params.t_prob or len(static) >= S - R:
        break
      static.append(b)
      cum += p[b]
    cand = []
    for b in order[len(static):]:
      if cum >= params.tr_prob:
        break
      cand.append(b)
      cum += p[b]
    for s, b in enumerate(static):
      index[t, s], weight[t, s] = b, 1.0
    if not cand or R == 0:
      continue
    mc = sum(p[b] for b in cand)
    raw = [max(p[b] / mc, params.u_prob) if mc > 0 else 1.0 for b in cand]
    zr = sum(raw)
    q = [r / zr for r in raw]
    counts = [0] * len(cand)
    for d in range(R):
      u = uniform(seed, batch, row, head, t, d)
      acc, pick = 0.0, len(cand) - 1
      for c, qc in enumerate(q):
        acc += qc
        if u < acc:
          pick = c
          break
      counts[pick] += 1
    s = len(static)
    for c, b in enumerate(cand):
      if counts[c]:
        index[t, s], weight[t, s] = b, counts[c] / (R * q[c])
        s += 1
  return index, weight


def sparse_attention(q, k, v, bias, key_valid, index, weight) -> torch.Tensor:
  """One attention row: q, k ``[N, D]`` (log2 units), v ``[N, Dv]``, bias ``[N, N]`` (log2
  units), key_valid ``[N]``, maps ``[T, S]``.  Returns ``[N, Dv]`` float64."""
  N = q.shape[0]
  dev = q.device                          # the oracle runs where its inputs live (CPU, or the GPU for large N)
  out = torch.zeros(N, v.shape[1], dtype=torch.float64, device=dev)
  qd, kd, vd, bd = q.double(), k.double(), v.double(), bias.double()
  for t in range(index.shape[0]):
    # a slot is used when its index names a key block and its weight is positive
    blocks = [(int(b), float(w)) for b, w in zip(index[t], weight[t]) if 0 <= b < index.shape[0] and w > 0]
    if not blocks:
      continue
    keys = torch.cat([torch.arange(BLOCK * b, min(N, BLOCK * b + BLOCK), device=dev) for b, _ in blocks])
    wk = torch.cat([torch.full((min(N, BLOCK * b + BLOCK) - BLOCK * b,), w, dtype=torch.float64, device=dev)
                    for b, w in blocks])
    ok = key_valid[keys]
    for i in range(BLOCK * t, min(N, BLOCK * t + BLOCK)):
      x = kd[keys] @ qd[i] + bd[i, keys]
      x = torch.where(ok, x, torch.full_like(x, -math.inf))
      e = torch.exp2(x - x.max()) * wk
      out[i] = (e[:, None] * vd[keys]).sum(0) / e.sum()
  return out


def grid_self_attention_ibs(act: torch.Tensor, seq_mask: torch.Tensor, p: dict, *, transpose: bool,
                            params: IBSParams, seed: int, maps=None, rows=None, return_maps: bool = False):
  """GridSelfAttention.forward (blocks.py:293-366) with IBS attention rows: LN, bias from the
  untransposed activations, per row q / k / v / gate projections, sparse attention, gate, output
  projection.  act ``[N, N, C]`` float32.  ``maps`` = (index ``[N, H, T, S]``, weight) replaces the
  sampler (map reuse).  Returns the update of the selected rows (``rows``: default all)
  ``[len(rows), N, C]`` and, with ``return_maps``, the maps of every row."""
  N = act.shape[0]
  H = p["q_projection.weight"].shape[0]
  D = p["q_projection.weight"].shape[1]
  T = (N + BLOCK - 1) // BLOCK
  scale = LOG2E / math.sqrt(D)
  x = layer_norm(act, p["act_norm.weight"], p.get("act_norm.bias"))
  bias = linear(x, p["pair_bias_projection.weight"]).movedim(-1, -3).contiguous() * LOG2E   # [H, N, N]
  xt = x.transpose(0, 1) if transpose else x
  seq = seq_mask.bool()
  rows = list(range(N)) if rows is None else list(rows)
  all_index = np.full((N, H, T, params.num_samples), -1, np.int32) if maps is None else maps[0]
  all_weight = np.zeros((N, H, T, params.num_samples), np.float32) if maps is None else maps[1]
  out = []
  for r in rows:
    xr = xt[r]
    q = linear(xr, p["q_projection.weight"], transpose_weights=True) * scale   # [N, H, D]
    k = linear(xr, p["k_projection.weight"], transpose_weights=True)
    v = linear(xr, p["v_projection.weight"])
    g = linear(xr, p["gating_query.weight"], transpose_weights=True, post_op="sigmoid")
    key_valid = seq & seq[r]
    o = torch.zeros(N, H, D, dtype=torch.float64, device=act.device)
    for h in range(H):
      if not bool(seq[r]):
        o[:, h] = v[:, h].double().mean(0)                  # every logit is -max: uniform over all keys
        continue
      if maps is None:
        masses = block_masses(q[:, h], k[:, h], bias[h], key_valid)
        idx, wt = select_blocks(masses, params, seed, 0, r, h)
        all_index[r, h], all_weight[r, h] = idx, wt
      o[:, h] = sparse_attention(q[:, h], k[:, h], v[:, h], bias[h], key_valid, all_index[r, h], all_weight[r, h])
    og = o.float().reshape(N, H * D) * g
    out.append(linear(og, p["output_projection.weight"]))
  upd = torch.stack(out)
  return (upd, (all_index, all_weight)) if return_maps else upd
