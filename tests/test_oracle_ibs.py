"""Pins of the IBS block-sparse triangle attention oracle (oracle/ibs.py) by what the
mathematics fixes.  Parity with the reference's own sampler (vecops' ibs_attention, an
un-vendored dependency) stays unpinned; these checks fix the sampler and the sparse attention
to their stated definitions."""
import math

import numpy as np
import pytest
import torch

from oracle import ibs
from oracle import modules as OM
from sparsefold_amd import workloads as W


def _case(N, seed=3, padded=False):
  mod, z, seq = W.make_triangle(N, C=16, H=2, seed=seed, sharp=True, padded=padded, dtype=torch.float32)
  return W.state_dict_f32(mod), z, seq


@pytest.mark.parametrize("N,transpose,padded", [(40, False, False), (100, True, True), (64, False, True)])
def test_all_blocks_selected_is_dense_attention(N, transpose, padded):
  """With num_samples >= the number of key blocks every valid block is selected with weight 1,
  and the sparse attention is the dense attention (the reference composite) exactly."""
  p, z, seq = _case(N, padded=padded)
  params = ibs.IBSParams(num_samples=16, num_rand_blocks=5)
  upd, (index, weight) = ibs.grid_self_attention_ibs(z, seq, p, transpose=transpose, params=params, seed=1,
                                                     return_maps=True)
  dense = OM.grid_self_attention(z, seq, p, transpose=transpose, return_update=True)
  got = upd.transpose(0, 1) if transpose else upd
  torch.testing.assert_close(got, dense, rtol=1e-4, atol=1e-5)
  T = (N + 31) // 32
  unmasked = [r for r in range(N) if seq[r]]
  assert (weight[unmasked] [index[unmasked] >= 0] == 1.0).all()
  assert ((index[unmasked] >= 0).sum(-1) == T - (0 if not padded else 0)).all() or padded


def _sparse_params():
  return ibs.IBSParams(num_samples=4, num_rand_blocks=2, t_prob=0.3, tr_prob=1.0, u_prob=0.02)


def test_maps_are_deterministic_in_the_seed():
  p, z, seq = _case(200, seed=5)
  params = _sparse_params()
  rows = [0, 7, 199]
  _, m1 = ibs.grid_self_attention_ibs(z, seq, p, transpose=False, params=params, seed=11, rows=rows, return_maps=True)
  _, m2 = ibs.grid_self_attention_ibs(z, seq, p, transpose=False, params=params, seed=11, rows=rows, return_maps=True)
  _, m3 = ibs.grid_self_attention_ibs(z, seq, p, transpose=False, params=params, seed=12, rows=rows, return_maps=True)
  assert np.array_equal(m1[0], m2[0]) and np.array_equal(m1[1], m2[1])
  assert not np.array_equal(m1[0][rows], m3[0][rows])
  # the hash is a pure function of its coordinates
  assert ibs.uniform(11, 0, 7, 1, 3, 0) == ibs.uniform(11, 0, 7, 1, 3, 0)
  assert ibs.uniform(11, 0, 7, 1, 3, 0) != ibs.uniform(11, 0, 7, 1, 3, 1)


def _tile_setup(seed=21, N=256):
  g = torch.Generator().manual_seed(seed)
  q = torch.randn(N, 8, generator=g)
  k = torch.randn(N, 8, generator=g)
  bias = 2.0 * torch.randn(N, N, generator=g)
  valid = torch.ones(N, dtype=torch.bool)
  return ibs.block_masses(q, k, bias, valid)


def test_static_blocks_are_the_heaviest_and_weights_normalise():
  masses = _tile_setup()
  params = _sparse_params()
  idx, wt = ibs.select_blocks(masses, params, seed=3, batch=0, row=0, head=0)
  S, R = params.num_samples, params.num_rand_blocks
  for t in range(masses.shape[0]):
    m = masses[t].numpy()
    p = m / m.sum()
    order = sorted(range(len(m)), key=lambda b: (-m[b], b))
    static = [b for b, w in zip(idx[t], wt[t]) if b >= 0 and w == 1.0][: S - R]
    # the static set is a prefix of the descending-mass order
    assert static == order[:len(static)]
    assert len(static) >= 1 and (p[static].sum() >= params.t_prob or len(static) == S - R)
    # the random slots: sum over draws of w * q is 1 (w = count / (R q))
    cand = order[len(static):]
    mc = p[cand].sum()
    raw = np.maximum(p[cand] / mc, params.u_prob)
    q = dict(zip(cand, raw / raw.sum()))
    rnd = [(b, w) for b, w in zip(idx[t][len(static):], wt[t][len(static):]) if b >= 0]
    assert rnd and math.isclose(sum(w * q[b] for b, w in rnd), 1.0, rel_tol=1e-5)
    assert len({b for b, _ in rnd}) == len(rnd)                      # repeated draws merged


def test_random_blocks_give_an_unbiased_estimate_of_the_candidates_mass():
  """Over many seeds, the importance-weighted mass of the drawn blocks averages to the candidates'
  total mass (the estimator the weights define)."""
  masses = _tile_setup(seed=22)
  params = _sparse_params()
  t = 2
  m = masses[t].numpy()
  p = m / m.sum()
  order = sorted(range(len(m)), key=lambda b: (-m[b], b))
  est = []
  for seed in range(3000):
    idx, wt = ibs.select_blocks(masses[t:t + 1], params, seed=seed, batch=0, row=0, head=0)
    n_static = sum(1 for w in wt[0] if w == 1.0)
    est.append(sum(w * p[b] for b, w in zip(idx[0][n_static:], wt[0][n_static:]) if b >= 0))
  truth = p[order[n_static:]].sum()
  mean, sd = float(np.mean(est)), float(np.std(est)) / math.sqrt(len(est))
  assert abs(mean - truth) < 4 * sd + 1e-9, (mean, truth, sd)


def test_tail_past_tr_prob_is_never_drawn():
  masses = _tile_setup(seed=23)
  params = ibs.IBSParams(num_samples=4, num_rand_blocks=2, t_prob=0.3, tr_prob=0.6, u_prob=0.02)
  for t in range(masses.shape[0]):
    m = masses[t].numpy()
    p = m / m.sum()
    order = sorted(range(len(m)), key=lambda b: (-m[b], b))
    cum = np.cumsum(p[order])
    allowed = set(order[: int(np.searchsorted(cum, params.tr_prob)) + 1])
    for seed in range(20):
      idx, _ = ibs.select_blocks(masses[t:t + 1], params, seed=seed, batch=0, row=0, head=0)
      assert {int(b) for b in idx[0] if b >= 0} <= allowed
