"""CPU model of the global and LDS accesses of the block-sparse (IBS) triangle attention kernels
(csrc/triangle.hip: tri_ibs_bias_mean_kernel, tri_ibs_index_kernel, ibs_exact_tile through
tri_ibs_attn_kernel and tri_ibs_flagged_kernel) and of
their host launch arithmetic, checked against the buffers the host carves, for N in
{1, 37, 97, 300, 768, 8192}.  The index expressions are the kernels' own, restated; nothing here
runs on a GPU."""
import numpy as np
import pytest

from sparsefold_amd import _lib

H, D = 4, 32


def _np(n):
  return (n + 127) & ~127


def _ql_off(r, h, NP, p, kk, hf):
  return ((((r * H + h) * (NP >> 5) + (p >> 5)) * 4 + kk * 2 + hf) * 256 + (p & 31) * 8)


def _vl_off(r, h, NP, c16, hf, d):
  return ((((r * H + h) * (NP >> 4) + c16) * 2 + hf) * 256 + d * 8)


def _bmean_off(h, G, KB, t, j):
  """ibs_bmean_off: [h][t / 32][j / 32][quad][t % 32][j % 4], quad = 2 ((j % 32) / 8) + (j / 4) % 2."""
  q4 = 2 * ((j & 31) >> 3) + ((j >> 2) & 1)
  return (((((h * G + (t >> 5)) * KB + (j >> 5)) * 8 + q4) * 32 + (t & 31)) * 4 + (j & 3))


def _bias_pos64(j):
  j32 = j & 31
  return (j & 32) + 16 * ((j32 >> 2) & 1) + 4 * (j32 >> 3) + (j32 & 3)


def test_bmean_layout_is_a_bijection_matching_the_sampler_reads():
  """Every (tile, key) of a head has its own slot, and the sampler's lane (half, li) finds the
  keys 32 b + 8 u + 4 half + e of tile 32 g + li at base + 1024 b + 128 half + 256 u + e."""
  T = 48
  G, KB = (T + 31) // 32, T
  offs = {_bmean_off(1, G, KB, t, j) for t in range(32 * G) for j in range(32 * KB)}
  assert len(offs) == 32 * G * 32 * KB
  for g in range(G):
    for li in (0, 5, 31):
      t = 32 * g + li
      base = _bmean_off(1, G, KB, t, 0)
      for b in (0, 7, KB - 1):
        for half in (0, 1):
          for u in range(4):
            for e in range(4):
              j = 32 * b + 8 * u + 4 * half + e
              assert _bmean_off(1, G, KB, t, j) == base + 1024 * b + 128 * half + 256 * u + e
  # the mean kernel's stored position -> key inverse of bias_pos64
  for j in range(64):
    sp = _bias_pos64(j)
    assert (sp & 32) + 8 * ((sp >> 2) & 3) + 4 * ((sp >> 4) & 1) + (sp & 3) == j


@pytest.mark.parametrize("N", [1, 37, 97, 300, 768, 8192])
def test_ibs_kernel_accesses_stay_in_bounds(N):
  NP, T = _np(N), (N + 31) // 32
  E = NP * NP * H * 32                      # elements of each of Q, K, V^T
  S = 16
  lane = np.arange(64)
  half, li = lane >> 5, lane & 31
  G = (T + 31) // 32
  nbm = H * G * T * 1024                           # tile-mean bias floats (tiles padded to 32 G)
  # bias mean: idx < H G KB 1024; the key's stored position js < NP, queries i < N
  idx = np.array([0, nbm - 1])
  c, tl, q4 = idx & 3, (idx >> 2) & 31, (idx >> 7) & 7
  rest = idx >> 10
  b, g, h = rest % T, (rest // T) % G, rest // (T * G)
  t = 32 * g + tl
  j = 32 * b + 8 * (q4 >> 1) + 4 * (q4 & 1) + c
  assert (_bmean_off(h, G, T, t, j) == idx).all()
  live = (t < T) & (j < N)
  js = (j & ~63) + np.array([_bias_pos64(int(x) & 63) for x in j])
  assert (js[live] < NP).all()
  i_last = np.minimum(N, 32 * t + 32) - 1
  assert ((h * NP + i_last) * NP + js)[live].max(initial=0) < H * NP * NP
  # sampler: grid N H G, lane tile t = 32 g + li (bias means) and tc = min(t, T - 1) (queries)
  for r, hh, g in [(0, 0, 0), (N - 1, H - 1, G - 1)]:
    t = 32 * g + li
    tc = np.minimum(t, T - 1)
    for it in (0, 7):                              # query sums: wave 3's tiles 32 g + 24 .. + 31
      tq = min(32 * g + 8 * 3 + it, T - 1)
      pc, p = lane >> 4, lane & 15
      q_last = _ql_off(r, hh, NP, 32 * tq, 0, 0) + pc * 256 + p * 8 + 128 + 7
      assert q_last.max() < E and 32 * tq + 31 < NP
    for b in (0, T - 1):
      jj = 32 * b + li
      assert (_ql_off(r, hh, NP, jj, 1, half) + 7).max() < E
      bp = np.array([_bmean_off(hh, G, T, int(x), 0) for x in t]) + 1024 * b + 128 * half + 256 * 3 + 3
      assert bp.max() < nbm
      assert ((bp - 3) % 4 == 0).all()             # f32x4 loads
    maps_last = ((r * H + hh) * T + tc) * S + S - 1
    assert maps_last.max() < N * H * T * S
  assert max(3 * T * 32 * 4, 32 * 4 * 8 * 4) <= 96 * 1024   # the sampler's dynamic LDS
  # flagged pairs: items b + k G < N H, their tiles t = wave, wave + 4, ... < T
  items, grid = N * H, min(N * H, 1024)
  for blk in (0, grid - 1):
    K = (items - blk + grid - 1) // grid
    assert blk + (K - 1) * grid < items and blk + K * grid >= items
  # attention: grid ceil(N H T / 4) x 4 waves, task < N H T
  tasks = N * H * T
  for task in (0, tasks - 1):
    t, hh, r = task % T, (task // T) % H, task // (T * H)
    i = 32 * t + li
    assert (i < NP).all()
    for b in (0, T - 1):
      assert (_ql_off(r, hh, NP, 32 * b + li, 1, half) + 7).max() < E
      assert (_vl_off(r, hh, NP, 2 * b + 1, half, li) + 7).max() < E
      bp = (hh * NP + i) * NP + 64 * (b >> 1) + 32 * (b & 1) + 16 * half + 15
      assert bp.max() < H * NP * NP
    ok = i < N
    za, zb = i, r
    assert ((hh * N * N + za * N + zb) * 32 + 16 * half + 15)[ok].max() < H * N * N * 32
    assert (task + 1) * S <= N * H * T * S


@pytest.mark.parametrize("N", [1, 37, 97, 300, 768, 8192])
def test_ibs_workspace_covers_dense_layout_and_means(N):
  lib = _lib.load()
  NP, T = _np(N), (N + 31) // 32
  dense = lib.sf_hip_triangle_workspace_bytes(N, 128, H, D)
  need = lib.sf_hip_triangle_ibs_workspace_bytes(N, 128, H, D)
  G = (T + 31) // 32
  assert need >= dense + H * G * T * 1024 * 4


def test_ibs_workspace_rejects_unsupported_sizes():
  lib = _lib.load()
  assert lib.sf_hip_triangle_ibs_workspace_bytes(8193, 128, H, D) == 0
  assert lib.sf_hip_triangle_ibs_workspace_bytes(64, 64, 2, D) == 0
  assert lib.sf_hip_triangle_ibs_workspace_bytes(0, 128, H, D) == 0
