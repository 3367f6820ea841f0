"""CPU model of the global and LDS accesses of the block-sparse (IBS) triangle attention kernels
(csrc/triangle.hip: tri_ibs_bias_mean_kernel, tri_ibs_index_kernel, tri_ibs_attn_kernel) and of
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


@pytest.mark.parametrize("N", [1, 37, 97, 300, 768, 8192])
def test_ibs_kernel_accesses_stay_in_bounds(N):
  NP, T = _np(N), (N + 31) // 32
  E = NP * NP * H * 32                      # elements of each of Q, K, V^T
  S = 16
  lane = np.arange(64)
  half, li = lane >> 5, lane & 31
  # bias mean: idx < H T NP -> bias[(h NP + i) NP + jp], i < N, jp < NP
  idx = np.array([0, H * T * NP - 1])
  jp, t, h = idx % NP, (idx // NP) % T, idx // (NP * T)
  i_last = np.minimum(N, 32 * t + 32) - 1
  assert ((h * NP + i_last) * NP + jp).max() < H * NP * NP
  # sampler: grid N H G, lane tile tc = min(32 g + li, T - 1)
  G = (T + 31) // 32
  for r, hh, g in [(0, 0, 0), (N - 1, H - 1, G - 1)]:
    tc = np.minimum(32 * g + li, T - 1)
    q_last = _ql_off(r, hh, NP, 32 * tc, 0, half) + 31 * 8 + 512 + 7
    assert q_last.max() < E and (32 * tc + 31 < NP).all()
    for b in (0, T - 1):
      j = 32 * b + li
      assert (_ql_off(r, hh, NP, j, 1, half) + 7).max() < E
      bp = ((hh * T + tc) * NP) + 64 * (b >> 1) + 32 * (b & 1) + 16 * half + 15
      assert bp.max() < H * T * NP
      assert ((((hh * T + tc) * NP) + 64 * (b >> 1) + 32 * (b & 1) + 16 * half) % 4 == 0).all()   # f32x4 loads
    maps_last = ((r * H + hh) * T + tc) * S + S - 1
    assert maps_last.max() < N * H * T * S
  assert 2 * T * 32 * 4 <= 64 * 1024                # the sampler's dynamic LDS
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
  assert need >= dense + H * T * NP * 4


def test_ibs_workspace_rejects_unsupported_sizes():
  lib = _lib.load()
  assert lib.sf_hip_triangle_ibs_workspace_bytes(8193, 128, H, D) == 0
  assert lib.sf_hip_triangle_ibs_workspace_bytes(64, 64, 2, D) == 0
  assert lib.sf_hip_triangle_ibs_workspace_bytes(0, 128, H, D) == 0
