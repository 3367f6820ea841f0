"""CPU model of every global memory access of the triangle multiplicative update's kernels
(csrc/trimul.hip: the prologue, the batched NT product through the library's GEMM, the epilogue)
and of the host's launch arithmetic, checked against the buffer sizes the host allocates, for
N in {1, 37, 64, 97, 384, 768} and both edges (97: N^2 = 9409 is not a multiple of the
32-position block, so the last block of the epilogue has lanes past the end).  The index expressions are the kernels' own, restated;
nothing here runs on a GPU."""
import numpy as np
import pytest

from sparsefold_amd import _lib

KC, KTW = 128, 8                 # channels, waves per workgroup of the position kernels
RESIDENT = 256                   # resident workgroups of the position kernels (one per CU)


def _pn(n):
  return (n + 63) & ~63


def _pp(n):
  return (n * n + 31) & ~31


def _grid(items):
  """launch_grid + the host's items-per-wave / group arithmetic."""
  waves = max(1, min(RESIDENT * KTW, items))
  ipw = (items + waves - 1) // waves
  groups = (items + ipw * KTW - 1) // (ipw * KTW)
  return ipw, groups


def _covered(items, ipw, groups):
  """Every item is processed by exactly one wave: workgroup g's wave w takes items
  g * KTW * ipw + k * KTW + w, k < ipw, until the first one past the end."""
  seen = np.zeros(items, np.int64)
  for g in range(groups):
    for w in range(KTW):
      for k in range(ipw):
        item = g * KTW * ipw + k * KTW + w
        if item >= items:
          break
        seen[item] += 1
  return bool((seen == 1).all())


def _proj_accesses(N, incoming):
  Pn = _pn(N)
  items = Pn * (Pn // 32)
  ipw, groups = _grid(items)
  assert _covered(items, ipw, groups)
  item = np.arange(items)[:, None]
  lane = np.arange(64)[None, :]
  half, li = lane >> 5, lane & 31
  cbs = Pn // 32
  R, cb = item // cbs, item % cbs
  col = 32 * cb + li
  za, zb = (col, R) if incoming else (R, col)
  ok = (za < N) & (zb < N)
  # z reads, every lane (unconditional): 8 x 16 bytes at element (za * N + zb) * 128 + 8 * half
  # + 16 kk, position 0 where not ok
  zfirst = np.where(ok, za * N + zb, 0) * KC + 8 * half
  zlast = zfirst + 16 * 7 + 7
  z_max = int(zlast.max())
  # mask reads, every lane: mask[za], mask[zb] where ok, mask[0] otherwise
  m_max = int(np.where(ok, np.maximum(za, zb), 0).max())
  # plane stores (2 bytes): lane (half, li) writes column col = 32 cb + li of plane row R for the
  # channels 32 nb + 8 (r / 4) + 4 half + r % 4, r = 0..15, nb = 0..3
  plane = Pn * Pn
  pbase = R * Pn + col
  # the kernel's byte address: uniform base dst + (32 nb + 8 (r / 4) + r % 4) plane * 2 plus the
  # 64-bit lane offset (4 half plane + pbase) * 2 -- the same element as below
  lofs = (4 * half * plane + pbase) * 2
  assert (lofs % 2 == 0).all() and (lofs >= 0).all()
  ch = np.array([[32 * nb + 8 * (r >> 2) + 4 * h + (r & 3) for nb in range(4) for r in range(16)] for h in (0, 1)])
  chl = ch[half[0]]                                        # [64 lanes, 64 channels]
  lo = int((chl.min(axis=1)[None, :] * plane + pbase).min())
  hi = int((chl.max(axis=1)[None, :] * plane + pbase).max())
  # every (channel, plane element) written exactly once
  writes = np.zeros((KC, Pn * Pn), np.int64)
  for h in (0, 1):
    lanes = np.flatnonzero(half[0] == h)
    for c in ch[h]:
      np.add.at(writes[c], pbase[:, lanes].ravel(), 1)
  return dict(items=items, z_max=z_max, m_max=m_max, plane_min=lo, plane_max=hi,
              plane_elems=KC * plane, row_writes=writes, aligned8=True)


def _gemm_accesses(N):
  """linear64_kernel, batched: loads clamp rows to M-1 / N-1 and read k0 + swizzled piece < K
  from rows of stride x_rs = K = Pn; stores y[b * y_bs + m * y_rs + n] for m < M, n < N."""
  Pn = _pn(N)
  M = Ng = N
  K = Pn
  x_rs, x_bs, y_rs, y_bs = Pn, Pn * Pn, N, _pp(N)
  out = {}
  for bm, bn in ((128, 128), (64, 128), (64, 64)):
    gm, gn = (M + bm - 1) // bm, (Ng + bn - 1) // bn
    # load rows: min(m0 + c * 8 + lane / 8, M - 1); columns k0 + rsw + 0..7 with k0 + 64 <= K
    max_row = M - 1
    max_col = K - 1                          # k0 <= K - 64, rsw + 7 <= 63
    x_max = (KC - 1) * x_bs + max_row * x_rs + max_col
    w_max = (KC - 1) * x_bs + (Ng - 1) * K + max_col
    y_max = (KC - 1) * y_bs + (M - 1) * y_rs + (Ng - 1)
    out[(bm, bn)] = (gm, gn, x_max, w_max, y_max)
  return out, KC * Pn * Pn, KC * y_bs


def _out_accesses(N):
  P, Pp = N * N, _pp(N)
  items = (P + 31) // 32
  ipw, groups = _grid(items)
  assert _covered(items, ipw, groups)
  item = np.arange(items)[:, None]
  lane = np.arange(64)[None, :]
  half, li = lane >> 5, lane & 31
  p = item * 32 + li
  ok = p < P
  qt = lane + 64 * np.arange(8)[:, None, None]            # the product loads: u = 0..7, every item
  ct, seg = qt >> 2, qt & 3
  t_start = ct * Pp + item[None] * 32 + 8 * seg
  assert (t_start % 8 == 0).all(), "16-byte product loads aligned"
  t_max = int((t_start + 7).max())
  # the wave's LDS rows hold 32 x kWS (136) elements; the staged block sits at pitch 34
  lds_store = (ct * 34 + 8 * seg + 7).max()
  kk, e = np.arange(8)[:, None, None, None], np.arange(4)[None, :, None, None]
  lds_read = ((16 * kk + 8 * half[None] + 2 * e + 1) * 34 + li[None]).max()
  assert max(lds_store, lds_read) < 32 * 136 and ((ct * 34 + 8 * seg) % 2 == 0).all()
  z_max = int((p * KC + 8 * half + 16 * 7 + 7)[ok].max())
  q = lane + 64 * np.arange(8)[:, None, None]             # the row-store loop: u = 0..7
  pos, c8 = q >> 4, (q & 15) * 8
  pp = item[None] * 32 + pos
  okw = pp < P
  out_max = int((pp * KC + c8 + 7)[okw].max())
  return dict(t_max=t_max, t_elems=KC * Pp, z_max=z_max, out_max=out_max, elems=P * KC)


@pytest.mark.parametrize("incoming", [False, True])
@pytest.mark.parametrize("N", [1, 37, 64, 97, 384, 768])
def test_trimul_kernel_accesses_stay_in_bounds(N, incoming):
  pr = _proj_accesses(N, incoming)
  assert pr["z_max"] < N * N * KC and pr["m_max"] < N
  assert 0 <= pr["plane_min"] and pr["plane_max"] < pr["plane_elems"]
  assert pr["aligned8"]
  assert (pr["row_writes"] == 1).all(), "every channel's padded plane element written exactly once (zeros included)"
  gemm, ab_elems, t_elems = _gemm_accesses(N)
  for (bm, bn), (gm, gn, x_max, w_max, y_max) in gemm.items():
    assert x_max < ab_elems and w_max < ab_elems and y_max < t_elems, (bm, bn)
    assert gm * gn * KC > 0 and gm < 2 ** 31 and KC <= 65535
  o = _out_accesses(N)
  assert o["t_max"] < o["t_elems"] and o["z_max"] < o["elems"] and o["out_max"] < o["elems"]


@pytest.mark.parametrize("N", [1, 37, 64, 384, 768])
def test_trimul_workspace_covers_the_modelled_buffers(N):
  lib = _lib.load()
  Pn, Pp = _pn(N), _pp(N)
  need = 2 * KC * Pn * Pn * 2 + KC * Pp * 2 + (4 * KC * KC + 2 * KC * KC) * 2 + 6 * KC * 4
  assert lib.sf_hip_triangle_mult_workspace_bytes(N, KC) >= need


@pytest.mark.parametrize("grid", [(6, 6, 128), (12, 12, 128), (1, 1, 8), (3, 2, 5), (320, 2, 5), (7, 3, 8)])
def test_batched_gemm_tile_remap_is_a_permutation(grid):
  """linear64_kernel's batched tile order (XCD-contiguous ranges when the tile count is a multiple
  of 8, dispatch order otherwise) visits every (x, y, z) tile exactly once."""
  gx, gy, gz = grid
  total = gx * gy * gz
  L = np.arange(total, dtype=np.int64)
  t = (L & 7) * (total >> 3) + (L >> 3) if total % 8 == 0 else L
  bx, by, bz = t % gx, (t // gx) % gy, t // (gx * gy)
  assert np.unique(bx + gx * (by + gy * bz)).size == total and bz.max() < gz
  if total % 8 == 0 and gz % 8 == 0:
    # each XCD (L % 8) holds whole batch members
    for x in range(8):
      members = np.unique(bz[(L & 7) == x])
      assert members.size == gz // 8
