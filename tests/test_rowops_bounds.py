"""CPU model of the global stores of the pair-logit kernel for C = 128 (csrc/rowops.hip:
pair_logits128_kernel with 16-byte stores) and of the loads and stores of the window projection
(csrc/modules.hip: adaln2_proj_kernel, one workgroup per side and worker), both of which store
unconditionally: a lane whose plane, positions or row lie
past the end stores the last valid plane's, chunk's or row's bytes again.  The host's tile
arithmetic and the kernels' index expressions are restated; nothing here runs on a GPU.  Checked:
every store lies inside the output, every output element is written, and a lane that repeats a
store writes the element its owner writes (so the bytes are identical)."""
import numpy as np
import pytest

W = 4                       # waves per pair-logit workgroup (kPLWaves)


def _pl_tiles(H):
  """The host's tile choice: 32-plane blocks per tile, tiles per workgroup, workgroups per worker."""
  hb = 1 if H <= 32 else 2
  g2 = 1 if (H <= 64 or (H - 1) % 128 < 64) else 2
  np_ = 32 * hb
  return hb, g2, (H + np_ * g2 - 1) // (np_ * g2)


def test_pair_logits_every_tile_holds_a_plane():
  for H in range(1, 1025):                  # the kernel's plane limit for C = 128
    hb, g2, hgroups = _pl_tiles(H)
    NP = 32 * hb
    assert hgroups * g2 * NP >= H
    for hg in range(hgroups):
      for g in range(g2):
        assert hg * g2 * NP + g * NP < H, (H, hg, g)


def _pl_stores(P, H, seg, grp, workers):
  """(element offset, plane, position) of every 16-byte store, and the element each lane's data
  belongs to, for one launch with `workers` position workers."""
  hb, g2, hgroups = _pl_tiles(H)
  NP, TPOS = 32 * hb, 32 * W
  LPP = TPOS // 8
  PPI, PPW = 64 // LPP, NP // W
  steps = (P + 31) // 32
  lane = np.arange(64)
  ch = lane % LPP
  out = []
  for worker in range(workers):
    for hg in range(hgroups):
      h0 = hg * g2 * NP
      base = worker * W
      while base < steps:
        for g in range(g2):
          p = base * 32 + 8 * ch
          pc = np.minimum(p, P - 8)
          chc = (pc - base * 32) >> 3
          plmax = H - 1 - h0 - g * NP
          for wave in range(W):
            for i in range(PPW // PPI):
              pl_own = wave * PPW + PPI * i + lane // LPP
              pl = np.minimum(pl_own, plmax)
              hh = h0 + g * NP + pl
              blk = hh // grp
              pos = (pc // seg) * grp * seg + pc % seg
              off = blk * grp * P + (hh - blk * grp) * seg + pos
              # the lane stores the tile row of plane pl, chunk chc: positions base*32 + 8 chc ..
              out.append((off, hh, base * 32 + 8 * chc))
        base += workers * W
  return out


@pytest.mark.parametrize("P,H,seg,grp", [(1320, 4, 1320, 4), (1320, 16, 1320, 16), (1320, 100, 1320, 100),
                                         (1320, 130, 1320, 130), (1320, 200, 1320, 200), (4096, 384, 4096, 384),
                                         (192, 96, 64, 8), (8, 1, 8, 1), (40, 64, 8, 16)])
@pytest.mark.parametrize("workers", [8, 16])
def test_pair_logits_16_byte_stores(P, H, seg, grp, workers):
  assert P % 8 == 0 and seg % 8 == 0 and P % seg == 0 and H % grp == 0
  stores = _pl_stores(P, H, seg, grp, workers)
  total = H * P
  written = np.zeros(total, np.int64)
  for off, hh, p0 in stores:
    assert (off >= 0).all() and (off + 7 < total).all()
    assert (hh < H).all() and (p0 + 7 < P).all()
    # the element a lane writes is the element of its data (plane hh, positions p0 ..): the
    # plane-major and segmented layouts place (hh, p) at the same offset formula
    blk = hh // grp
    expect = blk * grp * P + (hh - blk * grp) * seg + (p0 // seg) * grp * seg + p0 % seg
    assert (off == expect).all()
    for e in range(8):
      np.add.at(written, off + e, 1)
  assert (written >= 1).all(), "every (plane, position) written"


def _window_workers(blocks, resident=512):
  """The host's launch: two workgroups per worker (one per side), workers a multiple of 8."""
  return max(8, min(resident // 2, (blocks + 7) // 8 * 8) // 8 * 8)


@pytest.mark.parametrize("S,A", [(5, 256), (2, 96), (1, 32), (3, 8192), (5, 8192)])
@pytest.mark.parametrize("resident", [512, 64])
def test_window_projection_accesses(S, A, resident):
  """adaln2_proj_kernel: workgroup b serves side (b / 8) % 2 for worker 8 (b / 16) + b % 8; a worker
  takes blocks worker, worker + workers, ... of 32 rows (row = sample * A + atom); per block it
  loads x[min(row, rows - 1)] and its side's scale / shift of atom row % A, and wave w stores
  columns 32 w .. 32 w + 31 of yq [S*A, 256] (side 0) or ykv [S][A+1][256] (side 1) for row
  min(row, rows - 1); the side-1 workgroup of worker 0 zeroes row A of every sample's K/V block."""
  rows = S * A
  blocks = (rows + 31) // 32
  workers = _window_workers(blocks, resident)
  grid = 2 * workers
  seen = set()
  for b in range(grid):
    side, worker = (b >> 3) & 1, 8 * (b >> 4) + (b & 7)
    assert worker < workers
    seen.add((side, worker))
  assert len(seen) == grid, "every (side, worker) pair exactly once"
  li = np.arange(64) & 31
  half = np.arange(64) >> 5
  prow = np.arange(512) >> 4
  pc = np.arange(512) & 15
  yq = np.zeros(rows * 256, np.int64)
  ykv = np.zeros(S * (A + 1) * 256, np.int64)
  for side, worker in sorted(seen):
    for blk in range(worker, blocks, workers):
      lrow = np.minimum(blk * 32 + prow, rows - 1)      # step-1 loads: x and this side's terms
      assert (lrow * 128 + 8 * pc + 7 < rows * 128).all() and ((lrow % A) < A).all()
      row = blk * 32 + li
      rr = np.minimum(row, rows - 1)
      at, smp = rr % A, rr // A
      for wave in range(8):
        dst = (smp * (A + 1) + at) * 256 if side else rr * 256
        q = dst + 32 * wave + 16 * half
        buf = ykv if side else yq
        for e in range(16):
          assert ((q + e) < buf.size).all()
          np.add.at(buf, q + e, 1)
    if side == 1 and worker == 0:
      for e in range(S * 32):
        start = ((e >> 5) * (A + 1) + A) * 256 + 8 * (e & 31)
        assert start + 7 < ykv.size
        ykv[start:start + 8] += 1
  assert (yq >= 1).all() and (ykv >= 1).all()
