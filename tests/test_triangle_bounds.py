"""CPU model of the operand layouts and the global / LDS accesses of the dense triangle attention
fast path (csrc/triangle.hip: tri_proj_kernel, tri_attn_kernel, tri_fixup_kernel and
tri_out_kernel) for both of its instances -- KC = 2 (C = 128, head dim 32) and KC = 1 (C = 64,
head dim 16) -- checked against the buffers the host carves, for N in {1, 37, 65, 257, 768}.
The index expressions are the kernels' own, restated; nothing here runs on a GPU."""
import numpy as np
import pytest

from sparsefold_amd import _lib

H = 4
KT, TR, AW = 64, 4, 8                         # keys per tile, rows per task, waves per workgroup


def _np(n):
  return (n + 127) & ~127


def _ql_off(KC, r, h, NP, p, kk, hf):
  return ((((r * H + h) * (NP >> 5) + (p >> 5)) * (2 * KC) + kk * 2 + hf) * 256 + (p & 31) * 8)


def _vl_off(KC, r, h, NP, c16, hf, d):
  return ((((r * H + h) * (NP >> 4) + c16) * 2 + hf) * (128 * KC) + d * 8)


def _o_off(KC, h, r, i, hf, kk, N, NP):
  return ((((h * N + r) * (NP >> 5) + (i >> 5)) * (512 * KC)) + ((((KC * hf + kk) << 5) + (i & 31)) << 3))


def _bias_pos64(j):
  j32 = j & 31
  return (j & 32) + 16 * ((j32 >> 2) & 1) + 4 * (j32 >> 3) + (j32 & 3)


def _bias_off(h, i, j, NP):
  js = (j & ~63) + _bias_pos64(j & 63)
  jp, pc = js & 63, (js & 63) >> 3
  k, hf = 2 * (pc >> 2) + (pc & 1), (pc >> 1) & 1
  return ((((h * (NP >> 5) + (i >> 5)) * (NP >> 6) + (js >> 6)) << 11) + ((k * 64 + 32 * hf + (i & 31)) << 3) + (jp & 7))


@pytest.mark.parametrize("KC", [1, 2])
def test_operand_layouts_are_bijections(KC):
  """Q/K, V^T and o: every (row, head, position, dim group) has its own 8-element slot, and the
  slots tile the buffers with no gap."""
  D, NP, N = 16 * KC, 128, 100
  q = np.array([_ql_off(KC, r, h, NP, p, kk, hf) for r in range(3) for h in range(H) for p in range(NP)
                for kk in range(KC) for hf in range(2)])
  assert len(set(q.tolist())) == len(q) and q.max() + 8 == 3 * H * NP * D and (q % 8 == 0).all()
  v = np.array([_vl_off(KC, r, h, NP, c, hf, d) for r in range(3) for h in range(H) for c in range(NP // 16)
                for hf in range(2) for d in range(D)])
  assert len(set(v.tolist())) == len(v) and v.max() + 8 == 3 * H * NP * D
  o = np.array([_o_off(KC, h, r, i, hf, kk, N, NP) for h in range(H) for r in range(N) for i in range(0, NP, 1)
                for hf in range(2) for kk in range(KC)])
  assert len(set(o.tolist())) == len(o) and o.max() + 8 == H * N * NP * D
  # a 64-key tile of one row is 2 KC KB of contiguous K (and of V^T): the attention kernel's
  # 1 KB copies at j0 * 32 KC bytes past the row's base
  for j0 in (0, 64, NP - 64):
    ks = {_ql_off(KC, 1, 2, NP, p, kk, hf) for p in range(j0, j0 + 64) for kk in range(KC) for hf in range(2)}
    base = _ql_off(KC, 1, 2, NP, 0, 0, 0) + j0 * 16 * KC
    assert ks == set(range(base, base + 1024 * KC, 8))
    vs = {_vl_off(KC, 1, 2, NP, c, hf, d) for c in range(j0 // 16, j0 // 16 + 4) for hf in range(2) for d in range(D)}
    vb = _vl_off(KC, 1, 2, NP, 0, 0, 0) + j0 * 16 * KC
    assert vs == set(range(vb, vb + 1024 * KC, 8))


@pytest.mark.parametrize("KC", [1, 2])
def test_lds_tile_reads_match_the_copies(KC):
  """The K and V^T operand reads of a tile hit the 16-byte slots the copies filled with the
  wanted key / dim: K slot (rr, kb, kk, half, li) holds key 32 kb + li, k-chunk kk, lane half
  half of row rr; V^T slot (rr, c16, half, li) holds dim li (li mod 16 for KC = 1)."""
  row_bytes = KT * 16 * KC * 2
  k_bytes = TR * row_bytes
  cpw = 2 * k_bytes // 1024 // AW
  assert cpw == 2 * KC
  # copy: wave w chunk u -> LDS bytes (w cpw + u) KB; source = row (w mod 4) of K (w < 4) or V^T
  # (w >= 4), bytes u KB .. of that row's tile; lane L -> 16 L
  filled = {}
  for w in range(AW):
    for u in range(cpw):
      for L in range(64):
        filled[(w * cpw + u) * 1024 + 16 * L] = ("K" if w < 4 else "V", w % 4, u * 1024 + 16 * L)
  assert max(filled) + 16 <= 2 * k_bytes
  for rr in range(TR):
    for kb in range(2):
      for kk in range(KC):
        for half in range(2):
          for li in range(32):
            slot = rr * row_bytes + (kb * 2 * KC + kk * 2 + half) * 512 + li * 16
            src, row, off = filled[slot]
            # offset within the row's tile of K [key block][k-chunk][half][key 32][16 B]
            assert (src, row) == ("K", rr)
            assert off == ((kb * 2 * KC + kk * 2 + half) * 32 + li) * 16
    for c16 in range(4):
      for half in range(2):
        for li in range(32):
          d = li if KC == 2 else li & 15
          slot = k_bytes + rr * row_bytes + (c16 * 2 + half) * 256 * KC + d * 16
          src, row, off = filled[slot]
          assert (src, row) == ("V", rr)
          assert off == ((c16 * 2 + half) * 16 * KC + d) * 16


@pytest.mark.parametrize("KC", [1, 2])
@pytest.mark.parametrize("N", [1, 37, 65, 257, 768])
def test_fast_path_accesses_stay_in_bounds(KC, N):
  D, C = 16 * KC, 64 * KC
  NP = _np(N)
  E = NP * NP * H * D                       # elements of each of Q, K, V^T
  EO = N * NP * H * D                       # elements of o
  EB = NP * NP * H                          # bias elements
  lane = np.arange(64)
  half, li = lane >> 5, lane & 31
  # workspace: the host's size covers Q, K, V^T, bias and o (each rounded to 256 bytes) plus the
  # folded weight, offsets, flags and counters
  ws = int(_lib.load().sf_hip_triangle_workspace_bytes(N, C, H, D))
  assert ws >= 3 * 2 * E + 2 * EB + 2 * EO + (4 * C + 32) * C * 2
  # projection: rows r < NP, positions p < NP; Q/K stores of head hd (16 bytes), V^T stores
  r, p = NP - 1, NP - 1
  for hd in range(H):
    for kk in range(KC):
      assert _ql_off(KC, r, hd, NP, p, kk, 1) + 8 <= E
    assert _vl_off(KC, r, hd, NP, NP // 16 - 1, 1, D - 1) + 8 <= E
  assert max(_bias_off(H - 1, NP - 1, j, NP) for j in range(NP - 64, NP)) < EB
  # attention: persistent tasks (head, row group, block of 256 queries); K / V^T copies of the
  # last tile of the last row, the bias loads of the last query tile, Q of the last query
  r0 = NP - TR
  for w in range(AW):
    rr = w % 4
    base = _ql_off(KC, r0 + rr, H - 1, NP, 0, 0, 0) if w < 4 else _vl_off(KC, r0 + rr, H - 1, NP, 0, 0, 0)
    j0 = NP - KT
    hi = base + j0 * 16 * KC + (2 * KC - 1) * 512 + lane.max() * 8 + 8
    assert hi <= E
  qt = NP // 32 - 1
  bias_base = ((H - 1) * (NP >> 5) + qt) * (NP >> 6) << 11
  assert bias_base + (NP - KT) * 32 + 3 * 512 + lane.max() * 8 + 8 <= EB
  for rr in range(TR):
    for kk in range(KC):
      assert _ql_off(KC, r0 + rr, H - 1, NP, NP - 1, kk, 1) + 8 <= E
  # o stores (rows r < N, queries i < N) and the output stage's o reads
  for kk in range(KC):
    assert _o_off(KC, H - 1, N - 1, N - 1, 1, kk, N, NP) + 8 <= EO
  for ch in range(C // 16):
    hd, hf, k2 = (ch >> 1, ch & 1, 1) if KC == 2 else (ch, 1, 0)
    assert _o_off(KC, hd, N - 1, N - 1, hf, k2, N, NP) + 8 <= EO
  # output stage: a block of 32 queries (i0 = 32 ib < N) stores rows i0 + min(row, N - 1 - i0),
  # the rows past N storing the block's last valid row again (no branch around the stores)
  for i0 in range(0, N, 32):
    for row in range(32):
      ro = i0 + min(row, N - 1 - i0)
      assert 0 <= ro < N and (ro == i0 + row or i0 + row >= N)
  # fix-up: mean of V over every 16-key chunk (parts pp of 256 / D threads, 4 chunks per pass)
  npart = 256 // D
  chunks = set()
  for pp in range(npart):
    for c0 in range(pp, NP // 16, npart * 4):
      for u in range(8):
        c16 = c0 + npart * (u >> 1)
        if c16 < NP // 16:
          chunks.add(c16)
          assert _vl_off(KC, N - 1, H - 1, NP, c16, u & 1, D - 1) + 8 <= E
  assert chunks == set(range(NP // 16))
