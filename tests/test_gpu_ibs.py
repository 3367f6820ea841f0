"""Block-sparse (IBS) triangle attention on the GPU vs the oracle (oracle/ibs.py):

* with num_samples >= the key blocks the maps select every valid block with weight 1 and the
  result is the dense module's;
* with maps given (synthetic: random blocks, random weights, empty slots) the sparse attention
  matches the oracle's on the same maps;
* generated maps have the sampler's structure, the attention follows them, a call that reuses
  them reproduces the generating call, and the maps depend on the seed only;
* the sampler, run by the oracle on the operands the kernels read (decoded from the workspace:
  bf16 Q / K and bias planes), selects the same blocks with the same weights;
* the module path: runtime switch, parameters and map reuse between layers.
"""
import numpy as np
import pytest
import torch

from oracle import ibs
from oracle import modules as OM
from sparsefold_amd import backends
from sparsefold_amd import modules as M
from sparsefold_amd import workloads as W
from sparsefold_amd.backends.hip import ops
from sparsefold_amd.runtime import config
from tests._metrics import assert_close_bf16, bf16_round

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
  M.layer_stack_indices.clear()


def _prepared(mod):
  mod = mod.to(DEV)
  backends.prepare(mod)
  return mod


def _params(mod):
  rounded = {f"{name}.weight" for name, m in mod.named_modules() if isinstance(m, M.Linear)}
  return {k: (bf16_round(v.float().cpu()) if k in rounded else v.float().cpu()) for k, v in mod.state_dict().items()}


def _call(hip, z, seq, params: ibs.IBSParams, **kw):
  return ops.triangle_attention_ibs(z, seq, hip._hip_ln_w, hip._hip_ln_b, hip._hip_w_qkvgb, hip._hip_w_o,
                                    num_head=hip.config.num_head, transpose=hip.transpose,
                                    num_samples=params.num_samples, num_rand_blocks=params.num_rand_blocks,
                                    t_prob=params.t_prob, tr_prob=params.tr_prob, u_prob=params.u_prob,
                                    add_residual=False, **kw)


def _rows_of(upd, rows, transpose):
  """The update of attention rows ``rows`` in the attention frame (as the oracle returns it)."""
  return upd[:, rows].transpose(0, 1) if transpose else upd[rows]


def _block_valid(seq, T):
  return np.array([bool(seq[32 * b:32 * b + 32].any()) for b in range(T)])


@pytest.mark.parametrize("N,padded,transpose", [(64, False, False), (97, True, True), (200, True, False)])
def test_ibs_dense_when_every_block_fits(N, padded, transpose):
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=padded, seed=31, sharp=True)
  hip = _prepared(mod)
  T = (N + 31) // 32
  params = ibs.IBSParams(num_samples=T + 1, num_rand_blocks=2)
  upd, im, wm = _call(hip, z.to(DEV), seq.to(DEV), params, seed=5)
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert_close_bf16(upd, ref, f"IBS dense-equivalent N={N}", max_abs=2e-2 * ref.abs().max().item())
  im, wm = im.cpu().numpy(), wm.cpu().numpy()
  valid = np.flatnonzero(_block_valid(seq.numpy(), T))
  for r in range(N):
    if not seq[r]:
      assert (im[r] == -1).all() and (wm[r] == 0).all()
      continue
    expect = np.full(params.num_samples, -1)
    expect[:len(valid)] = valid
    assert (im[r] == expect).all(), f"row {r}"
    assert (wm[r][..., :len(valid)] == 1.0).all() and (wm[r][..., len(valid):] == 0.0).all()


def _synthetic_maps(N, H, S, seed):
  """Random maps: per tile 1..S distinct blocks, one of them block 0 (so that every tile sees a
  valid key: the attention of a tile without one is undefined), weights in [0.5, 3]."""
  rng = np.random.default_rng(seed)
  T = (N + 31) // 32
  im = np.full((N, H, T, S), -1, np.int32)
  wm = np.zeros((N, H, T, S), np.float32)
  for r in range(N):
    for h in range(H):
      for t in range(T):
        n = int(rng.integers(1, min(S, T) + 1))
        blocks = rng.choice(T, size=n, replace=False)
        if 0 not in blocks:
          blocks[rng.integers(n)] = 0
        im[r, h, t, :n] = blocks
        wm[r, h, t, :n] = rng.uniform(0.5, 3.0, size=n)
  return im, wm


@pytest.mark.parametrize("N,transpose,limit", [(200, False, 0.0), (200, True, 0.0), (200, False, 1.0),
                                              (520, False, 0.0), (520, True, 0.0)])
def test_ibs_given_maps_match_oracle(N, transpose, limit):
  """limit 1 flags every (row, head) of the tile pipeline (weight sums exceed 1), so the exact
  block-sparse kernel recomputes all of them.  N=520: 3 query blocks, the last half full, which a
  workgroup's tasks step through (waves idle in one task and active in the next)."""
  S = 4
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=True, seed=33, sharp=True)
  hip = _prepared(mod)
  im, wm = _synthetic_maps(N, 4, S, seed=3)
  params = ibs.IBSParams(num_samples=S, num_rand_blocks=1)
  upd, im_out, wm_out = _call(hip, z.to(DEV), seq.to(DEV), params, fixup_sum_limit=limit,
                              index_map=torch.from_numpy(im).to(DEV), weight_map=torch.from_numpy(wm).to(DEV))
  assert (im_out.cpu().numpy() == im).all() and (wm_out.cpu().numpy() == wm).all(), "given maps are not rewritten"
  rows = [0, 1, 63, 64, 150, N // 2 + 1, N - 1]       # N - 1: a masked row
  assert not seq[N - 1]
  ref = ibs.grid_self_attention_ibs(z.float(), seq, _params(hip), transpose=transpose, params=params, seed=0,
                                    maps=(im, wm), rows=rows).float()
  got = _rows_of(upd, rows, transpose).float().cpu()
  assert_close_bf16(got, ref, f"IBS given maps transpose={transpose} limit={limit}",
                    max_abs=2e-2 * ref.abs().max().item())
  if limit:
    default, _, _ = _call(hip, z.to(DEV), seq.to(DEV), params, index_map=im_out, weight_map=wm_out)
    assert not torch.equal(default, upd), "the exact kernel (fp32 weights) recomputed the rows"


def _check_structure(im, wm, seq, S, R, T):
  valid = _block_valid(seq, T)
  for r in range(im.shape[0]):
    if not seq[r]:
      assert (im[r] == -1).all()
      continue
    for h in range(im.shape[1]):
      for t in range(T):
        idx, w = im[r, h, t], wm[r, h, t]
        n = int((idx >= 0).sum())
        assert (idx[:n] >= 0).all() and (idx[n:] == -1).all() and (w[n:] == 0).all(), "filled slots form a prefix"
        assert n >= 1 and len(set(idx[:n].tolist())) == n and (idx[:n] < T).all()
        assert valid[idx[:n]].all(), "only blocks with a valid key"
        assert (w[:n] > 0).all()
        static = int(np.argmax(w[:n] != 1.0)) if (w[:n] != 1.0).any() else n
        assert static >= 1 and (static <= S - R or n == static)
        assert n - static <= R


@pytest.mark.parametrize("transpose", [False, True])
def test_ibs_generated_maps(transpose):
  N, S, R = 384, 6, 2
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=True, seed=35, sharp=True)
  hip = _prepared(mod)
  params = ibs.IBSParams(num_samples=S, num_rand_blocks=R, t_prob=0.5, tr_prob=0.95, u_prob=0.02)
  zd, sd = z.to(DEV), seq.to(DEV)
  upd, im, wm = _call(hip, zd, sd, params, seed=77)
  T = (N + 31) // 32
  imn, wmn = im.cpu().numpy(), wm.cpu().numpy()
  _check_structure(imn, wmn, seq.numpy(), S, R, T)
  assert (wmn != 1.0).any() and ((imn >= 0).sum(-1) < T).all(), "the maps are sparse and sampled"
  # the attention follows the maps it produced
  rows = [0, 5, 100, 200, 300, N - 1]
  ref = ibs.grid_self_attention_ibs(z.float(), seq, _params(hip), transpose=transpose, params=params, seed=0,
                                    maps=(imn, wmn), rows=rows).float()
  got = _rows_of(upd, rows, transpose).float().cpu()
  assert_close_bf16(got, ref, f"IBS generated maps transpose={transpose}", max_abs=2e-2 * ref.abs().max().item())
  # reuse reproduces the generating call; the seed alone decides the maps
  upd2, _, _ = _call(hip, zd, sd, params, index_map=im, weight_map=wm)
  assert torch.equal(upd2, upd)
  _, im3, wm3 = _call(hip, zd, sd, params, seed=77)
  assert torch.equal(im3, im) and torch.equal(wm3, wm)
  _, im4, _ = _call(hip, zd, sd, params, seed=78)
  assert not torch.equal(im4, im)


def _round_np(n):
  return (n + 127) & ~127


def _bias_pos64(j):
  j32 = j & 31
  return (j & 32) + 16 * ((j32 >> 2) & 1) + 4 * (j32 >> 3) + (j32 & 3)


def _decode_operands(ws, N, H):
  """Q, K [r][h][NP][32] and bias [h][NP][NP] (keys in natural order) from the workspace of the
  projection stage: Q / K pieces of 8 dims 16 kk + 8 (t / 4) + 4 hf + t % 4 per (32-position
  block, kk, hf, position); bias as 4 KB blocks per (head, 32 queries, 64 keys) of
  [k 4][hf 2][query 32][8 keys], piece k of lane half hf holding stored piece
  4 (k / 2) + 2 hf + k % 2, with keys permuted within 64-key tiles."""
  NP = _round_np(N)
  E = NP * NP * H * 32
  rup = lambda x: (x + 255) & ~255
  raw = ws.cpu()
  def bf(off, count):
    return raw[off:off + 2 * count].view(torch.bfloat16).float()
  dims = torch.tensor([16 * kk + 8 * (t // 4) + 4 * hf + t % 4 for kk in range(2) for hf in range(2) for t in range(8)])

  def layout(off):
    x = bf(off, E).reshape(NP, H, NP // 32, 2, 2, 32, 8)          # r h pb kk hf p t
    x = x.permute(0, 1, 2, 5, 3, 4, 6).reshape(NP, H, NP, 32)       # r h p (kk hf t)
    out = torch.empty_like(x)
    out[..., dims] = x
    return out
  q = layout(0)
  k = layout(rup(E * 2))
  bias_off = 3 * rup(E * 2)
  blocks = bf(bias_off, H * NP * NP).reshape(H, NP // 32, NP // 64, 2, 2, 2, 32, 8)  # h qt kt k2 k1 hf i e
  planes = blocks.permute(0, 1, 6, 2, 3, 5, 4, 7).reshape(H, NP, NP)                # h (qt i) (kt k2 hf k1 e)
  j = torch.arange(NP)
  stored = (j & ~63) + torch.tensor([_bias_pos64(int(x) & 63) for x in j])
  return q, k, planes[:, :, stored]


@pytest.mark.parametrize("transpose", [False, True])
def test_ibs_sampler_matches_oracle_on_kernel_operands(transpose):
  N, H, S, R = 300, 4, 5, 2
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=True, seed=37, sharp=True)
  hip = _prepared(mod)
  params = ibs.IBSParams(num_samples=S, num_rand_blocks=R, t_prob=0.5, tr_prob=0.95, u_prob=0.02)
  need = ops.triangle_ibs_workspace_bytes(N, 128, H, 32)
  ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
  _, im, wm = _call(hip, z.to(DEV), seq.to(DEV), params, seed=91, workspace=ws)
  torch.cuda.synchronize()
  q, k, bias = _decode_operands(ws, N, H)
  imn, wmn = im.cpu().numpy(), wm.cpu().numpy()
  same = total = 0
  for r in [0, 1, 2, 17, 64, 128, 199, 250, 269]:
    assert seq[r]
    key_valid = seq.clone()
    for h in range(H):
      masses = ibs.block_masses(q[r, h, :N], k[r, h, :N], bias[h, :N, :N], key_valid)
      idx, wt = ibs.select_blocks(masses, params, seed=91, batch=0, row=r, head=h)
      for t in range(idx.shape[0]):
        total += 1
        if (idx[t] == imn[r, h, t]).all():
          same += 1
          np.testing.assert_allclose(wmn[r, h, t], wt[t], rtol=1e-4, err_msg=f"weights r={r} h={h} t={t}")
  assert same >= 0.99 * total, f"sampler agrees on {same} of {total} tiles"


def test_ibs_module_switch_and_reuse():
  N = 160
  mod, z, seq = W.make_triangle(N, padded=True, seed=39, sharp=True)
  p = M.IBSAParameters(num_samples=3, num_rand_blocks=1, t_prob=0.5, tr_prob=0.95, u_prob=0.02)
  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda", hip_sparse_grid_attention=True)
  backends.init()
  reuse = lambda indices: (0,) if indices == (1,) else None
  sparse = M.GridSelfAttention(M.GridSelfAttention.Config(num_head=4), M.GlobalConfig(), False, num_channels=128,
                               name="pair_attention", ibsa_params=p, index_reuse_policy=reuse)
  sparse.load_state_dict(mod.state_dict())
  hip = _prepared(sparse)
  zd, sd = z.to(DEV).unsqueeze(0), seq.to(DEV)
  M.layer_stack_indices[:] = [0]
  out0 = hip(zd, sd)
  im0, wm0 = hip.last_maps
  assert im0.shape == (1, N, 4, 5, 3)
  upd, _, _ = _call(hip, zd[0], sd, ibs.IBSParams(3, 1, 0.5, 0.95, 0.02), index_map=im0[0], weight_map=wm0[0])
  assert_close_bf16(out0[0], zd[0].float() + upd.float(), "module = input + the op's update on its maps")
  M.layer_stack_indices[:] = [1]                        # reuses layer 0's maps
  out1 = hip(zd, sd)
  assert torch.equal(hip.last_maps[0], im0) and torch.equal(out1, out0)
  M.layer_stack_indices[:] = [2]                        # samples afresh (new seed)
  hip(zd, sd)
  assert not torch.equal(hip.last_maps[0], im0)
  # with the switch off the same module is dense
  config.configure_runtime(backend="hip", sdpa_implementation="hip", device="cuda")
  dense = hip(zd, sd, add_residual=False)[0]
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=False, return_update=True)
  assert_close_bf16(dense, ref, "switch off: dense", max_abs=2e-2 * ref.abs().max().item())


def _large_maps(N, H, S, seed):
  """Vectorised synthetic maps for large N: slot 0 = block 0 and slot 1 = the last block (so the
  tile kernel's per-wave table is filled to its last entry), the others random (repeats allowed:
  a repeated block is the same as one slot with the summed weight); weights in [0.5, 3], except
  that slot S-1 is unused -- index -1, weight 0 or a negative weight, by tile."""
  rng = np.random.default_rng(seed)
  T = (N + 31) // 32
  im = rng.integers(0, T, size=(N, H, T, S), dtype=np.int32)
  im[..., 0] = 0
  im[..., 1] = T - 1
  wm = rng.uniform(0.5, 3.0, size=(N, H, T, S)).astype(np.float32)
  kind = rng.integers(0, 3, size=(N, H, T))
  im[..., S - 1] = np.where(kind == 0, -1, im[..., S - 1])
  wm[..., S - 1] = np.where(kind == 1, 0.0, np.where(kind == 2, -1.5, wm[..., S - 1]))
  return im, wm


@pytest.mark.parametrize("N", [4096, 4100])
def test_ibs_given_maps_large(N):
  """N=4096: the tile kernel with its per-wave block table full (T = 128 blocks, the last one
  selected everywhere).  N=4100: above the table's limit, so every row runs on the exact
  block-sparse kernel alone.  Slots with a negative or zero weight count as unused in both.  A
  few rows against the oracle, which runs on the GPU here (its LayerNorm and bias planes over the
  N^2 positions would take minutes on the host)."""
  H, S = 4, 4
  print(f"[case] IBS given maps N={N}", flush=True)
  mod, _, _ = W.make_triangle(1, seed=41, sharp=True)       # the weights do not depend on N
  hip = _prepared(mod)
  g = torch.Generator(device=DEV).manual_seed(41)
  zd = torch.randn(N, N, 128, generator=g, device=DEV).to(torch.bfloat16)   # 4.3 GB: made on the GPU
  seq = torch.ones(N, dtype=torch.bool)
  im, wm = _large_maps(N, H, S, seed=4)
  params = ibs.IBSParams(num_samples=S, num_rand_blocks=1)
  upd, _, _ = _call(hip, zd, seq.to(DEV), params, index_map=torch.from_numpy(im).to(DEV),
                    weight_map=torch.from_numpy(wm).to(DEV))
  torch.cuda.synchronize()
  rows = [0, N // 2 + 1, N - 1]
  got = upd[rows].float().cpu()
  del upd
  pd = {k: v.to(DEV) for k, v in _params(hip).items()}
  ref = ibs.grid_self_attention_ibs(zd.float(), seq.to(DEV), pd, transpose=False, params=params, seed=0,
                                    maps=(im, wm), rows=rows).float().cpu()
  assert_close_bf16(got, ref, f"IBS given maps N={N}", max_abs=2e-2 * ref.abs().max().item())
