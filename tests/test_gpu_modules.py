"""Module-level parity: the HIP backend's four attention forms vs the oracle composites,
through the reference lifecycle (configure_runtime -> backends.init -> construct ->
load weights -> backends.prepare -> forward)."""
import pytest
import torch

from oracle import modules as OM
from sparsefold_amd import backends
from sparsefold_amd import workloads as W
from sparsefold_amd.runtime import config
from tests._metrics import BF16_ULP, assert_close_bf16, bf16_round

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


def _prepared(mod):
  mod = mod.to(DEV)
  counts = backends.prepare(mod)
  assert counts["opaque"] >= 1
  return mod


def _params(mod):
  """float32 copies of the weights as the HIP path sees them: projection matrices rounded
  to bf16 (the kernels' MFMA operands), norm parameters and biases kept in float32."""
  from sparsefold_amd import modules as M
  rounded = {f"{name}.weight" if name else "weight" for name, m in mod.named_modules() if isinstance(m, M.Linear)}
  return {k: (bf16_round(v.float().cpu()) if k in rounded else v.float().cpu()) for k, v in mod.state_dict().items()}


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_c1_n20_fp32(transpose):
  mod, z, seq = W.make_triangle(20, transpose=transpose, seed=1, dtype=torch.float32)
  hip = _prepared(mod)
  out = hip(z.to(DEV), seq.to(DEV))
  assert out.dtype == torch.float32
  p = _params(hip)
  ref = OM.grid_self_attention(z, seq, p, transpose=transpose)
  assert_close_bf16(out, ref, f"C1 triangle N=20 transpose={transpose}")
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False)
  ref_u = OM.grid_self_attention(bf16_round(z), seq, p, transpose=transpose, return_update=True)
  assert_close_bf16(upd, ref_u, "C1 update", max_abs=2e-2 * ref_u.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("N", [64, 97])
def test_triangle_sharp_update_padded(transpose, N):
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=True, seed=7, sharp=True, act_norm_bias=True)
  hip = _prepared(mod)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False)
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert_close_bf16(upd, ref, f"triangle sharp N={N} transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("N,padded", [(1, False), (3, False), (11, True), (65, True), (257, False)])
def test_triangle_edge_sizes(transpose, N, padded):
  """Sizes at the edges of the fast path's tiling: a single token, fewer tokens than one
  32-query block, one key past a 64-key tile (65: NP=128 with 63 padding keys), and one query
  past a 256-query workgroup block (257)."""
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=padded, seed=13, sharp=True)
  hip = _prepared(mod)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False)
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert torch.isfinite(upd).all()
  assert_close_bf16(upd, ref, f"triangle N={N} transpose={transpose}", max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("N,masked", [(100, "all"), (300, "leading"), (257, "every_other_group")])
def test_triangle_masked_row_groups(transpose, N, masked):
  """Row groups (4 attention rows) whose rows are all masked or past N are not scheduled: every
  token masked (no attention task runs; the fix-up writes every row), a masked prefix, and masks
  that leave every other row group empty."""
  mod, z, seq = W.make_triangle(N, transpose=transpose, seed=43, sharp=True)
  if masked == "all":
    seq[:] = False
  elif masked == "leading":
    seq[:37] = False
  else:
    seq[:] = torch.tensor([(i // 4) % 2 == 0 for i in range(N)])
  hip = _prepared(mod)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False)
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert torch.isfinite(upd).all()
  assert_close_bf16(upd, ref, f"triangle N={N} masked={masked} transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


def _triangle_update(hip, z, seq, add_residual=False, **kw):
  """The module's update through the C entry point with its packed weights (the module's own
  forward, plus the explicit test controls of ops.triangle_attention)."""
  from sparsefold_amd.backends.hip import ops
  return ops.triangle_attention(z, seq, hip._hip_ln_w, hip._hip_ln_b, hip._hip_w_qkvgb, hip._hip_w_o,
                                num_head=hip.config.num_head, transpose=hip.transpose, add_residual=add_residual,
                                **kw)


@pytest.mark.parametrize("limit", [1.0, 1500.0])
@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_exact_fixup(transpose, limit):
  """The attention kernel exponentiates logits against a fixed reference point and flags a
  (row, head) whose weight sum leaves [2^-100, limit]; the fix-up kernel recomputes those with
  an exact two-pass softmax.  A limit of 1 flags every row; 1500 lies near the 90th percentile
  of the per-(row, head) maximum weight sums of this input (N=200, sharp weights), so flagged
  and fast-path rows meet in one call.  Padded rows stay on the masked-row path.  The result
  must match the oracle either way."""
  mod, z, seq = W.make_triangle(200, transpose=transpose, padded=True, seed=11, sharp=True)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  upd_default = hip(zd, sd, add_residual=False)
  assert torch.equal(_triangle_update(hip, zd, sd), upd_default)
  upd = _triangle_update(hip, zd, sd, fixup_sum_limit=limit)
  # the exact path keeps fp32 weights (the fast path rounds them to bf16), so the attention rows
  # it recomputed differ from the default call: every unmasked row at limit 1, some at 1500
  rows = (upd != upd_default).transpose(0, 1) if transpose else (upd != upd_default)
  changed = rows.flatten(1).any(1).cpu()
  assert not changed[~seq].any()
  if limit == 1.0:
    assert changed[seq].all()
  else:
    assert 0 < int(changed[seq].sum()) < int(seq.sum())
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert_close_bf16(upd, ref, f"triangle exact fix-up N=200 limit={limit} transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())
  # the flags were cleared: the next default call is the fast path again, bit for bit
  assert torch.equal(hip(zd, sd, add_residual=False), upd_default)


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_c2_n384_padded(transpose):
  mod, z, seq = W.make_triangle(384, transpose=transpose, padded=True, seed=2)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  out = hip(zd, sd)
  p = _params(hip)
  ref = OM.grid_self_attention(z.float(), seq, p, transpose=transpose, chunk_size=128)
  assert_close_bf16(out, ref, f"C2 triangle N=384 transpose={transpose}")
  upd = hip(zd, sd, add_residual=False)
  ref_u = ref - z.float()
  assert_close_bf16(upd, ref_u, "C2 update", max_abs=2e-2 * ref_u.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_c3_n768_sampled_rows(transpose):
  mod, z, seq = W.make_triangle(768, transpose=transpose, seed=3)
  hip = _prepared(mod)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False).float().cpu()
  rows = [0, 1, 255, 383, 384, 511, 700, 767]
  ref = OM.grid_self_attention_rows(z.float(), seq, _params(hip), transpose=transpose, rows=rows)
  got = upd[:, rows].transpose(0, 1) if transpose else upd[rows]
  assert_close_bf16(got, ref, f"C3 triangle N=768 rows transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


_N768_CACHE: dict = {}


def _n768_sharp_padded(transpose: bool):
  """HIP update, oracle inputs and the shared LN / bias prologue of the sharp, padded N=768
  triangle case (computed once per node for the row-range tests below)."""
  if transpose not in _N768_CACHE:
    from oracle.primitives import layer_norm, linear
    mod, z, seq = W.make_triangle(768, transpose=transpose, padded=True, seed=17, sharp=True)
    hip = _prepared(mod)
    print(f"[case] triangle N=768 sharp padded transpose={transpose}", flush=True)
    upd = hip(z.to(DEV), seq.to(DEV), add_residual=False).float().cpu()
    p = _params(hip)
    zf = z.float()
    x = layer_norm(zf, p["act_norm.weight"], p.get("act_norm.bias"))
    bias = linear(x, p["pair_bias_projection.weight"]).movedim(-1, -3).contiguous()
    _N768_CACHE.clear()
    _N768_CACHE[transpose] = (upd.transpose(0, 1) if transpose else upd, zf, seq, p, bias)
  return _N768_CACHE[transpose]


# rows of the first and the last task of every persistent attention workgroup at N=768 (256
# workgroups x 9 tasks of 4 rows; task t of XCD x covers rows 4 ((t/3) mod 192)): the prologue
# with nothing to overlap and the final drain
_N768_FIRST_LAST = list(range(0, 44)) + list(range(340, 428)) + list(range(724, 768))


@pytest.mark.parametrize("transpose,rows", [(False, (0, 256)), (False, (256, 512)), (False, (512, 768)),
                                            (True, "first_last")])
def test_triangle_c3_n768_sharp_padded_rows(transpose, rows):
  """N=768 (the headline size) with sharp weights (a far-from-uniform softmax) and the last 76
  tokens padded, against the oracle row by row: every row of the starting node -- so every task
  boundary, where the next task's first tile and Q operands are loaded during the last tile --
  and, for the ending node, the rows of every workgroup's first and last task.  Covers the
  masked rows (fix-up kernel) and the padded keys of the last 64-key tile."""
  got_all, zf, seq, p, bias = _n768_sharp_padded(transpose)
  assert torch.isfinite(got_all).all()
  sel = list(range(*rows)) if rows != "first_last" else _N768_FIRST_LAST
  refs = [OM.grid_self_attention_rows(zf, seq, p, transpose=transpose, rows=sel[i:i + 32], bias=bias)
          for i in range(0, len(sel), 32)]
  ref = torch.cat(refs)
  got = got_all[sel]
  assert_close_bf16(got, ref, f"C3 triangle N=768 sharp padded rows {rows} transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())
  masked = [i for i, r in enumerate(sel) if not bool(seq[r])]
  if masked:                          # padded tokens attend uniformly: the mean of V, gated and projected
    assert got[masked].abs().max() > 0


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_n600_idle_waves(transpose):
  """N=600 pads to 640 positions: 3 blocks of 256 queries, the last with 128, so waves 4-7 of a
  workgroup are idle in its tasks of the last block, and since a workgroup's tasks step through
  the blocks (32 mod 3 != 0), they are active again in the next task.  Every row against the
  oracle, sharp weights (a wrong bias tile in any task's first tile shows)."""
  from oracle.primitives import layer_norm, linear
  mod, z, seq = W.make_triangle(600, transpose=transpose, padded=True, seed=23, sharp=True)
  hip = _prepared(mod)
  print(f"[case] triangle N=600 sharp padded transpose={transpose}", flush=True)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False).float().cpu()
  got_all = upd.transpose(0, 1) if transpose else upd
  p = _params(hip)
  zf = z.float()
  x = layer_norm(zf, p["act_norm.weight"], p.get("act_norm.bias"))
  bias = linear(x, p["pair_bias_projection.weight"]).movedim(-1, -3).contiguous()
  sel = list(range(600))
  ref = torch.cat([OM.grid_self_attention_rows(zf, seq, p, transpose=transpose, rows=sel[i:i + 40], bias=bias)
                   for i in range(0, 600, 40)])
  assert_close_bf16(got_all, ref, f"triangle N=600 sharp padded transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("C,N,transpose", [(128, 70, False), (128, 300, True), (128, 520, False),
                                            (128, 800, True), (128, 1100, False), (128, 1100, True),
                                            (128, 1300, False), (64, 520, True), (64, 1100, False)])
def test_triangle_schedule_classes(C, N, transpose):
  """Sizes across the attention kernel's schedule classes: 1 to 6 query blocks of 256 (NP =
  N rounded up to 128), a half-full last block whose waves 4-7 idle (70, 300, 520, 800, 1100,
  1300), blocks that a workgroup's tasks step through (32 mod QB != 0: 520, 1100, 1300) or not
  (300, 800), padded tokens, both nodes and both head dims.  Sampled rows: the first two row
  groups, the middle and the last, against the oracle with sharp weights."""
  mod, z, seq = W.make_triangle(N, C=C, H=4, transpose=transpose, padded=True, seed=29 + N, sharp=True)
  hip = _prepared(mod)
  print(f"[case] triangle C={C} N={N} transpose={transpose}", flush=True)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False).float().cpu()
  got_all = upd.transpose(0, 1) if transpose else upd
  rows = sorted({0, 3, 4, 7, N // 2, N // 2 + 1, N - 4, N - 1} & set(range(N)))
  ref = OM.grid_self_attention_rows(z.float(), seq, _params(hip), transpose=transpose, rows=rows)
  assert torch.isfinite(got_all[rows]).all()
  assert_close_bf16(got_all[rows], ref, f"triangle C={C} N={N} transpose={transpose} rows {rows}",
                    max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_n768_sharp_padded_repeatable(transpose):
  """Two calls on the same inputs give the same bits.  At N=768 every persistent attention
  workgroup runs 9 tasks, so the last tile of each task -- which loads the next task's first tile
  and Q operands behind partial waits -- runs 8 times per workgroup; a wait that let a load land
  late would show up as differing bits between calls."""
  mod, z, seq = W.make_triangle(768, transpose=transpose, padded=True, seed=17, sharp=True)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  first = hip(zd, sd, add_residual=False)
  for _ in range(3):
    assert torch.equal(hip(zd, sd, add_residual=False), first)
  assert torch.equal(hip(zd, sd), hip(zd, sd))


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("N,limit", [(768, 0.0), (768, 1.0), (384, 0.0), (200, 1500.0), (257, 0.0), (20, 0.0)])
def test_triangle_fused_output_stage(transpose, N, limit):
  """The opt-in fused kernel (SF_TRI_STAGE_FUSE: the attention epilogue writes each group's
  output rows once its four heads are done, flagged rows go to the post kernel) gives the same bits
  as the separate stages: every row and node, padded rows (mean of V in the epilogue), and rows
  recomputed by the exact fix-up (limit 1: every row deferred; 1500: some)."""
  from sparsefold_amd import _lib
  mod, z, seq = W.make_triangle(N, transpose=transpose, padded=True, seed=29, sharp=True)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  print(f"[case] fused output stage N={N} limit={limit} transpose={transpose}", flush=True)
  for residual in (False, True):
    ref = _triangle_update(hip, zd, sd, fixup_sum_limit=limit, add_residual=residual)
    fused = _triangle_update(hip, zd, sd, fixup_sum_limit=limit, add_residual=residual,
                             stages=_lib.TRI_STAGE_ALL | _lib.TRI_STAGE_FUSE)
    assert torch.isfinite(fused).all()
    assert torch.equal(fused, ref), f"max diff {(fused.float() - ref.float()).abs().max().item():.3e}"
  # the counters are reset for the next call: a second fused call gives the same bits
  again = _triangle_update(hip, zd, sd, fixup_sum_limit=limit, add_residual=True,
                           stages=_lib.TRI_STAGE_ALL | _lib.TRI_STAGE_FUSE)
  assert torch.equal(again, ref)


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("N,padded,sharp", [(96, True, True), (200, True, False), (37, False, True),
                                            (1, False, True), (65, True, True), (257, False, True),
                                            (600, True, True)])
def test_triangle_template_stack_shape(transpose, N, padded, sharp):
  """The template stack's PairFormer triangle attention (model/embeddings/template.py:122-127,
  304-313): C=64, H=4, so D=16 -- the head-dim-16 instance of the fast path (fold, projection
  into the attention layouts, tile attention, fix-up, gate and output projection).  Includes the
  tiling edges: one token, one key past a 64-key tile (65), one query past a 256-query block,
  and N=600, whose half-full last query block leaves waves idle in one task and active in the
  next."""
  mod, z, seq = W.make_triangle(N, C=64, H=4, transpose=transpose, padded=padded, seed=23, sharp=sharp)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  p = _params(hip)
  upd = hip(zd, sd, add_residual=False)
  ref_u = OM.grid_self_attention(z.float(), seq, p, transpose=transpose, return_update=True)
  assert torch.isfinite(upd).all()
  assert_close_bf16(upd, ref_u, f"template triangle N={N} transpose={transpose} update",
                    max_abs=2e-2 * ref_u.abs().max().item())
  out = hip(zd, sd)
  ref = OM.grid_self_attention(z.float(), seq, p, transpose=transpose)
  assert_close_bf16(out, ref, f"template triangle N={N} transpose={transpose}")


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("masked", ["all", "leading"])
def test_triangle_template_stack_masked_rows(transpose, masked):
  """Head dim 16 with masked attention rows: every token masked (no attention task runs; the
  fix-up writes the mean of V for every row) and a masked prefix."""
  mod, z, seq = W.make_triangle(100, C=64, H=4, transpose=transpose, seed=43, sharp=True)
  if masked == "all":
    seq[:] = False
  else:
    seq[:37] = False
  hip = _prepared(mod)
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False)
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert torch.isfinite(upd).all()
  assert_close_bf16(upd, ref, f"template triangle masked={masked} transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_template_stack_exact_fixup(transpose):
  """Head dim 16 with a weight-sum limit of 1: every unmasked (row, head) is flagged and
  recomputed by the exact two-pass softmax; the flags are cleared for the next call."""
  mod, z, seq = W.make_triangle(200, C=64, H=4, transpose=transpose, padded=True, seed=11, sharp=True)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  upd_default = hip(zd, sd, add_residual=False)
  upd = _triangle_update(hip, zd, sd, fixup_sum_limit=1.0)
  rows = (upd != upd_default).transpose(0, 1) if transpose else (upd != upd_default)
  changed = rows.flatten(1).any(1).cpu()
  assert not changed[~seq].any()
  assert changed[seq].all()
  ref = OM.grid_self_attention(z.float(), seq, _params(hip), transpose=transpose, return_update=True)
  assert_close_bf16(upd, ref, f"template triangle exact fix-up transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())
  assert torch.equal(hip(zd, sd, add_residual=False), upd_default)


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_template_stack_n768(transpose):
  """Head dim 16 at N=768, sharp weights, the last 76 tokens padded: the rows of every
  persistent attention workgroup's first and last task against the oracle, two calls bit for
  bit equal (9 tasks per workgroup: the next-task hand-off behind partial waits runs 8 times),
  and the single stages run one after another against one workspace give the same bits."""
  from oracle.primitives import layer_norm, linear
  from sparsefold_amd import _lib
  mod, z, seq = W.make_triangle(768, C=64, H=4, transpose=transpose, padded=True, seed=17, sharp=True)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  print(f"[case] template triangle N=768 transpose={transpose}", flush=True)
  first = hip(zd, sd, add_residual=False)
  for _ in range(2):
    assert torch.equal(hip(zd, sd, add_residual=False), first)
  ws = torch.empty(_lib.load().sf_hip_triangle_workspace_bytes(768, 64, 4, 16), dtype=torch.uint8, device=DEV)
  out = torch.empty_like(first)
  for st in (_lib.TRI_STAGE_PROJECT, _lib.TRI_STAGE_ATTEND, _lib.TRI_STAGE_OUTPUT):
    _triangle_update(hip, zd, sd, stages=st, workspace=ws, out=out)
  assert torch.equal(out, first)
  upd = (first.float().cpu().transpose(0, 1) if transpose else first.float().cpu())
  p = _params(hip)
  zf = z.float()
  x = layer_norm(zf, p["act_norm.weight"], p.get("act_norm.bias"))
  bias = linear(x, p["pair_bias_projection.weight"]).movedim(-1, -3).contiguous()
  sel = _N768_FIRST_LAST
  ref = torch.cat([OM.grid_self_attention_rows(zf, seq, p, transpose=transpose, rows=sel[i:i + 32], bias=bias)
                   for i in range(0, len(sel), 32)])
  assert_close_bf16(upd[sel], ref, f"template triangle N=768 transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_n768_exact_fixup_every_row(transpose):
  """N=768 with a weight-sum limit of 1: every unmasked (row, head) is flagged by the attention
  kernel and recomputed by the exact two-pass fix-up kernel."""
  mod, z, seq = W.make_triangle(768, transpose=transpose, padded=True, seed=19, sharp=True)
  hip = _prepared(mod)
  zd, sd = z.to(DEV), seq.to(DEV)
  upd = _triangle_update(hip, zd, sd, fixup_sum_limit=1.0).float().cpu()
  rows = list(range(0, 768, 37)) + [767]
  ref = OM.grid_self_attention_rows(z.float(), seq, _params(hip), transpose=transpose, rows=rows)
  got = upd[:, rows].transpose(0, 1) if transpose else upd[rows]
  assert_close_bf16(got, ref, f"triangle N=768 exact path transpose={transpose}",
                    max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("N,padded,sharp", [(96, True, True), (768, False, False)])
def test_single_attention_with_pair_bias(N, padded, sharp):
  mod, z, s, seq = W.make_single(N, seed=3, padded=padded, sharp=sharp)
  hip = _prepared(mod)
  out = hip(z.to(DEV), s.to(DEV), seq.to(DEV))
  ref = OM.single_act_update_attention(z.float(), s.float(), seq, _params(hip))
  assert_close_bf16(out, ref, f"single N={N}")
  upd = hip(z.to(DEV), s.to(DEV), seq.to(DEV), add_residual=False)
  d_ref = OM.single_act_update_attention(z.float(), s.float(), seq, _params(hip), return_update=True)
  assert_close_bf16(upd, d_ref, f"single N={N} update", max_abs=2e-2 * d_ref.abs().max().item())


@pytest.mark.parametrize("N,keys", [(333, "padded"), (512, "second_half"), (512, "first_tile"), (512, "none")])
def test_single_attention_key_slices(N, keys):
  """Grids this small split each query block's key range over several waves and merge the
  slices: slices whose keys are all masked, a reference point set by one slice only, ragged last
  slices and rows with no valid key at all."""
  mod, z, s, seq = W.make_single(N, seed=5, padded=keys == "padded", sharp=True)
  if keys == "second_half":
    seq[N // 2:] = False
  elif keys == "first_tile":
    seq[64:] = False
  elif keys == "none":
    seq[:] = False
  hip = _prepared(mod)
  upd = hip(z.to(DEV), s.to(DEV), seq.to(DEV), add_residual=False)
  d_ref = OM.single_act_update_attention(z.float(), s.float(), seq, _params(hip), return_update=True)
  assert_close_bf16(upd, d_ref, f"single N={N} keys={keys}", max_abs=2e-2 * d_ref.abs().max().item())


@pytest.mark.parametrize("N,S,padded,sharp", [(100, 2, True, True), (300, 1, True, True), (1024, 5, False, False)])
def test_diffusion_token_attention(N, S, padded, sharp):
  mod, act, cond, bias, mask = W.make_diffusion(N, S=S, seed=4, padded=padded, sharp=sharp)
  hip = _prepared(mod)
  args = (act.to(DEV), mask.to(DEV))
  kw = dict(pair_logits=bias.to(DEV), single_cond=cond.to(DEV))
  out = hip(*args, **kw)
  p = _params(hip)
  ref = OM.self_attention(act.float(), mask, p, pair_logits=bias.float(), single_cond=cond.float())
  assert_close_bf16(out, ref, f"diffusion N={N} S={S}")
  upd = hip(*args, **kw, add_residual=False)
  d_ref = OM.self_attention(act.float(), mask, p, pair_logits=bias.float(), single_cond=cond.float(),
                            return_update=True)
  assert_close_bf16(upd, d_ref, "diffusion update", max_abs=2e-2 * d_ref.abs().max().item())


@pytest.mark.parametrize("atoms,S,sharp", [(256, 2, True), (8192, 5, False)])
def test_windowed_atom_attention(atoms, S, sharp):
  mod, act, lay, qc, kc, bias = W.make_window(atoms, S=S, seed=5, sharp=sharp)
  hip = _prepared(mod)
  args = (act.to(DEV), lay.queries_mask.to(DEV), lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV),
          lay.keys_mask.to(DEV), qc.to(DEV), kc.to(DEV), bias.to(DEV))
  out = hip.forward_indexed(*args)
  p = _params(hip)
  oargs = (act.float(), lay.queries_mask, lay.gather_idxs, lay.gather_mask, lay.keys_mask, qc.float(), kc.float(),
           bias.float(), p)
  ref = OM.windowed_cross_attention(*oargs)
  assert_close_bf16(out, ref, f"window atoms={atoms}")
  upd = hip.forward_indexed(*args, add_residual=False)
  d_ref = OM.windowed_cross_attention(*oargs, return_update=True)
  assert_close_bf16(upd, d_ref, "window update", max_abs=2e-2 * d_ref.abs().max().item())


@pytest.mark.parametrize("atoms,S,sharp", [(256, 2, True), (8192, 5, False), (8192, 5, True)])
def test_windowed_per_atom_plan(atoms, S, sharp):
  """keys_single_cond=None: the keys' condition is the gathered queries' (as CrossAttTransformer
  builds it), so both sides' AdaLN terms are per atom, K/V are projected per atom and the
  attention gathers each window's rows (invalid keys: zero rows).  The workload's key condition is
  that gather, so the oracle and the general path see the same inputs."""
  mod, act, lay, qc, kc, bias = W.make_window(atoms, S=S, seed=5, sharp=sharp)
  U = atoms // 32
  ref_kc = OM.atom_layout_convert(lay.gather_idxs, lay.gather_mask, (U, 32), qc.float(), layout_axes=(-3, -2))
  assert torch.equal(kc.float(), ref_kc)
  hip = _prepared(mod)
  ad, qcd, bd = act.to(DEV), qc.to(DEV), bias.to(DEV)
  idx, gm = lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV)
  qm, km = lay.queries_mask.to(DEV), lay.keys_mask.to(DEV)
  out = hip.forward_indexed(ad, qm, idx, gm, km, qcd, None, bd)
  p = _params(hip)
  oargs = (act.float(), lay.queries_mask, lay.gather_idxs, lay.gather_mask, lay.keys_mask, qc.float(), kc.float(),
           bias.float(), p)
  ref = OM.windowed_cross_attention(*oargs)
  assert_close_bf16(out, ref, f"per-atom plan atoms={atoms} sharp={sharp}")
  upd = hip.forward_indexed(ad, qm, idx, gm, km, qcd, None, bd, add_residual=False)
  d_ref = OM.windowed_cross_attention(*oargs, return_update=True)
  assert_close_bf16(upd, d_ref, "per-atom plan update", max_abs=2e-2 * d_ref.abs().max().item())
  general = hip.forward_indexed(ad, qm, idx, gm, km, qcd, kc.to(DEV), bd, add_residual=False)
  assert_close_bf16(upd, general.float().cpu(), "per-atom plan vs general path", max_abs=2e-2 * d_ref.abs().max().item())
  # the conditioning is computed once per condition tensor, again after it changes in place
  first = hip._hip_cond_cache[2]
  hip.forward_indexed(ad, qm, idx, gm, km, qcd, None, bd)
  assert hip._hip_cond_cache[2] is first
  qcd.mul_(1.0)
  hip.forward_indexed(ad, qm, idx, gm, km, qcd, None, bd)
  assert hip._hip_cond_cache[2] is not first


def test_windowed_per_atom_plan_new_condition_at_a_freed_address():
  """A later example's condition is a new tensor of the same shape.  Even if the allocator would
  hand it the memory of the previous (freed) condition, the per-atom plan must not reuse that
  condition's cached AdaLN terms: the output follows the new values."""
  mod, act, lay, qc, kc, bias = W.make_window(256, S=2, seed=5, sharp=True)
  hip = _prepared(mod)
  ad, bd = act.to(DEV), bias.to(DEV)
  idx, gm = lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV)
  qm, km = lay.queries_mask.to(DEV), lay.keys_mask.to(DEV)
  first = hip.forward_indexed(ad, qm, idx, gm, km, qc.to(DEV), None, bd, add_residual=False).float().cpu()
  torch.cuda.synchronize()
  qc2 = torch.randn(qc.shape, generator=torch.Generator().manual_seed(77)).to(qc.dtype)
  second = hip.forward_indexed(ad, qm, idx, gm, km, qc2.to(DEV), None, bd, add_residual=False).float().cpu()
  p = _params(hip)
  kc2 = OM.atom_layout_convert(lay.gather_idxs, lay.gather_mask, (256 // 32, 32), qc2.float(), layout_axes=(-3, -2))
  ref2 = OM.windowed_cross_attention(act.float(), lay.queries_mask, lay.gather_idxs, lay.gather_mask, lay.keys_mask,
                                     qc2.float(), kc2, bias.float(), p, return_update=True)
  assert not torch.equal(first, second)
  assert_close_bf16(second, ref2, "per-atom plan, new condition", max_abs=2e-2 * ref2.abs().max().item())


@pytest.mark.parametrize("atoms,S,sharp", [(256, 2, True), (8192, 5, False)])
def test_cross_attention_explicit_keys(atoms, S, sharp):
  """The reference's own call into CrossAttention (transformer.py:671-683): keys gathered by
  convert() first, then cross_attention(x_q, x_k, ...).  That is the module entry with explicit
  key rows (no gather index); it must match forward_indexed on the same inputs and the oracle."""
  from sparsefold_amd.backends.hip import ops
  mod, act, lay, qc, kc, bias = W.make_window(atoms, S=S, seed=5, sharp=sharp)
  hip = _prepared(mod)
  U = atoms // 32
  ad, qcd, kcd, bd = act.to(DEV), qc.to(DEV), kc.to(DEV), bias.to(DEV)
  qm, km = lay.queries_mask.to(DEV), lay.keys_mask.to(DEV)
  keys = ops.window_gather(ad.reshape(S, U * 32, 128), lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV))
  keys = keys.view(S, U, 128, 128)
  # the gather is the reference's convert (its known answers pin the oracle's)
  ref_keys = OM.atom_layout_convert(lay.gather_idxs, lay.gather_mask, (U, 32), act.float(), layout_axes=(-3, -2))
  assert torch.equal(keys.float().cpu(), ref_keys)
  out = hip(ad, keys, qm, km, bd, qcd, kcd)
  idx = hip.forward_indexed(ad, qm, lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV), km, qcd, kcd, bd)
  assert torch.equal(out, idx), "explicit keys and the indexed entry must run the same arithmetic"
  p = _params(hip)
  oargs = (act.float(), lay.queries_mask, lay.gather_idxs, lay.gather_mask, lay.keys_mask, qc.float(), kc.float(),
           bias.float(), p)
  ref = OM.windowed_cross_attention(*oargs)
  assert_close_bf16(out, ref, f"cross attention explicit keys atoms={atoms}")
  upd = hip(ad, keys, qm, km, bd, qcd, kcd, add_residual=False)
  d_ref = OM.windowed_cross_attention(*oargs, return_update=True)
  assert_close_bf16(upd, d_ref, "cross attention explicit keys update", max_abs=2e-2 * d_ref.abs().max().item())


def test_cross_attention_op_level_path():
  """Arguments outside the module entry's contract (a per-sample key condition [S, U, Kw, C])
  take the op-level composition (AdaLN, linear, attention, linear kernels); with the condition
  identical across samples it must agree with the module entry and the oracle."""
  from sparsefold_amd.backends.hip import ops
  S, atoms = 2, 256
  mod, act, lay, qc, kc, bias = W.make_window(atoms, S=S, seed=29, sharp=True)
  hip = _prepared(mod)
  U = atoms // 32
  ad, qcd, kcd, bd = act.to(DEV), qc.to(DEV), kc.to(DEV), bias.to(DEV)
  qm, km = lay.queries_mask.to(DEV), lay.keys_mask.to(DEV)
  keys = ops.window_gather(ad.reshape(S, U * 32, 128), lay.gather_idxs.to(DEV), lay.gather_mask.to(DEV))
  keys = keys.view(S, U, 128, 128)
  kc4 = kcd.unsqueeze(0).expand(S, U, 128, 128).contiguous()
  assert not hip._native_ok(U, 32, 128, qm, km, bd, qcd, kc4)
  upd_op = hip(ad, keys, qm, km, bd, qcd, kc4, add_residual=False)
  upd_mod = hip(ad, keys, qm, km, bd, qcd, kcd, add_residual=False)
  p = _params(hip)
  d_ref = OM.windowed_cross_attention(act.float(), lay.queries_mask, lay.gather_idxs, lay.gather_mask,
                                      lay.keys_mask, qc.float(), kc.float(), bias.float(), p, return_update=True)
  tol = 2e-2 * d_ref.abs().max().item()
  assert_close_bf16(upd_op, d_ref, "cross attention op-level path", max_abs=tol)
  assert_close_bf16(upd_op, upd_mod.float().cpu(), "op-level vs module entry", max_abs=tol)


@pytest.mark.parametrize("transpose", [False, True])
def test_triangle_against_committed_fixture(transpose):
  """tests/golden/oracle_small.npz: sharp-weight, padded triangle attention at N=20 (float32)."""
  import os
  import numpy as np
  from sparsefold_amd import modules as M
  f = np.load(os.path.join(os.path.dirname(__file__), "golden", "oracle_small.npz"))
  tag = "end" if transpose else "start"
  pre = f"tri20_{tag}_param_"
  params = {k[len(pre):]: torch.from_numpy(f[k]) for k in f.files if k.startswith(pre)}
  mod = M.GridSelfAttention(M.GridSelfAttention.Config(num_head=4), M.GlobalConfig(), transpose,
                            num_channels=128, name="fixture")
  mod.load_state_dict(params, strict=True)
  hip = _prepared(mod)
  z = torch.from_numpy(f[f"tri20_{tag}_z"])
  seq = torch.from_numpy(f[f"tri20_{tag}_seq"])
  upd = hip(z.to(DEV), seq.to(DEV), add_residual=False)
  ref = torch.from_numpy(f[f"tri20_{tag}_update"])
  assert_close_bf16(upd, ref, f"fixture triangle N=20 {tag}", max_abs=2e-2 * ref.abs().max().item())


@pytest.mark.parametrize("N", [96, 37])
def test_transformer_pair_logit_pack(N):
  """transformer.py:430-438: 6 super-blocks x (4 blocks x 16 heads) = 384 planes in one pass
  (N=37: N*N is not a multiple of 4, the store tail)."""
  mod, pair_cond = W.make_transformer_pack(N, seed=6 + N)
  hip = _prepared(mod)
  out = hip.pair_logits_pack(pair_cond.to(DEV))
  assert out.shape == (6, 4, 16, N, N) and out.dtype == torch.bfloat16 and out.is_contiguous()
  ref = OM.transformer_pair_logits(pair_cond.float(), _params(hip), 4, None)
  # logits of several units are stored in bf16 by the reference too (transformer.py:438)
  assert_close_bf16(out.float().cpu(), ref, f"transformer pack N={N}", rtol=BF16_ULP)


@pytest.mark.parametrize("U,Qw,Kw,P", [(8, 32, 128, 16), (6, 5, 7, 128), (4, 32, 128, 128)])
def test_cross_att_pair_logit_pack(U, Qw, Kw, P):
  """transformer.py:655-662: [U, Q, K, P] -> [num_blocks, U, H, Q, K] written in place
  (P=16: one thread per position; P=128: the MFMA kernel, Q*K=35 takes the unaligned stores)."""
  mod, pair_cond = W.make_cross_pack(U, Qw=Qw, Kw=Kw, P=P, seed=U + P)
  hip = _prepared(mod)
  out = hip.pair_logits_pack(pair_cond.to(DEV))
  assert out.shape == (3, U, 4, Qw, Kw) and out.dtype == torch.bfloat16 and out.is_contiguous()
  ref = OM.cross_att_pair_logits(pair_cond.float(), _params(hip))
  assert_close_bf16(out.float().cpu(), ref, f"cross pack U={U} Q={Qw} K={Kw} P={P}", rtol=BF16_ULP)


# --------------------------------------------------------------------------------------
# Diffusion Transformer: every block's AdaLN conditioning in one call
# --------------------------------------------------------------------------------------

class _Transition(torch.nn.Module):
  """Stand-in for TransitionBlock (outside this library): halves the activations, exactly in bf16."""

  def forward(self, x, single_cond=None):
    return x * 0.5


class _NoCache:
  def get(self, *args, name=None, factory=None):
    return factory()


def _diffusion_stack(N: int, n_super: int = 2, sb: int = 2, seed: int = 40):
  """A diffusion Transformer of n_super x sb blocks: the package's pair-logit half plus the
  [super-block][block] stacks transformer.py:375-403 builds."""
  mod, pair_cond = W.make_transformer_pack(N, P=16, num_blocks=n_super * sb, super_block_size=sb, seed=seed)
  mod.self_attention = torch.nn.ModuleList(
      [torch.nn.ModuleList([W.make_diffusion(N, S=1, seed=seed + 10 * i + j, sharp=True)[0] for j in range(sb)])
       for i in range(n_super)])
  mod.transition_block = torch.nn.ModuleList(
      [torch.nn.ModuleList([_Transition() for _ in range(sb)]) for _ in range(n_super)])
  mod._cache = _NoCache()
  return _prepared(mod), pair_cond


@pytest.mark.parametrize("N", [100, 1])
def test_diffusion_conditioning_matches_oracle(N):
  """scale / shift / zero-gate of every block (transformer.py:80-96, :138-154) against the
  oracle's LayerNorm and Linear, layer by layer."""
  from oracle import primitives as OP
  mod, _ = _diffusion_stack(N)
  cond = torch.randn(N, 384, generator=torch.Generator().manual_seed(N)).to(torch.bfloat16)
  scale, shift, zgate = mod.diffusion_conditioning(cond.to(DEV))
  assert scale.shape == shift.shape == zgate.shape == (4, N, 768)
  blocks = [b for sb in mod.self_attention for b in sb]
  for layer, blk in enumerate(blocks):
    p = _params(blk)
    pre = "layer_norm."
    cn = OP.layer_norm(cond.float(), p[pre + "single_cond_layer_norm.weight"], None, compute_dtype=torch.float32)
    ref_scale = OP.linear(cn, p[pre + "single_cond_scale.weight"], p[pre + "single_cond_scale.bias"], post_op="sigmoid")
    ref_shift = OP.linear(cn, p[pre + "single_cond_bias.weight"])
    ref_zgate = OP.linear(cond.float(), p["zero_init.adaptive_zero_cond.weight"], p["zero_init.adaptive_zero_cond.bias"],
                          post_op="sigmoid")
    for got, ref, what in ((scale, ref_scale, "scale"), (shift, ref_shift, "shift"), (zgate, ref_zgate, "zgate")):
      assert_close_bf16(got[layer].float().cpu(), ref, f"conditioning N={N} layer {layer} {what}",
                        max_abs=2e-2 * max(ref.abs().max().item(), 1.0))


def test_transformer_conditioned_block_loop():
  """Transformer.forward (transformer.py:422-477) with the conditioning computed once: against the
  oracle chain and against the per-block path that conditions each block from single_cond."""
  N = 100
  mod, pair_cond = _diffusion_stack(N)
  _, act, cond, _, mask = W.make_diffusion(N, S=2, seed=99, padded=True)
  calls = []
  whole = mod.diffusion_conditioning
  mod.diffusion_conditioning = lambda c: (calls.append(c), whole(c))[1]
  out = mod(act.to(DEV), mask.to(DEV), cond.to(DEV), pair_cond.to(DEV))
  assert len(calls) == 1 and out.dtype == act.dtype and out.shape == act.shape
  blocks = [[b for b in sb] for sb in mod.self_attention]
  pack = mod.pair_logits_pack(pair_cond.to(DEV))
  x = act.to(DEV)
  opack = OM.transformer_pair_logits(pair_cond.float(), _params(mod), 2, None)
  ref = act.float()
  for i, row in enumerate(blocks):
    for j, blk in enumerate(row):
      x = blk(x, mask.to(DEV), pair_logits=pack[i][j], single_cond=cond.to(DEV)) * 0.5
      ref = OM.self_attention(ref, mask, _params(blk), pair_logits=opack[i][j], single_cond=cond.float()) * 0.5
  assert_close_bf16(out, x, "conditioned loop vs per-block conditioning", max_abs=2e-2 * x.abs().max().item())
  assert_close_bf16(out, ref, "conditioned loop vs oracle", max_abs=2e-2 * ref.abs().max().item())


# --------------------------------------------------------------------------------------
# Transitions (blocks.py:38-96, transformer.py:157-231)
# --------------------------------------------------------------------------------------

@pytest.mark.parametrize("sharp", [False, True])
@pytest.mark.parametrize("rows,C,lead", [(768, 384, ()), (37, 384, ()), (64, 128, (64,)), (5, 128, (3,))])
def test_trunk_transition(rows, C, lead, sharp):
  """The single transition of SingleActUpdate (C=384) and the pair transition (C=128 over [N, N]).
  The module output is checked at the configurations' weights (std 0.02); with sharp weights
  (std 1/sqrt(fan_in)) the update reaches magnitudes where a bf16 result's own rounding passes
  2e-2, so there the update is checked against 2% of its largest magnitude, as for the attention
  modules."""
  mod, act = W.make_transition(rows, C=C, lead=lead, seed=60 + rows, sharp=sharp)
  hip = _prepared(mod)
  p = _params(hip)
  if not sharp:
    out = hip(act.to(DEV))
    assert out.shape == act.shape and out.dtype == act.dtype
    ref = OM.transition_block(act.float(), p)
    assert_close_bf16(out, ref, f"trunk transition rows={rows} C={C}")
  upd = hip(act.to(DEV), add_residual=False)
  d_ref = OM.transition_block(act.float(), p, return_update=True)
  assert_close_bf16(upd, d_ref, f"trunk transition update rows={rows} C={C} sharp={sharp}",
                    max_abs=2e-2 * max(1.0, d_ref.abs().max().item()))


@pytest.mark.parametrize("sharp", [False, True])
@pytest.mark.parametrize("N,S,cond", [(100, 2, True), (1024, 5, True), (33, 1, False)])
def test_diffusion_transition(N, S, cond, sharp):
  mod, act, c = W.make_diffusion_transition(N, S=S, C_cond=384 if cond else None, seed=70 + N, sharp=sharp)
  hip = _prepared(mod)
  cd = None if c is None else c.to(DEV)
  p = _params(hip)
  cf = None if c is None else c.float()
  if not sharp:
    out = hip(act.to(DEV), single_cond=cd)
    ref = OM.diffusion_transition_block(act.float(), cf, p)
    assert_close_bf16(out, ref, f"diffusion transition N={N} S={S} cond={cond}")
  upd = hip(act.to(DEV), single_cond=cd, add_residual=False)
  d_ref = OM.diffusion_transition_block(act.float(), cf, p, return_update=True)
  assert_close_bf16(upd, d_ref, f"diffusion transition update N={N} sharp={sharp}",
                    max_abs=2e-2 * max(1.0, d_ref.abs().max().item()))


def test_diffusion_transition_precomputed_conditioning_is_the_same_call():
  """The transition's AdaLN from the one-call conditioning (pre_scale / pre_shift / pre_zgate)
  equals the transition conditioned from single_cond."""
  from sparsefold_amd.backends.hip import ops
  N = 96
  mod, act, c = W.make_diffusion_transition(N, S=2, seed=77)
  hip = _prepared(mod)
  lnc = hip._hip_ada_lnc_w[None]
  scale, shift, zgate = ops.diffusion_conditioning(c.to(DEV), lnc, hip._hip_ada_w_scale, hip._hip_ada_b_scale,
                                                   hip._hip_ada_w_shift, hip._hip_w_zc, hip._hip_b_zc)
  got = hip(act.to(DEV), adaptive_scale=scale[0], adaptive_bias=shift[0], zero_gate=zgate[0], add_residual=False)
  want = hip(act.to(DEV), single_cond=c.to(DEV), add_residual=False)
  d_ref = OM.diffusion_transition_block(act.float(), c.float(), _params(hip), return_update=True)
  tol = 2e-2 * d_ref.abs().max().item()
  assert_close_bf16(got, d_ref, "precomputed-conditioning transition", max_abs=tol)
  assert_close_bf16(got, want.float().cpu(), "precomputed vs per-call conditioning", max_abs=tol)


def test_single_act_update_with_transition():
  """SingleActUpdate.forward (blocks.py:739-763): pair-logit prologue, single attention, then
  the single transition."""
  N = 96
  mod, z, s, seq = W.make_single(N, seed=81, padded=True, sharp=True, transition=True)
  hip = _prepared(mod)
  assert getattr(hip.single_transition, "_native_prepared", False)
  out = hip(z.to(DEV), s.to(DEV), seq.to(DEV))
  p = _params(hip)
  mid = OM.single_act_update_attention(z.float(), s.float(), seq, p)
  sub = {k[len("single_transition."):]: v for k, v in p.items() if k.startswith("single_transition.")}
  ref = OM.transition_block(mid, sub)
  assert_close_bf16(out, ref, "SingleActUpdate with transition", max_abs=2e-2 * max(1.0, ref.abs().max().item()))


def test_transformer_conditioned_loop_with_hip_transitions():
  """Transformer.forward with HIP attention and HIP transition blocks: one conditioning call for
  all 8 layers (4 attention + 4 transition), against the oracle's block chain."""
  N = 64
  mod, pair_cond = W.make_transformer_pack(N, P=16, num_blocks=4, super_block_size=2, seed=90)
  mod.self_attention = torch.nn.ModuleList(
      [torch.nn.ModuleList([W.make_diffusion(N, S=1, seed=91 + 10 * i + j, sharp=True)[0] for j in range(2)])
       for i in range(2)])
  mod.transition_block = torch.nn.ModuleList(
      [torch.nn.ModuleList([W.make_diffusion_transition(N, seed=95 + 10 * i + j)[0] for j in range(2)])
       for i in range(2)])
  mod._cache = _NoCache()
  mod = _prepared(mod)
  assert mod._hip_dc_transitions
  _, act, cond, _, mask = W.make_diffusion(N, S=2, seed=99, padded=True)
  calls = []
  whole = mod.diffusion_conditioning
  mod.diffusion_conditioning = lambda c: (calls.append(c), whole(c))[1]
  out = mod(act.to(DEV), mask.to(DEV), cond.to(DEV), pair_cond.to(DEV))
  assert len(calls) == 1
  opack = OM.transformer_pair_logits(pair_cond.float(), _params(mod), 2, None)
  ref = act.float()
  for i in range(2):
    for j in range(2):
      ref = OM.self_attention(ref, mask, _params(mod.self_attention[i][j]), pair_logits=opack[i][j],
                              single_cond=cond.float())
      ref = OM.diffusion_transition_block(ref, cond.float(), _params(mod.transition_block[i][j]))
  assert_close_bf16(out, ref, "Transformer loop with HIP transitions", max_abs=2e-2 * ref.abs().max().item())


# --------------------------------------------------------------------------------------
# Triangle multiplicative update (blocks.py:425-566)
# --------------------------------------------------------------------------------------

@pytest.mark.parametrize("N,incoming,padded", [(64, False, False), (64, True, True), (37, False, True),
                                               (37, True, False), (1, False, False), (384, False, True),
                                               (384, True, True)])
def test_triangle_multiplication(N, incoming, padded):
  """Sharp weights (std 1/sqrt(fan_in)): the update reaches magnitudes of several units, so it is
  checked against 2% of its largest magnitude (the bf16 a / b planes and product carry the
  reference bf16 module's own rounding), as for the other modules' sharp-weight updates."""
  print(f"[case] trimul N={N} incoming={incoming} padded={padded}", flush=True)
  mod, z, mask = W.make_trimul(N, incoming=incoming, padded=padded, seed=7 + N)
  hip = _prepared(mod)
  eq = mod.EQUATIONS[int(incoming)]
  upd = hip(z.to(DEV), mask.to(DEV), add_residual=False)
  assert upd.dtype == z.dtype and upd.shape == z.shape and torch.isfinite(upd).all()
  d_ref = OM.triangle_multiplication(z.float(), mask, _params(hip), equation=eq, return_update=True)
  assert_close_bf16(upd, d_ref, f"trimul update N={N} incoming={incoming} padded={padded}",
                    max_abs=2e-2 * max(1.0, d_ref.abs().max().item()))
  # the residual form adds z to the same bf16 update in fp32 and rounds once more: bit-exact
  out = hip(z.to(DEV), mask.to(DEV))
  assert torch.equal(out, (upd.float() + z.to(DEV).float()).to(z.dtype)), "trimul residual != bf16(update + z)"


@pytest.mark.parametrize("N,incoming", [(768, False), (768, True), (96, False), (96, True)])
def test_triangle_multiplication_module_output(N, incoming):
  """The module output z + update at the configurations' weight scale (std 0.02) against the
  fp32 oracle at the full bar (max-abs 2e-2, rel-L2 1e-2), N=768 included, padded."""
  print(f"[case] trimul module N={N} incoming={incoming}", flush=True)
  mod, z, mask = W.make_trimul(N, incoming=incoming, padded=True, seed=71 + N, sharp=False)
  hip = _prepared(mod)
  out = hip(z.to(DEV), mask.to(DEV))
  ref = OM.triangle_multiplication(z.float(), mask, _params(hip), equation=mod.EQUATIONS[int(incoming)])
  assert_close_bf16(out, ref, f"trimul module N={N} incoming={incoming}")


def test_triangle_multiplication_n768_transpose_identity():
  """N=768: incoming edges of z equal the outgoing edges of z^T transposed back, with the same
  weights -- a size-independent property of the module (sharp weights)."""
  out_mod, z, mask = W.make_trimul(768, padded=True, seed=70)
  in_mod, _, _ = W.make_trimul(768, incoming=True, seed=70)
  in_mod.load_state_dict(out_mod.state_dict())
  hip_out, hip_in = _prepared(out_mod), _prepared(in_mod)
  zd, md = z.to(DEV), mask.to(DEV)
  inc = hip_in(zd, md, add_residual=False)
  out_t = hip_out(zd.transpose(0, 1).contiguous(), md, add_residual=False).transpose(0, 1)
  assert_close_bf16(inc, out_t, "trimul N=768 incoming vs outgoing of z^T",
                    max_abs=2e-2 * out_t.float().abs().max().item())


def test_precomputed_conditioning_op_level_path():
  """A per-sample key mask takes the op-level path (LayerNorm, linear, attention, linear); with a
  block's precomputed conditioning it must agree with the one-call path on the same values."""
  N, S = 100, 2
  mod, _ = _diffusion_stack(N, n_super=1, sb=2)
  _, act, cond, bias, mask = W.make_diffusion(N, S=S, seed=98, padded=True, sharp=True)
  scale, shift, zgate = mod.diffusion_conditioning(cond.to(DEV))
  blk = [b for b in mod.self_attention[0]][1]
  x, m = act.to(DEV), mask.to(DEV)
  pre = dict(adaptive_scale=scale[1], adaptive_bias=shift[1], zero_gate=zgate[1])
  fused = blk(x, m, pair_logits=bias.to(DEV), **pre)
  op_level = blk(x, m.expand(S, N).contiguous(), pair_logits=bias.to(DEV), **pre)
  assert_close_bf16(op_level, fused, "op-level vs one-call path, precomputed conditioning",
                    max_abs=2e-2 * fused.float().abs().max().item())
  ref = OM.self_attention(act.float(), mask, _params(blk), pair_logits=bias.float(), single_cond=cond.float())
  assert_close_bf16(op_level, ref, "op-level path vs oracle", rtol=BF16_ULP)
