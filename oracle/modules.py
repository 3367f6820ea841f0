"""Oracle restatements of the four gated pair-biased attention composites.

TEST INFRASTRUCTURE: imported only by tests, smoke() and bench's CPU baseline.

Parameters are passed as flat dicts keyed like the reference modules'
``state_dict`` (e.g. ``"q_projection.weight"``) with the reference's weight
layouts, so a module's ``state_dict()`` can be handed in directly.

Dtype behaviour follows the reference: ``Linear`` casts its input to the
weight dtype and its output back to the input dtype; ``LayerNorm`` computes in
its own dtype (input dtype when None) and casts back.  With float32 inputs and
weights (the parity configuration) every step is float32.
"""
from __future__ import annotations

import torch

from oracle.primitives import gated_linear_unit, layer_norm, linear
from oracle.sdpa import dot_product_attention


def _get(p: dict, name: str):
  return p.get(name)


# --------------------------------------------------------------------------------------
# Triangle attention: blocks.py:188-366 (GridSelfAttention)
# --------------------------------------------------------------------------------------

def grid_self_attention(act: torch.Tensor, seq_mask: torch.Tensor, p: dict, *,
                        transpose: bool, chunk_size: int | None = None,
                        return_update: bool = False) -> torch.Tensor:
  """blocks.py:293-366 (forward) with blocks.py:270-291 (_attention) per row chunk.

  act ``[*, N, N, C]``; seq_mask ``[N]`` bool.  ``chunk_size`` reproduces the
  row sub-batching of ``mapping.inference_subbatch`` (blocks.py:331-361,
  mapping.py:326-382), which is numerically neutral.  With
  ``return_update`` the residual ``act`` is not added (the module returns
  ``act + update``, blocks.py:366).
  """
  num_res = act.shape[-2]
  assert seq_mask.shape == (num_res,) and seq_mask.dtype == torch.bool
  pair_mask = seq_mask[:, None] & seq_mask[None, :]                 # :314
  x = layer_norm(act, p["act_norm.weight"], _get(p, "act_norm.bias"))  # :317
  bias = linear(x, p["pair_bias_projection.weight"])                 # :320  (*, B, N, H)
  bias = bias.movedim(-1, -3).unsqueeze(-4).contiguous()             # :329  (*, 1, H, B, N)
  if transpose:                                                      # :345-346
    x = x.transpose(-2, -3)
  if x.ndim > 3:
    pair_mask = pair_mask.expand(*x.shape[:-3], *pair_mask.shape)

  def attention(xc: torch.Tensor, mc: torch.Tensor) -> torch.Tensor:  # :270-291
    q = linear(xc, p["q_projection.weight"], transpose_weights=True)
    k = linear(xc, p["k_projection.weight"], transpose_weights=True)
    v = linear(xc, p["v_projection.weight"])
    o = dot_product_attention(q, k, v, mask_k=mc, bias=bias)
    o = o.reshape(*o.shape[:-2], -1)
    g = linear(xc, p["gating_query.weight"], transpose_weights=True, post_op="sigmoid")
    o = o * g
    return linear(o, p["output_projection.weight"])

  rows = x.shape[-3]
  step = rows if chunk_size is None else chunk_size
  outs = []
  for s in range(0, rows, step):
    outs.append(attention(x[..., s:s + step, :, :], pair_mask[..., s:s + step, :]))
  out = torch.cat(outs, dim=-3)
  if transpose:
    out = out.transpose(-2, -3)
  return out if return_update else act + out


def grid_self_attention_rows(act: torch.Tensor, seq_mask: torch.Tensor, p: dict, *, transpose: bool,
                             rows, bias: torch.Tensor | None = None) -> torch.Tensor:
  """Update of selected attention rows only (rows are independent given the shared bias):
  returns ``[len(rows), N, C]``, row r being ``update[r]`` (starting node) or
  ``update[:, r]`` (ending node).  ``bias`` ``[H, N, N]`` overrides the bias built from
  ``act`` (used by the ending-node identity test).  act ``[N, N, C]``."""
  pair_mask = seq_mask[:, None] & seq_mask[None, :]
  x = layer_norm(act, p["act_norm.weight"], _get(p, "act_norm.bias"))
  if bias is None:
    bias = linear(x, p["pair_bias_projection.weight"]).movedim(-1, -3).contiguous()
  if transpose:
    x = x.transpose(0, 1)
  idx = torch.as_tensor(list(rows), dtype=torch.long)
  xr = x[idx]
  q = linear(xr, p["q_projection.weight"], transpose_weights=True)
  k = linear(xr, p["k_projection.weight"], transpose_weights=True)
  v = linear(xr, p["v_projection.weight"])
  o = dot_product_attention(q, k, v, mask_k=pair_mask[idx], bias=bias.unsqueeze(0))
  o = o.reshape(*o.shape[:-2], -1)
  g = linear(xr, p["gating_query.weight"], transpose_weights=True, post_op="sigmoid")
  return linear(o * g, p["output_projection.weight"])


# --------------------------------------------------------------------------------------
# AdaLN / AdaLN-zero and SelfAttention: transformer.py:27-154, 234-345
# --------------------------------------------------------------------------------------

def adaptive_layer_norm(x: torch.Tensor, single_cond: torch.Tensor | None, p: dict, prefix: str,
                        dtype: torch.dtype | None) -> torch.Tensor:
  """transformer.py:80-96 (AdaptiveLayerNorm.forward)."""
  if single_cond is not None:
    orig = x.dtype
    x = layer_norm(x, None, None, compute_dtype=torch.float32)
    sc = layer_norm(single_cond, p[prefix + "single_cond_layer_norm.weight"],
                    _get(p, prefix + "single_cond_layer_norm.bias"), compute_dtype=torch.float32)
    sc = sc.to(dtype) if dtype is not None else sc
    scale = linear(sc, p[prefix + "single_cond_scale.weight"], p[prefix + "single_cond_scale.bias"],
                   post_op="sigmoid").to(orig)
    shift = linear(sc, p[prefix + "single_cond_bias.weight"]).to(orig)
    return scale * x + shift
  return layer_norm(x, p[prefix + "layer_norm.weight"], _get(p, prefix + "layer_norm.bias"),
                    compute_dtype=torch.float32)


def adaptive_zero_init(x: torch.Tensor, single_cond: torch.Tensor | None, p: dict, prefix: str,
                       dtype: torch.dtype | None) -> torch.Tensor:
  """transformer.py:138-154 (AdaptiveZeroInit.forward)."""
  orig = x.dtype
  x = x.to(dtype) if dtype is not None else x
  out = linear(x, p[prefix + "transition2.weight"])
  if single_cond is not None:
    c = single_cond.to(dtype) if dtype is not None else single_cond
    cond = linear(c, p[prefix + "adaptive_zero_cond.weight"], p[prefix + "adaptive_zero_cond.bias"],
                  post_op="sigmoid")
    out = cond * out
  return out.to(orig)


def self_attention(x: torch.Tensor, mask: torch.Tensor, p: dict, *, pair_logits=None,
                   single_cond=None, dtype: torch.dtype | None = None,
                   return_update: bool = False) -> torch.Tensor:
  """transformer.py:306-345 (SelfAttention.forward).  x ``[..., N, C]``;
  mask ``[..., N]``; pair_logits ``[..., H, N, N]``; single_cond ``[..., N, S]``."""
  residual = x
  orig = x.dtype
  h = adaptive_layer_norm(x, single_cond, p, "layer_norm.", dtype)
  h = h.to(dtype) if dtype is not None else h
  q = linear(h, p["q_projection.weight"], p["q_projection.bias"])
  k = linear(h, p["k_projection.weight"])
  v = linear(h, p["v_projection.weight"])
  o = dot_product_attention(q, k, v, mask_k=mask, bias=pair_logits)
  o = o.reshape(*o.shape[:-2], -1)
  g = linear(h, p["gating_query.weight"], post_op="sigmoid")
  o = o * g
  out = adaptive_zero_init(o, single_cond, p, "zero_init.", dtype).to(orig)
  return out if return_update else residual + out


def single_act_update_attention(pair_act: torch.Tensor, single_act: torch.Tensor, seq_mask: torch.Tensor,
                                p: dict, *, return_update: bool = False) -> torch.Tensor:
  """blocks.py:739-763 up to and including the attention (the SwiGLU transition
  that follows, blocks.py:760-762, is not part of the attention path)."""
  pl = layer_norm(pair_act, p["single_pair_logits_norm.weight"], _get(p, "single_pair_logits_norm.bias"))
  pl = linear(pl, p["single_pair_logits_projection.weight"])          # (*, B, N, H)
  pl = pl.movedim(-1, -3).contiguous()                                # (*, H, B, N)
  sub = {k[len("single_attention."):]: v for k, v in p.items() if k.startswith("single_attention.")}
  return self_attention(single_act, seq_mask, sub, pair_logits=pl, return_update=return_update)


def pair_logits_from_pair(pair_act: torch.Tensor, norm_w, norm_b, proj_w) -> torch.Tensor:
  """LN + projection + ``b n h -> h b n`` (blocks.py:745-749): ``[N,N,C] -> [H,N,N]``."""
  pl = layer_norm(pair_act, norm_w, norm_b)
  return linear(pl, proj_w).movedim(-1, -3).contiguous()


def transformer_pair_logits(pair_cond: torch.Tensor, p: dict, super_block_size: int,
                            dtype: torch.dtype | None) -> torch.Tensor:
  """transformer.py:430-447: ``[N,N,P] -> [n_super, super_block_size, H, N, N]``."""
  pair_act = layer_norm(pair_cond, p["pair_input_layer_norm.weight"], None)
  pack = []
  sb = 0
  while f"pair_logits_projection.{sb}.weight" in p:
    w = p[f"pair_logits_projection.{sb}.weight"]                      # [P, S, H]
    pl = linear(pair_act, w)                                          # [N, N, S, H]
    pack.append(pl.permute(2, 3, 0, 1))                               # "b n s h -> s h b n"
    sb += 1
  out = torch.stack(pack)
  return (out.to(dtype) if dtype is not None else out).contiguous()


# --------------------------------------------------------------------------------------
# Windowed atom attention: transformer.py:480-693, atom_layout.py:52-83
# --------------------------------------------------------------------------------------

def atom_layout_convert(gather_idxs: torch.Tensor, gather_mask: torch.Tensor, input_shape,
                        arr: torch.Tensor, layout_axes: tuple[int, ...] = (0,)) -> torch.Tensor:
  """atom_layout.py:61-83 (convert): flat-index gather over the layout axes,
  masked positions filled with 0."""
  layout_axes = tuple(i if i >= 0 else i + arr.ndim for i in layout_axes)
  if not layout_axes or any(i < 0 or i >= arr.ndim for i in layout_axes):
    raise ValueError("layout_axes must contain valid axes")
  begin, end = layout_axes[0], layout_axes[-1] + 1
  if layout_axes != tuple(range(begin, end)):
    raise ValueError(f"layout_axes must be continuous. Got {layout_axes}.")
  layout_shape = tuple(arr.shape[begin:end])
  expected = tuple(int(x) for x in input_shape)
  vol = 1
  for s in layout_shape:
    vol *= s
  exp_vol = 1
  for s in expected:
    exp_vol *= s
  same_volume = vol == exp_vol
  leading_padding = (len(layout_shape) == len(expected) and bool(expected)
                     and layout_shape[0] >= expected[0] and layout_shape[1:] == expected[1:])
  if not expected or any(s < 0 for s in expected) or not (same_volume or leading_padding):
    raise ValueError(f"Input layout {layout_shape} incompatible with gather shape {expected}")
  batch_shape = arr.shape[:begin]
  feat_shape = arr.shape[end:]
  flat = arr.reshape(batch_shape + (-1,) + feat_shape)
  out = flat[(slice(None),) * begin + (gather_idxs.long(), ...)]
  mshape = (1,) * len(batch_shape) + tuple(gather_mask.shape) + (1,) * len(feat_shape)
  return out.masked_fill(~gather_mask.reshape(mshape), 0.0)


def cross_attention(x_q: torch.Tensor, x_k: torch.Tensor, mask_q: torch.Tensor, mask_k: torch.Tensor,
                    p: dict, *, pair_logits=None, single_cond_q=None, single_cond_k=None,
                    dtype: torch.dtype | None = None, return_update: bool = False) -> torch.Tensor:
  """transformer.py:549-585 (CrossAttention.forward)."""
  residual = x_q
  orig = x_q.dtype
  hq = adaptive_layer_norm(x_q, single_cond_q, p, "q_layernorm.", dtype)
  hk = adaptive_layer_norm(x_k, single_cond_k, p, "k_layernorm.", dtype)
  if dtype is not None:
    hq, hk = hq.to(dtype), hk.to(dtype)
  q = linear(hq, p["q_projection.weight"], p["q_projection.bias"])
  k = linear(hk, p["k_projection.weight"])
  v = linear(hk, p["v_projection.weight"])
  o = dot_product_attention(q, k, v, mask_q=mask_q, mask_k=mask_k, bias=pair_logits).to(orig)
  o = o.reshape(*o.shape[:-2], -1)
  g = linear(hq, p["gating_query.weight"], post_op="sigmoid").to(orig)
  o = o * g
  out = adaptive_zero_init(o, single_cond_q, p, "zero_init.", dtype)
  return out if return_update else residual + out


def cross_att_pair_logits(pair_cond: torch.Tensor, p: dict) -> torch.Tensor:
  """transformer.py:655-666: ``[U,Q,K,P] -> [num_blocks, U, H, Q, K]``."""
  pair_act = layer_norm(pair_cond, p["pair_input_layer_norm.weight"], None)
  pl = linear(pair_act, p["pair_logits_projection.weight"])          # [U, Q, K, nb, H]
  return pl.permute(3, 0, 4, 1, 2).contiguous()


def windowed_cross_attention(queries_act: torch.Tensor, queries_mask: torch.Tensor,
                             gather_idxs: torch.Tensor, gather_mask: torch.Tensor, keys_mask: torch.Tensor,
                             queries_single_cond: torch.Tensor, keys_single_cond: torch.Tensor,
                             pair_logits: torch.Tensor, p: dict, *, dtype=None,
                             return_update: bool = False) -> torch.Tensor:
  """One CrossAttTransformer block's attention (transformer.py:668-682): keys
  gathered from the queries by ``queries_to_keys`` (layout axes (-3,-2)), then
  CrossAttention.  queries_act ``[..., U, Qw, C]``; gather ``[U, Kw]``."""
  U, Qw = queries_act.shape[-3:-1]
  keys_act = atom_layout_convert(gather_idxs, gather_mask, (U, Qw), queries_act, layout_axes=(-3, -2))
  return cross_attention(queries_act, keys_act, queries_mask, keys_mask, p, pair_logits=pair_logits,
                         single_cond_q=queries_single_cond, single_cond_k=keys_single_cond,
                         dtype=dtype, return_update=return_update)


# --------------------------------------------------------------------------------------
# Transitions: blocks.py:38-96 (trunk), transformer.py:157-231 (diffusion transformer)
# --------------------------------------------------------------------------------------

def transition_block(act: torch.Tensor, p: dict, *, return_update: bool = False) -> torch.Tensor:
  """blocks.py:84-96 (TransitionBlock.forward): LN, SwiGLU of transition1 (its ``[C, 2I]`` weight
  viewed as ``"a (i2 n) -> a i2 n"``), transition2 with the input as residual."""
  x = layer_norm(act, p["input_layer_norm.weight"], _get(p, "input_layer_norm.bias"))
  w1 = p["transition1.weight"]
  c = gated_linear_unit(x, w1.reshape(w1.shape[0], 2, -1))
  out = linear(c, p["transition2.weight"])
  return out if return_update else act + out


def diffusion_transition_block(x: torch.Tensor, single_cond: torch.Tensor | None, p: dict, *,
                               dtype: torch.dtype | None = None, return_update: bool = False) -> torch.Tensor:
  """transformer.py:209-231 (TransitionBlock.forward of the diffusion transformer): AdaLN with the
  ``layer_norm.`` parameters, SwiGLU of ``transition``, AdaLN-zero output (``zero_init.``)."""
  residual = x
  orig = x.dtype
  h = adaptive_layer_norm(x, single_cond, p, "layer_norm.", dtype)
  h = h.to(dtype) if dtype is not None else h
  w1 = p["transition.weight"]
  c = gated_linear_unit(h, w1.reshape(w1.shape[0], 2, -1))
  out = adaptive_zero_init(c.to(orig), single_cond, p, "zero_init.", dtype)
  return out if return_update else residual + out


# --------------------------------------------------------------------------------------
# Triangle multiplicative update: blocks.py:425-566
# --------------------------------------------------------------------------------------

TRIMUL_EQUATIONS = {"...ikc,...jkc->...ijc": "cik,cjk->cij", "...kjc,...kic->...ijc": "ckj,cki->cij"}


def triangle_multiplication(act: torch.Tensor, mask: torch.Tensor, p: dict, *, equation: str,
                            return_update: bool = False) -> torch.Tensor:
  """blocks.py:486-566 (TriangleMultiplication.forward, not distributed).  act ``[N, N, C]``,
  mask ``[N]`` bool.  The gated linear unit is primitives.py:586-631: the combined weight
  stacks (gate, projection) on dim 1 and the first half of the product is the gated one."""
  C = act.shape[-1]
  pair = (mask[:, None] & mask[None, :])[None]                                   # :501
  x = layer_norm(act, p["left_norm_input.weight"], _get(p, "left_norm_input.bias"))
  w_glu = torch.stack((p["gate_projection.weight"], p["projection.weight"]), dim=1)   # (C, 2, 2C), :513
  y = x @ w_glu.reshape(C, 4 * C).to(x.dtype)                                    # primitives.py:616-624
  gate, proj = torch.tensor_split(y, 2, dim=-1)
  glu = (torch.sigmoid(gate) * proj).to(x.dtype)                                 # primitives.py:628-630
  glu = glu.permute(2, 0, 1).masked_fill(~pair, 0.0)                             # "... b n c2 -> ... c2 b n"
  a, b = glu.reshape(C, 2, *glu.shape[1:]).unbind(1)                             # "(c i2) b n -> i2 c b n"
  t = torch.einsum(TRIMUL_EQUATIONS[equation], a, b)                             # :555
  t = layer_norm(t.permute(1, 2, 0), p["center_norm.weight"], _get(p, "center_norm.bias"))   # dim=-3, :556-559
  out = linear(t, p["output_projection.weight"])
  out = out * linear(x, p["gating_linear.weight"], post_op="sigmoid")            # :561-563
  return out if return_update else act + out
