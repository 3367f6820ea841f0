"""HIP module replacements for the four gated pair-biased attention forms.

Each replacement is a mixin over a module with the reference's parameter layout (this
package's ``sparsefold_amd.modules`` classes, or -- when integrated -- the reference classes
themselves).  ``prepare_native()`` runs after strict checkpoint loading and packs bf16 /
fp32 copies of the weights into *non-persistent* buffers; parameters and ``state_dict`` are
untouched (as ``backends/vecops/modules.py:436-444`` / ``tests/test_native_preparation.py:107-132``
require).  ``forward`` before ``prepare_native`` raises the reference's "not prepared" error
(``backends/vecops/modules.py:88-94``).  Every numeric step runs in libsparsefold_hip.

Replaced reference forwards:
* ``GridSelfAttentionHip.forward``   blocks.py:293-366
* ``SelfAttentionHip.forward``       transformer.py:306-345 (with AdaLN :80-96, AdaLN-zero :138-154)
* ``CrossAttentionHip.forward``      transformer.py:549-585; ``forward_indexed`` additionally
                                     gathers the key windows (transformer.py:671-673)
* ``SingleActUpdateHip.forward``     blocks.py:739-763 (attention half)
* ``TriangleMultiplicationHip.forward``  blocks.py:486-566 (outgoing and incoming edges, C = 128)
* ``TransitionBlockHip.forward``     blocks.py:84-96 (trunk transition: pair / single)
* ``DiffusionTransitionBlockHip.forward``  transformer.py:209-231 (diffusion transformer transition)
* ``TransformerHipMixin``            transformer.py:430-447 -- the cached pair-logit pack
                                     ``[n_super, super_block, H, N, N]`` in one pass over pair_cond;
                                     with condition-only HIP attention blocks, also every block's
                                     AdaLN conditioning in one call before the block loop (the
                                     native Transformer's, backends/vecops/modules.py:1093-1183)
* ``CrossAttTransformerHipMixin``    transformer.py:655-666 -- the cached pack
                                     ``[num_blocks, U, H, Q, K]``, written in that layout directly
The pair-logit pack replaces only the factory of the ``ValueCache`` entry ``"pair_logits"``, so
cache keys and ``enable_cache`` behave as in the reference; the transition blocks always run as
they are.
"""
from __future__ import annotations

import functools

import torch

from sparsefold_amd import modules as base
from sparsefold_amd.runtime import config as runtime_config
from sparsefold_amd.backends.hip import graphs, ops
from sparsefold_amd.backends.hip.attention import dot_product_attention

BF16 = torch.bfloat16


def _begin_preparation(module: torch.nn.Module) -> None:
  module._native_prepared = False
  graphs.clear(module)                                  # captured graphs hold the old weight buffers
  devices = {p.device.type for p in module.parameters()}
  if devices - {"cuda"}:
    raise RuntimeError("HIP kernels need the module's parameters on the GPU; move the model to 'cuda' first")


def _require_native_preparation(function):
  @functools.wraps(function)
  def wrapped(self, *args, **kwargs):
    if not getattr(self, "_native_prepared", False):
      raise RuntimeError("Native buffers are not prepared; call backends.prepare(model) after strict checkpoint loading")
    return function(self, *args, **kwargs)
  return wrapped


def _buf(module: torch.nn.Module, name: str, value: torch.Tensor | None) -> None:
  module.register_buffer(name, None if value is None else value.detach().contiguous(), persistent=False)


def _bf(t: torch.Tensor) -> torch.Tensor:
  return t.detach().to(BF16).contiguous()


def _f32(t: torch.Tensor | None) -> torch.Tensor | None:
  return None if t is None else t.detach().to(torch.float32).contiguous()


# ---------------------------------------------------------------------------------------
# Triangle attention
# ---------------------------------------------------------------------------------------

class GridSelfAttentionHipMixin:
  """GridSelfAttention.forward (blocks.py:293-366) as one library call per pair block.  With the
  runtime's ``hip_sparse_grid_attention`` on, the attention rows are block-sparse (IBS) with the
  native backend's parameters and map reuse (backends/vecops/modules.py:1399-1640):
  ``ibsa_params`` (parameters or a provider of them per layer-stack indices) and
  ``index_reuse_policy``; otherwise they are dense, as in the reference's torch path."""

  def __init__(self, *args, index_reuse_policy=base.default_reuse_policy,
               ibsa_params=base.IBSAParameters.default, **kwargs):
    super().__init__(*args, **kwargs)
    if isinstance(ibsa_params, base.IBSAParameters):
      self.ibsa_params_provider = lambda _indices: ibsa_params
    else:
      self.ibsa_params_provider = ibsa_params
    self.index_reuse_policy = index_reuse_policy
    self._hip_reusers: dict = {}          # (act shape, mask shape) -> IndexReuser
    self.last_maps = None                 # (index_map, weight_map) of the last block-sparse call

  def prepare_native(self) -> bool:
    _begin_preparation(self)
    H, C, D = self.config.num_head, self.num_channels, self.qkv_dim
    HD = H * D
    wq = self.q_projection.weight.reshape(HD, C)                       # [H, D, C]
    wk = self.k_projection.weight.reshape(HD, C)
    wv = self.v_projection.weight.reshape(C, HD).t()                   # [C, H, D]
    wg = self.gating_query.weight.reshape(HD, C)                       # [H*D, C]
    wb = self.pair_bias_projection.weight.t()                          # [C, H]
    _buf(self, "_hip_w_qkvgb", _bf(torch.cat([wq, wk, wv, wg, wb], 0)))
    _buf(self, "_hip_w_o", _bf(self.output_projection.weight.t()))      # [H*D, C] -> [C, H*D]
    _buf(self, "_hip_ln_w", _f32(self.act_norm.weight))
    _buf(self, "_hip_ln_b", _f32(getattr(self.act_norm, "bias", None)))
    self._native_prepared = True
    return True

  @_require_native_preparation
  def forward(self, act: torch.Tensor, seq_mask: torch.Tensor, *, add_residual: bool = True) -> torch.Tensor:
    assert act.ndim >= 3
    N = act.shape[-2]
    assert act.shape[-1] == self.num_channels
    assert seq_mask.shape == (N,) and seq_mask.dtype == torch.bool
    assert act.shape[-3] == N, "triangle attention needs the full [N, N] pair block on one GPU"
    if runtime_config.hip_sparse_grid_attention:    # per-call seeds and map reuse: never graphed
      flat = act.reshape(-1, N, N, act.shape[-1])
      outs = self._forward_sparse(act, flat, seq_mask, add_residual)
      out = outs[0].unsqueeze(0) if len(outs) == 1 else torch.stack(outs)
      return out.reshape(act.shape).to(act.dtype)
    return self._forward_dense(act, seq_mask, add_residual=add_residual)

  @graphs.graphed
  def _forward_dense(self, act: torch.Tensor, seq_mask: torch.Tensor, *, add_residual: bool) -> torch.Tensor:
    N = act.shape[-2]
    flat = act.reshape(-1, N, N, act.shape[-1])
    outs = [ops.triangle_attention(z, seq_mask, self._hip_ln_w, self._hip_ln_b, self._hip_w_qkvgb, self._hip_w_o,
                                   num_head=self.config.num_head, transpose=self.transpose,
                                   add_residual=add_residual) for z in flat]
    out = outs[0].unsqueeze(0) if len(outs) == 1 else torch.stack(outs)
    return out.reshape(act.shape).to(act.dtype)

  def _forward_sparse(self, act, flat, seq_mask, add_residual):
    """Block-sparse rows; maps ``[B, N, H, T, S]`` sampled or taken from the layer the reuse
    policy names (modules.py:1589-1626 of the vecops backend)."""
    indices = tuple(base.layer_stack_indices)
    p = self.ibsa_params_provider(indices)
    key = (tuple(act.shape), tuple(seq_mask.shape))
    reuser = self._hip_reusers.setdefault(key, base.IndexReuser(self.index_reuse_policy))
    maps, _ = reuser.get(indices)
    outs, index_maps, weight_maps = [], [], []
    for b, z in enumerate(flat):
      im, wm = (None, None) if maps is None else (maps[0][b], maps[1][b])
      o, im, wm = ops.triangle_attention_ibs(
          z, seq_mask, self._hip_ln_w, self._hip_ln_b, self._hip_w_qkvgb, self._hip_w_o,
          num_head=self.config.num_head, transpose=self.transpose, num_samples=p.num_samples,
          num_rand_blocks=p.num_rand_blocks, t_prob=p.t_prob, tr_prob=p.tr_prob, u_prob=p.u_prob,
          index_map=im, weight_map=wm, add_residual=add_residual)
      outs.append(o)
      index_maps.append(im)
      weight_maps.append(wm)
    self.last_maps = (torch.stack(index_maps), torch.stack(weight_maps))
    if maps is None:
      reuser.set(indices, self.last_maps)
    return outs


# ---------------------------------------------------------------------------------------
# AdaLN helpers shared by SelfAttention and CrossAttention
# ---------------------------------------------------------------------------------------

def _prepare_adaln(module: torch.nn.Module, ada: base.AdaptiveLayerNorm, prefix: str) -> None:
  if ada.single_cond:
    _buf(module, prefix + "lnc_w", _f32(ada.single_cond_layer_norm.weight))
    _buf(module, prefix + "lnc_b", _f32(getattr(ada.single_cond_layer_norm, "bias", None)))
    _buf(module, prefix + "w_scale", _bf(ada.single_cond_scale.weight.t()))   # [S, C] -> [C, S]
    _buf(module, prefix + "b_scale", _f32(ada.single_cond_scale.bias))
    _buf(module, prefix + "w_shift", _bf(ada.single_cond_bias.weight.t()))
  else:
    _buf(module, prefix + "ln_w", _f32(ada.layer_norm.weight))
    _buf(module, prefix + "ln_b", _f32(getattr(ada.layer_norm, "bias", None)))


def _adaln(module, prefix: str, x: torch.Tensor, cond: torch.Tensor | None) -> torch.Tensor:
  if cond is None:
    return ops.layer_norm(x, getattr(module, prefix + "ln_w"), getattr(module, prefix + "ln_b"))
  c = ops.layer_norm(cond, getattr(module, prefix + "lnc_w"), getattr(module, prefix + "lnc_b"))
  scale = ops.linear(c, getattr(module, prefix + "w_scale"), getattr(module, prefix + "b_scale"), post_sigmoid=True)
  shift = ops.linear(c, getattr(module, prefix + "w_shift"))
  return ops.layer_norm(x, scale=scale.reshape(-1, scale.shape[-1]), shift=shift.reshape(-1, shift.shape[-1]))


def _prepare_zero_init(module: torch.nn.Module, zi: base.AdaptiveZeroInit) -> None:
  _buf(module, "_hip_w_t2", _bf(zi.transition2.weight.t()))            # [HD, C] -> [C, HD]
  if zi.single_cond:
    _buf(module, "_hip_w_zc", _bf(zi.adaptive_zero_cond.weight.t()))  # [S, C] -> [C, S]
    _buf(module, "_hip_b_zc", _f32(zi.adaptive_zero_cond.bias))


def _zero_init_residual(module, o: torch.Tensor, cond: torch.Tensor | None, residual: torch.Tensor | None) -> torch.Tensor:
  """AdaLN-zero output (transformer.py:138-154) plus the caller's residual add, one GEMM."""
  mul = None
  if cond is not None:
    mul = ops.linear(cond, module._hip_w_zc, module._hip_b_zc, post_sigmoid=True)
    mul = mul.reshape(-1, mul.shape[-1])
  return ops.linear(o, module._hip_w_t2, mul=mul, residual=residual)


# ---------------------------------------------------------------------------------------
# SelfAttention (single representation with pair bias; diffusion token attention)
# ---------------------------------------------------------------------------------------

class SelfAttentionHipMixin:
  def prepare_native(self) -> bool:
    _begin_preparation(self)
    H, D = self.num_head, self.key_dim
    C = self.q_projection.weight.shape[0]
    HD = H * D
    wq = self.q_projection.weight.reshape(C, HD).t()
    wk = self.k_projection.weight.reshape(C, HD).t()
    wv = self.v_projection.weight.reshape(C, HD).t()
    wg = self.gating_query.weight.reshape(C, HD).t()
    _buf(self, "_hip_w_qkvg", _bf(torch.cat([wq, wk, wv, wg], 0)))    # [4HD, C]
    b = torch.zeros(4 * HD, dtype=torch.float32, device=wq.device)
    b[:HD] = self.q_projection.bias.detach().reshape(HD).float()
    _buf(self, "_hip_b_qkvg", b)
    _prepare_adaln(self, self.layer_norm, "_hip_ada_")
    _prepare_zero_init(self, self.zero_init)
    self._native_prepared = True
    return True

  def _native_weights(self) -> dict:
    w = {"w_qkvg": self._hip_w_qkvg, "b_qkvg": self._hip_b_qkvg, "w_t2": self._hip_w_t2}
    for key in ("ln_w", "ln_b", "lnc_w", "lnc_b", "w_scale", "b_scale", "w_shift"):
      w[key] = getattr(self, "_hip_ada_" + key, None)
    w["w_zc"], w["b_zc"] = getattr(self, "_hip_w_zc", None), getattr(self, "_hip_b_zc", None)
    return w

  @_require_native_preparation
  @graphs.graphed
  def forward(self, x: torch.Tensor, mask: torch.Tensor, *, pair_logits: torch.Tensor | None = None,
              single_cond: torch.Tensor | None = None, add_residual: bool = True,
              adaptive_scale: torch.Tensor | None = None, adaptive_bias: torch.Tensor | None = None,
              zero_gate: torch.Tensor | None = None) -> torch.Tensor:
    """``adaptive_scale`` / ``adaptive_bias`` / ``zero_gate`` ``[N, C]``: this layer's precomputed
    conditioning (``TransformerHipMixin.diffusion_conditioning``; the reference's
    ``forward_prepared``, backends/vecops/modules.py:1171-1176), used in place of ``single_cond``."""
    H, D = self.num_head, self.key_dim
    HD = H * D
    lead, N = x.shape[:-2], x.shape[-2]
    S = x.numel() // max(N * x.shape[-1], 1)
    pre = None
    if adaptive_scale is not None:
      pre = (adaptive_scale, adaptive_bias, zero_gate)
      assert all(t is not None for t in pre), "adaptive_scale, adaptive_bias and zero_gate go together"
    native = (mask is None or tuple(mask.shape) == (N,)) and \
        (pair_logits is None or tuple(pair_logits.shape) in {(H, N, N), (S, H, N, N)}) and \
        (single_cond is None or (single_cond.dim() == 2 and single_cond.shape[0] == N)) and \
        (single_cond is not None or pre is not None or hasattr(self, "_hip_ada_ln_w")) and \
        (pre is None or all(tuple(t.shape) == (N, x.shape[-1]) and t.stride(-1) == 1 and
                            t.stride(0) == adaptive_scale.stride(0) for t in pre))
    if native:                                        # the whole module in one library call
      out = ops.self_attention_module(x, mask, pair_logits, None if pre else single_cond, self._native_weights(),
                                      num_head=H, head_dim=D, add_residual=add_residual, pre=pre)
      return out.to(x.dtype)
    if pre is not None:
      xh = ops.layer_norm(x, scale=adaptive_scale.reshape(-1, adaptive_scale.shape[-1]),
                          shift=adaptive_bias.reshape(-1, adaptive_bias.shape[-1]))
    else:
      xh = _adaln(self, "_hip_ada_", x, single_cond)
    y = ops.linear(xh, self._hip_w_qkvg, self._hip_b_qkvg)              # [..., N, 4HD]
    q, k, v, g = (y[..., i * HD:(i + 1) * HD].unflatten(-1, (H, D)) for i in range(4))
    o = dot_product_attention(q, k, v, mask_k=mask, bias=pair_logits, gate=g)
    o = o.reshape(*lead, N, HD)
    if pre is not None:
      return ops.linear(o, self._hip_w_t2, mul=zero_gate.reshape(-1, zero_gate.shape[-1]),
                        residual=x if add_residual else None).to(x.dtype)
    return _zero_init_residual(self, o, single_cond, x if add_residual else None).to(x.dtype)


# ---------------------------------------------------------------------------------------
# CrossAttention (windowed atom attention)
# ---------------------------------------------------------------------------------------

class CrossAttentionHipMixin:
  def prepare_native(self) -> bool:
    _begin_preparation(self)
    H, D = self.num_head, self.key_dim
    C = self.q_projection.weight.shape[0]
    HD = H * D
    wq = self.q_projection.weight.reshape(C, HD).t()
    wg = self.gating_query.weight.reshape(C, HD).t()
    wk = self.k_projection.weight.reshape(C, HD).t()
    wv = self.v_projection.weight.reshape(C, HD).t()
    _buf(self, "_hip_w_qg", _bf(torch.cat([wq, wg], 0)))               # [2HD, C]
    b = torch.zeros(2 * HD, dtype=torch.float32, device=wq.device)
    b[:HD] = self.q_projection.bias.detach().reshape(HD).float()
    _buf(self, "_hip_b_qg", b)
    _buf(self, "_hip_w_kv", _bf(torch.cat([wk, wv], 0)))               # [2HD, C]
    _prepare_adaln(self, self.q_layernorm, "_hip_adq_")
    _prepare_adaln(self, self.k_layernorm, "_hip_adk_")
    _prepare_zero_init(self, self.zero_init)
    self._hip_cond_cache = None
    if self.q_layernorm.single_cond and self.k_layernorm.single_cond and self.zero_init.single_cond:
      # both sides' conditioning as two layers of one diffusion_conditioning call (the k side's
      # zero gate is computed and dropped, as the native plan does)
      _buf(self, "_hip_pc_lnc_w", torch.stack([self._hip_adq_lnc_w, self._hip_adk_lnc_w]))
      _buf(self, "_hip_pc_w_scale", torch.cat([self._hip_adq_w_scale, self._hip_adk_w_scale], 0))   # [2C, Cs]
      _buf(self, "_hip_pc_b_scale", torch.cat([self._hip_adq_b_scale, self._hip_adk_b_scale]))
      _buf(self, "_hip_pc_w_shift", torch.cat([self._hip_adq_w_shift, self._hip_adk_w_shift], 0))
      _buf(self, "_hip_pc_w_zc", torch.cat([self._hip_w_zc, self._hip_w_zc], 0))
      _buf(self, "_hip_pc_b_zc", torch.cat([self._hip_b_zc, self._hip_b_zc]))
    self._native_prepared = True
    return True

  def cross_conditioning(self, queries_single_cond: torch.Tensor) -> dict:
    """Both sides' AdaLN terms per atom from the queries' condition ``[U, Qw, C]``, cached per
    condition tensor (the native plan's per-example conditioning, backends/vecops/modules.py:
    1302-1351): q_scale, q_shift, k_scale, k_shift, zgate, each ``[U*Qw, C]``.

    The cache holds the condition tensor itself and matches it by identity and version counter:
    while it is held, its memory cannot be handed to another tensor, so a new condition that
    happens to land at a freed address is never mistaken for the cached one, and an in-place
    change bumps the version."""
    cached = self._hip_cond_cache
    if (cached is not None and cached[0] is queries_single_cond
        and cached[1] == queries_single_cond._version):
      return cached[2]
    scale, shift, zgate = ops.diffusion_conditioning(queries_single_cond, self._hip_pc_lnc_w, self._hip_pc_w_scale,
                                                     self._hip_pc_b_scale, self._hip_pc_w_shift, self._hip_pc_w_zc,
                                                     self._hip_pc_b_zc)
    terms = {"q_scale": scale[0], "q_shift": shift[0], "k_scale": scale[1], "k_shift": shift[1], "zgate": zgate[0]}
    self._hip_cond_cache = (queries_single_cond, queries_single_cond._version, terms)
    return terms

  def _native_weights(self) -> dict:
    w = {"w_qg": self._hip_w_qg, "b_qg": self._hip_b_qg, "w_kv": self._hip_w_kv, "w_t2": self._hip_w_t2,
         "w_zc": getattr(self, "_hip_w_zc", None), "b_zc": getattr(self, "_hip_b_zc", None)}
    for side in ("q", "k"):
      for key in ("lnc_w", "lnc_b", "w_scale", "b_scale", "w_shift"):
        w[f"{key}_{side}"] = getattr(self, f"_hip_ad{side}_{key}", None)
    return w

  def _native_ok(self, U, Qw, Kw, mask_q, mask_k, pair_logits, cq, ck) -> bool:
    return (cq is not None and ck is not None and hasattr(self, "_hip_adq_w_scale")
            and hasattr(self, "_hip_adk_w_scale") and getattr(self, "_hip_w_zc", None) is not None
            and tuple(cq.shape[-3:-1]) == (U, Qw) and cq.dim() == 3 and tuple(ck.shape[-3:-1]) == (U, Kw)
            and ck.dim() == 3 and (mask_q is None or tuple(mask_q.shape) == (U, Qw))
            and (mask_k is None or tuple(mask_k.shape) == (U, Kw))
            and (pair_logits is None or tuple(pair_logits.shape) == (U, self.num_head, Qw, Kw)))

  @_require_native_preparation
  @graphs.graphed
  def forward(self, x_q: torch.Tensor, x_k: torch.Tensor, mask_q: torch.Tensor, mask_k: torch.Tensor,
              pair_logits: torch.Tensor | None = None, single_cond_q: torch.Tensor | None = None,
              single_cond_k: torch.Tensor | None = None, *, add_residual: bool = True) -> torch.Tensor:
    H, D = self.num_head, self.key_dim
    HD = H * D
    if x_q.dim() >= 3 and x_k.dim() == x_q.dim() and x_k.shape[:-2] == x_q.shape[:-2] and \
        self._native_ok(x_q.shape[-3], x_q.shape[-2], x_k.shape[-2], mask_q, mask_k, pair_logits,
                        single_cond_q, single_cond_k):
      out = ops.cross_attention_module(x_q, x_k, None, None, mask_q, mask_k, pair_logits, single_cond_q,
                                       single_cond_k, self._native_weights(), num_head=H, head_dim=D,
                                       add_residual=add_residual)
      return out.to(x_q.dtype)
    hq = _adaln(self, "_hip_adq_", x_q, single_cond_q)
    hk = _adaln(self, "_hip_adk_", x_k, single_cond_k)
    yq = ops.linear(hq, self._hip_w_qg, self._hip_b_qg)                 # [..., Q, 2HD]
    yk = ops.linear(hk, self._hip_w_kv)                                 # [..., K, 2HD]
    q, g = yq[..., :HD].unflatten(-1, (H, D)), yq[..., HD:].unflatten(-1, (H, D))
    k, v = yk[..., :HD].unflatten(-1, (H, D)), yk[..., HD:].unflatten(-1, (H, D))
    o = dot_product_attention(q, k, v, mask_q=mask_q, mask_k=mask_k, bias=pair_logits, gate=g)
    o = o.reshape(*o.shape[:-2], HD)
    return _zero_init_residual(self, o, single_cond_q, x_q if add_residual else None).to(x_q.dtype)

  @_require_native_preparation
  @graphs.graphed
  def forward_indexed(self, queries_act: torch.Tensor, queries_mask: torch.Tensor, gather_idxs: torch.Tensor,
                      gather_mask: torch.Tensor, keys_mask: torch.Tensor, queries_single_cond: torch.Tensor,
                      keys_single_cond: torch.Tensor, pair_logits: torch.Tensor | None = None, *,
                      add_residual: bool = True) -> torch.Tensor:
    """CrossAttTransformer block attention (transformer.py:668-682): keys are gathered from
    the queries by ``queries_to_keys`` (flat index over ``[U, Qw]``, masked -> 0).
    ``keys_single_cond=None`` states that the keys' condition is the gathered queries' condition
    (as CrossAttTransformer builds it, atom.py:279-281): the per-atom plan then runs, with both
    sides' conditioning computed once per ``queries_single_cond`` (cross_conditioning)."""
    lead = queries_act.shape[:-3]
    U, Qw, Cn = queries_act.shape[-3:]
    Kw = gather_idxs.shape[-1]
    if keys_single_cond is None:
      ok = (hasattr(self, "_hip_pc_lnc_w") and queries_single_cond is not None
            and tuple(queries_single_cond.shape) == (U, Qw, Cn) and tuple(gather_idxs.shape) == (U, Kw)
            and self._native_ok(U, Qw, Kw, queries_mask, keys_mask, pair_logits, queries_single_cond,
                                queries_single_cond.new_empty(U, Kw, Cn)))
      if not ok:
        raise ValueError("forward_indexed without keys_single_cond needs the conditioned module, "
                         "queries_single_cond [U, Qw, C] and [U, Kw] gather indices")
      out = ops.cross_attention_module(queries_act, None, gather_idxs, gather_mask, queries_mask, keys_mask,
                                       pair_logits, None, None, self._native_weights(), num_head=self.num_head,
                                       head_dim=self.key_dim, add_residual=add_residual,
                                       pre=self.cross_conditioning(queries_single_cond))
      return out.to(queries_act.dtype)
    if tuple(gather_idxs.shape) == (U, Kw) and self._native_ok(U, Qw, Kw, queries_mask, keys_mask, pair_logits,
                                                               queries_single_cond, keys_single_cond):
      out = ops.cross_attention_module(queries_act, None, gather_idxs, gather_mask, queries_mask, keys_mask,
                                       pair_logits, queries_single_cond, keys_single_cond, self._native_weights(),
                                       num_head=self.num_head, head_dim=self.key_dim, add_residual=add_residual)
      return out.to(queries_act.dtype)
    S = 1
    for s in lead:
      S *= s
    keys = ops.window_gather(queries_act.reshape(S, U * Qw, Cn), gather_idxs, gather_mask)
    keys = keys.view(*lead, U, gather_idxs.shape[-1], Cn)
    return self.forward(queries_act, keys, queries_mask, keys_mask, pair_logits, queries_single_cond,
                        keys_single_cond, add_residual=add_residual)


# ---------------------------------------------------------------------------------------
# Transitions (trunk: blocks.py:38-96; diffusion transformer: transformer.py:157-231)
# ---------------------------------------------------------------------------------------

def _glu_rows(weight: torch.Tensor) -> torch.Tensor:
  """The reference's ``[C, 2I]`` GLU weight (first I columns through swish) as the kernel's
  ``[2I, C]`` K-contiguous rows, interleaved: row 2i = column i, row 2i + 1 = column I + i."""
  wt = weight.detach().t()
  I = wt.shape[0] // 2
  return _bf(torch.stack([wt[:I], wt[I:]], 1).reshape(2 * I, wt.shape[1]))


class TransitionBlockHipMixin:
  """TransitionBlock.forward (blocks.py:84-96) as one library call."""

  def prepare_native(self) -> bool:
    _begin_preparation(self)
    _buf(self, "_hip_ln_w", _f32(self.input_layer_norm.weight))
    _buf(self, "_hip_ln_b", _f32(getattr(self.input_layer_norm, "bias", None)))
    _buf(self, "_hip_w1", _glu_rows(self.transition1.weight))
    _buf(self, "_hip_w2", _bf(self.transition2.weight.t()))           # [I, C] -> [C, I]
    self._native_prepared = True
    return True

  @_require_native_preparation
  @graphs.graphed
  def forward(self, act: torch.Tensor, *, broadcast_dim: int | None = 0, add_residual: bool = True) -> torch.Tensor:
    w = {"ln_w": self._hip_ln_w, "ln_b": self._hip_ln_b, "w1": self._hip_w1, "w2": self._hip_w2}
    rows = act.reshape(-1, act.shape[-1])
    out = ops.transition_module(rows, None, w, add_residual=add_residual)
    return out.view(act.shape).to(act.dtype)


class DiffusionTransitionHipMixin:
  """TransitionBlock.forward of the diffusion transformer (transformer.py:209-231) as one call."""

  def prepare_native(self) -> bool:
    _begin_preparation(self)
    _prepare_adaln(self, self.layer_norm, "_hip_ada_")
    _buf(self, "_hip_w1", _glu_rows(self.transition.weight))
    _prepare_zero_init(self, self.zero_init)                           # _hip_w_t2 = W2 [C, I]
    self._native_prepared = True
    return True

  def _native_weights(self) -> dict:
    w = {"w1": self._hip_w1, "w2": self._hip_w_t2, "w_zc": getattr(self, "_hip_w_zc", None),
         "b_zc": getattr(self, "_hip_b_zc", None)}
    for key in ("ln_w", "ln_b", "lnc_w", "lnc_b", "w_scale", "b_scale", "w_shift"):
      w[key] = getattr(self, "_hip_ada_" + key, None)
    return w

  @_require_native_preparation
  @graphs.graphed
  def forward(self, x: torch.Tensor, *, single_cond: torch.Tensor | None = None, add_residual: bool = True,
              adaptive_scale: torch.Tensor | None = None, adaptive_bias: torch.Tensor | None = None,
              zero_gate: torch.Tensor | None = None) -> torch.Tensor:
    """``adaptive_scale`` / ``adaptive_bias`` / ``zero_gate`` ``[N, C]``: this layer's precomputed
    conditioning (``TransformerHipMixin.diffusion_conditioning``), used in place of ``single_cond``."""
    N = x.shape[-2]
    pre = None
    if adaptive_scale is not None:
      pre = (adaptive_scale, adaptive_bias, zero_gate)
    elif single_cond is not None and not (single_cond.dim() == 2 and single_cond.shape[0] == N):
      raise ValueError(f"diffusion transition: single_cond must be [N, Cs], got {tuple(single_cond.shape)}")
    if single_cond is None and pre is None and not hasattr(self, "_hip_ada_ln_w"):
      raise ValueError("diffusion transition: this block is conditioned; pass single_cond")
    out = ops.transition_module(x, None if pre else single_cond, self._native_weights(), add_residual=add_residual,
                                pre=pre)
    return out.to(x.dtype)


# ---------------------------------------------------------------------------------------
# SingleActUpdate: pair-logit prologue + single attention
# ---------------------------------------------------------------------------------------

class SingleActUpdateHipMixin:
  def prepare_native(self) -> bool:
    _begin_preparation(self)
    _buf(self, "_hip_pl_ln_w", _f32(self.single_pair_logits_norm.weight))
    _buf(self, "_hip_pl_ln_b", _f32(getattr(self.single_pair_logits_norm, "bias", None)))
    _buf(self, "_hip_pl_w", _bf(self.single_pair_logits_projection.weight.t()))   # [Cz, H] -> [H, Cz]
    if getattr(self.single_attention, "prepare_native", None) is None:
      raise RuntimeError("single_attention is not a HIP module; select backend 'hip' before construction")
    _prepare_hip_children(self)                                         # the attention and the transition
    self._native_prepared = True
    return True

  @_require_native_preparation
  @graphs.graphed
  def forward(self, pair_act: torch.Tensor, single_act: torch.Tensor, seq_mask: torch.Tensor, *,
              add_residual: bool = True) -> torch.Tensor:
    N = pair_act.shape[-2]
    pl = ops.pair_logits(pair_act, self._hip_pl_ln_w, self._hip_pl_ln_b, self._hip_pl_w)
    pl = pl.view(self.num_head, *pair_act.shape[:-1])                   # [H, B, N]
    out = self.single_attention(single_act, seq_mask, pair_logits=pl, add_residual=add_residual)
    transition = getattr(self, "single_transition", None)
    if transition is not None and add_residual:                         # reference transition, when present
      out = transition(out, broadcast_dim=None)
    assert out.shape[-2] == N
    return out


# ---------------------------------------------------------------------------------------
# Transformer / CrossAttTransformer: the cached pair-logit packs
# ---------------------------------------------------------------------------------------

class _PackFactory:
  """Stands in for a ``ValueCache`` during one ``forward``: ``get`` of the entry ``name``
  uses ``factory`` in place of the caller's; everything else goes to the wrapped cache."""

  def __init__(self, cache, name: str, factory):
    self._cache, self._name, self._factory = cache, name, factory

  def get(self, *args, name=None, factory=None):
    if name == self._name:
      factory = self._factory
    return self._cache.get(*args, name=name, factory=factory)

  def __getattr__(self, attr):
    return getattr(self._cache, attr)


def _with_pack_factory(module, factory, call):
  cache = module._cache
  module._cache = _PackFactory(cache, "pair_logits", factory)
  try:
    return call()
  finally:
    module._cache = cache


def _prepare_hip_children(module: torch.nn.Module) -> None:
  """A container's ``prepare_native`` also prepares the HIP modules inside it (``prepare``
  stops at the first HIP module it meets on each branch)."""
  for child in module.modules():
    if child is not module and isinstance(child, HIP_TYPES) and not getattr(child, "_native_prepared", False):
      child.prepare_native()


class TransformerHipMixin:
  def prepare_native(self) -> bool:
    _begin_preparation(self)
    projections = list(self.pair_logits_projection)
    Pc = self.pair_input_layer_norm.weight.shape[0]
    w = [proj.weight.reshape(Pc, -1).t() for proj in projections]      # [P, S, H] -> [S*H, P]
    _buf(self, "_hip_pack_w", _bf(torch.cat(w, 0)))                    # planes (super-block, s, h)
    _buf(self, "_hip_pack_ln_w", _f32(self.pair_input_layer_norm.weight))
    _buf(self, "_hip_pack_ln_b", _f32(getattr(self.pair_input_layer_norm, "bias", None)))
    self._hip_pack_shape = (len(projections),) + tuple(projections[0].weight.shape[1:])
    _prepare_hip_children(self)
    self._prepare_conditioning()
    self._native_prepared = True
    return True

  def _attention_layers(self) -> list | None:
    """The SelfAttention blocks in call order (super-block, block), or None when the stacks are
    not [super-block][block] containers of prepared, condition-only HIP blocks."""
    try:
      layers = [[a for a in sb] for sb in self.self_attention]
      trans = [[t for t in sb] for sb in self.transition_block]
    except (AttributeError, TypeError):
      return None
    if [len(x) for x in layers] != [len(x) for x in trans]:
      return None
    flat = [a for sb in layers for a in sb]
    ok = bool(flat) and all(isinstance(a, SelfAttentionHipMixin) and getattr(a, "_hip_ada_lnc_w", None) is not None
                            and getattr(a, "_hip_ada_lnc_b", None) is None and getattr(a, "_hip_w_zc", None) is not None
                            for a in flat)
    return flat if ok else None

  def _transition_layers(self) -> list | None:
    """The transition blocks in call order when every one is a conditioned HIP transition (then
    their AdaLN conditioning joins the attention blocks' one call), else None."""
    try:
      flat = [t for sb in self.transition_block for t in sb]
    except (AttributeError, TypeError):
      return None
    ok = bool(flat) and all(isinstance(t, DiffusionTransitionHipMixin) and getattr(t, "_hip_ada_lnc_w", None) is not None
                            and getattr(t, "_hip_ada_lnc_b", None) is None and getattr(t, "_hip_w_zc", None) is not None
                            for t in flat)
    return flat if ok else None

  def _prepare_conditioning(self) -> None:
    """Stacks every block's AdaLN / AdaLN-zero condition weights -- the attention blocks', then the
    transition blocks' when those are conditioned HIP transitions -- so that one call conditions
    them all (the reference packs them per super-block, backends/vecops/modules.py:1040-1081)."""
    self._hip_dc = None
    flat = self._attention_layers()
    if flat is None:
      return
    trans = self._transition_layers()
    self._hip_dc_transitions = trans is not None
    layers = flat + (trans or [])
    zeros = lambda a: torch.zeros(a._hip_ada_w_scale.shape[0], dtype=torch.float32, device=a._hip_ada_w_scale.device)
    self._hip_dc = {
        "lnc_w": torch.stack([a._hip_ada_lnc_w for a in layers]).contiguous(),
        "w_scale": torch.cat([a._hip_ada_w_scale for a in layers]).contiguous(),
        "b_scale": torch.cat([a._hip_ada_b_scale if a._hip_ada_b_scale is not None else zeros(a) for a in layers]),
        "w_shift": torch.cat([a._hip_ada_w_shift for a in layers]).contiguous(),
        "w_zc": torch.cat([a._hip_w_zc for a in layers]).contiguous(),
        "b_zc": torch.cat([a._hip_b_zc if a._hip_b_zc is not None else zeros(a) for a in layers]),
    }

  @_require_native_preparation
  def diffusion_conditioning(self, single_cond: torch.Tensor):
    """Every block's AdaLN scale, shift and AdaLN-zero gate from ``single_cond [N, Cs]`` in one
    call: (scale, shift, zgate), each ``[L, N, C]`` (L = number of blocks; scale and zgate after
    the sigmoid).  The reference computes them per super-block (DiffusionConditioning.cpp)."""
    d = self._hip_dc
    return ops.diffusion_conditioning(single_cond, d["lnc_w"], d["w_scale"], d["b_scale"], d["w_shift"],
                                      d["w_zc"], d["b_zc"])

  @_require_native_preparation
  def pair_logits_pack(self, pair_cond: torch.Tensor) -> torch.Tensor:
    """``pair_cond [N, N, P]`` -> ``[n_super, super_block, H, N, N]`` (transformer.py:431-438)."""
    assert pair_cond.ndim == 3, "pair_cond must be [N, N, P]"
    N0, N1 = pair_cond.shape[:2]
    planes = ops.pair_logits(pair_cond, self._hip_pack_ln_w, self._hip_pack_ln_b, self._hip_pack_w)
    pack = planes.view(*self._hip_pack_shape, N0, N1)
    return pack.to(self.dtype or pair_cond.dtype)

  def forward(self, act, mask, single_cond, pair_cond=None):
    if getattr(self, "_hip_dc", None) is not None and isinstance(single_cond, torch.Tensor) and \
        single_cond.is_cuda and single_cond.dim() == 2 and single_cond.shape[0] == act.shape[-2]:
      return self._forward_conditioned(act, mask, single_cond, pair_cond)
    if pair_cond is None:
      return super().forward(act, mask, single_cond, pair_cond)
    return _with_pack_factory(self, lambda: self.pair_logits_pack(pair_cond),
                              lambda: super(TransformerHipMixin, self).forward(act, mask, single_cond, pair_cond))

  def _forward_conditioned(self, act, mask, single_cond, pair_cond):
    """Transformer.forward (transformer.py:422-477) with every block's conditioning computed once
    up front: the native Transformer's loop (backends/vecops/modules.py:1093-1183) -- the
    attention blocks take their precomputed layer, the transition blocks run as they are."""
    pack = None
    if pair_cond is not None:
      pack = self._cache.get(name="pair_logits", factory=lambda: self.pair_logits_pack(pair_cond))
    scale, shift, zgate = self.diffusion_conditioning(single_cond)
    x = act.to(self.dtype) if getattr(self, "dtype", None) is not None else act
    layer = 0
    n_att = sum(len(sb) for sb in self.self_attention)
    for sb, (attentions, transitions) in enumerate(zip(self.self_attention, self.transition_block)):
      for b, (attention, transition) in enumerate(zip(attentions, transitions)):
        x = attention(x, mask, pair_logits=None if pack is None else pack[sb][b], single_cond=single_cond,
                      adaptive_scale=scale[layer], adaptive_bias=shift[layer], zero_gate=zgate[layer])
        if self._hip_dc_transitions:
          t = n_att + layer
          x = transition(x, single_cond=single_cond, adaptive_scale=scale[t], adaptive_bias=shift[t],
                         zero_gate=zgate[t])
        else:
          x = transition(x, single_cond=single_cond)
        layer += 1
    return x.to(act.dtype)


class CrossAttTransformerHipMixin:
  def prepare_native(self) -> bool:
    _begin_preparation(self)
    w = self.pair_logits_projection.weight                              # [P, num_blocks, H]
    _buf(self, "_hip_pack_w", _bf(w.reshape(w.shape[0], -1).t()))        # planes (block, h)
    _buf(self, "_hip_pack_ln_w", _f32(self.pair_input_layer_norm.weight))
    _buf(self, "_hip_pack_ln_b", _f32(getattr(self.pair_input_layer_norm, "bias", None)))
    self._hip_pack_shape = tuple(w.shape[1:])
    _prepare_hip_children(self)
    self._native_prepared = True
    return True

  @_require_native_preparation
  def pair_logits_pack(self, pair_cond: torch.Tensor) -> torch.Tensor:
    """``pair_cond [U, Q, K, P]`` -> ``[num_blocks, U, H, Q, K]`` (transformer.py:655-662),
    stored by the kernel in that order (no permute pass)."""
    assert pair_cond.ndim == 4, "pair_cond must be [num_subsets, num_queries, num_keys, P]"
    U, Qn, Kn = pair_cond.shape[:3]
    nb, H = self._hip_pack_shape
    pack = ops.pair_logits(pair_cond, self._hip_pack_ln_w, self._hip_pack_ln_b, self._hip_pack_w,
                           seg=Qn * Kn, group=H)                        # [nb, U, H, Q*K]
    return pack.view(nb, U, H, Qn, Kn).to(pair_cond.dtype)

  def forward(self, queries_act, queries_mask, queries_to_keys, keys_mask, queries_single_cond,
              keys_single_cond, pair_cond):
    return _with_pack_factory(
        self, lambda: self.pair_logits_pack(pair_cond),
        lambda: super(CrossAttTransformerHipMixin, self).forward(
            queries_act, queries_mask, queries_to_keys, keys_mask, queries_single_cond, keys_single_cond,
            pair_cond))


class GridSelfAttentionHip(GridSelfAttentionHipMixin, base.GridSelfAttention):
  pass


class SelfAttentionHip(SelfAttentionHipMixin, base.SelfAttention):
  pass


class CrossAttentionHip(CrossAttentionHipMixin, base.CrossAttention):
  pass


class SingleActUpdateHip(SingleActUpdateHipMixin, base.SingleActUpdate):
  pass


class TransformerPairLogitsHip(TransformerHipMixin, base.TransformerPairLogits):
  pass


class CrossAttTransformerPairLogitsHip(CrossAttTransformerHipMixin, base.CrossAttTransformerPairLogits):
  pass


class TriangleMultiplicationHipMixin:
  """TriangleMultiplication.forward (blocks.py:486-566) as one library call."""

  def prepare_native(self) -> bool:
    _begin_preparation(self)
    C = self.num_channels
    if C != 128:
      raise ValueError(f"TriangleMultiplicationHip: {C} channels; the HIP module handles 128")

    def split(w):  # [C, 2C] (in, out) -> rows of channels 2c (a) then 2c + 1 (b), K contiguous
      wt = w.detach().t()
      return torch.cat([wt[0::2], wt[1::2]], 0)

    _buf(self, "_hip_w_glu", _bf(torch.cat([split(self.gate_projection.weight), split(self.projection.weight)], 0)))
    _buf(self, "_hip_ln_w", _f32(self.left_norm_input.weight))
    _buf(self, "_hip_ln_b", _f32(getattr(self.left_norm_input, "bias", None)))
    _buf(self, "_hip_cn_w", _f32(self.center_norm.weight))
    _buf(self, "_hip_cn_b", _f32(getattr(self.center_norm, "bias", None)))
    _buf(self, "_hip_w_out", _bf(self.output_projection.weight.t()))   # [C in, C out] -> [out, in]
    _buf(self, "_hip_w_gate", _bf(self.gating_linear.weight.t()))
    self._native_prepared = True
    return True

  # incoming edges, in the config's form and in the per-channel form the reference module stores
  # (blocks.py:447-451)
  INCOMING_EQUATIONS = ("...kjc,...kic->...ijc", "...ckj,...cki->...cij")

  @_require_native_preparation
  @graphs.graphed
  def forward(self, act: torch.Tensor, mask: torch.Tensor, *, add_residual: bool = True) -> torch.Tensor:
    w = {k: getattr(self, "_hip_" + k) for k in ("ln_w", "ln_b", "w_glu", "cn_w", "cn_b", "w_out", "w_gate")}
    out = ops.triangle_multiplication(act, mask, w, incoming=self.equation in self.INCOMING_EQUATIONS,
                                      add_residual=add_residual)
    return out.to(act.dtype)


class TriangleMultiplicationHip(TriangleMultiplicationHipMixin, base.TriangleMultiplication):
  pass


class TransitionBlockHip(TransitionBlockHipMixin, base.TransitionBlock):
  pass


class DiffusionTransitionBlockHip(DiffusionTransitionHipMixin, base.DiffusionTransitionBlock):
  pass


HIP_TYPES = (TriangleMultiplicationHipMixin, GridSelfAttentionHipMixin, SelfAttentionHipMixin, CrossAttentionHipMixin,
             SingleActUpdateHipMixin, TransformerHipMixin, CrossAttTransformerHipMixin, TransitionBlockHipMixin,
             DiffusionTransitionHipMixin)
