"""Tensor-level wrappers over the C ABI (include/sparsefold_hip.h).

Each wrapper checks devices, shapes and dtypes in Python (ValueError, as the reference's
native wrappers do, ``backends/vecops/kernels/registry.py:2910-2929``), allocates outputs and
workspaces with torch on the input's device, and launches on torch's current HIP stream.
Nothing here computes on the host: every numeric result comes from libsparsefold_hip.
"""
from __future__ import annotations

import ctypes as C
import itertools
import math

import torch

from sparsefold_amd import _lib

BF16 = torch.bfloat16


def _vp(t: torch.Tensor | None):
  return None if t is None else C.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor):
  """torch's current stream on t's device (the raw handle; the public accessor builds a Stream
  object per call, which costs more than some of the kernels it launches)."""
  if _raw_stream is not None:
    return C.c_void_p(_raw_stream(t.device.index))
  return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_cuda(*ts: torch.Tensor | None) -> torch.device:
  dev = None
  for t in ts:
    if t is None:
      continue
    if t.device.type != "cuda":
      raise ValueError(f"HIP kernels need device tensors, got a tensor on {t.device}")
    if dev is None:
      dev = t.device
    elif t.device != dev:
      raise ValueError(f"tensors on different devices: {dev} and {t.device}")
  if dev is None:
    raise ValueError("no device tensor given")
  return dev


def _require(cond: bool, msg: str) -> None:
  if not cond:
    raise ValueError(msg)


def _bf16(t: torch.Tensor) -> torch.Tensor:
  return t if t.dtype == BF16 else t.to(BF16)


def _f32(t: torch.Tensor | None) -> torch.Tensor | None:
  return None if t is None else t.to(torch.float32).contiguous()


def _u8(t: torch.Tensor) -> torch.Tensor:
  """Byte mask: a bool tensor is reinterpreted in place (torch stores bool as 0/1 bytes)."""
  if t.dtype == torch.uint8:
    return t
  if t.dtype == torch.bool:
    return t.view(torch.uint8)
  return (t != 0).view(torch.uint8)


def _rows(t: torch.Tensor, last: int) -> torch.Tensor:
  """2-D row view ``[M, last]`` with unit last stride and 16-byte aligned rows."""
  t2 = t.reshape(-1, last)
  if t2.stride(-1) != 1 or t2.stride(0) % 8 != 0 or t2.data_ptr() % 16 != 0:
    t2 = t2.contiguous()
  return t2


# ---------------------------------------------------------------------------------------
# attention core
# ---------------------------------------------------------------------------------------

def attention(q, k, v, *, scale: float, bias=None, mask_q=None, mask_k=None, gate=None, out=None,
              schedule: int = 0):
  """Core launch on 2-level batched views.

  q ``[B0,B1,Q,H,D]``, k ``[B0,B1,K,H,D]``, v ``[B0,B1,K,H,Dv]``, gate like the output
  ``[B0,B1,Q,H,Dv]``; bias ``[B0,B1,H,Q,K]`` (zero strides allowed), masks ``[B0,B1,Q]`` /
  ``[B0,B1,K]`` uint8.  All bf16 with unit last stride.  ``schedule``: 0 chooses the work
  decomposition from the sizes, 1 / 2 force shared-tile / per-wave tasks, 3 the shared-bias
  kernel (5 samples, head dim 48, one bias for all samples; refused otherwise).  Returns ``out``.
  """
  dev = _require_cuda(q, k, v, bias, mask_q, mask_k, gate, out)
  _require(q.ndim == 5 and k.ndim == 5 and v.ndim == 5, "attention: q/k/v must be [B0,B1,L,H,D]")
  B0, B1, Q, H, D = q.shape
  K, Dv = k.shape[2], v.shape[-1]
  _require(tuple(k.shape) == (B0, B1, K, H, D), f"attention: k shape {tuple(k.shape)} vs q {tuple(q.shape)}")
  _require(tuple(v.shape[:4]) == (B0, B1, K, H), f"attention: v shape {tuple(v.shape)}")
  for name, t in (("q", q), ("k", k), ("v", v), ("gate", gate), ("bias", bias)):
    if t is not None:
      _require(t.dtype == BF16, f"attention: {name} must be bfloat16, got {t.dtype}")
      _require(t.stride(-1) == 1, f"attention: {name} needs a unit last stride")
  if out is None:
    out = torch.empty((B0, B1, Q, H, Dv), dtype=BF16, device=dev)
  _require(tuple(out.shape) == (B0, B1, Q, H, Dv) and out.stride(-1) == 1, "attention: bad out")
  a = _lib.AttentionArgs()
  a.B0, a.B1, a.Q, a.K, a.H, a.D, a.Dv = B0, B1, Q, K, H, D, Dv
  a.scale = float(scale)
  a.q, a.q_s = _vp(q), (C.c_int64 * 4)(*q.stride()[:4])
  a.k, a.k_s = _vp(k), (C.c_int64 * 4)(*k.stride()[:4])
  a.v, a.v_s = _vp(v), (C.c_int64 * 4)(*v.stride()[:4])
  if bias is not None:
    _require(tuple(bias.shape) == (B0, B1, H, Q, K), f"attention: bias shape {tuple(bias.shape)}")
    a.bias, a.bias_s = _vp(bias), (C.c_int64 * 4)(*bias.stride()[:4])
  if mask_q is not None:
    _require(tuple(mask_q.shape) == (B0, B1, Q) and mask_q.dtype == torch.uint8, "attention: bad mask_q")
    a.mask_q, a.mq_s = _vp(mask_q), (C.c_int64 * 3)(*mask_q.stride())
  if mask_k is not None:
    _require(tuple(mask_k.shape) == (B0, B1, K) and mask_k.dtype == torch.uint8, "attention: bad mask_k")
    a.mask_k, a.mk_s = _vp(mask_k), (C.c_int64 * 3)(*mask_k.stride())
  if gate is not None:
    _require(tuple(gate.shape) == (B0, B1, Q, H, Dv), f"attention: gate shape {tuple(gate.shape)}")
    a.gate, a.g_s = _vp(gate), (C.c_int64 * 4)(*gate.stride()[:4])
  a.out, a.o_s = _vp(out), (C.c_int64 * 4)(*out.stride()[:4])
  _require(schedule in (0, 1, 2, 3), f"attention: schedule {schedule} is not 0, 1, 2 or 3")
  a.schedule = schedule
  lib = _lib.load()
  _lib.check(lib.sf_hip_attention_fwd(C.byref(a), _stream(q)), "sf_hip_attention_fwd")
  return out


# ---------------------------------------------------------------------------------------
# row kernels
# ---------------------------------------------------------------------------------------

def layer_norm(x: torch.Tensor, gamma=None, beta=None, *, eps: float = 1e-5, scale=None, shift=None):
  """LN over the last dim (bf16 in / out).  With ``scale``/``shift`` ([R, C] bf16) this is
  the AdaLN modulation, row m using condition row ``m % R``."""
  _require_cuda(x, gamma, beta, scale, shift)
  Cn = x.shape[-1]
  x2 = _rows(_bf16(x), Cn)
  y = torch.empty(x2.shape, dtype=BF16, device=x.device)
  a = _lib.LayerNormArgs()
  a.M, a.C, a.eps = x2.shape[0], Cn, float(eps)
  a.x, a.x_rs = _vp(x2), x2.stride(0)
  g, b = _f32(gamma), _f32(beta)
  a.gamma, a.beta = _vp(g), _vp(b)
  if scale is not None:
    s2, h2 = _rows(_bf16(scale), Cn), _rows(_bf16(shift), Cn)
    _require(s2.shape == h2.shape, "layer_norm: scale/shift shapes differ")
    a.scale, a.shift, a.cond_rows, a.cond_rs = _vp(s2), _vp(h2), s2.shape[0], s2.stride(0)
  a.y, a.y_rs = _vp(y), y.stride(0)
  _lib.check(_lib.load().sf_hip_layer_norm_fwd(C.byref(a), _stream(x)), "sf_hip_layer_norm_fwd")
  return y.view(*x.shape[:-1], Cn)


def linear(x: torch.Tensor, wt: torch.Tensor, bias=None, *, residual=None, mul=None,
           post_sigmoid: bool = False, ycols: int | None = None, yt=None, tcol0: int = 0,
           want_y: bool = True):
  """``post(x @ wt.T + bias) * mul + residual`` with ``wt`` ``[N, K]`` bf16 (K contiguous).

  ``mul`` ``[R, N]`` multiplies row m by ``mul[m % R]``.  ``yt`` (``[T, M]`` bf16) receives
  columns ``[tcol0, tcol0+T)`` transposed.  Returns ``y`` ``[..., ycols or N]`` or None."""
  _require_cuda(x, wt, bias, residual, mul, yt)
  N, K = wt.shape
  _require(x.shape[-1] == K, f"linear: x last dim {x.shape[-1]} != weight K {K}")
  _require(K % 8 == 0, "linear: K must be a multiple of 8")
  _require(wt.dtype == BF16 and wt.is_contiguous(), "linear: wt must be contiguous bf16 [N, K]")
  x2 = _rows(_bf16(x), K)
  M = x2.shape[0]
  a = _lib.LinearArgs()
  a.M, a.N, a.K = M, N, K
  a.x, a.x_rs, a.wt = _vp(x2), x2.stride(0), _vp(wt)
  bias_f = _f32(bias)
  a.bias = _vp(bias_f)
  ycols = N if ycols is None else ycols
  y = None
  if want_y:
    y = torch.empty((M, ycols), dtype=BF16, device=x.device)
    a.y, a.y_rs, a.ycols = _vp(y), y.stride(0), ycols
  if residual is not None:
    r2 = _bf16(residual).reshape(M, -1)
    _require(r2.shape[1] == ycols and r2.stride(-1) == 1, "linear: residual shape")
    a.residual, a.r_rs = _vp(r2), r2.stride(0)
  if mul is not None:
    m2 = _bf16(mul).reshape(-1, N)
    _require(m2.stride(-1) == 1, "linear: mul needs a unit last stride")
    a.mul, a.mul_rows, a.mul_rs = _vp(m2), m2.shape[0], m2.stride(0)
  else:
    a.mul_rows = 1
  a.post_sigmoid = int(bool(post_sigmoid))
  if yt is not None:
    _require(yt.dtype == BF16 and yt.shape[-1] == M and yt.stride(-1) == 1, "linear: yt shape")
    a.tcol0, a.tcols, a.yt, a.yt_rs = tcol0, yt.shape[0], _vp(yt), yt.stride(0)
  _lib.check(_lib.load().sf_hip_linear_fwd(C.byref(a), _stream(x)), "sf_hip_linear_fwd")
  return None if y is None else y.view(*x.shape[:-1], ycols)


def pair_logits(z: torch.Tensor, ln_w, ln_b, w_t: torch.Tensor, *, seg: int = 0, group: int = 0) -> torch.Tensor:
  """``[..., C]`` pair activations -> LN + projection logits planes.

  ``seg == 0``: ``[H, P]``.  ``seg > 0``: ``[H // group, P // seg, group, seg]`` (plane
  ``blk * group + h``, position ``u * seg + r``), the CrossAttTransformer pack layout."""
  _require_cuda(z, ln_w, ln_b, w_t)
  H, Cn = w_t.shape
  z2 = _rows(_bf16(z), Cn)
  P = z2.shape[0]
  _require(z2.stride(0) == Cn, "pair_logits: z rows must be contiguous")
  if seg:
    _require(P % seg == 0 and group > 0 and H % group == 0, "pair_logits: P % seg and H % group must be 0")
    out = torch.empty((H // group, P // seg, group, seg), dtype=BF16, device=z.device)
  else:
    out = torch.empty((H, P), dtype=BF16, device=z.device)
  lw, lb = _f32(ln_w), _f32(ln_b)
  wt = _bf16(w_t).contiguous()
  a = _lib.PairLogitsArgs()
  a.P, a.C, a.H = P, Cn, H
  a.z, a.ln_w, a.ln_b, a.w_t, a.out = _vp(z2), _vp(lw), _vp(lb), _vp(wt), _vp(out)
  a.seg, a.group = int(seg), int(group) if seg else 0
  _lib.check(_lib.load().sf_hip_pair_logits_fwd(C.byref(a), _stream(z)), "sf_hip_pair_logits_fwd")
  return out


def window_gather(src: torch.Tensor, idx: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
  """``src [S, rows, C]`` -> ``[S, UK, C]`` by flat index ``idx [UK]`` (masked -> 0)."""
  _require_cuda(src, idx, mask)
  S, rows, Cn = src.shape
  src = _bf16(src).contiguous()
  idx32 = idx.reshape(-1).to(torch.int32).contiguous()
  m8 = _u8(mask.reshape(-1)).contiguous()
  _require(idx32.numel() == m8.numel(), "window_gather: idx / mask sizes differ")
  UK = idx32.numel()
  keys = torch.empty((S, UK, Cn), dtype=BF16, device=src.device)
  a = _lib.WindowGatherArgs()
  a.S, a.rows, a.C, a.UK = S, rows, Cn, UK
  a.src, a.idx, a.mask, a.keys = _vp(src), _vp(idx32), _vp(m8), _vp(keys)
  _lib.check(_lib.load().sf_hip_window_gather_fwd(C.byref(a), _stream(src)), "sf_hip_window_gather_fwd")
  return keys


# ---------------------------------------------------------------------------------------
# triangle attention module
# ---------------------------------------------------------------------------------------

def triangle_workspace_bytes(N: int, C_: int, H: int, D: int) -> int:
  return int(_lib.load().sf_hip_triangle_workspace_bytes(N, C_, H, D))


def triangle_attention(z: torch.Tensor, seq_mask: torch.Tensor, ln_w, ln_b, w_qkvgb: torch.Tensor,
                       w_o: torch.Tensor, *, num_head: int, transpose: bool, add_residual: bool = True,
                       workspace: torch.Tensor | None = None, stages: int = _lib.TRI_STAGE_ALL,
                       out: torch.Tensor | None = None, fixup_sum_limit: float = 0.0) -> torch.Tensor:
  """GridSelfAttention on ``z [N, N, C]`` (bf16).  Weights packed as the C ABI documents.
  ``stages`` selects a subset of the pipeline (projection / attention / output projection)
  against a caller-held ``workspace``.  ``fixup_sum_limit`` > 0 lowers the weight-sum limit
  above which a (row, head) is recomputed by the exact two-pass softmax (0 = the default 2^100)."""
  _require_cuda(z, seq_mask, ln_w, ln_b, w_qkvgb, w_o, workspace)
  _require(z.ndim == 3 and z.shape[0] == z.shape[1], f"triangle: z must be [N, N, C], got {tuple(z.shape)}")
  N, _, Cn = z.shape
  HD = w_o.shape[1]
  _require(HD % num_head == 0, "triangle: output projection width not divisible by heads")
  D = HD // num_head
  _require(tuple(w_qkvgb.shape) == (4 * HD + num_head, Cn), f"triangle: w_qkvgb shape {tuple(w_qkvgb.shape)}")
  _require(tuple(w_o.shape) == (Cn, HD), f"triangle: w_o shape {tuple(w_o.shape)}")
  _require(seq_mask.shape == (N,), "triangle: seq_mask must be [N]")
  zc = _bf16(z).contiguous()
  m8 = _u8(seq_mask).contiguous()
  lw, lb = _f32(ln_w), _f32(ln_b)
  need = triangle_workspace_bytes(N, Cn, num_head, D)
  if workspace is None or workspace.numel() < need:
    workspace = torch.empty(need, dtype=torch.uint8, device=z.device)
  if out is None:
    out = torch.empty_like(zc)
  a = _lib.TriangleArgs()
  a.N, a.C, a.H, a.D = N, Cn, num_head, D
  a.transpose, a.add_residual = int(bool(transpose)), int(bool(add_residual))
  a.z, a.seq_mask, a.ln_w, a.ln_b = _vp(zc), _vp(m8), _vp(lw), _vp(lb)
  a.w_qkvgb, a.w_o, a.out = _vp(w_qkvgb), _vp(w_o), _vp(out)
  _require(fixup_sum_limit >= 0.0, "triangle: fixup_sum_limit must be >= 0")
  a.fixup_sum_limit = float(fixup_sum_limit)
  if stages == _lib.TRI_STAGE_ALL:
    rc = _lib.load().sf_hip_triangle_attn_fwd(C.byref(a), _vp(workspace), workspace.numel(), _stream(z))
  else:
    rc = _lib.load().sf_hip_triangle_stage_fwd(C.byref(a), stages, _vp(workspace), workspace.numel(), _stream(z))
  _lib.check(rc, "sf_hip_triangle_attn_fwd")
  return out


# per-call seeds of the block sampler when the caller gives none (the reference draws them from a
# process-wide counter, backends/vecops/kernels/registry.py:3033)
_ibs_seed_counter = itertools.count()


def triangle_ibs_workspace_bytes(N: int, C_: int, H: int, D: int) -> int:
  return int(_lib.load().sf_hip_triangle_ibs_workspace_bytes(N, C_, H, D))


def triangle_attention_ibs(z: torch.Tensor, seq_mask: torch.Tensor, ln_w, ln_b, w_qkvgb: torch.Tensor,
                           w_o: torch.Tensor, *, num_head: int, transpose: bool, num_samples: int,
                           num_rand_blocks: int, t_prob: float, tr_prob: float, u_prob: float,
                           index_map: torch.Tensor | None = None, weight_map: torch.Tensor | None = None,
                           seed: int | None = None, add_residual: bool = True,
                           workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                           fixup_sum_limit: float = 0.0):
  """GridSelfAttention on ``z [N, N, C]`` with block-sparse (IBS) attention rows; returns
  ``(out, index_map, weight_map)``, maps int32 / float32 ``[N, H, ceil(N/32), num_samples]``.
  Given maps (both or neither, as backends/vecops/kernels/registry.py:2985-3002 requires) are
  reused; otherwise they are sampled with ``seed`` (default: the next value of a process-wide
  counter).  ``fixup_sum_limit`` > 0 lowers the weight-sum limit above which a (row, head) is
  recomputed by the exact block-sparse kernel (0 = the default 2^100)."""
  _require_cuda(z, seq_mask, ln_w, ln_b, w_qkvgb, w_o, workspace, index_map, weight_map)
  _require(fixup_sum_limit >= 0.0, "triangle_ibs: fixup_sum_limit must be >= 0")
  _require(z.ndim == 3 and z.shape[0] == z.shape[1], f"triangle_ibs: z must be [N, N, C], got {tuple(z.shape)}")
  _require((index_map is None) == (weight_map is None), "index_map and weight_map must be both present or both omitted")
  N, _, Cn = z.shape
  HD = w_o.shape[1]
  _require(HD % num_head == 0, "triangle_ibs: output projection width not divisible by heads")
  D = HD // num_head
  _require(tuple(w_qkvgb.shape) == (4 * HD + num_head, Cn), f"triangle_ibs: w_qkvgb shape {tuple(w_qkvgb.shape)}")
  _require(tuple(w_o.shape) == (Cn, HD), f"triangle_ibs: w_o shape {tuple(w_o.shape)}")
  _require(seq_mask.shape == (N,), "triangle_ibs: seq_mask must be [N]")
  need = triangle_ibs_workspace_bytes(N, Cn, num_head, D)
  _require(need > 0, f"triangle_ibs: unsupported sizes N={N} C={Cn} H={num_head} D={D} "
           "(block-sparse rows need C = 128, H = 4, D = 32, N <= 8192)")
  T = (N + 31) // 32
  shape = (N, num_head, T, int(num_samples))
  generate = index_map is None
  if generate:
    index_map = torch.empty(shape, dtype=torch.int32, device=z.device)
    weight_map = torch.empty(shape, dtype=torch.float32, device=z.device)
  else:
    _require(tuple(index_map.shape) == shape and tuple(weight_map.shape) == shape,
             f"triangle_ibs: maps must be {shape}, got {tuple(index_map.shape)} / {tuple(weight_map.shape)}")
    _require(index_map.dtype == torch.int32 and weight_map.dtype == torch.float32,
             "triangle_ibs: index_map int32 and weight_map float32")
    index_map, weight_map = index_map.contiguous(), weight_map.contiguous()
  zc = _bf16(z).contiguous()
  m8 = _u8(seq_mask).contiguous()
  lw, lb = _f32(ln_w), _f32(ln_b)
  if workspace is None or workspace.numel() < need:
    workspace = torch.empty(need, dtype=torch.uint8, device=z.device)
  if out is None:
    out = torch.empty_like(zc)
  a = _lib.TriangleArgs()
  a.N, a.C, a.H, a.D = N, Cn, num_head, D
  a.transpose, a.add_residual = int(bool(transpose)), int(bool(add_residual))
  a.z, a.seq_mask, a.ln_w, a.ln_b = _vp(zc), _vp(m8), _vp(lw), _vp(lb)
  a.w_qkvgb, a.w_o, a.out = _vp(w_qkvgb), _vp(w_o), _vp(out)
  a.fixup_sum_limit = float(fixup_sum_limit)
  p = _lib.IbsArgs()
  p.num_samples, p.num_rand_blocks = int(num_samples), int(num_rand_blocks)
  p.t_prob, p.tr_prob, p.u_prob = float(t_prob), float(tr_prob), float(u_prob)
  p.generate_maps = int(generate)
  p.seed = (next(_ibs_seed_counter) if seed is None else int(seed)) & ((1 << 64) - 1)
  p.index_map, p.weight_map = _vp(index_map), _vp(weight_map)
  rc = _lib.load().sf_hip_triangle_attn_ibs_fwd(C.byref(a), C.byref(p), _vp(workspace), workspace.numel(), _stream(z))
  _lib.check(rc, "sf_hip_triangle_attn_ibs_fwd")
  return out, index_map, weight_map


def default_scale(d: int) -> float:
  return 1.0 / math.sqrt(d)


# ---------------------------------------------------------------------------------------
# whole attention modules (one C call each; see sf_hip_self_attention_fwd /
# sf_hip_cross_attention_fwd)
# ---------------------------------------------------------------------------------------

def _u8_or_none(t):
  return None if t is None else _u8(t).contiguous()


def self_attention_module(x: torch.Tensor, mask, bias, cond, w: dict, *, num_head: int, head_dim: int,
                          add_residual: bool = True, pre=None, noalloc: bool = False) -> torch.Tensor:
  """SelfAttention.forward as one call.  ``x`` ``[..., N, C]`` (leading dims = samples),
  ``mask`` ``[N]`` or None, ``bias`` ``[H, N, N]`` (shared) or ``[S, H, N, N]`` or None,
  ``cond`` ``[N, Cs]`` or None; ``w`` holds the packed weights (keys as in the C struct).
  ``pre`` = (scale, shift, zgate) ``[N, C]`` views with one row stride (one layer of
  ``diffusion_conditioning``) replaces the AdaLN computation from ``cond``.  ``noalloc`` runs
  the allocation-free entry point (the library's fixed per-GPU scratch; no workspace)."""
  _require_cuda(x, mask, bias, cond, *(pre or ()))
  N, Cn = x.shape[-2], x.shape[-1]
  S = x.numel() // max(N * Cn, 1)
  H, D = num_head, head_dim
  x3 = _bf16(x).reshape(S, N, Cn).contiguous()
  out = torch.empty_like(x3)
  a = _lib.SelfAttentionArgs()
  a.S, a.N, a.C, a.H, a.D = S, N, Cn, H, D
  a.scale, a.add_residual = 0.0, int(bool(add_residual))
  a.x, a.out = _vp(x3), _vp(out)
  m8 = _u8_or_none(mask)
  a.mask = _vp(m8)
  if bias is not None:
    b = _bf16(bias)
    _require(b.stride(-1) == 1, "self_attention: bias keys must be contiguous")
    if b.dim() == 3:
      a.bias_s[0], a.bias_s[1], a.bias_s[2] = 0, b.stride(0), b.stride(1)
    else:
      a.bias_s[0], a.bias_s[1], a.bias_s[2] = b.stride(0), b.stride(1), b.stride(2)
    a.bias = _vp(b)
  c2 = None
  if cond is not None:
    c2 = _bf16(cond).contiguous()
    a.cond, a.Cs = _vp(c2), c2.shape[-1]
  for key in ("ln_w", "ln_b", "lnc_w", "lnc_b", "w_scale", "b_scale", "w_shift", "w_qkvg", "b_qkvg",
              "w_t2", "w_zc", "b_zc"):
    setattr(a, key, _vp(w.get(key)))
  if pre is not None:
    ps, pb, pz = pre
    rs = ps.stride(0)
    for t in pre:
      _require(t.dtype == torch.bfloat16 and tuple(t.shape) == (N, Cn) and t.stride() == (rs, 1),
               "self_attention: precomputed conditioning must be bf16 [N, C] views with one row stride")
    a.pre_scale, a.pre_shift, a.pre_zgate, a.pre_rs = _vp(ps), _vp(pb), _vp(pz), rs
  lib = _lib.load()
  if noalloc:      # the library's fixed per-GPU scratch instead of a workspace
    _lib.check(lib.sf_hip_self_attention_fwd_noalloc(C.byref(a), _stream(x)), "sf_hip_self_attention_fwd_noalloc")
    return out.view(x.shape)
  ws = torch.empty(int(lib.sf_hip_self_attention_workspace_bytes(C.byref(a))), dtype=torch.uint8, device=x.device)
  _lib.check(lib.sf_hip_self_attention_fwd(C.byref(a), _vp(ws), ws.numel(), _stream(x)), "sf_hip_self_attention_fwd")
  return out.view(x.shape)


def transition_module(x: torch.Tensor, cond, w: dict, *, add_residual: bool = True, pre=None) -> torch.Tensor:
  """A transition block as one call (sf_hip_transition_fwd).  ``x`` ``[..., N, C]`` (leading dims =
  samples sharing the condition), ``cond`` ``[N, Cs]`` or None; ``w`` holds the packed weights
  (``w1`` ``[2I, C]`` interleaved, ``w2`` ``[C, I]``, LayerNorm / AdaLN / zero-gate terms as in
  the C struct).  ``pre`` = (scale, shift, zgate) ``[N, C]`` views with one row stride."""
  _require_cuda(x, cond, *(pre or ()))
  N, Cn = x.shape[-2], x.shape[-1]
  S = x.numel() // max(N * Cn, 1)
  w1, w2 = w["w1"], w["w2"]
  I = w2.shape[1]
  _require(tuple(w1.shape) == (2 * I, Cn) and tuple(w2.shape) == (Cn, I), "transition: weight shapes")
  x3 = _bf16(x).reshape(S, N, Cn).contiguous()
  out = torch.empty_like(x3)
  a = _lib.TransitionArgs()
  a.S, a.N, a.C, a.I = S, N, Cn, I
  a.add_residual = int(bool(add_residual))
  a.x, a.out = _vp(x3), _vp(out)
  c2 = None
  if cond is not None and pre is None:
    c2 = _bf16(cond).contiguous()
    _require(tuple(c2.shape[:-1]) == (N,), "transition: cond must be [N, Cs]")
    a.cond, a.Cs = _vp(c2), c2.shape[-1]
  for key in ("ln_w", "ln_b", "lnc_w", "lnc_b", "w_scale", "b_scale", "w_shift", "w1", "w2", "w_zc", "b_zc"):
    setattr(a, key, _vp(w.get(key)))
  if pre is not None:
    ps, pb, pz = pre
    rs = ps.stride(0)
    for t in pre:
      _require(t.dtype == torch.bfloat16 and tuple(t.shape) == (N, Cn) and t.stride() == (rs, 1),
               "transition: precomputed conditioning must be bf16 [N, C] views with one row stride")
    a.pre_scale, a.pre_shift, a.pre_zgate, a.pre_rs = _vp(ps), _vp(pb), _vp(pz), rs
  lib = _lib.load()
  ws = torch.empty(int(lib.sf_hip_transition_workspace_bytes(C.byref(a))), dtype=torch.uint8, device=x.device)
  _lib.check(lib.sf_hip_transition_fwd(C.byref(a), _vp(ws), ws.numel(), _stream(x)), "sf_hip_transition_fwd")
  return out.view(x.shape)


def cross_attention_module(xq: torch.Tensor, xk, gather_idx, gather_mask, mask_q, mask_k, bias, cond_q, cond_k,
                           w: dict, *, num_head: int, head_dim: int, add_residual: bool = True,
                           pre: dict | None = None) -> torch.Tensor:
  """CrossAttention.forward as one call.  ``xq`` ``[..., U, Qw, C]``; keys either ``xk``
  ``[..., U, Kw, C]`` or gathered from the query rows by ``gather_idx`` / ``gather_mask``
  ``[U, Kw]``; masks ``[U, Qw]`` / ``[U, Kw]``; ``bias`` ``[U, H, Qw, Kw]``; conditions
  ``[U, Qw, C]`` / ``[U, Kw, C]``.  ``pre`` (with ``gather_idx``): the per-atom plan -- the
  keys' condition is the gathered queries', and ``pre`` holds both sides' AdaLN terms per atom
  (``q_scale``, ``q_shift``, ``k_scale``, ``k_shift``, ``zgate``: ``[U*Qw, C]`` views with one
  row stride, as cross_conditioning returns them); the conditions are then not read."""
  _require_cuda(xq, xk, gather_idx, gather_mask, mask_q, mask_k, bias, cond_q, cond_k,
                *([] if pre is None else pre.values()))
  _require(pre is None or gather_idx is not None, "cross_attention: the per-atom plan gathers its keys")
  U, Qw, Cn = xq.shape[-3:]
  S = xq.numel() // max(U * Qw * Cn, 1)
  Kw = gather_idx.shape[-1] if gather_idx is not None else xk.shape[-2]
  xq4 = _bf16(xq).reshape(S, U, Qw, Cn).contiguous()
  out = torch.empty_like(xq4)
  a = _lib.CrossAttentionArgs()
  a.S, a.U, a.Qw, a.Kw, a.C, a.H, a.D = S, U, Qw, Kw, Cn, num_head, head_dim
  a.scale, a.add_residual = 0.0, int(bool(add_residual))
  a.xq, a.out = _vp(xq4), _vp(out)
  keep = []
  if gather_idx is not None:
    idx32 = gather_idx.reshape(-1).to(torch.int32).contiguous()
    gm8 = _u8(gather_mask.reshape(-1)).contiguous()
    _require(idx32.numel() == U * Kw and gm8.numel() == U * Kw, "cross_attention: gather sizes")
    a.gather_idx, a.gather_mask = _vp(idx32), _vp(gm8)
    keep += [idx32, gm8]
  else:
    xk4 = _bf16(xk).reshape(S, U, Kw, Cn).contiguous()
    a.xk = _vp(xk4)
    keep.append(xk4)
  mq8, mk8 = _u8_or_none(mask_q), _u8_or_none(mask_k)
  a.mask_q, a.mask_k = _vp(mq8), _vp(mk8)
  b = None if bias is None else _bf16(bias).contiguous()
  a.bias = _vp(b)
  if pre is None:
    cq, ck = _bf16(cond_q).contiguous(), _bf16(cond_k).contiguous()
    a.cond_q, a.cond_k = _vp(cq), _vp(ck)
  else:
    terms = [pre[k] for k in ("q_scale", "q_shift", "k_scale", "k_shift", "zgate")]
    rs = terms[0].stride(0)
    for t in terms:
      _require(t.dtype == torch.bfloat16 and tuple(t.shape) == (U * Qw, Cn) and t.stride() == (rs, 1),
               "cross_attention: pre terms must be bf16 [U*Qw, C] views with one row stride")
    a.pre_q_scale, a.pre_q_shift, a.pre_k_scale, a.pre_k_shift, a.pre_zgate = (_vp(t) for t in terms)
    a.pre_rs = rs
  for key in ("lnc_w_q", "lnc_b_q", "w_scale_q", "b_scale_q", "w_shift_q", "lnc_w_k", "lnc_b_k", "w_scale_k",
              "b_scale_k", "w_shift_k", "w_qg", "b_qg", "w_kv", "w_t2", "w_zc", "b_zc"):
    setattr(a, key, _vp(w.get(key)))
  lib = _lib.load()
  ws = torch.empty(int(lib.sf_hip_cross_attention_workspace_bytes(C.byref(a))), dtype=torch.uint8, device=xq.device)
  _lib.check(lib.sf_hip_cross_attention_fwd(C.byref(a), _vp(ws), ws.numel(), _stream(xq)), "sf_hip_cross_attention_fwd")
  return out.view(xq.shape)


def diffusion_conditioning(cond: torch.Tensor, lnc_w: torch.Tensor, w_scale: torch.Tensor, b_scale, w_shift: torch.Tensor,
                           w_zc: torch.Tensor, b_zc) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
  """AdaLN conditioning of L layers from one condition, one call (sf_hip_diffusion_conditioning_fwd;
  the reference's diffusion_conditioning_packed, backends/vecops/kernels/registry.py:720-760).
  ``cond`` ``[..., N, Cs]``; ``lnc_w`` f32 ``[L, Cs]``; weights bf16 ``[L*C, Cs]``; biases f32
  ``[L*C]``.  Returns (scale, shift, zgate), each ``[L, rows, C]`` (rows = cond's leading dims x N)
  as per-layer views of one ``[rows, L*C]`` buffer; scale and zgate after the sigmoid."""
  _require_cuda(cond, lnc_w, w_scale, b_scale, w_shift, w_zc, b_zc)
  L, Cs = lnc_w.shape
  LC = w_scale.shape[0]
  _require(LC % L == 0 and cond.shape[-1] == Cs, "diffusion_conditioning: shapes do not match")
  Cn = LC // L
  for t, n in ((w_scale, "w_scale"), (w_shift, "w_shift"), (w_zc, "w_zc")):
    _require(tuple(t.shape) == (LC, Cs) and t.dtype == torch.bfloat16 and t.is_contiguous(),
             f"diffusion_conditioning: {n} must be contiguous bf16 [L*C, Cs]")
  c2 = _bf16(cond).reshape(-1, Cs).contiguous()
  rows = c2.shape[0]
  outs = [torch.empty(rows, LC, dtype=torch.bfloat16, device=cond.device) for _ in range(3)]
  a = _lib.DiffusionConditioningArgs()
  a.rows, a.L, a.C, a.Cs = rows, L, Cn, Cs
  g = lnc_w.float().contiguous()
  bs = None if b_scale is None else b_scale.float().contiguous()
  bz = None if b_zc is None else b_zc.float().contiguous()
  a.cond, a.lnc_w, a.w_scale, a.b_scale, a.w_shift = _vp(c2), _vp(g), _vp(w_scale), _vp(bs), _vp(w_shift)
  a.w_zc, a.b_zc = _vp(w_zc), _vp(bz)
  a.scale, a.shift, a.zgate, a.out_rs = _vp(outs[0]), _vp(outs[1]), _vp(outs[2]), LC
  lib = _lib.load()
  ws = torch.empty(int(lib.sf_hip_diffusion_conditioning_workspace_bytes(C.byref(a))), dtype=torch.uint8,
                   device=cond.device)
  _lib.check(lib.sf_hip_diffusion_conditioning_fwd(C.byref(a), _vp(ws), ws.numel(), _stream(cond)),
             "sf_hip_diffusion_conditioning_fwd")
  return tuple(o.view(rows, L, Cn).transpose(0, 1) for o in outs)


def triangle_multiplication(z: torch.Tensor, mask, w: dict, *, incoming: bool, add_residual: bool = True) -> torch.Tensor:
  """TriangleMultiplication.forward (blocks.py:486-566) as one call (sf_hip_triangle_mult_fwd).
  ``z`` ``[N, N, 128]``, ``mask`` ``[N]`` bool or None; ``w`` holds the packed weights (keys as in
  the C struct)."""
  _require_cuda(z, mask)
  _require(z.dim() == 3 and z.shape[0] == z.shape[1], "triangle_multiplication: z must be [N, N, C]")
  N, Cn = z.shape[0], z.shape[2]
  z3 = _bf16(z).contiguous()
  out = torch.empty_like(z3)
  lib = _lib.load()
  ws_bytes = int(lib.sf_hip_triangle_mult_workspace_bytes(N, Cn))
  _require(ws_bytes > 0, f"triangle_multiplication: unsupported sizes N={N} C={Cn} (C must be 128)")
  a = _lib.TriangleMultArgs()
  a.N, a.C, a.incoming, a.add_residual = N, Cn, int(bool(incoming)), int(bool(add_residual))
  m8 = _u8_or_none(mask)
  a.z, a.mask, a.out = _vp(z3), _vp(m8), _vp(out)
  for key in ("ln_w", "ln_b", "w_glu", "cn_w", "cn_b", "w_out", "w_gate"):
    setattr(a, key, _vp(w.get(key)))
  ws = torch.empty(ws_bytes, dtype=torch.uint8, device=z.device)
  _lib.check(lib.sf_hip_triangle_mult_fwd(C.byref(a), _vp(ws), ws.numel(), _stream(z)), "sf_hip_triangle_mult_fwd")
  return out.to(z.dtype) if z.dtype != torch.bfloat16 else out
