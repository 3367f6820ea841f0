"""ctypes binding of ``libsparsefold_hip.so`` (the C ABI declared in include/sparsefold_hip.h).

The structures below mirror the header field for field; ``tests/test_abi.py`` compiles the
header with gcc and checks every size and offset against these definitions.  Loading fails
loudly: there is no fallback implementation behind this module.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsparsefold_hip.so"
ABI_VERSION = 11
TRI_STAGE_PROJECT, TRI_STAGE_ATTEND, TRI_STAGE_OUTPUT, TRI_STAGE_ALL, TRI_STAGE_FUSE = 1, 2, 4, 7, 8
NOALLOC_SCRATCH_BYTES = 64 << 20           # SF_HIP_NOALLOC_SCRATCH_BYTES

_i32, _i64, _f32, _vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p
_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)


class AttentionArgs(C.Structure):
  _fields_ = [
      ("B0", _i32), ("B1", _i32), ("Q", _i32), ("K", _i32), ("H", _i32), ("D", _i32), ("Dv", _i32),
      ("scale", _f32),
      ("q", _vp), ("q_s", _i64 * 4),
      ("k", _vp), ("k_s", _i64 * 4),
      ("v", _vp), ("v_s", _i64 * 4),
      ("bias", _vp), ("bias_s", _i64 * 4),
      ("mask_q", _vp), ("mq_s", _i64 * 3),
      ("mask_k", _vp), ("mk_s", _i64 * 3),
      ("gate", _vp), ("g_s", _i64 * 4),
      ("out", _vp), ("o_s", _i64 * 4),
      ("schedule", _i32),
      ("kv_index", _vp), ("kv_mask", _vp), ("kvi_s", _i64), ("kv_zero_row", _i32),
  ]


class LayerNormArgs(C.Structure):
  _fields_ = [
      ("M", _i64), ("C", _i32), ("eps", _f32),
      ("x", _vp), ("x_rs", _i64),
      ("gamma", _vp), ("beta", _vp),
      ("scale", _vp), ("shift", _vp),
      ("cond_rows", _i64), ("cond_rs", _i64),
      ("y", _vp), ("y_rs", _i64),
      ("gather_idx", _vp), ("gather_mask", _vp), ("gather_rows", _i64), ("gather_src_rows", _i64),
  ]


class LinearArgs(C.Structure):
  _fields_ = [
      ("M", _i64), ("N", _i32), ("K", _i32),
      ("x", _vp), ("x_rs", _i64),
      ("wt", _vp),
      ("bias", _vp),
      ("residual", _vp), ("r_rs", _i64),
      ("mul", _vp), ("mul_rows", _i64), ("mul_rs", _i64),
      ("post_sigmoid", _i32),
      ("y", _vp), ("y_rs", _i64), ("ycols", _i32),
      ("tcol0", _i32), ("tcols", _i32), ("yt", _vp), ("yt_rs", _i64),
      ("glu", _i32),
      ("batch", _i32), ("x_bs", _i64), ("w_bs", _i64), ("y_bs", _i64),
  ]


class TriangleArgs(C.Structure):
  _fields_ = [
      ("N", _i32), ("C", _i32), ("H", _i32), ("D", _i32),
      ("transpose", _i32), ("add_residual", _i32),
      ("z", _vp), ("seq_mask", _vp),
      ("ln_w", _vp), ("ln_b", _vp),
      ("w_qkvgb", _vp), ("w_o", _vp),
      ("out", _vp),
      ("fixup_sum_limit", _f32),
  ]


class IbsArgs(C.Structure):
  _fields_ = [
      ("num_samples", _i32), ("num_rand_blocks", _i32),
      ("t_prob", _f32), ("tr_prob", _f32), ("u_prob", _f32),
      ("generate_maps", _i32), ("seed", C.c_uint64),
      ("index_map", _vp), ("weight_map", _vp),
  ]


class PairLogitsArgs(C.Structure):
  _fields_ = [
      ("P", _i64), ("C", _i32), ("H", _i32),
      ("z", _vp), ("ln_w", _vp), ("ln_b", _vp), ("w_t", _vp), ("out", _vp),
      ("seg", _i64), ("group", _i32), ("reserved", _i32),
  ]


class WindowGatherArgs(C.Structure):
  _fields_ = [
      ("S", _i32), ("rows", _i32), ("C", _i32), ("UK", _i32),
      ("src", _vp), ("idx", _vp), ("mask", _vp), ("keys", _vp),
  ]


class SelfAttentionArgs(C.Structure):
  _fields_ = [
      ("S", _i32), ("N", _i32), ("C", _i32), ("H", _i32), ("D", _i32), ("Cs", _i32),
      ("scale", _f32), ("add_residual", _i32),
      ("x", _vp), ("mask", _vp), ("bias", _vp), ("bias_s", _i64 * 3), ("cond", _vp),
      ("ln_w", _vp), ("ln_b", _vp), ("lnc_w", _vp), ("lnc_b", _vp),
      ("w_scale", _vp), ("b_scale", _vp), ("w_shift", _vp),
      ("w_qkvg", _vp), ("b_qkvg", _vp), ("w_t2", _vp), ("w_zc", _vp), ("b_zc", _vp),
      ("out", _vp),
      ("pre_scale", _vp), ("pre_shift", _vp), ("pre_zgate", _vp), ("pre_rs", _i64),
  ]


class CrossAttentionArgs(C.Structure):
  _fields_ = [
      ("S", _i32), ("U", _i32), ("Qw", _i32), ("Kw", _i32), ("C", _i32), ("H", _i32), ("D", _i32),
      ("scale", _f32), ("add_residual", _i32),
      ("xq", _vp), ("xk", _vp), ("gather_idx", _vp), ("gather_mask", _vp),
      ("mask_q", _vp), ("mask_k", _vp), ("bias", _vp), ("cond_q", _vp), ("cond_k", _vp),
      ("lnc_w_q", _vp), ("lnc_b_q", _vp), ("w_scale_q", _vp), ("b_scale_q", _vp), ("w_shift_q", _vp),
      ("lnc_w_k", _vp), ("lnc_b_k", _vp), ("w_scale_k", _vp), ("b_scale_k", _vp), ("w_shift_k", _vp),
      ("w_qg", _vp), ("b_qg", _vp), ("w_kv", _vp), ("w_t2", _vp), ("w_zc", _vp), ("b_zc", _vp),
      ("out", _vp),
      ("pre_q_scale", _vp), ("pre_q_shift", _vp), ("pre_k_scale", _vp), ("pre_k_shift", _vp),
      ("pre_zgate", _vp), ("pre_rs", _i64),
  ]


class DiffusionConditioningArgs(C.Structure):
  _fields_ = [
      ("rows", _i64), ("L", _i32), ("C", _i32), ("Cs", _i32),
      ("cond", _vp), ("lnc_w", _vp), ("w_scale", _vp), ("b_scale", _vp), ("w_shift", _vp),
      ("w_zc", _vp), ("b_zc", _vp), ("scale", _vp), ("shift", _vp), ("zgate", _vp), ("out_rs", _i64),
  ]


class TransitionArgs(C.Structure):
  _fields_ = [
      ("S", _i32), ("N", _i32), ("C", _i32), ("I", _i32), ("Cs", _i32), ("add_residual", _i32),
      ("x", _vp), ("cond", _vp), ("ln_w", _vp), ("ln_b", _vp), ("lnc_w", _vp), ("lnc_b", _vp),
      ("w_scale", _vp), ("b_scale", _vp), ("w_shift", _vp), ("w1", _vp), ("w2", _vp),
      ("w_zc", _vp), ("b_zc", _vp), ("out", _vp),
      ("pre_scale", _vp), ("pre_shift", _vp), ("pre_zgate", _vp), ("pre_rs", _i64),
  ]


class TriangleMultArgs(C.Structure):
  _fields_ = [
      ("N", _i32), ("C", _i32), ("incoming", _i32), ("add_residual", _i32),
      ("z", _vp), ("mask", _vp), ("ln_w", _vp), ("ln_b", _vp), ("w_glu", _vp),
      ("cn_w", _vp), ("cn_b", _vp), ("w_out", _vp), ("w_gate", _vp), ("out", _vp),
  ]


STRUCTS = {
    "sf_attention_args": AttentionArgs,
    "sf_layer_norm_args": LayerNormArgs,
    "sf_linear_args": LinearArgs,
    "sf_triangle_args": TriangleArgs,
    "sf_ibs_args": IbsArgs,
    "sf_pair_logits_args": PairLogitsArgs,
    "sf_window_gather_args": WindowGatherArgs,
    "sf_self_attention_args": SelfAttentionArgs,
    "sf_cross_attention_args": CrossAttentionArgs,
    "sf_diffusion_conditioning_args": DiffusionConditioningArgs,
    "sf_triangle_mult_args": TriangleMultArgs,
    "sf_transition_args": TransitionArgs,
}

# (name, restype, argtypes) of every exported entry point.
SIGNATURES = [
    ("sf_hip_abi_version", C.c_int, []),
    ("sf_hip_last_error", C.c_size_t, [C.c_char_p, C.c_size_t]),
    ("sf_hip_attention_fwd", C.c_int, [C.POINTER(AttentionArgs), _vp]),
    ("sf_hip_layer_norm_fwd", C.c_int, [C.POINTER(LayerNormArgs), _vp]),
    ("sf_hip_linear_fwd", C.c_int, [C.POINTER(LinearArgs), _vp]),
    ("sf_hip_triangle_workspace_bytes", C.c_size_t, [_i32, _i32, _i32, _i32]),
    ("sf_hip_triangle_attn_fwd", C.c_int, [C.POINTER(TriangleArgs), _vp, C.c_size_t, _vp]),
    ("sf_hip_triangle_stage_fwd", C.c_int, [C.POINTER(TriangleArgs), _i32, _vp, C.c_size_t, _vp]),
    ("sf_hip_triangle_ibs_workspace_bytes", C.c_size_t, [_i32, _i32, _i32, _i32]),
    ("sf_hip_triangle_attn_ibs_fwd", C.c_int, [C.POINTER(TriangleArgs), C.POINTER(IbsArgs), _vp, C.c_size_t, _vp]),
    ("sf_hip_pair_logits_fwd", C.c_int, [C.POINTER(PairLogitsArgs), _vp]),
    ("sf_hip_window_gather_fwd", C.c_int, [C.POINTER(WindowGatherArgs), _vp]),
    ("sf_hip_self_attention_workspace_bytes", C.c_size_t, [C.POINTER(SelfAttentionArgs)]),
    ("sf_hip_self_attention_fwd", C.c_int, [C.POINTER(SelfAttentionArgs), _vp, C.c_size_t, _vp]),
    ("sf_hip_self_attention_fwd_noalloc", C.c_int, [C.POINTER(SelfAttentionArgs), _vp]),
    ("sf_hip_cross_attention_workspace_bytes", C.c_size_t, [C.POINTER(CrossAttentionArgs)]),
    ("sf_hip_cross_attention_fwd", C.c_int, [C.POINTER(CrossAttentionArgs), _vp, C.c_size_t, _vp]),
    ("sf_hip_diffusion_conditioning_workspace_bytes", C.c_size_t, [C.POINTER(DiffusionConditioningArgs)]),
    ("sf_hip_diffusion_conditioning_fwd", C.c_int, [C.POINTER(DiffusionConditioningArgs), _vp, C.c_size_t, _vp]),
    ("sf_hip_transition_workspace_bytes", C.c_size_t, [C.POINTER(TransitionArgs)]),
    ("sf_hip_transition_fwd", C.c_int, [C.POINTER(TransitionArgs), _vp, C.c_size_t, _vp]),
    ("sf_hip_triangle_mult_workspace_bytes", C.c_size_t, [_i32, _i32]),
    ("sf_hip_triangle_mult_fwd", C.c_int, [C.POINTER(TriangleMultArgs), _vp, C.c_size_t, _vp]),
]

_lib: C.CDLL | None = None


def load() -> C.CDLL:
  """Loads the HIP library once; raises RuntimeError when it is missing or mismatched."""
  global _lib
  if _lib is not None:
    return _lib
  if not LIB_PATH.exists():
    raise RuntimeError(f"{LIB_PATH.name} is not built; run __graft_entry__.build() or "
                       "python -m sparsefold_amd._build (no fallback implementation exists)")
  lib = C.CDLL(str(LIB_PATH))
  for name, res, args in SIGNATURES:
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = args
  ver = lib.sf_hip_abi_version()
  if ver != ABI_VERSION:
    raise RuntimeError(f"libsparsefold_hip ABI version {ver} != expected {ABI_VERSION}")
  _lib = lib
  return lib


def last_error() -> str:
  lib = load()
  buf = C.create_string_buffer(1024)
  lib.sf_hip_last_error(buf, len(buf))
  return buf.value.decode(errors="replace")


def check(rc: int, what: str) -> None:
  if rc != 0:
    raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")
