"""Parameter-layout mirrors of the reference attention modules.

Each class has the reference constructor signature and registers the same sub-modules and
parameters (names and shapes), so a reference ``state_dict`` loads strictly.  They carry no
compute of their own: ``forward`` is provided by the HIP backend, which ``backends.init()``
installs over these factories (exactly as the reference's vecops ``apply()`` replaces module
factories, ``src/sparsefold/backends/vecops/backend.py:187-248``).  Calling ``forward`` on an
unreplaced class raises.

Mirrored layouts (reference file:line):
* ``Linear``            primitives.py:178-280 -- weight ``[*in, *out]``, or ``[*out, *in]``
                        with ``transpose_weights``; optional bias ``[*out]``
* ``LayerNorm``         primitives.py:375-430 -- weight ``[C]``, optional bias ``[C]``
* ``GridSelfAttention`` blocks.py:188-267; with it the block-sparse parameters and map reuse
                        (``IBSAParameters``, ``IndexReuser``, ``default_reuse_policy``,
                        blocks.py:368-422) and ``layer_stack_indices`` (primitives.py:535)
* ``AdaptiveLayerNorm`` / ``AdaptiveZeroInit`` / ``SelfAttention`` transformer.py:27-304
* ``CrossAttention``    transformer.py:480-547
* ``SingleActUpdate``   blocks.py:692-737 (pair-logit prologue, single attention and, with a
                        ``transition_config``, the single transition)
* ``TransitionBlock``   blocks.py:38-96 (trunk transition)
* ``DiffusionTransitionBlock`` transformer.py:157-231 (the diffusion transformer's transition)
* ``TransformerPairLogits``         transformer.py:398-419 -- the pair-conditioning sub-modules
                        of ``Transformer`` (``pair_input_layer_norm``, ``pair_logits_projection``)
* ``CrossAttTransformerPairLogits`` transformer.py:611-620 -- the same for ``CrossAttTransformer``
  (the self-attention / transition stacks of both are outside the attention path; parameter
  names match, so those keys of a reference ``state_dict`` load into these mirrors)
"""
from __future__ import annotations

import dataclasses
import numbers
from collections.abc import Callable, Sequence
from typing import Any

import torch


@dataclasses.dataclass
class GlobalConfig:
  """model/config.py:15-27 (the fields the attention modules read)."""
  bfloat16: str = "all"
  final_init: str = "zeros"
  pair_attention_chunk_size: Sequence = ((1536, 128), (None, 32))


def _shape(x) -> tuple[int, ...]:
  return (int(x),) if isinstance(x, numbers.Integral) else tuple(int(v) for v in x)


class Linear(torch.nn.Module):
  def __init__(self, num_input, num_output, *, bias: bool = False, transpose_weights: bool = False,
               dtype: torch.dtype | None = None, device=None, name: str | None = None, **_):
    super().__init__()
    self.name = name
    self.input_shape, self.output_shape = _shape(num_input), _shape(num_output)
    self.transpose_weights = transpose_weights
    self.use_bias = bias
    ws = self.output_shape + self.input_shape if transpose_weights else self.input_shape + self.output_shape
    self.weight = torch.nn.Parameter(torch.empty(ws, dtype=dtype or torch.float32, device=device))
    if bias:
      self.bias = torch.nn.Parameter(torch.empty(self.output_shape, dtype=dtype or torch.float32, device=device))
    else:
      self.register_parameter("bias", None)


class LayerNorm(torch.nn.Module):
  def __init__(self, normalized_shape: int, *, eps: float = 1e-5, elementwise_affine: bool = True,
               bias: bool = True, dtype=None, device=None, name: str | None = None):
    super().__init__()
    self.name = name
    self.eps = eps
    self.normalized_shape = _shape(normalized_shape)
    if elementwise_affine:
      self.weight = torch.nn.Parameter(torch.empty(self.normalized_shape, dtype=dtype or torch.float32, device=device))
      if bias:
        self.bias = torch.nn.Parameter(torch.empty(self.normalized_shape, dtype=dtype or torch.float32, device=device))
      else:
        self.register_parameter("bias", None)
    else:
      self.register_parameter("weight", None)
      self.register_parameter("bias", None)


# ---------------------------------------------------------------------------------------
# Block-sparse (IBS) grid attention parameters and map reuse (blocks.py:368-422).  Index and
# weight maps of one layer can be reused by another: the policy maps a layer's stack indices to
# those of the layer whose maps it takes (None: sample new ones).
# ---------------------------------------------------------------------------------------

# Indices of the layer being run inside nested layer stacks (primitives.py:535); a layer-stack
# runner sets the last entry per layer.
layer_stack_indices: list[int] = []

IndexReusePolicy = Callable[[tuple[int, ...]], "tuple[int, ...] | None"]


def _normalize_slice(indices) -> tuple[int, ...]:
  if isinstance(indices, Sequence):
    return tuple(int(x) for x in indices)
  return (int(indices),)


def default_reuse_policy(indices) -> tuple[int, ...] | None:
  """No reuse (blocks.py:376-377)."""
  return None


class IndexReuser:
  """Maps kept per layer (blocks.py:379-403); ``get`` returns (maps or None, source indices)."""

  def __init__(self, policy: IndexReusePolicy):
    self.policy = policy
    self.cached_indices: dict[tuple[int, ...], Any] = {}

  def get(self, indices):
    from sparsefold_amd.runtime import config
    if not config.enable_gsa_index_reuse:
      return None, None
    target = self.policy(_normalize_slice(indices))
    if target is None:
      return None, None
    target = _normalize_slice(target)
    return self.cached_indices.get(target), target

  def set(self, indices, maps) -> None:
    self.cached_indices[_normalize_slice(indices)] = maps


@dataclasses.dataclass(frozen=True)
class IBSAParameters:
  """Index-based sparse attention parameters (blocks.py:405-418)."""
  num_samples: int = 16
  num_rand_blocks: int = 6
  t_prob: float = 0.90
  tr_prob: float = 0.95
  u_prob: float = 0.02

  @classmethod
  def default(cls, *args, **kwargs) -> "IBSAParameters":
    """The runtime's ``sparse_attention_parameters`` over the field defaults."""
    from sparsefold_amd.runtime import config
    return cls(**config.sparse_attention_parameters)


IBSAParametersProvider = Callable[[tuple[int, ...]], IBSAParameters]
IBSAParametersOrProvider = "IBSAParameters | IBSAParametersProvider"


class _NoTorchPath:
  def forward(self, *args, **kwargs):
    raise RuntimeError(f"{type(self).__name__} has no Torch compute path in this package; "
                       "configure_runtime(backend='hip') and backends.init() before constructing it")


class GridSelfAttention(_NoTorchPath, torch.nn.Module):
  """blocks.py:188-267: triangle attention, starting (transpose=False) / ending node."""

  @dataclasses.dataclass
  class Config:
    num_head: int = 4

  def __init__(self, config: Config, global_config: GlobalConfig, transpose: bool, *, num_channels: int,
               distributed: bool = False, name: str = "", **kwargs):
    super().__init__()
    self.name = name
    self.distributed = False
    if distributed:
      raise ValueError("GridSelfAttention: the multi-rank path is not part of this build")
    self.transpose = transpose
    self.config = config
    self.num_channels = num_channels
    self.pair_attention_chunk_size = global_config.pair_attention_chunk_size
    assert num_channels % config.num_head == 0
    qkv_dim = max(num_channels // config.num_head, 16)
    self.qkv_dim = qkv_dim
    H = config.num_head
    self.q_projection = Linear(num_channels, (H, qkv_dim), transpose_weights=True, name="q_projection")
    self.k_projection = Linear(num_channels, (H, qkv_dim), transpose_weights=True, name="k_projection")
    self.v_projection = Linear(num_channels, (H, qkv_dim), name="v_projection")
    self.gating_query = Linear(num_channels, H * qkv_dim, transpose_weights=True, name="gating_query")
    self.output_projection = Linear(H * qkv_dim, num_channels, name="output_projection")
    # bias-free as in the reference (blocks.py:260-264); a checkpoint that carries an
    # act_norm.bias still loads (see _load_from_state_dict)
    self.act_norm = LayerNorm(num_channels, bias=kwargs.pop("act_norm_bias", False), name="act_norm")
    self.pair_bias_projection = Linear(num_channels, H, name="pair_bias_projection")

  def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
    key = prefix + "act_norm.bias"
    if key in state_dict and self.act_norm.bias is None:
      w = self.act_norm.weight
      self.act_norm.bias = torch.nn.Parameter(torch.empty(w.shape, dtype=w.dtype, device=w.device))
    super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)


class TriangleMultiplication(_NoTorchPath, torch.nn.Module):
  """blocks.py:425-485: gated triangle multiplicative update, outgoing
  (``"...ikc,...jkc->...ijc"``) or incoming (``"...kjc,...kic->...ijc"``) edges."""

  @dataclasses.dataclass
  class Config:
    equation: str = "...ikc,...jkc->...ijc"
    use_glu_kernel: bool = True

  EQUATIONS = ("...ikc,...jkc->...ijc", "...kjc,...kic->...ijc")

  def __init__(self, config: Config, global_config: GlobalConfig, *, num_channels: int,
               distributed: bool = False, name: str = "", **kwargs):
    super().__init__()
    if config.equation not in self.EQUATIONS:
      raise ValueError(f"TriangleMultiplication: unknown equation {config.equation!r}")
    if distributed:
      raise ValueError("TriangleMultiplication: the multi-rank path is not part of this build")
    self.name = name
    self.config = config
    self.distributed = False
    self.num_channels = num_channels
    self.equation = config.equation
    self.use_glu_kernel = config.use_glu_kernel
    C = num_channels
    self.left_norm_input = LayerNorm(C, bias=True, name="left_norm_input")
    self.projection = Linear(C, C * 2, bias=False, name="projection")
    self.gate_projection = Linear(C, C * 2, bias=False, name="gate")
    self.center_norm = LayerNorm(C, bias=True, name="center_norm")
    self.output_projection = Linear(C, C, bias=False, name="output_projection")
    self.gating_linear = Linear(C, C, bias=False, name="gating_linear")


class AdaptiveLayerNorm(torch.nn.Module):
  """transformer.py:27-78."""

  def __init__(self, hidden_size, single_cond_size, *, dtype=None, name: str = ""):
    super().__init__()
    self.name = name
    self.dtype = dtype
    self.single_cond = single_cond_size is not None
    if self.single_cond:
      self.layer_norm = LayerNorm(hidden_size, elementwise_affine=False, dtype=torch.float32, name="layer_norm")
      self.single_cond_layer_norm = LayerNorm(single_cond_size, bias=False, dtype=torch.float32,
                                              name="single_cond_layer_norm")
      self.single_cond_scale = Linear(single_cond_size, hidden_size, bias=True, dtype=dtype, name="single_cond_scale")
      self.single_cond_bias = Linear(single_cond_size, hidden_size, bias=False, dtype=dtype, name="single_cond_bias")
    else:
      self.layer_norm = LayerNorm(hidden_size, dtype=torch.float32, name="layer_norm")


class AdaptiveZeroInit(torch.nn.Module):
  """transformer.py:99-136."""

  def __init__(self, global_config, *, num_channels: int, hidden_size: int, single_cond_size, dtype=None,
               name: str = ""):
    super().__init__()
    self.name = name
    self.dtype = dtype
    self.single_cond = single_cond_size is not None
    self.transition2 = Linear(hidden_size, num_channels, bias=False, dtype=dtype, name="transition2")
    if self.single_cond:
      self.adaptive_zero_cond = Linear(single_cond_size, num_channels, bias=True, dtype=dtype,
                                       name="adaptive_zero_cond")


class SelfAttention(_NoTorchPath, torch.nn.Module):
  """transformer.py:234-304: single-representation / diffusion token attention."""

  @dataclasses.dataclass
  class Config:
    num_head: int = 16
    key_dim: int | None = None
    value_dim: int | None = None

  def __init__(self, config: Config, global_config: GlobalConfig, *, num_channels: int,
               single_cond_size: int | None = None, dtype: torch.dtype | None = None,
               distributed: bool = False, name: str = ""):
    super().__init__()
    self.name = name
    self.dtype = dtype
    if distributed:
      raise ValueError("SelfAttention: the multi-rank path is not part of this build")
    self.distributed = False
    self.layer_norm = AdaptiveLayerNorm(num_channels, single_cond_size, dtype=dtype, name="")
    key_dim = config.key_dim if config.key_dim is not None else num_channels
    value_dim = config.value_dim if config.value_dim is not None else num_channels
    H = config.num_head
    assert key_dim % H == 0 and value_dim % H == 0
    self.num_head = H
    self.key_dim = key_dim = key_dim // H
    self.value_dim = value_dim = value_dim // H
    assert key_dim == value_dim
    self.q_projection = Linear(num_channels, (H, key_dim), bias=True, dtype=dtype, name="q_projection")
    self.k_projection = Linear(num_channels, (H, key_dim), bias=False, dtype=dtype, name="k_projection")
    self.v_projection = Linear(num_channels, (H, value_dim), bias=False, dtype=dtype, name="v_projection")
    self.gating_query = Linear(num_channels, H * value_dim, bias=False, dtype=dtype, name="gating_query")
    self.zero_init = AdaptiveZeroInit(global_config, num_channels=num_channels, hidden_size=num_channels,
                                      single_cond_size=single_cond_size, dtype=dtype, name="")


class CrossAttention(_NoTorchPath, torch.nn.Module):
  """transformer.py:480-547: windowed atom cross attention."""

  @dataclasses.dataclass
  class Config:
    num_head: int = 4
    key_dim: int = 128
    value_dim: int = 128

  def __init__(self, config: Config, global_config: GlobalConfig, *, num_channels: int,
               dtype: torch.dtype | None = None, name: str = ""):
    super().__init__()
    self.name = name
    self.dtype = dtype
    self.q_layernorm = AdaptiveLayerNorm(num_channels, num_channels, dtype=dtype, name="q")
    self.k_layernorm = AdaptiveLayerNorm(num_channels, num_channels, dtype=dtype, name="k")
    assert config.key_dim % config.num_head == 0 and config.value_dim % config.num_head == 0
    H = config.num_head
    self.num_head = H
    self.key_dim = key_dim = config.key_dim // H
    self.value_dim = value_dim = config.value_dim // H
    assert key_dim == value_dim
    self.q_projection = Linear(num_channels, (H, key_dim), bias=True, dtype=dtype, name="q_projection")
    self.k_projection = Linear(num_channels, (H, key_dim), bias=False, dtype=dtype, name="k_projection")
    self.v_projection = Linear(num_channels, (H, value_dim), bias=False, dtype=dtype, name="v_projection")
    self.gating_query = Linear(num_channels, H * value_dim, bias=False, dtype=dtype, name="gating_query")
    self.zero_init = AdaptiveZeroInit(global_config, num_channels=num_channels, hidden_size=num_channels,
                                      single_cond_size=num_channels, dtype=dtype, name="")


class SingleActUpdate(_NoTorchPath, torch.nn.Module):
  """blocks.py:692-737: pair-logit prologue + single attention with pair bias."""

  def __init__(self, global_config: GlobalConfig, num_channels: int, seq_channels: int,
               attn_config: SelfAttention.Config, transition_config=None, distributed: bool = False, **kwargs):
    super().__init__()
    self.name = "<none>"
    if distributed:
      raise ValueError("SingleActUpdate: the multi-rank path is not part of this build")
    self.distributed = False
    self.num_channels = num_channels
    self.seq_channels = seq_channels
    self.num_head = attn_config.num_head
    self.qkv_dim = seq_channels // self.num_head
    self.single_pair_logits_norm = LayerNorm(num_channels, name="single_pair_logits_norm")
    self.single_pair_logits_projection = Linear(num_channels, attn_config.num_head,
                                                name="single_pair_logits_projection")
    self.single_attention = SelfAttention(attn_config, global_config, num_channels=seq_channels,
                                          name="single_attention_")
    if transition_config is not None:
      self.num_intermediate = int(seq_channels * transition_config.num_intermediate_factor)
      self.single_transition = TransitionBlock(transition_config, global_config, num_channels=seq_channels,
                                               name="single_transition")


class TransitionBlock(_NoTorchPath, torch.nn.Module):
  """blocks.py:38-96: the trunk transition -- LayerNorm, SwiGLU of ``transition1`` (``[C, 2I]``:
  the first I columns through swish, times the last I), ``transition2`` plus the residual."""

  @dataclasses.dataclass
  class Config:
    num_intermediate_factor: int = 4
    use_glu_kernel: bool = True

  def __init__(self, config: Config, global_config: GlobalConfig, *, num_channels: int, name: str = "", **kwargs):
    super().__init__()
    self.name = name
    self.num_channels = num_channels
    self.num_intermediate_factor = config.num_intermediate_factor
    self.use_glu_kernel = config.use_glu_kernel
    self.num_intermediate = int(num_channels * config.num_intermediate_factor)
    self.input_layer_norm = LayerNorm(num_channels, name="input_layer_norm")
    self.transition1 = Linear(num_channels, self.num_intermediate * 2, name="transition1")
    self.transition2 = Linear(self.num_intermediate, num_channels, name="transition2")


class DiffusionTransitionBlock(_NoTorchPath, torch.nn.Module):
  """transformer.py:157-231 (``TransitionBlock`` of the diffusion transformer): AdaLN (``ffw_``),
  SwiGLU of ``transition`` (``[C, 2I]``), AdaLN-zero output (``transition2`` times the sigmoid
  gate of the condition) plus the residual."""

  def __init__(self, global_config: GlobalConfig, *, num_channels: int, num_intermediate_factor: int,
               single_cond_size: int | None = None, use_glu_kernel: bool = True, dtype=None, name: str = ""):
    super().__init__()
    self.name = name
    self.dtype = dtype
    self.use_glu_kernel = use_glu_kernel
    self.num_intermediates = num_intermediate_factor * num_channels
    self.layer_norm = AdaptiveLayerNorm(num_channels, single_cond_size, dtype=dtype, name="ffw_")
    self.transition = Linear(num_channels, self.num_intermediates * 2, bias=False, dtype=dtype,
                             name="ffw_transition1")
    self.zero_init = AdaptiveZeroInit(global_config, num_channels=num_channels, hidden_size=self.num_intermediates,
                                      single_cond_size=single_cond_size, dtype=dtype, name="ffw_")


class TransformerPairLogits(_NoTorchPath, torch.nn.Module):
  """transformer.py:398-419: ``pair_input_layer_norm`` (no bias) and one
  ``Linear(pair_cond_size, (super_block_size, num_head))`` per super-block."""

  def __init__(self, *, num_blocks: int = 24, super_block_size: int = 4, num_head: int = 16,
               pair_cond_size: int = 128, dtype: torch.dtype | None = None, name: str = "transformer"):
    super().__init__()
    assert num_blocks % super_block_size == 0
    self.name = name
    self.dtype = dtype
    self.super_block_size = super_block_size
    self.num_head = num_head
    self.pair_logits_projection = torch.nn.ModuleList(
        [Linear(pair_cond_size, (super_block_size, num_head), bias=False, name="pair_logits_projection")
         for _ in range(num_blocks // super_block_size)])
    self.pair_input_layer_norm = LayerNorm(pair_cond_size, bias=False, name="pair_input_layer_norm")


class CrossAttTransformerPairLogits(_NoTorchPath, torch.nn.Module):
  """transformer.py:611-620: ``pair_input_layer_norm`` (no bias) and
  ``Linear(pair_cond_size, (num_blocks, num_head))``."""

  def __init__(self, *, num_blocks: int = 3, num_head: int = 4, pair_cond_size: int = 16,
               dtype: torch.dtype | None = None, name: str = "transformer"):
    super().__init__()
    self.name = name
    self.dtype = dtype
    self.num_head = num_head
    self.pair_input_layer_norm = LayerNorm(pair_cond_size, bias=False, name="pair_input_layer_norm")
    self.pair_logits_projection = Linear(pair_cond_size, (num_blocks, num_head), bias=False,
                                         name="pair_logits_projection")
