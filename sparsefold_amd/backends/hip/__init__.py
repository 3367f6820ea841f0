"""Lifecycle hooks of the HIP (MI355X / gfx950) backend.

Same hook set as the reference backends (``src/sparsefold/backends/__init__.py:25``):
``apply`` replaces the attention module factories before model construction (selected by
``native_ops`` names from ``src/sparsefold/config.py:24-35``, as
``backends/vecops/backend.py:187-248`` does), ``unapply`` restores them, ``prepare`` packs
weights into non-persistent buffers after strict loading, and the remaining hooks are
trivial because nothing is JIT-compiled (the kernels are built ahead of time into
``libsparsefold_hip.so``).  ``apply`` loads that library first, so a missing build fails here,
before any model exists.
"""
from __future__ import annotations

import importlib
from contextlib import nullcontext

import torch

from sparsefold_amd import _lib
from sparsefold_amd import modules as _modules
from sparsefold_amd.runtime import config

# native.ops name -> [(factory attribute, HIP class attribute in backends.hip.modules)]
_REPLACE_MAP = {
    "grid_self_attn": [("GridSelfAttention", "GridSelfAttentionHip")],
    "evoformer_single_act_update": [("SingleActUpdate", "SingleActUpdateHip")],
    "triangle_multiplication": [("TriangleMultiplication", "TriangleMultiplicationHip")],
    "evoformer_transition_block": [("TransitionBlock", "TransitionBlockHip")],
    "diffusion_transition_block": [("DiffusionTransitionBlock", "DiffusionTransitionBlockHip")],
    "diffusion_self_attention": [("SelfAttention", "SelfAttentionHip"),
                                 ("TransformerPairLogits", "TransformerPairLogitsHip")],
    "diffusion_cross_attention": [("CrossAttention", "CrossAttentionHip"),
                                  ("CrossAttTransformerPairLogits", "CrossAttTransformerPairLogitsHip")],
}


class _FactoryPatches:
  """The module factories this backend has replaced, each with the original to put back.

  Keyed by (owner identity, attribute name): the first replacement of a factory records the
  original, later ones (``apply`` called again) only swap the implementation, so ``restore``
  always returns the reference's own class."""

  def __init__(self) -> None:
    self._originals: dict[tuple[int, str], tuple[object, object]] = {}

  def replace(self, owner, name: str, implementation) -> None:
    self._originals.setdefault((id(owner), name), (owner, getattr(owner, name)))
    setattr(owner, name, implementation)

  def restore(self) -> None:
    originals, self._originals = self._originals, {}
    for (_, name), (owner, original) in originals.items():
      setattr(owner, name, original)


_patches = _FactoryPatches()


def unapply() -> None:
  _patches.restore()


def apply() -> None:
  _lib.load()
  hip_modules = importlib.import_module("sparsefold_amd.backends.hip.modules")
  selected = list(config.native_ops)
  if "*" in selected or "all" in selected:
    selected = list(_REPLACE_MAP)
  for key, pairs in _REPLACE_MAP.items():
    if key in selected:
      for factory, impl in pairs:
        _patches.replace(_modules, factory, getattr(hip_modules, impl))


def manual_seed(seed: int) -> None:
  torch.manual_seed(seed)


def prepare(module: torch.nn.Module) -> dict[str, int]:
  """Prepare every HIP module once (children of a prepared fused module are covered)."""
  hip_modules = importlib.import_module("sparsefold_amd.backends.hip.modules")
  counts = {"packed": 0, "fallback": 0, "opaque": 0}
  visited: set[int] = set()

  def visit(current: torch.nn.Module) -> None:
    if id(current) in visited:
      return
    visited.add(id(current))
    if isinstance(current, hip_modules.HIP_TYPES):
      current.prepare_native()
      counts["opaque"] += 1
      for child in current.modules():
        visited.add(id(child))
      return
    for child in current.children():
      visit(child)

  visit(module)
  return counts


def materialize(*, parallelism: int | None = None) -> int:
  _lib.load()
  return 0


def precompile(module, *args, **kwargs):
  return None


def is_precompiling() -> bool:
  return False


def execution_context():
  return nullcontext()
