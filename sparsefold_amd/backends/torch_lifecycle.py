"""Lifecycle hooks of the reference Torch backend (``src/sparsefold/backends/torch/__init__.py``).

Selecting ``torch`` leaves the module factories untouched; every hook is a no-op.  (The
Torch math compute path itself is not part of this package.)
"""
from contextlib import nullcontext

import torch


def apply() -> None:
  return None


def manual_seed(seed: int) -> None:
  torch.manual_seed(seed)


def prepare(module) -> dict[str, int]:
  return {"packed": 0, "fallback": 0, "opaque": 0}


def materialize(*, parallelism: int | None = None) -> int:
  return 0


def precompile(module, *args, **kwargs):
  return None


def is_precompiling() -> bool:
  return False


def execution_context():
  return nullcontext()
