"""Backend lifecycle dispatcher -- mirror of ``src/sparsefold/backends/__init__.py``.

Same hooks and semantics: ``register_library(apply_fn, name, fn_redirects)``, ``init()``
selects the backend named by ``runtime.config.acclib_implementation`` and runs its
``apply()`` before model construction; ``manual_seed / prepare / precompile / materialize /
is_precompiling / execution_context`` dispatch to the selected backend.  Registered here:
``torch`` (no-op lifecycle: the reference's Torch backend, ``backends/torch/__init__.py``) and
``hip`` (this package's MI355X kernels).  ``vecops`` is declared but cannot load here.
"""
from __future__ import annotations

import importlib
from collections.abc import Callable
from contextlib import nullcontext
from dataclasses import dataclass

from sparsefold_amd.runtime import config


@dataclass(frozen=True)
class _Library:
  name: str
  apply: Callable[[], None]
  fn_redirects: dict[str, Callable]


_registered_impl: dict[str, _Library] = {}
_current_library: _Library | None = None
_applied_libraries: set[str] = set()
_HOOKS = ("manual_seed", "prepare", "precompile", "materialize", "is_precompiling", "execution_context")
_BUILTIN = {"torch": "sparsefold_amd.backends.torch_lifecycle", "hip": "sparsefold_amd.backends.hip"}


def register_library(apply_fn: Callable[[], None], name: str, fn_redirects: dict[str, Callable] | None = None):
  if name in _registered_impl:
    raise KeyError(f"Library {name!r} already registered")
  _registered_impl[name] = _Library(name, apply_fn, fn_redirects or {})


def available_libraries() -> list[str]:
  return list(dict.fromkeys(["torch", "vecops", "hip", *_registered_impl]))


def _load_library(name: str) -> _Library:
  if name not in _registered_impl and name in _BUILTIN:
    try:
      module = importlib.import_module(_BUILTIN[name])
    except ImportError as error:
      raise RuntimeError(f"Cannot load backend {name!r}: {error}") from error
    register_library(module.apply, name, {hook: getattr(module, hook) for hook in _HOOKS})
  if name == "vecops" and name not in _registered_impl:
    raise RuntimeError("Backend 'vecops' requires the external vecops package, which this build does not ship")
  if name not in _registered_impl:
    raise KeyError(f"Backend {name!r} is not registered")
  return _registered_impl[name]


def init(apply: bool = True):
  """Select the configured backend (idempotent); model construction must follow."""
  global _current_library
  name = config.normalize_backend(config.acclib_implementation)
  if name == "hip":
    from sparsefold_amd.backends.hip.policy import validate_hip_device, validate_hip_ops
    validate_hip_device(config.device)
    validate_hip_ops(config.native_ops)
  lib = _load_library(name)
  if _current_library is not None and _current_library.name != name:
    if _current_library.name == "hip" and "hip" in _applied_libraries:
      importlib.import_module("sparsefold_amd.backends.hip").unapply()
      _applied_libraries.discard("hip")
    elif _current_library.name not in {"torch", "hip"} and _current_library.name in _applied_libraries:
      raise RuntimeError("Cannot safely switch from an applied custom backend")
  if apply and name not in _applied_libraries:
    try:
      lib.apply()
    except Exception as error:
      if name == "hip":
        importlib.import_module("sparsefold_amd.backends.hip").unapply()
      raise RuntimeError(f"Failed to apply backend {name!r}: {error}") from error
    _applied_libraries.add(name)
  _current_library = lib


def _dispatch_redirect_call(name: str, *args, **kwargs):
  lib = _current_library or _load_library("torch")
  fn = lib.fn_redirects.get(name)
  return fn(*args, **kwargs) if fn is not None else None


def manual_seed(seed: int):
  return _dispatch_redirect_call("manual_seed", seed)


def prepare(module):
  return _dispatch_redirect_call("prepare", module)


def precompile(module, *args, use_real_tensors: bool = False, parallelism: int | None = None,
               capture_graph: bool = False, graph_name: str | None = None, **kwargs):
  return _dispatch_redirect_call("precompile", module, *args, use_real_tensors=use_real_tensors,
                                 parallelism=parallelism, capture_graph=capture_graph,
                                 graph_name=graph_name, **kwargs)


def materialize(*, parallelism: int | None = None):
  return _dispatch_redirect_call("materialize", parallelism=parallelism)


def is_precompiling() -> bool:
  return bool(_dispatch_redirect_call("is_precompiling"))


def execution_context():
  return _dispatch_redirect_call("execution_context") or nullcontext()
