"""Backend selection and lifecycle hooks.

The plugin interface is the reference's (``src/sparsefold/backends/__init__.py``): a backend is
a set of hooks -- ``apply`` (replace module factories before model construction) plus
``manual_seed``, ``prepare``, ``precompile``, ``materialize``, ``is_precompiling`` and
``execution_context`` -- registered under a name with ``register_library``; ``init()`` activates
the backend that ``runtime.config.acclib_implementation`` names, and the module-level hook
functions forward to the active backend (to ``torch`` before any ``init``).

Built-in backends: ``torch`` (hooks that change nothing: the reference's Torch path) and
``hip`` (this package's MI355X kernels).  ``vecops`` is a known name whose native package this
build does not ship, so selecting it fails with an explanation.
"""
from __future__ import annotations

import importlib
from collections.abc import Callable
from contextlib import nullcontext
from types import SimpleNamespace

from sparsefold_amd.runtime import config

HOOK_NAMES = ("manual_seed", "prepare", "precompile", "materialize", "is_precompiling", "execution_context")
_BUILT_IN_MODULES = {"torch": "sparsefold_amd.backends.torch_lifecycle", "hip": "sparsefold_amd.backends.hip"}


class _Selection:
  """Which backends exist, which one is active, and which have had ``apply`` run."""

  def __init__(self) -> None:
    self.backends: dict[str, SimpleNamespace] = {}
    self.active: SimpleNamespace | None = None
    self.applied: set[str] = set()

  def add(self, name: str, apply_fn: Callable[[], None], hooks: dict[str, Callable], unapply=None) -> None:
    if name in self.backends:
      raise KeyError(f"A backend named {name!r} is already registered")
    self.backends[name] = SimpleNamespace(name=name, apply=apply_fn, unapply=unapply, hooks=dict(hooks))

  def get(self, name: str) -> SimpleNamespace:
    if name not in self.backends and name in _BUILT_IN_MODULES:
      try:
        module = importlib.import_module(_BUILT_IN_MODULES[name])
      except ImportError as error:
        raise RuntimeError(f"Backend {name!r} could not be imported: {error}") from error
      self.add(name, module.apply, {h: getattr(module, h) for h in HOOK_NAMES}, getattr(module, "unapply", None))
    if name not in self.backends:
      if name == "vecops":
        raise RuntimeError("Backend 'vecops' needs the external vecops package, which is not part of this build")
      raise KeyError(f"No backend named {name!r} is registered")
    return self.backends[name]

  def leave_active(self) -> None:
    """Undoes the active backend's factory replacements before another one takes over."""
    old = self.active
    if old is None or old.name not in self.applied:
      return
    if old.unapply is not None:
      old.unapply()
      self.applied.discard(old.name)
    elif old.name != "torch":
      raise RuntimeError(f"Backend {old.name!r} replaced module factories and cannot restore them")

  def activate(self, name: str, apply: bool) -> None:
    backend = self.get(name)
    if self.active is not None and self.active is not backend:
      self.leave_active()
    if apply and name not in self.applied:
      try:
        backend.apply()
      except Exception as error:
        if backend.unapply is not None:
          backend.unapply()
        raise RuntimeError(f"Backend {name!r} could not be applied: {error}") from error
      self.applied.add(name)
    self.active = backend

  def hook(self, hook_name: str) -> Callable | None:
    backend = self.active if self.active is not None else self.get("torch")
    return backend.hooks.get(hook_name)


_selection = _Selection()


def register_library(apply_fn: Callable[[], None], name: str, fn_redirects: dict[str, Callable] | None = None):
  """Registers a backend: ``apply_fn`` runs when it is activated, ``fn_redirects`` maps hook
  names to its implementations (missing hooks do nothing)."""
  _selection.add(name, apply_fn, fn_redirects or {})


def available_libraries() -> list[str]:
  """Known backend names (whether each one can load is checked by ``init``)."""
  names = ["torch", "vecops", "hip"]
  return names + [n for n in _selection.backends if n not in names]


def init(apply: bool = True):
  """Activates the configured backend; model construction must come after.  Activating the
  same backend again changes nothing; moving to another one restores the factories the
  previous one replaced."""
  name = config.normalize_backend(config.acclib_implementation)
  if name == "hip":
    from sparsefold_amd.backends.hip.policy import validate_hip_device, validate_hip_ops
    validate_hip_device(config.device)
    validate_hip_ops(config.native_ops)
  _selection.activate(name, apply)


def _forward(hook_name: str, *args, **kwargs):
  fn = _selection.hook(hook_name)
  return None if fn is None else fn(*args, **kwargs)


def manual_seed(seed: int):
  return _forward("manual_seed", seed)


def prepare(module):
  return _forward("prepare", module)


def precompile(module, *args, use_real_tensors: bool = False, parallelism: int | None = None,
               capture_graph: bool = False, graph_name: str | None = None, **kwargs):
  return _forward("precompile", module, *args, use_real_tensors=use_real_tensors, parallelism=parallelism,
                  capture_graph=capture_graph, graph_name=graph_name, **kwargs)


def materialize(*, parallelism: int | None = None):
  return _forward("materialize", parallelism=parallelism)


def is_precompiling() -> bool:
  return bool(_forward("is_precompiling"))


def execution_context():
  return _forward("execution_context") or nullcontext()
