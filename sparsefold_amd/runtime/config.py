"""Runtime settings for backend selection -- mirror of ``src/sparsefold/runtime/config.py``.

Same API (``configure_runtime(**overrides)``, ``backend=`` alias, ``normalize_backend``,
``get_runtime_options``, ``reset``, module attribute access) and the same environment
variables (``SPARSEFOLD_*``, legacy ``AF3_*``), restricted to the settings that select the
attention path.  The value sets are those of the reference (config.py:271-285) extended with
the HIP backend: ``acclib_implementation`` (``[native] impl``) and ``sdpa_implementation``
(``[precision] sdpa``) both accept ``"hip"``.
"""
from __future__ import annotations

import copy
import os
import warnings
from typing import Any

SDPA_IMPLEMENTATIONS = frozenset({"math", "flash", "efficient", "hip"})
BACKENDS = frozenset({"torch", "vecops", "hip"})

# name -> (legacy env var, default); runtime/config.py:13-28
_LEGACY: dict[str, tuple[str, Any]] = {
    "device": ("AF3_DEVICE", "cpu"),
    "enable_sharding": ("AF3_ENABLE_SHARDING", "0"),
    "acclib_implementation": ("AF3_ACCLIB_IMPLEMENTATION", "torch"),
    "native_ops": ("AF3_NATIVE_OPS", "*"),
    "sdpa_implementation": ("AF3_SDPA_IMPLEMENTATION", "math"),
    "diffusion_precision": ("AF3_DIFFUSION_PRECISION", "fp32"),
    # HIP backend only, no reference counterpart: replay repeated module calls as HIP graphs
    "hip_graphs": ("AF3_HIP_GRAPHS", "0"),
}
_BOOL_FIELDS = {"enable_sharding", "hip_graphs"}
_state: dict[str, Any] | None = None


def normalize_backend(value: str) -> str:
  """runtime/config.py:42-49: ``none`` -> ``torch``, deprecated ``cpp`` -> ``vecops``."""
  value = value.lower()
  if value == "none":
    return "torch"
  if value == "cpp":
    warnings.warn("backend 'cpp' is deprecated; use 'vecops'", DeprecationWarning, stacklevel=2)
    return "vecops"
  return value


def _environment_value(name: str) -> Any:
  legacy, default = _LEGACY[name]
  current = legacy.replace("AF3_", "SPARSEFOLD_", 1)
  if current in os.environ:
    raw = os.environ[current]
  elif legacy in os.environ:
    raw = os.environ[legacy]
    warnings.warn(f"{legacy} is deprecated; use {current} or configure_runtime()",
                  DeprecationWarning, stacklevel=3)
  else:
    raw = default
  if name == "native_ops":
    return [p.strip() for p in raw.split(",") if p.strip()]
  if name in _BOOL_FIELDS:
    return str(raw).lower() in {"1", "true", "yes", "on"}
  if name == "acclib_implementation":
    return normalize_backend(raw)
  return raw


def _validate(state: dict[str, Any]) -> None:
  if state["sdpa_implementation"] not in SDPA_IMPLEMENTATIONS:
    raise ValueError(f"Unsupported SDPA implementation: {state['sdpa_implementation']!r}")
  if state["acclib_implementation"] not in BACKENDS:
    raise ValueError(f"Unsupported backend: {state['acclib_implementation']!r}")


def configure_runtime(**overrides: Any) -> None:
  """runtime/config.py:93-111.  ``backend=`` is an alias for ``acclib_implementation``."""
  global _state
  if "backend" in overrides:
    if "acclib_implementation" in overrides:
      raise ValueError("Pass either backend or acclib_implementation")
    overrides["acclib_implementation"] = overrides.pop("backend")
  unknown = overrides.keys() - _LEGACY.keys()
  if unknown:
    raise TypeError(f"Unknown runtime settings: {sorted(unknown)}")
  state = {name: _environment_value(name) for name in _LEGACY}
  state.update(overrides)
  state["acclib_implementation"] = normalize_backend(state["acclib_implementation"])
  state["native_ops"] = list(state["native_ops"])
  _validate(state)
  _state = state


def get_runtime_options() -> dict[str, Any]:
  return copy.deepcopy({name: __getattr__(name) for name in _LEGACY})


def uses_hip() -> bool:
  return __getattr__("acclib_implementation") == "hip"


def reset() -> None:
  global _state
  _state = None


def __getattr__(name: str) -> Any:
  if name in _LEGACY:
    return _state[name] if _state is not None else _environment_value(name)
  raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
