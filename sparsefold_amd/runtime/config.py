"""Runtime settings that select the attention path.

Interface kept from the reference (``src/sparsefold/runtime/config.py``), because callers and
configuration files depend on it:

* ``configure_runtime(**settings)`` resolves every setting once (explicit values win over the
  environment); ``backend=`` is accepted in place of ``acclib_implementation``;
* the environment names ``SPARSEFOLD_<SETTING>`` and their deprecated ``AF3_<SETTING>`` forms;
* module attribute access (``config.device``, ``config.acclib_implementation`` ...),
  ``get_runtime_options()`` (an independent copy) and ``reset()``;
* backend names: ``none`` means ``torch``, ``cpp`` is the deprecated name of ``vecops``.

Only the settings that matter to the attention path are modelled.  The allowed values are the
reference's (``src/sparsefold/config.py:271-285``) plus ``"hip"`` for both the native backend
(``[native] impl``) and the SDPA implementation (``[precision] sdpa``).
"""
from __future__ import annotations

import ast
import dataclasses
import os
import warnings
from typing import Any, Callable

SDPA_IMPLEMENTATIONS = frozenset({"math", "flash", "efficient", "hip"})
BACKENDS = frozenset({"torch", "vecops", "hip"})


def normalize_backend(value: str) -> str:
  """Canonical backend name: lower case, ``none`` -> ``torch``, ``cpp`` -> ``vecops``."""
  name = str(value).strip().lower()
  aliases = {"none": "torch"}
  if name == "cpp":
    warnings.warn("the backend name 'cpp' is deprecated; select 'vecops'", DeprecationWarning, stacklevel=2)
    return "vecops"
  return aliases.get(name, name)


def _flag(text: str) -> bool:
  return str(text).strip().lower() in ("1", "true", "yes", "on")


def _names(text: str) -> list[str]:
  return [item.strip() for item in str(text).split(",") if item.strip()]


def _literal_dict(text) -> dict:
  """A Python dict literal (the reference parses this setting with ast.literal_eval)."""
  value = ast.literal_eval(text) if isinstance(text, str) else dict(text)
  if not isinstance(value, dict):
    raise ValueError(f"sparse_attention_parameters must be a dict, got {value!r}")
  return dict(value)


@dataclasses.dataclass(frozen=True)
class _Setting:
  """One runtime setting: its environment suffix, default text and parser."""
  env: str
  default: str
  parse: Callable[[str], Any] = str


_SETTINGS: dict[str, _Setting] = {
    "device": _Setting("DEVICE", "cpu"),
    "enable_sharding": _Setting("ENABLE_SHARDING", "0", _flag),
    "acclib_implementation": _Setting("ACCLIB_IMPLEMENTATION", "torch", normalize_backend),
    "native_ops": _Setting("NATIVE_OPS", "*", _names),
    "sdpa_implementation": _Setting("SDPA_IMPLEMENTATION", "math"),
    "diffusion_precision": _Setting("DIFFUSION_PRECISION", "fp32"),
    "sparse_attention_parameters": _Setting("SPARSE_ATTENTION_PARAMETERS", "{}", _literal_dict),
    "enable_gsa_index_reuse": _Setting("ENABLE_GSA_INDEX_REUSE", "1", _flag),
    # no counterpart in the reference: replay repeated HIP module calls as captured graphs
    "hip_graphs": _Setting("HIP_GRAPHS", "0", _flag),
    # no counterpart in the reference (whose native grid attention is always block-sparse and
    # whose torch path is always dense): the HIP grid attention's rows are block-sparse (IBS)
    "hip_sparse_grid_attention": _Setting("HIP_SPARSE_GRID_ATTENTION", "0", _flag),
}

_resolved: dict[str, Any] | None = None


def _from_environment(name: str) -> Any:
  spec = _SETTINGS[name]
  current, legacy = "SPARSEFOLD_" + spec.env, "AF3_" + spec.env
  text = os.environ.get(current)
  if text is None and legacy in os.environ:
    warnings.warn(f"{legacy} is deprecated; set {current} or call configure_runtime()",
                  DeprecationWarning, stacklevel=4)
    text = os.environ[legacy]
  return spec.parse(spec.default if text is None else text)


def _check(settings: dict[str, Any]) -> None:
  if settings["sdpa_implementation"] not in SDPA_IMPLEMENTATIONS:
    raise ValueError(f"Unsupported SDPA implementation {settings['sdpa_implementation']!r}; "
                     f"choose one of {sorted(SDPA_IMPLEMENTATIONS)}")
  if settings["acclib_implementation"] not in BACKENDS:
    raise ValueError(f"Unsupported backend {settings['acclib_implementation']!r}; choose one of {sorted(BACKENDS)}")


def configure_runtime(**settings: Any) -> None:
  """Resolves all settings: the given ones, the environment for the rest."""
  global _resolved
  if "backend" in settings:
    if "acclib_implementation" in settings:
      raise ValueError("Pass either backend or acclib_implementation, not both")
    settings["acclib_implementation"] = settings.pop("backend")
  extra = sorted(set(settings) - set(_SETTINGS))
  if extra:
    raise TypeError(f"Unknown runtime settings: {extra}")
  resolved = {name: settings[name] if name in settings else _from_environment(name) for name in _SETTINGS}
  resolved["acclib_implementation"] = normalize_backend(resolved["acclib_implementation"])
  resolved["native_ops"] = list(resolved["native_ops"])
  resolved["sparse_attention_parameters"] = _literal_dict(resolved["sparse_attention_parameters"])
  _check(resolved)
  _resolved = resolved


def _value(name: str) -> Any:
  return _resolved[name] if _resolved is not None else _from_environment(name)


def get_runtime_options() -> dict[str, Any]:
  """A copy of the current settings that ``configure_runtime(**options)`` accepts back."""
  def copy(v):
    return list(v) if isinstance(v, list) else dict(v) if isinstance(v, dict) else v
  return {name: copy(_value(name)) for name in _SETTINGS}


def uses_hip() -> bool:
  return _value("acclib_implementation") == "hip"


def reset() -> None:
  """Forgets explicit settings: values come from the environment again."""
  global _resolved
  _resolved = None


def __getattr__(name: str) -> Any:
  if name in _SETTINGS:
    return _value(name)
  raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
