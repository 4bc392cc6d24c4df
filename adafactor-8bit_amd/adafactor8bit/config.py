"""Dictionary policies over generated parameter groups (the reference's config.py).

A policy is a mapping with up to three sections:

* ``defaults``: constructor options applied to every generated group;
* ``presets``: named custom presets, each ``{"preset": <base>, **options}``
  with a built-in or another custom preset as base (no cycles, no shadowing of
  a built-in name);
* ``mapping``: per route name (``one_d``, ``matrix``, ``apollo``, ...) an
  optional ``preset`` plus options.

Precedence, lowest first: the generated group, ``defaults``, the mapped
preset, the mapped options (config.py:83-89).  Resolving a preset resets every
semantic option to the constructor default before applying the preset's own
values, so a mapped preset fully determines the update path.  Error types and
messages are the reference's.
"""
from copy import deepcopy
from inspect import signature
from typing import Any, Dict, List, Mapping

from .optimizer import Adafactor8Bit
from .presets import PRESETS
from .routing import _ROUTE_NAMES, _validate_route_options

__all__ = ["validate_policy", "apply_policy"]

_CTOR = signature(Adafactor8Bit.__init__).parameters
_CONFIG_KEYS = frozenset(_CTOR) - {"self", "params"}
# Options that define an update path: everything any preset sets, plus the rank.
_SEMANTIC_KEYS = frozenset({"apollo_rank"}.union(*(set(s.primary) | set(s.fallback or {})
                                                   for s in PRESETS.values())))


def _check_options(options: Mapping[str, Any], where: str) -> None:
    if not isinstance(options, Mapping):
        raise TypeError(f"{where} must be a mapping")
    unknown = set(options) - _CONFIG_KEYS
    if unknown:
        raise TypeError(f"Unknown optimizer options in {where}: {sorted(unknown)}")
    _validate_route_options(where, options)


def _resolve_preset(name: str, custom: Mapping[str, Any], chain=()) -> Dict[str, Any]:
    """Options of a built-in or custom preset, inheritance resolved
    (config.py:32-51)."""
    if not isinstance(name, str):
        raise TypeError("Policy preset names must be strings")
    spec = PRESETS.get(name)
    if spec is not None:
        out = {k: deepcopy(_CTOR[k].default) for k in _SEMANTIC_KEYS}
        out.update(deepcopy(spec.primary))
        out["apollo_rank"] = spec.default_apollo_rank
        return out
    if name not in custom:
        raise ValueError(f"Unknown policy preset {name!r}")
    if name in chain:
        raise ValueError(f"Cyclic policy preset inheritance: {' -> '.join((*chain, name))}")
    own = dict(custom[name])
    base = own.pop("preset", None)
    if base is None:
        raise ValueError(f"Custom preset {name!r} requires a base 'preset'")
    out = _resolve_preset(base, custom, (*chain, name))
    out.update(deepcopy(own))
    return out


def validate_policy(policy: Mapping[str, Any]) -> None:
    """Check a policy without a model (config.py:54-80)."""
    if not isinstance(policy, Mapping):
        raise TypeError("policy must be a mapping")
    extra = set(policy) - {"defaults", "presets", "mapping"}
    if extra:
        raise TypeError(f"Unknown policy sections: {sorted(extra)}")
    _check_options(policy.get("defaults", {}), "policy.defaults")
    custom = policy.get("presets", {})
    mapping = policy.get("mapping", {})
    if not isinstance(custom, Mapping) or not isinstance(mapping, Mapping):
        raise TypeError("policy.presets and policy.mapping must be mappings")
    for name, body in custom.items():
        if not isinstance(name, str) or not name:
            raise TypeError("Custom preset names must be non-empty strings")
        if name in PRESETS:
            raise ValueError(f"Custom preset {name!r} shadows a built-in; choose a distinct name")
        if not isinstance(body, Mapping):
            raise TypeError(f"Custom preset {name!r} must be a mapping")
        _check_options({k: v for k, v in body.items() if k != "preset"}, f"presets.{name}")
    for name in custom:
        _resolve_preset(name, custom)
    for route, entry in mapping.items():
        if route not in _ROUTE_NAMES:
            raise ValueError(f"Unknown policy route {route!r}; expected one of {sorted(_ROUTE_NAMES)}")
        if not isinstance(entry, Mapping):
            raise TypeError(f"mapping.{route} must be a mapping")
        _check_options({k: v for k, v in entry.items() if k != "preset"}, f"mapping.{route}")
        if "preset" in entry:
            _resolve_preset(entry["preset"], custom)


def apply_policy(groups: List[Dict[str, Any]], policy: Mapping[str, Any]) -> List[Dict[str, Any]]:
    """New group dicts with the policy laid over ``groups`` (config.py:83-108);
    parameter lists and group order are kept.  Routes named in the mapping but
    absent from the model are allowed."""
    validate_policy(policy)
    defaults = policy.get("defaults", {})
    custom = policy.get("presets", {})
    mapping = policy.get("mapping", {})
    out = []
    for g in groups:
        merged = dict(g)
        merged.update(deepcopy(dict(defaults)))
        entry = dict(mapping.get(g["group_name"], {}))
        preset = entry.pop("preset", None)
        if preset is not None:
            merged.update(_resolve_preset(preset, custom))
        merged.update(deepcopy(entry))
        rank = merged.get("apollo_rank", 0)
        if not isinstance(rank, int) or isinstance(rank, bool) or rank < 0:
            raise ValueError("apollo_rank must be an integer >= 0")
        if rank and any(p.ndim != 2 or min(p.shape) < rank for p in merged["params"]):
            raise ValueError(f"Route {g['group_name']!r} contains parameters ineligible for APOLLO rank {rank}")
        out.append(merged)
    return out
