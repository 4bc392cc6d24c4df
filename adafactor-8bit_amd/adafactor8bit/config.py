"""Dictionary policies over generated parameter groups.

A policy is a mapping with up to three sections:

* ``defaults``: constructor options applied to every generated group;
* ``presets``: named custom presets, each ``{"preset": <base>, **options}`` whose
  base is a built-in or another custom preset (no cycles, no reuse of a built-in
  name);
* ``mapping``: per route name (``one_d``, ``matrix``, ``apollo``, ...) an optional
  ``preset`` and options.

The interface is the reference's (adafactor8bit/config.py:22-108): the same
sections, error types and messages, and the same precedence, lowest first: the
generated group, ``defaults``, the mapped preset, the mapped options.  A preset
sets every option that defines an update path (the constructor default where
the preset is silent), so a mapped preset fully determines the route's update.

Here a policy is parsed once into a ``_Policy``: each section is checked as it is
read, custom presets are resolved by walking their inheritance chain down to the
built-in they rest on (memoised per name), and groups are then built by laying
the four option layers over each generated group.
"""
from copy import deepcopy
from inspect import signature
from typing import Any, Dict, List, Mapping, Optional, Tuple

from .optimizer import Adafactor8Bit
from .presets import PRESETS
from .routing import _ROUTE_NAMES, _validate_route_options

__all__ = ["validate_policy", "apply_policy"]

_SECTIONS = ("defaults", "presets", "mapping")
_CTOR_DEFAULTS = {name: prm.default for name, prm in signature(Adafactor8Bit.__init__).parameters.items()
                  if name not in ("self", "params")}
# Options that define an update path: whatever a built-in preset sets, and the rank.
_PATH_KEYS = sorted({"apollo_rank"}.union(*(set(spec.primary) | set(spec.fallback or {})
                                            for spec in PRESETS.values())))


def _options(value: Any, label: str) -> Dict[str, Any]:
    """A checked option mapping: only constructor keywords, valid route options."""
    if not isinstance(value, Mapping):
        raise TypeError(f"{label} must be a mapping")
    bad = sorted(set(value) - set(_CTOR_DEFAULTS))
    if bad:
        raise TypeError(f"Unknown optimizer options in {label}: {bad}")
    _validate_route_options(label, value)
    return dict(value)


def _builtin(name: str) -> Dict[str, Any]:
    spec = PRESETS[name]
    opts = {k: deepcopy(_CTOR_DEFAULTS[k]) for k in _PATH_KEYS}
    opts.update(deepcopy(spec.primary))
    opts["apollo_rank"] = spec.default_apollo_rank
    return opts


class _Policy:
    def __init__(self, policy: Any):
        if not isinstance(policy, Mapping):
            raise TypeError("policy must be a mapping")
        extra = sorted(set(policy) - set(_SECTIONS))
        if extra:
            raise TypeError(f"Unknown policy sections: {extra}")
        self.defaults = _options(policy.get("defaults", {}), "policy.defaults")
        self.custom = policy.get("presets", {})
        mapping = policy.get("mapping", {})
        if not isinstance(self.custom, Mapping) or not isinstance(mapping, Mapping):
            raise TypeError("policy.presets and policy.mapping must be mappings")
        self._resolved: Dict[str, Dict[str, Any]] = {}
        self._read_custom_presets()
        for name in self.custom:
            self.preset(name)
        self.routes: Dict[str, Tuple[Optional[str], Dict[str, Any]]] = {}
        for route, entry in mapping.items():
            if route not in _ROUTE_NAMES:
                raise ValueError(f"Unknown policy route {route!r}; expected one of {sorted(_ROUTE_NAMES)}")
            if not isinstance(entry, Mapping):
                raise TypeError(f"mapping.{route} must be a mapping")
            opts = _options({k: v for k, v in entry.items() if k != "preset"}, f"mapping.{route}")
            name = entry.get("preset") if "preset" in entry else None
            if "preset" in entry:
                self.preset(entry["preset"])
            self.routes[route] = (name, opts)

    def _read_custom_presets(self):
        for name, body in self.custom.items():
            if not isinstance(name, str) or not name:
                raise TypeError("Custom preset names must be non-empty strings")
            if name in PRESETS:
                raise ValueError(f"Custom preset {name!r} shadows a built-in; choose a distinct name")
            if not isinstance(body, Mapping):
                raise TypeError(f"Custom preset {name!r} must be a mapping")
            _options({k: v for k, v in body.items() if k != "preset"}, f"presets.{name}")

    def preset(self, name: Any) -> Dict[str, Any]:
        """Options of a built-in or custom preset, inheritance applied."""
        lineage: List[str] = []   # custom presets from `name` down to the built-in
        cur = name
        while True:
            if not isinstance(cur, str):
                raise TypeError("Policy preset names must be strings")
            if cur in PRESETS or cur in self._resolved:
                break
            if cur not in self.custom:
                raise ValueError(f"Unknown policy preset {cur!r}")
            if cur in lineage:
                raise ValueError("Cyclic policy preset inheritance: " + " -> ".join(lineage + [cur]))
            lineage.append(cur)
            cur = self.custom[cur].get("preset")
            if cur is None:
                raise ValueError(f"Custom preset {lineage[-1]!r} requires a base 'preset'")
        opts = _builtin(cur) if cur in PRESETS else deepcopy(self._resolved[cur])
        for child in reversed(lineage):
            opts.update(deepcopy({k: v for k, v in self.custom[child].items() if k != "preset"}))
            self._resolved[child] = deepcopy(opts)
        return deepcopy(opts)

    def group(self, generated: Dict[str, Any]) -> Dict[str, Any]:
        """The four layers over one generated group, then the APOLLO eligibility check."""
        name, opts = self.routes.get(generated["group_name"], (None, {}))
        layers = [deepcopy(self.defaults)]
        if name is not None:
            layers.append(self.preset(name))
        layers.append(deepcopy(opts))
        out = dict(generated)
        for layer in layers:
            out.update(layer)
        rank = out.get("apollo_rank", 0)
        if not isinstance(rank, int) or isinstance(rank, bool) or rank < 0:
            raise ValueError("apollo_rank must be an integer >= 0")
        if rank and any(p.ndim != 2 or min(p.shape) < rank for p in out["params"]):
            raise ValueError(f"Route {generated['group_name']!r} contains parameters ineligible for APOLLO rank "
                             f"{rank}")
        return out


def validate_policy(policy: Mapping[str, Any]) -> None:
    """Check a policy without a model (config.py:54-80)."""
    _Policy(policy)


def apply_policy(groups: List[Dict[str, Any]], policy: Mapping[str, Any]) -> List[Dict[str, Any]]:
    """New group dicts with the policy laid over ``groups`` (config.py:83-108);
    parameter lists and group order are kept.  Routes named in the mapping but
    absent from the model are allowed."""
    parsed = _Policy(policy)
    return [parsed.group(g) for g in groups]
