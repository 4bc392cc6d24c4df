"""Model-aware parameter groups for Adafactor8Bit (the reference's routing.py).

``build_param_groups(model, preset, grouping, ...)`` returns ordinary PyTorch
parameter-group dicts with the same names, membership, order and options as the
reference's builder (routing.py:512-789), so a training script that builds its
groups there builds identical ones here.

How a parameter is placed:

1. Every trainable Parameter is visited once, in module order, with all the
   names it is reachable under (routing.py:126-181).
2. Its role is ``one_d`` (ndim <= 1, owned by a norm layer, or named ``bias``),
   ``embedding`` (an ``nn.Embedding`` or a name containing ``embed``/``wte``,
   positional and time embeddings excluded), ``lm_head``, ``matrix`` (other 2-D)
   or ``nd`` (routing.py:184-204).  A tied embedding/LM head is an embedding.
3. Under an APOLLO preset a 2-D weight whose name contains a target substring and
   whose smaller side is at least ``rank * multiplier`` goes to ``apollo``;
   protected roles only when targeted explicitly (routing.py:207-238, 645-652).
4. The grouping decides which roles share a group (routing.py:654-672):
   G0 one group (``apollo`` + ``fallback`` for APOLLO), G1 ``one_d``,
   ``embedding``, ``lm_head``, ``apollo``, ``other``, G2 ``one_d``,
   ``embedding``, ``lm_head``, ``apollo``, ``matrix``, ``nd``.

Route options (``<route>_<option>=value``) override a group's state formats,
block sizes, learning rate and quantization; algorithm options (``beta1``,
``eps``, ...) override the preset.  Error types, messages and warnings are the
reference's.
"""
from __future__ import annotations

import warnings
from collections import defaultdict
from dataclasses import dataclass
from typing import Any, Dict, List, Mapping, Optional, Sequence, Tuple, Union

from torch import nn

from .presets import PRESETS, PresetSpec, _preset_names

__all__ = ["build_param_groups"]

# Accepted spellings of the three groupings (routing.py:55-59); "auto" is
# matched case-insensitively on its own.
_GROUPING_ALIASES = {"G0": "G0", "g0": "G0", "bare": "G0",
                     "G1": "G1", "g1": "G1", "protected": "G1",
                     "G2": "G2", "g2": "G2", "topology": "G2"}

# Every group name the builder can produce (routing.py:62-65).
_ROUTE_NAMES = {"all", "fallback", "other", "one_d", "embedding", "lm_head", "apollo", "matrix", "nd"}

# Route option suffixes, tried in this order so that the longer of two
# overlapping suffixes wins (``m_block_size`` before ``block_size``).
_ROUTE_OPTION_SUFFIXES = ("m_quant_type", "v_quant_type", "c_quant_type", "stochastic_round_writeback",
                          "min_8bit_size", "m_block_size", "block_size", "quantize", "lr")

_M_TYPES = {"fp32", "uf4", "uf8", "d4", "d8"}
_VC_TYPES = {"fp32", "al8", "al16"}

# Algorithm overrides that reach both an APOLLO preset's primary and fallback
# paths, and those that reach only the primary one (routing.py:80-95).
_COMMON_OVERRIDE_KEYS = {"beta1", "beta2", "beta2_decay", "bias_correction", "relative_step",
                         "scale_parameter", "scale_weight_decay", "d", "eps", "fira_margin", "lag_norm",
                         "momentum_only_1d", "enable_fira_for_adafactor", "stochastic_round_writeback"}
_PRIMARY_OVERRIDE_KEYS = {"beta3", "eps_came", "apollo_factorize", "apollo_update_proj_gap",
                          "apollo_scale_type", "apollo_scale", "apollo_scale_front", "apollo_eps",
                          "apollo_cache_proj", "enable_fira_for_apollo"}

_PROTECTED = ("one_d", "embedding", "lm_head")
_PRECISION_KEYS = ("m_quant_type", "v_quant_type", "c_quant_type", "min_8bit_size", "m_block_size", "block_size")

_NORM_TYPES = tuple(getattr(nn, n) for n in (
    "BatchNorm1d", "BatchNorm2d", "BatchNorm3d", "SyncBatchNorm", "InstanceNorm1d", "InstanceNorm2d",
    "InstanceNorm3d", "LayerNorm", "GroupNorm", "LocalResponseNorm", "RMSNorm") if hasattr(nn, n))


# ----------------------------------------------------------------------------
# Parameter discovery and roles
# ----------------------------------------------------------------------------

def _is_excluded_embedding_name(name: str) -> bool:
    low = name.lower()
    return any(s in low for s in ("position", "pos_embed", "wpe", "time"))


@dataclass
class _Param:
    param: nn.Parameter
    names: List[Tuple[str, nn.Module, str]]   # (qualified name, owning module, attribute name)

    @property
    def aliases(self) -> Tuple[str, ...]:
        return tuple(n for n, _, _ in self.names)

    @property
    def embedding_aliases(self) -> Tuple[str, ...]:
        out = []
        for name, owner, _ in self.names:
            if _is_excluded_embedding_name(name):
                continue
            low = name.lower()
            if isinstance(owner, nn.Embedding) or "embed" in low or "wte" in low:
                out.append(name)
        return tuple(out)

    @property
    def lm_head_aliases(self) -> Tuple[str, ...]:
        return tuple(n for n in self.aliases if "lm_head" in n.lower())

    def role(self) -> str:
        """routing.py:184-204"""
        p = self.param
        if (p.ndim <= 1 or any(isinstance(m, _NORM_TYPES) for _, m, _ in self.names)
                or any(local.lower() == "bias" for _, _, local in self.names)):
            return "one_d"
        if self.embedding_aliases:
            return "embedding"
        if self.lm_head_aliases:
            return "lm_head"
        return "matrix" if p.ndim == 2 else "nd"


def _collect_params(model: nn.Module) -> List[_Param]:
    """One entry per trainable Parameter in first-seen order, with every name it
    is reachable under, shared submodules included (routing.py:126-181)."""
    found: Dict[int, _Param] = {}
    try:
        modules = model.named_modules(remove_duplicate=False)
    except TypeError:
        modules = model.named_modules()
    for mod_name, mod in modules:
        for local, p in mod.named_parameters(recurse=False):
            if p.requires_grad:
                entry = found.setdefault(id(p), _Param(p, []))
                entry.names.append((f"{mod_name}.{local}" if mod_name else local, mod, local))
    # Parameters reachable only through a module's own named_parameters().
    for name, p in model.named_parameters():
        if p.requires_grad and id(p) not in found:
            found[id(p)] = _Param(p, [(name, model, name.rsplit(".", 1)[-1])])
    return list(found.values())


def _name_hits(names: Sequence[str], targets: Sequence[str]) -> bool:
    return any(t.lower() in n.lower() for n in names for t in targets)


def _apollo_target(rec: _Param, role: str, targets: Optional[Sequence[str]], explicit: bool) -> Tuple[bool, bool]:
    """(matches, matched only through the LM-head name of a tied embedding),
    routing.py:207-232.  ``targets=None`` matches everything."""
    if targets is None:
        return True, False
    if not targets or not _name_hits(rec.aliases, targets):
        return False, False
    if explicit and role == "embedding" and rec.lm_head_aliases and not _name_hits(rec.embedding_aliases, targets):
        return False, True
    return True, False


# ----------------------------------------------------------------------------
# Option handling
# ----------------------------------------------------------------------------

def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _validate_route_options(route: str, opts: Mapping[str, Any]):
    """Type and range checks of route options (routing.py:241-295)."""
    if "stochastic_round_writeback" in opts and not isinstance(opts["stochastic_round_writeback"], bool):
        raise TypeError(f"{route}_stochastic_round_writeback must be bool")
    if "m_quant_type" in opts and opts["m_quant_type"] not in _M_TYPES:
        raise ValueError(f"Invalid {route}_m_quant_type={opts['m_quant_type']!r}; "
                         f"expected one of {sorted(_M_TYPES)}")
    if "v_quant_type" in opts and opts["v_quant_type"] not in _VC_TYPES:
        raise ValueError(f"Invalid {route}_v_quant_type={opts['v_quant_type']!r}; "
                         f"expected one of {sorted(_VC_TYPES)}")
    if "c_quant_type" in opts and opts["c_quant_type"] is not None and opts["c_quant_type"] not in _VC_TYPES:
        raise ValueError(f"Invalid {route}_c_quant_type={opts['c_quant_type']!r}; "
                         f"expected None or one of {sorted(_VC_TYPES)}")
    if "lr" in opts:
        v = opts["lr"]
        if v is None or not isinstance(v, (int, float)) or isinstance(v, bool) or v < 0:
            raise ValueError(f"Invalid {route}_lr={v!r}; expected a number >= 0")
    if "quantize" in opts:
        v = opts["quantize"]
        if not isinstance(v, bool) and not (isinstance(v, str) and v.lower() == "auto"):
            raise TypeError(f"{route}_quantize must be True, False, or 'auto'")
    if "block_size" in opts:
        v = opts["block_size"]
        if not _is_int(v) or v < 128 or v % 128 != 0:
            raise ValueError(f"{route}_block_size must be >= 128 and a multiple of 128")
    if "m_block_size" in opts:
        v = opts["m_block_size"]
        if not _is_int(v) or v < 32 or v % 4 != 0:
            raise ValueError(f"{route}_m_block_size must be >= 32 and a multiple of 4")
    if "min_8bit_size" in opts:
        v = opts["min_8bit_size"]
        if not _is_int(v) or v < 0:
            raise ValueError(f"{route}_min_8bit_size must be an integer >= 0")


def _split_overrides(overrides: Mapping[str, Any]):
    """Split keyword overrides into algorithm options and per-route options
    (routing.py:298-330)."""
    algorithm: Dict[str, Any] = {}
    routes: Dict[str, Dict[str, Any]] = defaultdict(dict)
    for key, value in overrides.items():
        if key in _COMMON_OVERRIDE_KEYS or key in _PRIMARY_OVERRIDE_KEYS:
            algorithm[key] = value
            continue
        suffix = next((s for s in _ROUTE_OPTION_SUFFIXES if key.endswith("_" + s)), None)
        if suffix is None:
            if key == "factored":
                raise TypeError("build_param_groups() owns 'factored' per route; edit the returned "
                                "group dict for expert overrides.")
            raise TypeError(f"Unknown build_param_groups() override: {key!r}")
        route = key[:-len(suffix) - 1]
        if route not in _ROUTE_NAMES:
            raise TypeError(f"Unknown route prefix {route!r} in {key!r}. Known routes: {sorted(_ROUTE_NAMES)}")
        routes[route][suffix] = value
    for route, opts in routes.items():
        _validate_route_options(route, opts)
    return algorithm, dict(routes)


def _full_rank(semantics: Mapping[str, Any], drop_momentum: bool = False) -> Dict[str, Any]:
    """Unfactored, unscaled, unclipped, no confidence; beta2 untouched
    (routing.py:347-359)."""
    out = dict(semantics, factored=False, scale_parameter=False, d=0.0, beta3=None)
    if drop_momentum:
        out["beta1"] = None
    return out


def _default_quantize(preset: str, grouping: str, route: str, auto_profile: bool) -> Optional[bool]:
    """Quantization a route gets when its ``quantize`` option is ``"auto"``;
    None keeps the optimizer's own setting (routing.py:362-392).  G1 keeps
    vectors full precision and, when chosen explicitly, embeddings and LM heads
    too; the automatic profile quantizes those two except under Adafactor and
    RMSprop.  G2 keeps vectors and embeddings full precision."""
    if grouping == "G1":
        if route == "one_d":
            return False
        if route in ("embedding", "lm_head") and (not auto_profile or preset in ("adafactor", "rmsprop")):
            return False
        if route in ("embedding", "lm_head"):
            return None
    if grouping == "G2" and route in ("one_d", "embedding"):
        return False
    return None


@dataclass
class _Build:
    preset: str
    grouping: str
    auto_profile: bool
    route_options: Mapping[str, Mapping[str, Any]]

    def group(self, name: str, params: List[nn.Parameter], semantics: Mapping[str, Any],
              wd_zero: bool = False, rank: Optional[int] = None) -> Optional[Dict[str, Any]]:
        """One group dict, or None when it would be empty (routing.py:410-478)."""
        if not params:
            return None
        g: Dict[str, Any] = {"params": list(params), "group_name": name, **semantics,
                             "apollo_rank": 0 if rank is None else int(rank)}
        if wd_zero:
            g["weight_decay"] = 0.0
        raw = self.route_options.get(name, {})
        explicit = raw.get("quantize", "auto")
        if isinstance(explicit, str):
            q = _default_quantize(self.preset, self.grouping, name, self.auto_profile)
        else:
            q = explicit
        if q is not None:
            g["quantize"] = q
        if q is False and isinstance(explicit, str) and any(k in raw for k in _PRECISION_KEYS):
            warnings.warn(f"Route {name!r} is unquantized by its auto policy, so explicit "
                          "precision/block options are inactive unless "
                          f"{name}_quantize=True is also set.", UserWarning, stacklevel=3)
        g.update((k, v) for k, v in raw.items() if k != "quantize")
        if g.get("quantize", True):
            if g.get("beta1") is None and ("m_quant_type" in raw or "m_block_size" in raw):
                warnings.warn(f"Route {name!r} has beta1=None, so its explicit M-state "
                              "quantization options are currently inactive.", UserWarning, stacklevel=3)
            if g.get("beta3") is None and "c_quant_type" in raw:
                warnings.warn(f"Route {name!r} has beta3=None, so its explicit C-state "
                              "quantization option is currently inactive.", UserWarning, stacklevel=3)
        return g


def _grouping_of(spec: PresetSpec, grouping) -> Tuple[str, bool]:
    if grouping is None:
        raise TypeError("grouping=None is ambiguous; use 'auto' or G0/G1/G2")
    if isinstance(grouping, str) and grouping.lower() == "auto":
        return spec.default_grouping, True
    key = _GROUPING_ALIASES.get(str(grouping))
    if key is None:
        raise ValueError(f"Unknown grouping {grouping!r}; use 'auto', G0/bare, G1/protected or G2/topology.")
    return key, False


def _targets_of(spec: PresetSpec, value) -> Tuple[Optional[Tuple[str, ...]], bool]:
    if isinstance(value, str):
        if value.lower() != "auto":
            raise TypeError("apollo_targets must be 'auto' or a sequence such as ['attn', 'mlp']")
        return (None if spec.default_apollo_targets is None else tuple(spec.default_apollo_targets)), False
    if value is None:
        raise TypeError("apollo_targets=None is ambiguous; use 'auto' or an explicit sequence")
    targets = tuple(value)
    if any(not isinstance(t, str) or not t for t in targets):
        raise TypeError("apollo_targets entries must be non-empty strings")
    return targets, True


def _multiplier_of(spec: PresetSpec, value) -> int:
    if isinstance(value, str) and value.lower() == "auto":
        return spec.default_apollo_min_dim_multiplier
    if not _is_int(value) or value < 1:
        raise ValueError("apollo_min_dim_multiplier must be 'auto' or an integer >= 1")
    return value


# ----------------------------------------------------------------------------
# The builder
# ----------------------------------------------------------------------------

def build_param_groups(
    model: nn.Module,
    preset: str,
    grouping: str = "auto",
    *,
    apollo_rank: Optional[int] = None,
    apollo_targets: Union[str, Sequence[str]] = "auto",
    apollo_min_dim_multiplier: Union[str, int] = "auto",
    nd_factored: Optional[bool] = None,
    policy: Optional[Mapping[str, Any]] = None,
    **overrides: Any,
) -> List[Dict[str, Any]]:
    """Parameter groups for ``model`` under ``preset`` (routing.py:512-789).

    ``grouping`` is ``"auto"`` (the preset's default, G1, with the automatic
    quantization profile) or G0/G1/G2 and their aliases.  ``apollo_*`` apply to
    the APOLLO preset only.  ``policy`` is a ``{"defaults", "presets",
    "mapping"}`` dict applied last (see :mod:`adafactor8bit.config`).  Keyword
    ``overrides`` are algorithm options or ``<route>_<option>`` route options.
    Parameter values and dtypes are never touched.
    """
    if not isinstance(model, nn.Module):
        raise TypeError("build_param_groups() expects an nn.Module, not model.parameters()")
    preset_key = str(preset).lower()
    if preset_key not in PRESETS:
        raise ValueError(f"Unknown preset {preset!r}. Available presets: {', '.join(_preset_names())}")
    spec = PRESETS[preset_key]
    grouping_key, auto_profile = _grouping_of(spec, grouping)

    if nd_factored is not None:
        if not isinstance(nd_factored, bool):
            raise TypeError("nd_factored must be bool or None")
        if grouping_key != "G2":
            raise ValueError("nd_factored is only meaningful with G2/topology grouping")
        if nd_factored and preset_key not in ("adafactor", "came"):
            raise ValueError(f"nd_factored=True is not part of the {preset_key!r} preset semantics; "
                             "use adafactor/came or edit the returned nd group explicitly.")

    algorithm, route_options = _split_overrides(overrides)
    primary = dict(spec.primary)
    fallback = dict(spec.fallback if spec.fallback is not None else spec.primary)
    for k, v in algorithm.items():
        primary[k] = v
        if k in _COMMON_OVERRIDE_KEYS:
            fallback[k] = v

    apollo_preset = spec.default_apollo_rank > 0
    if not apollo_preset:
        for arg, given in (("apollo_rank", apollo_rank is not None),
                           ("apollo_targets", apollo_targets != "auto"),
                           ("apollo_min_dim_multiplier", apollo_min_dim_multiplier != "auto")):
            if given:
                raise ValueError(f"{arg} requires an APOLLO-capable preset; got {preset_key!r}")
        rank, targets, explicit, multiplier = 0, (), False, 1
    else:
        if apollo_rank is None:
            rank = spec.default_apollo_rank
        elif not _is_int(apollo_rank):
            raise TypeError("apollo_rank must be an integer >= 0 or None")
        else:
            rank = apollo_rank
        if rank < 0:
            raise ValueError("apollo_rank must be >= 0")
        targets, explicit = _targets_of(spec, apollo_targets)
        multiplier = _multiplier_of(spec, apollo_min_dim_multiplier)
        if rank == 0:
            if explicit and targets:
                warnings.warn("apollo_rank=0 disables APOLLO; explicit apollo_targets are ignored.",
                              UserWarning, stacklevel=2)
            targets = ()

    if policy is not None:
        from .config import apply_policy

    params = _collect_params(model)
    if not params:
        return apply_policy([], policy) if policy is not None else []

    tied = any(r.embedding_aliases and r.lm_head_aliases for r in params)
    tied_override_warned = "lm_head" in route_options and tied
    if tied_override_warned:
        warnings.warn("A token embedding and lm_head share the same Parameter. The shared tensor "
                      "is routed as 'embedding', so lm_head_* overrides do not apply to that tied "
                      "Parameter; any untied lm_head parameters still use the lm_head route.",
                      UserWarning, stacklevel=2)

    buckets: Dict[str, List[nn.Parameter]] = defaultdict(list)
    warned_tied_target = False
    for rec in params:
        role = rec.role()
        hit, tied_head_only = _apollo_target(rec, role, targets, explicit)
        if tied_head_only and not warned_tied_target:
            warnings.warn("apollo_targets matched only the lm_head alias of a tied embedding/lm_head "
                          "Parameter. The shared tensor is treated as 'embedding' and remains on the "
                          "embedding route unless an embedding alias is explicitly targeted.",
                          UserWarning, stacklevel=2)
            warned_tied_target = True
        p = rec.param
        shape_ok = rank > 0 and p.ndim == 2 and min(p.shape) >= rank * multiplier
        protected = role in _PROTECTED
        low_rank = (apollo_preset and hit and shape_ok
                    and (not protected or (explicit and role in ("embedding", "lm_head"))))
        if low_rank:
            route = "apollo"
        elif grouping_key == "G0":
            route = "fallback" if apollo_preset else "all"
        elif grouping_key == "G1":
            route = role if protected else "other"
        else:
            route = role
        buckets[route].append(p)

    # Group layout per grouping: (route, semantics, weight decay forced to 0, carries the rank).
    base = fallback if apollo_preset else primary
    if grouping_key == "G0":
        layout = [("apollo", primary, False, True), ("fallback", fallback, False, False)] if apollo_preset \
            else [("all", primary, False, False)]
    elif grouping_key == "G1":
        layout = [("one_d", base, True, False), ("embedding", base, True, False), ("lm_head", base, True, False),
                  ("apollo", primary, False, True), ("other", base, False, False)]
    else:
        nd_fact = spec.default_nd_factored if nd_factored is None else nd_factored
        layout = [("one_d", base, True, False), ("embedding", _full_rank(base, drop_momentum=True), True, False),
                  ("lm_head", _full_rank(base), True, False), ("apollo", primary, False, True),
                  ("matrix", base, False, False), ("nd", dict(base) if nd_fact else _full_rank(base), False, False)]

    b = _Build(preset_key, grouping_key, auto_profile, route_options)
    groups = []
    for route, semantics, wd_zero, carries_rank in layout:
        g = b.group(route, buckets.get(route, []), semantics, wd_zero, rank if carries_rank else None)
        if g is not None:
            groups.append(g)

    placed = [id(p) for g in groups for p in g["params"]]
    if len(placed) != len(set(placed)) or set(placed) != {id(r.param) for r in params}:
        raise RuntimeError("Internal routing error: parameters were duplicated or omitted")

    made = {g["group_name"] for g in groups}
    for route in route_options:
        if route in made or (route == "lm_head" and tied_override_warned):
            continue
        warnings.warn(f"Route override for {route!r} did not match a generated group.", UserWarning, stacklevel=2)

    if policy is not None:
        groups = apply_policy(groups, policy)
    return groups
