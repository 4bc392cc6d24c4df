"""Semantic presets for :func:`adafactor8bit.build_param_groups`.

The table mirrors presets.py:15-169 of the reference key for key and value for
value: a preset is a named set of constructor options that selects an update
path (SGD, Adafactor, AdamW, RMSprop, CAME, APOLLO), and a group built from it
must configure the optimizer exactly as the reference's would.  Learning rate,
weight decay and state formats are not part of a preset; they stay constructor
or route options.
"""
from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

__all__ = ["PresetSpec", "PRESETS"]


@dataclass(frozen=True)
class PresetSpec:
    """One preset (presets.py:15-24).

    ``primary`` configures the preset's own path; ``fallback`` (APOLLO only)
    configures parameters the low-rank path does not take.  The ``default_*``
    fields are what ``build_param_groups`` uses for its ``"auto"`` arguments.
    """
    name: str
    default_grouping: str
    primary: Dict[str, Any]
    fallback: Optional[Dict[str, Any]] = None
    default_apollo_rank: int = 0
    default_apollo_targets: Optional[Tuple[str, ...]] = None
    default_apollo_min_dim_multiplier: int = 1
    default_nd_factored: bool = False


# Options every non-factored, constant-step preset turns off (no RMS scaling of
# the step, no scaled weight decay, no update clipping).
_PLAIN = {"beta2_decay": None, "beta3": None, "factored": False, "relative_step": False,
          "scale_parameter": False, "scale_weight_decay": False, "d": 0.0}

# presets.py:30-40: no moments at all, the optimizer's SGD mode.
_SGD = dict(_PLAIN, beta1=None, beta2=None)

# presets.py:42-49: factored second moment with the step-dependent decay -0.8.
_ADAFACTOR = {"beta1": None, "beta2": None, "beta2_decay": -0.8, "beta3": None,
              "factored": True, "relative_step": False}

# presets.py:51-62
_ADAMW = dict(_PLAIN, beta1=0.9, beta2=0.999, eps=(1e-8, 1e-3))

# presets.py:64-75
_RMSPROP = dict(_PLAIN, beta1=None, beta2=0.99, eps=(1e-8, 1e-3))

# presets.py:77-88: factored V and confidence with update clipping d = 1.
_CAME = dict(_PLAIN, beta1=0.9, beta2=0.999, beta3=0.9999, factored=True, d=1.0, eps_came=1e-16)

# presets.py:90-104: full-rank Adam for what APOLLO does not take, with APOLLO's eps.
_APOLLO_FALLBACK = dict(_PLAIN, beta1=0.9, beta2=0.999, eps=(1e-6, 1e-3))

# presets.py:106-125
_APOLLO = dict(_APOLLO_FALLBACK, apollo_eps=1e-6, apollo_factorize=False, apollo_update_proj_gap=200,
               apollo_scale_type="channel", apollo_scale=1.0, apollo_scale_front=False,
               apollo_cache_proj=True, enable_fira_for_apollo=True)

# presets.py:128-165
PRESETS: Dict[str, PresetSpec] = {
    "sgd": PresetSpec("sgd", "G1", _SGD),
    "adafactor": PresetSpec("adafactor", "G1", _ADAFACTOR),
    "adamw": PresetSpec("adamw", "G1", _ADAMW),
    "rmsprop": PresetSpec("rmsprop", "G1", _RMSPROP),
    "came": PresetSpec("came", "G1", _CAME),
    "apollo": PresetSpec("apollo", "G1", _APOLLO, fallback=_APOLLO_FALLBACK, default_apollo_rank=256,
                         default_apollo_targets=("attn", "mlp"), default_apollo_min_dim_multiplier=1),
}


def _preset_names() -> Tuple[str, ...]:
    return tuple(PRESETS)
