"""Models and calls that pin ``build_param_groups`` and policies.

Shared by ``gen_routing.py`` (which records what the reference builder returns
for each call) and ``tests/test_routing.py`` (which replays the calls on this
package).  A call's outcome is serialised by ``describe``: the groups (name,
parameters by qualified name, every other option), the warnings raised, or the
exception type and message.
"""
import copy
import warnings

import torch
from torch import nn


# ----------------------------------------------------------------------------
# Models (all tiny; weights are never used)
# ----------------------------------------------------------------------------

def demo_model():
    """Every G2 route once (the layout of examples/auto_presets.py:34-41)."""
    torch.manual_seed(0)
    m = nn.Module()
    m.token_embed = nn.Embedding(32, 256)
    m.norm = nn.LayerNorm(256)
    m.attn = nn.Linear(256, 256, bias=False)
    m.mlp = nn.Linear(256, 512, bias=False)
    m.output_projection = nn.Linear(512, 256, bias=False)
    m.lm_head = nn.Linear(256, 32, bias=False)
    m.conv = nn.Conv2d(3, 16, kernel_size=3, bias=False)
    return m


class _Block(nn.Module):
    def __init__(self, h):
        super().__init__()
        self.input_layernorm = nn.RMSNorm(h)
        self.q_proj = nn.Linear(h, h, bias=True)
        self.k_proj = nn.Linear(h, h // 2, bias=False)
        self.mlp = nn.Sequential(nn.Linear(h, 2 * h, bias=False), nn.Linear(2 * h, h, bias=False))
        self.gain = nn.Parameter(torch.ones(h))


def tied_model():
    """Decoder-like: tied token embedding / LM head, biases, RMSNorm, a
    positional embedding, a frozen weight, a 3-D parameter and a shared block."""
    torch.manual_seed(0)
    h = 48
    m = nn.Module()
    m.embed_tokens = nn.Embedding(96, h)
    m.pos_embedding = nn.Embedding(16, h)
    m.layers = nn.ModuleList([_Block(h), _Block(h)])
    m.shared = m.layers[0].k_proj            # a second name for one module
    m.frozen = nn.Linear(h, h)
    m.frozen.weight.requires_grad_(False)
    m.kernel3d = nn.Parameter(torch.zeros(4, h, 3))
    m.final_norm = nn.LayerNorm(h)
    m.lm_head = nn.Linear(h, 96, bias=False)
    m.lm_head.weight = m.embed_tokens.weight
    return m


def gpt_model():
    """GPT-2 style names (wte / wpe / c_attn / c_fc), untied head, a time embedding."""
    torch.manual_seed(0)
    m = nn.Module()
    m.transformer = nn.Module()
    m.transformer.wte = nn.Embedding(80, 40)
    m.transformer.wpe = nn.Embedding(20, 40)
    m.transformer.time_embed = nn.Linear(8, 40)
    m.transformer.h = nn.ModuleList()
    for _ in range(2):
        blk = nn.Module()
        blk.ln_1 = nn.LayerNorm(40)
        blk.attn = nn.Module()
        blk.attn.c_attn = nn.Linear(40, 120)
        blk.mlp = nn.Module()
        blk.mlp.c_fc = nn.Linear(40, 160)
        blk.mlp.c_proj = nn.Linear(160, 40)
        m.transformer.h.append(blk)
    m.lm_head = nn.Linear(40, 80, bias=False)
    return m


class TinyTextEncoder(nn.Module):
    """The encoder of examples/optimizer_from_config.py:18-32 (nn.TransformerEncoder)."""

    def __init__(self):
        super().__init__()
        torch.manual_seed(0)
        self.token_embed = nn.Embedding(256, 64)
        self.position_embed = nn.Embedding(32, 64)
        self.layers = nn.TransformerEncoder(
            nn.TransformerEncoderLayer(64, 4, 128, dropout=0.0, batch_first=True), num_layers=2,
            enable_nested_tensor=False)
        self.norm = nn.LayerNorm(64)


def empty_model():
    m = nn.Module()
    m.frozen = nn.Linear(4, 4)
    for p in m.frozen.parameters():
        p.requires_grad_(False)
    return m


MODELS = {"demo": demo_model, "tied": tied_model, "gpt": gpt_model, "encoder": TinyTextEncoder,
          "empty": empty_model}

# The policy of examples/custom_policy.json, as data.
EXAMPLE_POLICY = {
    "defaults": {"beta1": 0.9, "beta2": 0.999, "weight_decay": 0.001, "relative_step": False,
                 "scale_parameter": False, "scale_weight_decay": False, "block_size": 256,
                 "m_block_size": 256, "enable_fira_for_adafactor": True, "fira_margin": 0.01},
    "presets": {
        "adam": {"preset": "adamw", "factored": False, "beta3": None, "d": 0.0, "eps": [1e-8, 0.001]},
        "apollo_training": {"preset": "apollo", "beta3": None, "d": 0.0, "eps": [1e-8, 0.001],
                            "apollo_rank": 8, "apollo_update_proj_gap": 200, "apollo_scale_type": "channel",
                            "apollo_scale": 1.0, "apollo_eps": 1e-8, "apollo_factorize": False,
                            "apollo_cache_proj": False, "enable_fira_for_apollo": True},
    },
    "mapping": {
        "one_d": {"preset": "adam", "weight_decay": 0.0, "quantize": False},
        "embedding": {"preset": "adam", "beta1": None, "weight_decay": 0.0, "quantize": False},
        "matrix": {"preset": "adam", "quantize": True, "m_quant_type": "uf8", "v_quant_type": "al8"},
        "apollo": {"preset": "apollo_training", "quantize": True, "m_block_size": 128, "m_quant_type": "uf4",
                   "v_quant_type": "al8"},
    },
}


def _policy(**edits):
    p = copy.deepcopy(EXAMPLE_POLICY)
    for path, value in edits.items():
        keys = path.split("__")
        d = p
        for k in keys[:-1]:
            d = d.setdefault(k, {})
        if value is _DROP:
            d.pop(keys[-1], None)
        else:
            d[keys[-1]] = value
    return p


_DROP = object()


def _cases():
    out = []
    presets = ("sgd", "adafactor", "adamw", "rmsprop", "came", "apollo")
    for model in ("demo", "tied", "gpt"):
        for preset in presets:
            for grouping in ("auto", "G0", "bare", "G1", "protected", "G2", "topology"):
                kw = {"preset": preset, "grouping": grouping}
                if preset == "apollo" and model != "demo":
                    kw["apollo_rank"] = 16
                out.append((model, kw))
    # APOLLO targeting and rank
    out += [
        ("demo", dict(preset="apollo", grouping="G2", apollo_rank=128, apollo_targets=("attn", "mlp"),
                      embedding_lr=1e-4, embedding_quantize=False)),
        ("demo", dict(preset="apollo", apollo_rank=300)),
        ("demo", dict(preset="apollo", grouping="G1", apollo_rank=16, apollo_targets=("embed", "lm_head"))),
        ("demo", dict(preset="apollo", grouping="G0", apollo_rank=8, apollo_min_dim_multiplier=4)),
        ("demo", dict(preset="apollo", grouping="G2", apollo_rank=0, apollo_targets=("attn",))),
        ("demo", dict(preset="apollo", grouping="G2", apollo_rank=0)),
        ("tied", dict(preset="apollo", grouping="G2", apollo_rank=16, apollo_targets=("lm_head",))),
        ("tied", dict(preset="apollo", grouping="G2", apollo_rank=16, apollo_targets=("embed_tokens", "proj"))),
        ("tied", dict(preset="apollo", grouping="G1", apollo_rank=16, apollo_targets=["mlp", "shared", "kernel"])),
        ("gpt", dict(preset="apollo", grouping="G1", apollo_rank=32, apollo_targets=("c_attn", "c_fc", "wpe"),
                     apollo_min_dim_multiplier="AUTO")),
        ("encoder", dict(preset="apollo", grouping="G2", apollo_rank=8,
                         apollo_targets=("self_attn", "linear1", "linear2"))),
        # algorithm and route overrides
        ("demo", dict(preset="apollo", grouping="G1", apollo_rank=64, beta1=0.8, eps_came=1e-20, beta3=0.99,
                      apollo_scale_type="tensor", d=1.0, stochastic_round_writeback=True)),
        ("demo", dict(preset="adamw", grouping="G1", other_m_quant_type="uf4", other_block_size=256,
                      other_lr=3e-4, one_d_block_size=256)),
        ("demo", dict(preset="adamw", grouping="G1", one_d_quantize=True, one_d_block_size=256,
                      embedding_quantize="auto", embedding_m_block_size=64)),
        ("demo", dict(preset="rmsprop", grouping="G2", matrix_m_quant_type="d8", nd_c_quant_type="al16",
                      lm_head_stochastic_round_writeback=True, lm_head_min_8bit_size=0)),
        ("demo", dict(preset="came", grouping="G2", embedding_c_quant_type="al8", embedding_quantize=True,
                      matrix_c_quant_type=None, apollo_lr=1.0)),
        ("demo", dict(preset="adafactor", grouping="auto", embedding_quantize="Auto", lm_head_v_quant_type="al16")),
        ("tied", dict(preset="adamw", grouping="G1", lm_head_lr=1e-5, other_lr=1e-3)),
        ("tied", dict(preset="adamw", grouping="G2", lm_head_lr=1e-5, matrix_lr=2e-3, nd_quantize=False)),
        ("gpt", dict(preset="sgd", grouping="G0", beta1=0.9, all_m_quant_type="d4", momentum_only_1d=True)),
        ("gpt", dict(preset="adafactor", grouping="G2", nd_factored=True)),
        ("gpt", dict(preset="came", grouping="topology", nd_factored=False)),
        ("tied", dict(preset="came", grouping="G2", nd_factored=True)),
        ("tied", dict(preset="adafactor", grouping="G2", nd_factored=False, bias_correction=True, lag_norm=True,
                      fira_margin=0.05, enable_fira_for_adafactor=True, relative_step=True, scale_parameter=True,
                      scale_weight_decay=True, eps=(1e-30, 1e-3), beta2_decay=-0.5, beta2=None)),
        ("empty", dict(preset="adamw")),
        ("empty", dict(preset="apollo", policy=EXAMPLE_POLICY)),
        # errors
        ("demo", dict(preset="lion")),
        ("demo", dict(preset="ADAMW")),
        ("demo", dict(preset="adamw", grouping="G3")),
        ("demo", dict(preset="adamw", grouping="BARE")),
        ("demo", dict(preset="adamw", grouping=None)),
        ("demo", dict(preset="adamw", grouping="G1", nd_factored=True)),
        ("demo", dict(preset="adamw", grouping="G2", nd_factored=True)),
        ("demo", dict(preset="came", grouping="G2", nd_factored=1)),
        ("demo", dict(preset="adamw", apollo_rank=8)),
        ("demo", dict(preset="adamw", apollo_targets=("attn",))),
        ("demo", dict(preset="adamw", apollo_min_dim_multiplier=2)),
        ("demo", dict(preset="apollo", apollo_rank=True)),
        ("demo", dict(preset="apollo", apollo_rank=-1)),
        ("demo", dict(preset="apollo", apollo_rank=8.0)),
        ("demo", dict(preset="apollo", apollo_targets="attn")),
        ("demo", dict(preset="apollo", apollo_targets=None)),
        ("demo", dict(preset="apollo", apollo_targets=("attn", ""))),
        ("demo", dict(preset="apollo", apollo_min_dim_multiplier=0)),
        ("demo", dict(preset="apollo", apollo_min_dim_multiplier="two")),
        ("demo", dict(preset="adamw", factored=True)),
        ("demo", dict(preset="adamw", momentum=0.9)),
        ("demo", dict(preset="adamw", lr=1e-3)),
        ("demo", dict(preset="adamw", head_lr=1e-3)),
        ("demo", dict(preset="adamw", other_block_size=100)),
        ("demo", dict(preset="adamw", other_block_size=True)),
        ("demo", dict(preset="adamw", other_m_block_size=30)),
        ("demo", dict(preset="adamw", other_m_block_size=34)),
        ("demo", dict(preset="adamw", other_lr=-1.0)),
        ("demo", dict(preset="adamw", other_lr=None)),
        ("demo", dict(preset="adamw", other_quantize="yes")),
        ("demo", dict(preset="adamw", other_m_quant_type="int8")),
        ("demo", dict(preset="adamw", other_v_quant_type="uf8")),
        ("demo", dict(preset="adamw", other_c_quant_type="d8")),
        ("demo", dict(preset="adamw", other_min_8bit_size=-1)),
        ("demo", dict(preset="adamw", other_stochastic_round_writeback=1)),
        ("params", dict(preset="adamw")),
        # policies
        ("encoder", dict(preset="apollo", grouping="G2", apollo_rank=8,
                         apollo_targets=("self_attn", "linear1", "linear2"), policy=EXAMPLE_POLICY)),
        ("demo", dict(preset="adamw", grouping="G2", policy=EXAMPLE_POLICY)),
        ("demo", dict(preset="adamw", grouping="G1", policy={"defaults": {"lr": 5e-4},
                                                             "mapping": {"other": {"preset": "came"}}})),
        ("demo", dict(preset="came", grouping="G2", policy={
            "presets": {"a": {"preset": "b", "beta1": 0.7}, "b": {"preset": "rmsprop", "lr": 2e-3}},
            "mapping": {"matrix": {"preset": "a"}, "nd": {"preset": "sgd", "beta1": 0.5}}})),
        ("demo", dict(preset="apollo", grouping="G2", apollo_rank=16,
                      policy={"mapping": {"apollo": {"preset": "apollo", "apollo_rank": 8}}})),
        ("demo", dict(preset="adamw", policy={"extra": {}})),
        ("demo", dict(preset="adamw", policy=[("defaults", {})])),
        ("demo", dict(preset="adamw", policy={"defaults": {"momentum": 0.9}})),
        ("demo", dict(preset="adamw", policy={"defaults": {"block_size": 100}})),
        ("demo", dict(preset="adamw", policy={"defaults": []})),
        ("demo", dict(preset="adamw", policy={"presets": []})),
        ("demo", dict(preset="adamw", policy={"presets": {"adamw": {"preset": "sgd"}}})),
        ("demo", dict(preset="adamw", policy={"presets": {"": {"preset": "sgd"}}})),
        ("demo", dict(preset="adamw", policy={"presets": {"x": 3}})),
        ("demo", dict(preset="adamw", policy={"presets": {"x": {"beta1": 0.5}}})),
        ("demo", dict(preset="adamw", policy={"presets": {"x": {"preset": "y"}, "y": {"preset": "x"}}})),
        ("demo", dict(preset="adamw", policy={"presets": {"x": {"preset": 3}}})),
        ("demo", dict(preset="adamw", policy={"presets": {"x": {"preset": "nope"}}})),
        ("demo", dict(preset="adamw", policy={"mapping": {"attention": {}}})),
        ("demo", dict(preset="adamw", policy={"mapping": {"other": 1}})),
        ("demo", dict(preset="adamw", policy={"mapping": {"other": {"preset": "nope"}}})),
        ("demo", dict(preset="adamw", policy={"mapping": {"other": {"m_quant_type": "q"}}})),
        ("demo", dict(preset="adamw", grouping="G1", policy={"mapping": {"other": {"apollo_rank": 1024}}})),
        ("demo", dict(preset="adamw", grouping="G1", policy={"mapping": {"one_d": {"apollo_rank": 4}}})),
        ("demo", dict(preset="adamw", grouping="G1", policy={"mapping": {"other": {"apollo_rank": -2}}})),
        ("demo", dict(preset="adamw", grouping="G1", policy={"mapping": {"other": {"apollo_rank": 2.0}}})),
    ]
    return out


CASES = _cases()


def _plain(v):
    if isinstance(v, (tuple, list)):
        return [_plain(x) for x in v]
    if isinstance(v, dict):
        return {k: _plain(x) for k, x in v.items()}
    if isinstance(v, float) and v != v:
        return "nan"
    return v


def describe(build, model_name, kwargs):
    """Run ``build(model, **kwargs)`` and serialise its outcome."""
    if model_name == "params":
        model = demo_model().parameters()
        names = {}
    else:
        model = MODELS[model_name]()
        names = {}
        for n, p in model.named_parameters(remove_duplicate=False):
            names.setdefault(id(p), n)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        try:
            groups = build(model, **copy.deepcopy(kwargs))
        except Exception as e:   # the outcome being recorded
            return {"error": [type(e).__name__, str(e)],
                    "warnings": [str(w.message) for w in caught]}
    out = []
    for g in groups:
        d = {k: _plain(v) for k, v in g.items() if k != "params"}
        d["params"] = [names[id(p)] for p in g["params"]]
        out.append(d)
    return {"groups": out, "warnings": [str(w.message) for w in caught]}
