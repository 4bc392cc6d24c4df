"""build_param_groups and dictionary policies against the reference's outcomes.

The builder (routing.py:512-789) and policy overlay (config.py:83-108) are host
logic; ``tests/golden/routing_groups.json`` holds what the reference returned for
every call in ``routing_cases.CASES``: group names and order, parameter
membership, every option, warnings and error messages.  Each call is replayed on
this package and must match exactly.  The groups must also construct an
optimizer (constructor validation only; no step runs here).
"""
import json
import os

import pytest

import routing_cases

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "routing_groups.json")) as f:
    GOLDEN = json.load(f)


def test_fixture_covers_every_case():
    assert GOLDEN["cases"] == len(routing_cases.CASES)


@pytest.mark.parametrize("idx", range(len(routing_cases.CASES)),
                         ids=[f"{i}-{m}-{kw.get('preset')}-{kw.get('grouping', 'auto')}"
                              for i, (m, kw) in enumerate(routing_cases.CASES)])
def test_matches_reference(idx):
    from adafactor8bit import build_param_groups
    model, kw = routing_cases.CASES[idx]
    got = routing_cases.describe(build_param_groups, model, kw)
    want = GOLDEN["outcomes"][idx]
    assert json.loads(json.dumps(got)) == want


def test_groups_construct_the_optimizer():
    from adafactor8bit import Adafactor8Bit, build_param_groups
    model = routing_cases.TinyTextEncoder()
    groups = build_param_groups(model, preset="apollo", grouping="G2", apollo_rank=8,
                                apollo_targets=("self_attn", "linear1", "linear2"),
                                policy=routing_cases.EXAMPLE_POLICY)
    opt = Adafactor8Bit(groups, lr=1e-4)
    names = [g["group_name"] for g in opt.param_groups]
    assert names == [g["group_name"] for g in groups]
    assert sum(len(g["params"]) for g in opt.param_groups) == sum(1 for p in model.parameters() if p.requires_grad)
    ap = next(g for g in opt.param_groups if g["group_name"] == "apollo")
    assert ap["apollo_rank"] == 8 and ap["m_quant_type"] == "uf4" and ap["m_block_size"] == 128


def test_public_api():
    import adafactor8bit
    assert set(adafactor8bit.__all__) == {"Adafactor8Bit", "build_param_groups"}
    from adafactor8bit.config import apply_policy, validate_policy  # noqa: F401
    from adafactor8bit.presets import PRESETS
    assert tuple(PRESETS) == ("sgd", "adafactor", "adamw", "rmsprop", "came", "apollo")
