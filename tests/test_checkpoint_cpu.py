"""load_state_dict / state_dict on the host (no kernels run): reference checkpoints
(tests/golden/ckpt_*.npz) load with every state tensor in its stored dtype, the
codec tags, step counts and seed counters restored, and round-trip exactly
(the reference's load path, optimizer.py:1463-1553)."""
import pytest
import torch

from test_gpu_checkpoint import SCENARIOS, _load, _params, checkpoint


def _points(name):
    meta, kw, z = _load(name)
    return [(meta, kw, z, tag) for tag in meta["points"]]


CASES = [(n, i) for n in SCENARIOS for i in range(len(_load(n)[0]["points"]))]


def _same(a, b):
    if torch.is_tensor(a) or torch.is_tensor(b):
        return torch.is_tensor(a) and torch.is_tensor(b) and a.dtype == b.dtype and a.shape == b.shape and \
            torch.equal(a.cpu(), b.cpu())
    if isinstance(a, (torch.Size, tuple, list)) and isinstance(b, (torch.Size, tuple, list)):
        return list(a) == list(b)
    return a == b


@pytest.mark.parametrize("name,point", CASES, ids=[f"{n}-ph{i}" for n, i in CASES])
def test_reference_checkpoint_loads_and_round_trips(name, point):
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = _load(name)
    tag = sorted(meta["points"])[point]
    ck = checkpoint(meta, z, tag)
    params = _params(meta, dev="cpu")
    opt = Adafactor8Bit(params, **kw)
    opt.load_state_dict(ck)
    for idx, saved in ck["state"].items():
        st = opt.state[params[idx]]
        apollo = "apollo_seed" in saved
        for k, v in saved.items():
            if apollo and k in ("m", "m_q", "m_scale"):
                continue
            assert k in st and _same(st[k], v), (tag, idx, k)
        assert isinstance(st["step"], int)
    again = opt.state_dict()
    assert again["_apollo_seed_counter"] == ck["_apollo_seed_counter"]
    assert again["_sr_seed_counter"] == ck["_sr_seed_counter"]
    for idx, saved in ck["state"].items():
        for k, v in saved.items():
            assert _same(again["state"][idx][k], v), (tag, idx, k)
    for g, sg in zip(again["param_groups"], ck["param_groups"]):
        for k, v in sg.items():
            assert _same(g[k], v), k


def test_bf16_parameters_keep_fp32_state():
    """The base loader would cast floating-point state to the parameter dtype."""
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = _load("ckpt_adamw_bf16_sr_policy")
    ck = checkpoint(meta, z, "ph0")
    params = _params(meta, dev="cpu")
    assert params[0].dtype == torch.bfloat16
    opt = Adafactor8Bit(params, **kw)
    opt.load_state_dict(ck)
    small = opt.state[params[1]]          # 300 elements: fp32 state
    assert small["variance"].dtype == torch.float32 and small["m"].dtype == torch.float32
    big = opt.state[params[0]]
    assert big["variance_q"].dtype == torch.uint8 and big["variance_scale"].dtype == torch.float32


@pytest.mark.parametrize("current", [True, False])
def test_sr_policy_backfilled_only_when_missing(current):
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = _load("ckpt_adamw_bf16_sr_policy")
    ck = checkpoint(meta, z, "ph0")
    params = _params(meta, dev="cpu")
    opt = Adafactor8Bit(params, **dict(kw, stochastic_round_writeback=current))
    del ck["param_groups"][0]["stochastic_round_writeback"]     # a checkpoint from before the option
    opt.load_state_dict(ck)
    assert opt.param_groups[0]["stochastic_round_writeback"] is current
    ck = checkpoint(meta, z, "ph0")                              # saved explicitly (False): kept
    opt = Adafactor8Bit(_params(meta, dev="cpu"), **dict(kw, stochastic_round_writeback=True))
    opt.load_state_dict(ck)
    assert opt.param_groups[0]["stochastic_round_writeback"] is False


def test_apollo_full_rank_momentum_dropped_and_tags_defaulted():
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = _load("ckpt_apollo_quant_flip")
    ck = checkpoint(meta, z, "ph0")
    ck["state"][0]["m"] = torch.ones(3)
    ck["state"][0]["m_q"] = torch.ones(3, dtype=torch.uint8)
    del ck["state"][1]["v_quant_type"]
    del ck["state"][1]["m_quant_type"]
    del ck["_apollo_seed_counter"]
    params = _params(meta, dev="cpu")
    opt = Adafactor8Bit(params, **kw)
    opt.load_state_dict(ck)
    st0, st1 = opt.state[params[0]], opt.state[params[1]]
    assert "m" not in st0 and "m_q" not in st0 and "apollo_seed" in st0
    assert st1["v_quant_type"] == "al8" and st1["m_quant_type"] == "uf8"
    assert opt._apollo_seed_counter == 0
