"""Checkpoints and configuration changes against the reference, on the GPU.

Fixtures (tests/golden/ckpt_*.npz, written by gen_checkpoints.py from the
reference's CPU path) hold ``state_dict()`` after phases of training.  Before a
phase the script may change group options: a ``quantize`` flip (codes <-> fp32
for every slot, the reference's _migrate_quantize_flag, optimizer.py:976-1045),
codec and block-size changes (a momentum reset or a full reset), CAME switched
on and off, APOLLO state, bf16 parameters with fp32 state.

Two checks per scenario:
* replay: this build runs the same phases from the same start and its
  ``state_dict()`` at every save point matches the fixture's;
* resume: the fixture's checkpoint at a save point is loaded into a fresh
  optimizer (``load_state_dict``), which then runs the next phase; the result
  matches the fixture's next save point.

Layout is held exactly: the same state keys, dtypes, shapes, tags, step counts,
seed counters and parameter-group options.  Values are held to the golden
tolerances (tests/test_gpu_golden.py and tests/test_gpu_apollo.py): codes
equal except where the reference's CPU decode (torch.pow, 1 ulp off on ~2% of
inputs) moves a near-tie, fp32 states rtol 2e-6, parameters rtol 1e-5 except
elements whose code flipped.
"""
import json
import os

import numpy as np
import pytest
import torch

import golden_util as gu
import inputs
from test_gpu_apollo import _cmp_params as _cmp_params_apollo
from test_gpu_apollo import _cmp_state as _cmp_state_apollo
from test_gpu_golden import _cmp_state as _cmp_state_golden

SCENARIOS = ["ckpt_adamw_quant_flip", "ckpt_adamw_codec_changes", "ckpt_adamw_d4_flip", "ckpt_adamw_start_fp32",
             "ckpt_came_quant_flip", "ckpt_adafactor_came_toggle", "ckpt_apollo_quant_flip", "ckpt_apollo_bf16",
             "ckpt_adamw_bf16_sr_policy"]


def _load(name):
    z = np.load(os.path.join(gu.GOLDEN, name + ".npz"), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    kw = dict(meta["kwargs"])
    if kw.get("eps") is not None:
        kw["eps"] = tuple(kw["eps"])
    return meta, kw, z


def _from_json(rec):
    kind, val = rec
    if kind == "v":
        return val
    if kind == "size":
        return torch.Size(val)
    items = [_from_json(x) for x in val]
    return tuple(items) if kind == "tuple" else items


def _tensor(z, key, dt):
    t = torch.from_numpy(z[key].copy())
    return t.view(torch.bfloat16) if dt == "bf16" else t


def checkpoint(meta, z, tag):
    """The reference's state_dict() at save point ``tag``, rebuilt."""
    ent = meta["points"][tag]
    state = {}
    for idx, rec in ent["state"].items():
        state[int(idx)] = {k: (_tensor(z, f"{tag}/state/{idx}/{k}", v[1]) if v[0] == "tensor" else _from_json(v))
                           for k, v in rec.items()}
    groups = [{k: _from_json(v) for k, v in g.items()} for g in ent["groups"]]
    return {"state": state, "param_groups": groups, "_apollo_seed_counter": ent["counters"][0],
            "_sr_seed_counter": ent["counters"][1]}


def _pdtype(meta):
    return torch.bfloat16 if meta["dtype"] == "bf16" else torch.float32


def _np_param(p):
    t = p.detach().cpu()
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def _compare(name, meta, z, tag, opt, params, v_low_steps=None):
    """This build's state_dict() and parameters against the fixture's point ``tag``.
    ``v_low_steps``: relative room of fp32 low-rank V that was decoded from codes."""
    mine = opt.state_dict()
    ref = checkpoint(meta, z, tag)
    assert mine["_apollo_seed_counter"] == ref["_apollo_seed_counter"], tag
    assert mine["_sr_seed_counter"] == ref["_sr_seed_counter"], tag
    assert len(mine["param_groups"]) == len(ref["param_groups"])
    for gm, gr in zip(mine["param_groups"], ref["param_groups"]):
        for k, v in gr.items():
            if k != "use_cuda_kernel":
                assert k in gm and gm[k] == v, (tag, k, gm.get(k), v)
    assert sorted(mine["state"]) == sorted(ref["state"]), tag
    factored = "came" in name or "adafactor" in name
    apollo = "apollo" in name
    for idx, sr in ref["state"].items():
        sm = mine["state"][idx]
        assert sorted(sm) == sorted(sr), (tag, idx, sorted(set(sm) ^ set(sr)))
        key = f"{tag}/state/{idx}"
        for k, v in sr.items():
            if torch.is_tensor(v):
                continue
            mv = sm[k]
            if isinstance(v, (torch.Size, tuple, list)):
                assert mv is not None and list(mv) == list(v), (tag, idx, k, mv, v)
            else:
                assert mv == v, (tag, idx, k, mv, v)
        tens = {k: v for k, v in sr.items() if torch.is_tensor(v)}
        zz = {f"{key}/{k}": (v.view(torch.int16) if v.dtype == torch.bfloat16 else v).numpy() for k, v in tens.items()}
        st_view = {k: v for k, v in opt.state[params[idx]].items()}
        if apollo:
            # fp32 low-rank V decoded from codes (a flip to fp32) inherits the room the
            # golden APOLLO comparison gives those codes (two code steps, see
            # test_gpu_apollo); norms drift over bf16 steps as in the fp16 fixtures
            fp32_rtol = {}
            if v_low_steps is not None and "v_low" in tens:
                fp32_rtol["v_low"] = v_low_steps
            _cmp_state_apollo("apollo_ckpt", key, st_view, zz, list(tens), norm_rtol=1e-4, fp32_rtol=fp32_rtol)
        else:
            # fp32 row / column statistics carry the reference's float32 sums over up to
            # 300 terms: (n - 1) 2^-24 <= 1.8e-5 relative; every factored update element
            # (and CAME's momentum, an EMA of it) inherits that, so near-zero fp32 entries
            # are held to 2e-5 of the state's largest magnitude
            _cmp_state_golden("came_ckpt" if factored else "ckpt", key, st_view, zz, list(tens), [],
                              stat_rtol=2e-5, floor_frac=2e-5 if factored else 1e-6)
    for i, p in enumerate(params):
        want = z[f"{tag}/p{i}"]
        got = _np_param(p)
        init = z["init/p0".replace("0", str(i))]
        if apollo or want.dtype == np.int16:
            _cmp_params_apollo(name, f"{tag}/p{i}", got, want, init, frac=1e-2)
            continue
        disp = float(np.abs(want - init).max())
        slack = 1e-4 * disp if factored else 0.0
        close = np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-8 + slack
        assert (~close).mean() <= 1e-4 + 1.0 / got.size, f"{name} {tag} p{i}"
        np.testing.assert_allclose(got, want, rtol=2e-3, atol=1e-8 + 1e-2 * disp, err_msg=f"{name} {tag} p{i}")


def _params(meta, dev="cuda"):
    dt = _pdtype(meta)
    return [torch.nn.Parameter(inputs.make_param(tuple(s), i, 0, kind=k).to(dev, dt))
            for i, (s, k) in enumerate(meta["params"])]


def _step(opt, params, meta, t):
    dt = _pdtype(meta)
    for i, p in enumerate(params):
        p.grad = inputs.make_grad(tuple(p.shape), i, t, 0, kind=meta["grad_kind"]).to(dt).cuda()
    opt.step()


@pytest.fixture
def det_proj(monkeypatch):
    import adafactor8bit.optimizer as O
    monkeypatch.setattr(O, "stable_randn", inputs.make_proj)


@pytest.mark.gpu
@pytest.mark.parametrize("name", SCENARIOS)
def test_replay_matches_reference_checkpoints(name, det_proj):
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = _load(name)
    print(f"[ckpt replay] {name}", flush=True)
    params = _params(meta)
    opt = Adafactor8Bit(params, **kw)
    t = 0
    steps2 = None   # two AL8 code steps of the widest low-rank V block, once V went to fp32
    for ph, (changes, nsteps, save) in enumerate(meta["phases"]):
        for g in opt.param_groups:
            g.update(changes)
            if changes.get("quantize") is False and ph > 0:
                prev = checkpoint(meta, z, f"ph{ph - 1}")["state"]
                scales = [st["v_low_scale"].max().item() for st in prev.values() if torch.is_tensor(
                    st.get("v_low_scale"))]
                if scales:
                    steps2 = 2.0 ** (2.0 * max(scales) / 254.0) - 1.0
        for _ in range(nsteps):
            t += 1
            _step(opt, params, meta, t)
        if save:
            torch.cuda.synchronize()
            _compare(name, meta, z, f"ph{ph}", opt, params, v_low_steps=steps2)


@pytest.mark.gpu
@pytest.mark.parametrize("name", SCENARIOS)
def test_resume_from_reference_checkpoints(name, det_proj):
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = _load(name)
    print(f"[ckpt resume] {name}", flush=True)
    phases = meta["phases"]
    t = 0
    for ph in range(len(phases) - 1):
        t += phases[ph][1]
        tag, nxt = f"ph{ph}", f"ph{ph + 1}"
        if tag not in meta["points"] or nxt not in meta["points"]:
            continue
        params = _params(meta)
        with torch.no_grad():
            for i, p in enumerate(params):
                p.copy_(_tensor(z, f"{tag}/p{i}", meta["dtype"]).to(p.device))
        opt = Adafactor8Bit(params, **kw)
        opt.load_state_dict(checkpoint(meta, z, tag))
        for k, st in opt.state.items():   # stored dtypes survive the load, whatever the parameter's dtype
            ref = checkpoint(meta, z, tag)["state"][[id(q) for q in params].index(id(k))]
            for key, v in st.items():
                if torch.is_tensor(v) and key != "step":
                    assert v.dtype == ref[key].dtype and v.is_cuda, (tag, key, v.dtype, ref[key].dtype)
        changes, nsteps, _ = phases[ph + 1]
        for g in opt.param_groups:
            g.update(changes)
        for s in range(nsteps):
            _step(opt, params, meta, t + s + 1)
        torch.cuda.synchronize()
        _compare(name, meta, z, nxt, opt, params)


HANDOFF = [
    ("adamw_uf8_al8", dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
                           scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-4),
     [(33, 517), (300,), (5000,)], False),
    ("came_uf8_al16", dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True,
                           relative_step=False, scale_parameter=False, scale_weight_decay=False, d=1.0, lr=1e-4,
                           v_quant_type="al16", c_quant_type="al16", block_size=256, m_block_size=128),
     [(64, 300), (300, 64), (64,)], True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,shapes,factored", HANDOFF, ids=[h[0] for h in HANDOFF])
def test_oracle_continues_this_builds_checkpoint(name, kw, shapes, factored):
    """This build's state_dict(), handed to the CPU oracle (a restatement of the
    reference's own step), continues there as it does here: three steps on the
    GPU, then two more on each side, compared with the golden tolerances."""
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer
    print(f"[ckpt handoff] {name}", flush=True)
    pg = [torch.nn.Parameter(inputs.make_param(s, i, 4).cuda()) for i, s in enumerate(shapes)]
    init = [p.detach().cpu().numpy() for p in pg]
    og = Adafactor8Bit(pg, **kw)
    for t in range(1, 4):
        for i, p in enumerate(pg):
            p.grad = inputs.make_grad(tuple(p.shape), i, t, 4, kind="logscale").cuda()
        og.step()
    sd = og.state_dict()
    pc = [torch.nn.Parameter(p.detach().cpu().clone()) for p in pg]
    oc = OracleOptimizer(pc, **kw)
    for idx, p in enumerate(pc):
        oc.state[id(p)] = {k: (v.detach().cpu().clone() if torch.is_tensor(v) else v)
                           for k, v in sd["state"][idx].items()}
    for t in range(4, 6):
        for i, (a, b) in enumerate(zip(pc, pg)):
            g = inputs.make_grad(tuple(a.shape), i, t, 4, kind="logscale")
            a.grad, b.grad = g, g.cuda()
        oc.step()
        og.step()
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(pc, pg)):
        key = f"s5/p{i}"
        ref_st = {k: v.numpy() for k, v in oc.state[id(a)].items() if torch.is_tensor(v)}
        zz = {f"{key}/{k}": v for k, v in ref_st.items()}
        _cmp_state_golden("came_handoff" if factored else "handoff", key, og.state[b], zz, list(ref_st), [])
        ref_p, mine_p = a.detach().numpy(), b.detach().cpu().numpy()
        disp = float(np.abs(ref_p - init[i]).max())
        slack = 1e-4 * disp if factored else 0.0
        close = np.abs(mine_p - ref_p) <= 1e-5 * np.abs(ref_p) + 1e-8 + slack
        assert (~close).mean() <= 1e-4 + 1.0 / mine_p.size, f"{name} p{i}"
        np.testing.assert_allclose(mine_p, ref_p, rtol=2e-3, atol=1e-8 + 1e-2 * disp, err_msg=f"{name} p{i}")
