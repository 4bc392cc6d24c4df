"""Write checkpoint fixtures from the reference's pure-PyTorch path.

Run ONLY in the build container, where the reference is mounted read-only:

    python tests/golden/gen_checkpoints.py /root/reference

Each scenario steps the reference's ``Adafactor8Bit`` (``use_cuda_kernel=False``)
on seeded inputs through phases.  Before a phase it may change options of the
parameter group, as a training script does between runs (a ``quantize`` flip, a
codec or block-size change, CAME switched on or off).  After selected phases it
records ``opt.state_dict()`` in full (every state tensor, every tag, the
parameter groups and the seed counters) and the parameters.  What these pin,
and nothing else does: ``state_dict`` / ``load_state_dict`` (optimizer.py:1463-1553)
and the state reconciliation of ``_init_group`` with its migrations
(optimizer.py:976-1045, 1618-1864) across those changes.  Nothing of the
reference is stored except these input/output vectors.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from inputs import make_grad, make_param, make_proj  # noqa: E402

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False, relative_step=False,
             scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-4)
CAME = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True, relative_step=False,
            scale_parameter=False, scale_weight_decay=False, d=1.0, eps_came=1e-16, lr=1e-4,
            v_quant_type="al16", c_quant_type="al16", block_size=256, m_block_size=128)
ADAFACTOR_M = dict(beta1=0.9, beta2=None, beta2_decay=-0.8, beta3=None, factored=True, relative_step=False,
                   lr=1e-3, block_size=256, m_block_size=128)
APOLLO = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False, relative_step=False,
              scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-6, 1e-3), apollo_eps=1e-6,
              apollo_update_proj_gap=200, apollo_scale_type="channel", apollo_cache_proj=True,
              enable_fira_for_apollo=True, apollo_rank=16, block_size=128, m_block_size=32, lr=1e-3)

P_1D = [((33, 517), "normal"), ((300,), "ones"), ((5000,), "normal")]
P_FACT = [((64, 300), "normal"), ((300, 64), "normal"), ((64,), "ones")]
P_APOLLO = [((128, 96), "normal"), ((64, 160), "normal"), ((96,), "ones")]

# name, kwargs, params, grad kind, param dtype, phases: (group changes, steps, save after)
SCENARIOS = [
    ("ckpt_adamw_quant_flip", ADAMW, P_1D, "normal_zeros", "f32",
     [({}, 3, True), ({"quantize": False}, 2, True), ({"quantize": True}, 2, True)]),
    ("ckpt_adamw_codec_changes", dict(ADAMW, m_quant_type="uf4"), P_1D, "student_t", "f32",
     [({}, 2, True), ({"m_quant_type": "d8"}, 1, True), ({"v_quant_type": "al16"}, 1, True),
      ({"block_size": 1024, "m_block_size": 128}, 1, True), ({"m_quant_type": "fp32"}, 2, True)]),
    ("ckpt_adamw_d4_flip", dict(ADAMW, m_quant_type="d4", v_quant_type="al16"), P_1D, "logscale", "f32",
     [({}, 2, True), ({"quantize": False}, 1, True), ({"quantize": True}, 2, True)]),
    ("ckpt_adamw_start_fp32", ADAMW, P_1D, "normal_zeros", "f32",
     [({"quantize": False}, 2, True), ({"quantize": True}, 2, True)]),
    ("ckpt_came_quant_flip", CAME, P_FACT, "logscale", "f32",
     [({}, 3, True), ({"quantize": False}, 2, True), ({"quantize": True}, 2, True)]),
    ("ckpt_adafactor_came_toggle", ADAFACTOR_M, P_FACT, "student_t", "f32",
     [({}, 2, True), ({"beta3": 0.999, "beta2": 0.999, "beta2_decay": None}, 2, True),
      ({"beta3": None}, 1, True)]),
    ("ckpt_apollo_quant_flip", APOLLO, P_APOLLO, "normal_zeros", "f32",
     [({}, 3, True), ({"quantize": False}, 2, True), ({"quantize": True}, 2, True)]),
    ("ckpt_apollo_bf16", APOLLO, P_APOLLO, "normal_zeros", "bf16",
     [({}, 2, True), ({}, 2, True)]),
    ("ckpt_adamw_bf16_sr_policy", dict(ADAMW, stochastic_round_writeback=False), P_1D, "normal_zeros", "bf16",
     [({}, 2, True), ({}, 1, True)]),
]


def _np(v):
    v = v.detach().cpu().contiguous()
    if v.dtype == torch.bfloat16:
        return v.view(torch.int16).numpy().copy(), "bf16"
    return v.numpy().copy(), str(v.dtype).replace("torch.", "")


def _jsonable(v):
    """(kind, value) for a non-tensor state or group entry."""
    if v is None or isinstance(v, (bool, int, float, str)):
        return ["v", v]
    if isinstance(v, torch.Size):
        return ["size", list(v)]
    if isinstance(v, tuple):
        return ["tuple", [_jsonable(x) for x in v]]
    if isinstance(v, list):
        return ["list", [_jsonable(x) for x in v]]
    raise TypeError(f"cannot record {type(v)}")


def record(arrays, meta, tag, opt, params):
    sd = opt.state_dict()
    entry = {"groups": [], "state": {}, "counters": [sd.get("_apollo_seed_counter"), sd.get("_sr_seed_counter")]}
    for g in sd["param_groups"]:
        entry["groups"].append({k: _jsonable(v) for k, v in g.items()})
    for idx, st in sd["state"].items():
        rec = {}
        for k, v in st.items():
            if torch.is_tensor(v):
                arr, dt = _np(v)
                arrays[f"{tag}/state/{idx}/{k}"] = arr
                rec[k] = ["tensor", dt]
            else:
                rec[k] = _jsonable(v)
        entry["state"][str(idx)] = rec
    for i, p in enumerate(params):
        arrays[f"{tag}/p{i}"] = _np(p.data)[0]
    meta["points"][tag] = entry


def run(mod, name, kwargs, pspecs, gkind, pdtype, phases, outdir):
    dt = {"bf16": torch.bfloat16}.get(pdtype, torch.float32)
    params = [torch.nn.Parameter(make_param(s, i, 0, kind=k).to(dt)) for i, (s, k) in enumerate(pspecs)]
    opt = mod.Adafactor8Bit(params, use_cuda_kernel=False, **kwargs)
    arrays = {}
    meta = {"scenario": name, "kwargs": {k: (list(v) if isinstance(v, tuple) else v) for k, v in kwargs.items()},
            "params": [[list(s), k] for s, k in pspecs], "grad_kind": gkind, "dtype": pdtype,
            "phases": [[ch, n, save] for ch, n, save in phases], "torch": torch.__version__, "points": {}}
    for i, p in enumerate(params):
        arrays[f"init/p{i}"] = _np(p.data)[0]
    t = 0
    for ph, (changes, nsteps, save) in enumerate(phases):
        for g in opt.param_groups:
            g.update(changes)
        for _ in range(nsteps):
            t += 1
            for i, p in enumerate(params):
                p.grad = make_grad(tuple(p.shape), i, t, 0, kind=gkind).to(dt)
            opt.step()
        if save:
            record(arrays, meta, f"ph{ph}", opt, params)
    np.savez_compressed(os.path.join(outdir, f"{name}.npz"), meta=np.array(json.dumps(meta)), **arrays)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    import adafactor8bit.optimizer as mod  # the reference package
    mod.stable_randn = make_proj
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    only = set(sys.argv[2:])
    for sc in SCENARIOS:
        if only and sc[0] not in only:
            continue
        run(mod, *sc, outdir=HERE)
        print("wrote", sc[0], flush=True)


if __name__ == "__main__":
    main()
