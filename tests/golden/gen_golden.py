"""Write golden optimizer-step fixtures from the reference's pure-PyTorch path.

Run ONLY in the build container, where the reference is mounted read-only:

    python tests/golden/gen_golden.py /root/reference

It imports ``adafactor8bit`` from that path with ``use_cuda_kernel=False`` on
every group (so no kernel is compiled), runs each configuration below for a few
steps on seeded inputs from ``inputs.py`` and stores, after selected steps, the
parameters and every tensor/scalar state entry in ``<name>.npz``.  The multi-step
trajectories of ``Adafactor8Bit.step`` (adafactor8bit/optimizer.py:1866-1938 and
the CPU branches of ``_update_param_8bit``, optimizer.py:1944-2552) are pinned
by nothing else, which is why they are recorded here.  Nothing of the reference
is stored except these input/output vectors.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from inputs import make_grad, make_param, make_proj  # noqa: E402

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False,
             relative_step=False, scale_parameter=False, scale_weight_decay=False,
             d=0.0, eps=(1e-8, 1e-3))
ADAFACTOR = dict(beta1=None, beta2=None, beta2_decay=-0.8, beta3=None, factored=True,
                 relative_step=False)
CAME = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True,
            relative_step=False, scale_parameter=False, scale_weight_decay=False,
            d=1.0, eps_came=1e-16)
RMSPROP = dict(beta1=None, beta2=0.99, beta2_decay=None, beta3=None, factored=False,
               relative_step=False, scale_parameter=False, scale_weight_decay=False,
               d=0.0, eps=(1e-8, 1e-3))
SGD = dict(beta1=None, beta2=None, beta2_decay=None, beta3=None, factored=False,
           relative_step=False, scale_parameter=False, scale_weight_decay=False, d=0.0)

# (shape, init kind).  Shapes are chosen so V blocks, M blocks and the last
# partial block of each state all occur.
P_ADAMW = [((61, 1003), "normal"), ((2048,), "ones"), ((5000,), "normal")]
P_SMALL = [((33, 517), "normal"), ((300,), "ones")]
P_FACT = [((64, 300), "normal"), ((300, 64), "normal"), ((2, 40, 130), "normal"),
          ((64,), "ones")]
P_EMB = [((500, 64), "normal"), ((64, 48), "normal")]
P_CAME = [((64, 300), "normal"), ((128, 64), "normal"), ((64,), "ones")]
# APOLLO: a right-side (R >= C) and a left-side (R < C) matrix, and a vector that
# takes the full-rank route of the same group.
P_APOLLO = [((128, 96), "normal"), ((64, 160), "normal"), ((96,), "ones")]
APOLLO = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False,
              relative_step=False, scale_parameter=False, scale_weight_decay=False, d=0.0,
              eps=(1e-6, 1e-3), apollo_eps=1e-6, apollo_factorize=False, apollo_update_proj_gap=3,
              apollo_scale_type="channel", apollo_scale=1.0, apollo_scale_front=False,
              apollo_cache_proj=True, enable_fira_for_apollo=True, apollo_rank=16,
              block_size=128, m_block_size=32)

CONFIGS = [
    # name, kwargs, params, grad kind, steps, save steps
    ("adamw_uf8_al8", dict(ADAMW, lr=1e-4), P_ADAMW, "normal_zeros", 10, (1, 2, 10)),
    ("adamw_uf8_al16", dict(ADAMW, lr=1e-4, v_quant_type="al16"), P_SMALL, "normal_zeros", 4, (1, 4)),
    ("adamw_uf4_al8", dict(ADAMW, lr=1e-4, m_quant_type="uf4"), P_SMALL, "normal_zeros", 4, (1, 4)),
    ("adamw_d8_al8", dict(ADAMW, lr=1e-4, m_quant_type="d8"), P_SMALL, "normal_zeros", 4, (1, 4)),
    ("adamw_d4_al8", dict(ADAMW, lr=1e-4, m_quant_type="d4"), P_SMALL, "normal_zeros", 4, (1, 4)),
    ("adamw_bv256_mb128", dict(ADAMW, lr=1e-4, block_size=256, m_block_size=128), P_SMALL,
     "student_t", 4, (1, 4)),
    ("adamw_clip_fira_wd", dict(ADAMW, lr=1e-3, d=1.0, weight_decay=0.1, scale_weight_decay=True,
                                enable_fira_for_adafactor=True), P_SMALL, "logscale", 5, (1, 5)),
    ("adamw_fp32_state", dict(ADAMW, lr=1e-4, quantize=False), P_SMALL, "normal_zeros", 4, (1, 4)),
    # fp32 V with quantised momentum (the reference's PyTorch branch, optimizer.py:2185-2191)
    ("adamw_fp32v_uf8m", dict(ADAMW, lr=1e-4, v_quant_type="fp32", d=1.0, weight_decay=0.1,
                              scale_weight_decay=True), P_ADAMW, "student_t", 4, (1, 4)),
    ("rmsprop_al8", dict(RMSPROP, lr=1e-4), P_SMALL, "normal_zeros", 4, (1, 4)),
    ("adafactor_mom1d", dict(ADAFACTOR, lr=1e-3, beta1=0.9, factored=False), P_SMALL,
     "student_t", 4, (1, 4)),
    ("adafactor_mom1d_fp32v_uf8m", dict(ADAFACTOR, lr=1e-3, beta1=0.9, factored=False, v_quant_type="fp32",
                                        enable_fira_for_adafactor=True), P_ADAMW, "logscale", 4, (1, 4)),
    ("adafactor_mom1d_fira", dict(ADAFACTOR, lr=1e-3, beta1=0.9, factored=False,
                                  enable_fira_for_adafactor=True, fira_margin=0.01), P_SMALL,
     "logscale", 5, (1, 5)),
    ("adafactor_factored_al8", dict(ADAFACTOR, lr=1e-3, block_size=256), P_FACT, "student_t",
     10, (1, 2, 10)),
    ("adafactor_factored_emb", dict(ADAFACTOR, lr=1e-3, block_size=256), P_EMB, "sparse_rows",
     4, (1, 4)),
    ("adafactor_factored_m_uf8", dict(ADAFACTOR, lr=1e-3, block_size=256, beta1=0.9), P_FACT,
     "student_t", 4, (1, 4)),
    ("came_uf8_al16_fira", dict(CAME, lr=1e-4, v_quant_type="al16", c_quant_type="al16",
                                enable_fira_for_adafactor=True, fira_margin=0.01), P_CAME,
     "logscale", 10, (1, 2, 10)),
    ("came_uf8_al8", dict(CAME, lr=1e-4), P_CAME, "normal_zeros", 4, (1, 4)),
    ("sgd_momentum_uf8", dict(SGD, lr=1e-2, beta1=0.9), P_SMALL, "normal_zeros", 4, (1, 4)),
    ("apollo_uf8_al8", dict(APOLLO, lr=1e-3), P_APOLLO, "normal_zeros", 7, (1, 3, 4, 7)),
    ("apollo_tensor_clip_wd", dict(APOLLO, lr=1e-3, apollo_scale_type="tensor", d=1.0,
                                   weight_decay=0.1, scale_weight_decay=True, apollo_scale=2.0,
                                   apollo_scale_front=True, enable_fira_for_apollo=False,
                                   apollo_cache_proj=False, m_quant_type="uf4"),
     P_APOLLO, "student_t", 5, (1, 5)),
    ("apollo_fp32_states", dict(APOLLO, lr=1e-3, quantize=False), P_APOLLO, "logscale", 4, (1, 4)),
    ("apollo_bf16_det", dict(APOLLO, lr=1e-3), P_APOLLO, "normal_zeros", 4, (1, 4), "bf16"),
    # CAME on the low-rank gradient (beta3) and the factorised low-rank second moment
    ("apollo_came_uf8_al8", dict(APOLLO, lr=1e-3, beta3=0.9999, d=1.0, eps_came=1e-16),
     P_APOLLO, "normal_zeros", 5, (1, 2, 5)),
    ("apollo_came_al16_tensor", dict(APOLLO, lr=1e-3, beta3=0.99, d=1.0, eps_came=1e-16,
                                     v_quant_type="al16", c_quant_type="al16", m_quant_type="uf4",
                                     apollo_scale_type="tensor", weight_decay=0.1),
     P_APOLLO, "student_t", 4, (1, 4)),
    ("apollo_came_fp32", dict(APOLLO, lr=1e-3, beta3=0.9999, d=1.0, eps_came=1e-16, quantize=False),
     P_APOLLO, "logscale", 4, (1, 4)),
    ("apollo_fact_uf8", dict(APOLLO, lr=1e-3, apollo_factorize=True), P_APOLLO, "student_t", 5,
     (1, 2, 5)),
    ("apollo_fact_nomom", dict(APOLLO, lr=1e-3, apollo_factorize=True, beta1=None, beta2=None,
                               beta2_decay=-0.8, relative_step=False, d=1.0,
                               apollo_scale_type="tensor"), P_APOLLO, "logscale", 4, (1, 4)),
    ("apollo_fact_came", dict(APOLLO, lr=1e-3, apollo_factorize=True, beta3=0.9999, d=1.0,
                              eps_came=1e-16), P_APOLLO, "normal_zeros", 5, (1, 2, 5)),
    ("apollo_fact_came_fp32", dict(APOLLO, lr=1e-3, apollo_factorize=True, beta3=0.999, d=1.0,
                                   eps_came=1e-16, quantize=False, weight_decay=0.05,
                                   scale_weight_decay=True), P_APOLLO, "student_t", 4, (1, 4)),
    ("apollo_came_bf16", dict(APOLLO, lr=1e-3, beta3=0.9999, d=1.0, eps_came=1e-16), P_APOLLO,
     "normal_zeros", 4, (1, 4), "bf16"),
    # fp16 parameters: projection of grad.float(), fp16 rounding of the decayed and updated values
    ("apollo_fp16_det", dict(APOLLO, lr=1e-3, weight_decay=0.1, scale_weight_decay=True), P_APOLLO,
     "normal_zeros", 4, (1, 4), "fp16"),
    ("apollo_fp16_tensor", dict(APOLLO, lr=1e-3, apollo_scale_type="tensor", scale_parameter=True,
                                relative_step=True, d=1.0), P_APOLLO, "student_t", 4, (1, 4), "fp16"),
]


def _to_np(v):
    # copy: parameters and fp32 states are updated in place by later steps
    if v.dtype == torch.bfloat16:
        return v.detach().view(torch.int16).numpy().copy()
    return v.detach().cpu().contiguous().numpy().copy()


def run_config(mod, name, kwargs, pspecs, gkind, steps, save_steps, pdtype="f32", outdir=".", seed=0):
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}.get(pdtype, torch.float32)
    params = []
    for i, (shape, init) in enumerate(pspecs):
        params.append(torch.nn.Parameter(make_param(shape, i, seed, kind=init).to(dt)))
    opt = mod.Adafactor8Bit(params, use_cuda_kernel=False, **kwargs)
    arrays = {}
    meta = {"config": name, "kwargs": {k: (list(v) if isinstance(v, tuple) else v)
                                       for k, v in kwargs.items()},
            "params": [[list(s), init] for s, init in pspecs], "grad_kind": gkind,
            "seed": seed, "steps": steps, "save_steps": list(save_steps), "dtype": pdtype,
            "torch": torch.__version__, "scalars": {}}
    for i, p in enumerate(params):
        arrays[f"init/p{i}"] = _to_np(p.data)
    for t in range(1, steps + 1):
        for i, p in enumerate(params):
            p.grad = make_grad(tuple(p.shape), i, t, seed, kind=gkind).to(dt)
        opt.step()
        if t in save_steps:
            for i, p in enumerate(params):
                arrays[f"s{t}/p{i}/param"] = _to_np(p.data)
                st = opt.state[p]
                sc = {}
                for k, v in st.items():
                    if torch.is_tensor(v):
                        arrays[f"s{t}/p{i}/{k}"] = _to_np(v)
                    elif isinstance(v, (int, float, str, bool)) or v is None:
                        sc[k] = v
                    elif isinstance(v, (torch.Size, tuple, list)):
                        sc[k] = list(v)
                meta["scalars"][f"s{t}/p{i}"] = sc
    np.savez_compressed(os.path.join(outdir, f"{name}.npz"), meta=np.array(json.dumps(meta)),
                        **arrays)
    return meta


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    import adafactor8bit.optimizer as mod  # the reference package
    # APOLLO projections from a host-independent generator (see inputs.make_proj)
    mod.stable_randn = make_proj
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    outdir = HERE
    only = set(sys.argv[2:])
    for cfg in CONFIGS:
        if only and cfg[0] not in only:
            continue
        run_config(mod, *cfg, outdir=outdir)
        print("wrote", cfg[0], flush=True)


if __name__ == "__main__":
    main()
