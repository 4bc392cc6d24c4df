"""Load golden fixtures and replay their inputs."""
import glob
import json
import os

import numpy as np
import torch

from inputs import make_grad, make_param

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def names():
    """Step-trajectory fixtures (the checkpoint fixtures, ckpt_*.npz, have a format of their own)."""
    return sorted(os.path.splitext(os.path.basename(f))[0]
                  for f in glob.glob(os.path.join(GOLDEN, "*.npz")) if not os.path.basename(f).startswith("ckpt_"))


def load(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    kw = dict(meta["kwargs"])
    if "eps" in kw and kw["eps"] is not None:
        kw["eps"] = tuple(kw["eps"])
    return meta, kw, z


def param_dtype(meta):
    return {"bf16": torch.bfloat16, "fp16": torch.float16}.get(meta.get("dtype", "f32"), torch.float32)


def init_params(meta, device="cpu", dtype=None):
    dtype = param_dtype(meta) if dtype is None else dtype
    out = []
    for i, (shape, init) in enumerate(meta["params"]):
        out.append(torch.nn.Parameter(make_param(tuple(shape), i, meta["seed"], kind=init)
                                      .to(device=device, dtype=dtype)))
    return out


def grads_for(meta, params, step):
    return [make_grad(tuple(p.shape), i, step, meta["seed"], kind=meta["grad_kind"]).to(param_dtype(meta))
            for i, p in enumerate(params)]


def code_mismatch(a, b):
    """(fraction of codes that differ, max |difference|) on unsigned code values."""
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.int16:
        a = a.astype(np.int64) & 0xFFFF
        b = b.astype(np.int64) & 0xFFFF
    a = a.astype(np.int64)
    b = b.astype(np.int64)
    if a.size == 0:
        return 0.0, 0
    diff = np.abs(a - b)
    return float((diff != 0).mean()), int(diff.max())
