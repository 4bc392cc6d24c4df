"""The CPU oracle reproduces the reference's own step trajectories (golden fixtures)."""
import numpy as np
import pytest
import torch

import golden_util as gu
import inputs
import oracle.fallback as F
from oracle.fallback import OracleOptimizer

ORACLE_NAMES = [n for n in gu.names()]


def _np(t):
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("name", ORACLE_NAMES)
def test_oracle_matches_golden(name, monkeypatch):
    # APOLLO projections: the generator the fixtures were written with
    monkeypatch.setattr(F, "stable_randn", inputs.make_proj)
    meta, kw, z = gu.load(name)
    params = gu.init_params(meta)
    opt = OracleOptimizer(params, **kw)
    for t in range(1, meta["steps"] + 1):
        for p, g in zip(params, gu.grads_for(meta, params, t)):
            p.grad = g
        opt.step()
        if t not in meta["save_steps"]:
            continue
        for i, p in enumerate(params):
            key = f"s{t}/p{i}"
            ref_p = z[f"{key}/param"]
            assert np.array_equal(_np(p.data), ref_p), f"{name} {key} param"
            st = opt.state[id(p)]
            ref_keys = [k[len(key) + 1:] for k in z.files if k.startswith(key + "/")]
            for k in ref_keys:
                if k == "param":
                    continue
                assert k in st, f"{name} {key}: oracle lacks state key {k}"
                mine = st[k]
                mine = _np(mine) if torch.is_tensor(mine) else np.asarray(mine)
                ref = z[f"{key}/{k}"]
                assert mine.dtype == ref.dtype, (k, mine.dtype, ref.dtype)
                assert mine.shape == ref.shape, (k, mine.shape, ref.shape)
                assert np.array_equal(mine, ref, equal_nan=True), f"{name} {key}/{k}"
            sc = meta["scalars"][key]
            for k, v in sc.items():
                if k in st and not torch.is_tensor(st[k]):
                    mv = list(st[k]) if isinstance(st[k], tuple) else st[k]
                    assert mv == v, (name, key, k, mv, v)
