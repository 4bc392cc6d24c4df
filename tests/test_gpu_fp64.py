"""fp64 parameters against the CPU oracle.

The reference's kernels dispatch double (AT_DISPATCH_FLOATING_TYPES_AND2,
kernels.cu:840); its PyTorch path reads the gradient as fp32 (grad.float()) and
updates the float64 parameter in double: p.mul_(decay), p.add_(u, alpha=-step)
(optimizer.py:866-875, 2034-2039).  Here the kernels read g as fp32 and apply
the update in double: p * decay, then fma(-step, u, p), where step * u, a
product of two floats, is exact in double, so the result is the double add's.

Parameters start near 16 (16 + N(0, 0.02^2)), where an fp32 rounding of p is
~1e-6 -- a hundred times the bound below -- so a path that stored p through
fp32 would fail.  Bound: 99.9% of the elements within 4 double ulps plus 1e-5
of the largest displacement the oracle's steps made (a step size that depends on
a norm -- RMS clip, Fira -- takes that norm as a float sum in another order,
which moves it by a few fp32 ulps); every element within 1% of that
displacement (a code that flipped near a rounding boundary moves one element's
update by one code step).  Codes to the parity bar.
"""
import numpy as np
import pytest
import torch

import golden_util as gu
from inputs import make_grad, make_param

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
             scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-3)
CASES = [
    ("adamw_uf8_al8_wd", dict(ADAMW, weight_decay=0.1), [(300, 200), (5000,), (300,)]),
    ("adamw_clip_fira", dict(ADAMW, d=1.0, enable_fira_for_adafactor=True), [(300, 200), (4096,), (64,)]),
    ("adamw_fp32_state", dict(ADAMW, quantize=False), [(300, 200), (100,)]),
    ("adafactor_factored", dict(beta1=None, beta2=None, beta2_decay=-0.8, factored=True, relative_step=False,
                                lr=1e-3, block_size=256, scale_parameter=False, d=1.0),
     [(256, 300), (130, 64), (64,)]),
    ("came_uf8_al16", dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True,
                           relative_step=False, scale_parameter=False, d=1.0, eps_came=1e-16, lr=1e-3,
                           v_quant_type="al16", c_quant_type="al16"), [(256, 300), (64,)]),
    ("sgd_momentum", dict(beta1=0.9, beta2=None, beta2_decay=None, factored=False, relative_step=False,
                          lr=1e-2, weight_decay=0.01, scale_parameter=False), [(300, 200), (100,)]),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,shapes", CASES, ids=[c[0] for c in CASES])
def test_fp64_params_match_oracle(name, kw, shapes):
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    print(f"[fp64] {name}", flush=True)
    init = [(16.0 + make_param(s, i, 5).double()) for i, s in enumerate(shapes)]
    pc = [torch.nn.Parameter(x.clone()) for x in init]
    pg = [torch.nn.Parameter(x.clone().cuda()) for x in init]
    oc, og = F.OracleOptimizer(pc, **kw), Adafactor8Bit(pg, **kw)
    # factored statistics are means over a matrix: the kernels sum them in double
    # and round once, so the oracle does too (the reference-order fp32 sums move
    # AL16 statistics codes, which CAME's 1/sqrt(confidence) magnifies)
    old = F.set_exact_reductions(bool(kw.get("factored")))
    try:
        for t in range(1, 5):
            for i, (a, b) in enumerate(zip(pc, pg)):
                g = make_grad(tuple(a.shape), i, t, 5, kind="student_t").double()
                a.grad, b.grad = g, g.cuda()
            oc.step()
            og.step()
    finally:
        F.set_exact_reductions(old)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(pc, pg)):
        assert b.dtype == torch.float64
        ref, mine, p0 = a.detach().numpy(), b.detach().cpu().numpy(), init[i].numpy()
        disp = float(np.abs(ref - p0).max())
        assert disp > 0, f"{name} p{i}: no update"
        err = np.abs(mine - ref)
        tight = 4 * np.spacing(np.abs(ref)) + 1e-5 * disp
        frac_ok = float((err <= tight).mean())
        print(f"  p{i} {tuple(a.shape)}: {frac_ok:.6f} within the tight bound, max err {err.max():.3e}, "
              f"disp {disp:.3e}", flush=True)
        assert frac_ok >= 0.999, f"{name} p{i}: only {frac_ok:.5f} within the double-precision bound"
        assert err.max() <= 1e-2 * disp, f"{name} p{i}: max error {err.max():.3e} vs displacement {disp:.3e}"
        sc, sg = oc.state[id(a)], og.state[b]
        for k, v in sc.items():
            if torch.is_tensor(v) and k.endswith("_q") and k in sg:
                frac, mx = gu.code_mismatch(v.reshape(-1).numpy(), sg[k].reshape(-1).cpu().numpy())
                assert frac <= 1e-4 + 1.0 / v.numel() and mx <= 1, f"{name} p{i} {k}: {frac:.2e} differ, max {mx}"


@pytest.mark.gpu
def test_fp64_scale_parameter_raises_as_the_reference():
    """With scale_parameter the reference takes ||p|| with dtype=float32
    (_compute_alpha, optimizer.py:850-852), which torch refuses for a float64
    tensor; the oracle meets the same error, and so does this build, before any
    state changes."""
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer
    kw = dict(ADAMW, scale_parameter=True)
    pc = torch.nn.Parameter(torch.ones(300, 200, dtype=torch.float64))
    pg = torch.nn.Parameter(torch.ones(300, 200, dtype=torch.float64, device="cuda"))
    pc.grad = torch.ones_like(pc)
    pg.grad = torch.ones_like(pg)
    with pytest.raises(RuntimeError) as ec:
        OracleOptimizer([pc], **kw).step()
    opt = Adafactor8Bit([pg], **kw)
    with pytest.raises(RuntimeError) as eg:
        opt.step()
    assert "Double" in str(ec.value) and "Double" in str(eg.value)
    assert opt.state[pg].get("step", 0) == 0


# APOLLO on fp64 parameters: the reference projects grad.float() and writes the
# update into the float64 parameter in double (p.mul_(decay), then addcmul_ with
# the fp32 channel scale, or add_ with the fp32 tensor scale; optimizer.py:2601,
# 3074-3080).  Here G is copied to fp32, projected with the fp32 GEMM, and the
# writeback runs in double.  The oracle gets this library's projection output
# (glow_hook) and reduces exactly.  Bounds: every element within 4 double ulps
# plus 2e-4 of the largest displacement (a low-rank V code that flips at a
# rounding boundary moves its channel's scale, as in the rank-256 APOLLO test),
# and at least 95% within 4 ulps plus 1e-5 of it -- a path that stored p through
# fp32 would be off by ~1e-6 near 16, fifty times that.
APOLLO = dict(lr=1e-3, beta1=0.9, beta2=0.999, relative_step=False, scale_parameter=False, apollo_rank=32,
              apollo_update_proj_gap=200, apollo_cache_proj=True, enable_fira_for_apollo=True, d=0.0)
APOLLO_CASES = [
    ("apollo_uf8_al8_wd", dict(APOLLO, weight_decay=0.01)),
    ("apollo_tensor_fp32_states", dict(APOLLO, quantize=False, apollo_scale_type="tensor", d=1.0)),
    ("apollo_bv384_bm96", dict(APOLLO, block_size=384, m_block_size=96, enable_fira_for_apollo=False)),
    ("apollo_came", dict(APOLLO, beta3=0.9999, d=1.0, eps_came=1e-16)),
    ("apollo_fact", dict(APOLLO, apollo_factorize=True)),
]
APOLLO_SHAPES = [(300, 200), (160, 420)]


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", APOLLO_CASES, ids=[c[0] for c in APOLLO_CASES])
def test_fp64_apollo_matches_oracle(name, kw, monkeypatch):
    import adafactor8bit.optimizer as O
    import inputs
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    monkeypatch.setattr(O, "stable_randn", inputs.make_proj)
    monkeypatch.setattr(F, "stable_randn", inputs.make_proj)
    print(f"[fp64 apollo] {name}", flush=True)
    init = [(16.0 + make_param(s, i, 23).double()) for i, s in enumerate(APOLLO_SHAPES)]
    pc = [torch.nn.Parameter(x.clone()) for x in init]
    pg = [torch.nn.Parameter(x.clone().cuda()) for x in init]
    oc, og = F.OracleOptimizer(pc, **kw), Adafactor8Bit(pg, **kw)
    lows = [(R, 32) if R >= C else (32, C) for R, C in APOLLO_SHAPES]
    glows = {}
    oc.glow_hook = lambda p, _g, _pt: glows[id(p)]
    old = F.set_exact_reductions(True)
    try:
        for t in range(1, 5):
            for i, (a, b) in enumerate(zip(pc, pg)):
                g = make_grad(APOLLO_SHAPES[i], i, t, 23, kind="student_t").double()
                a.grad, b.grad = g, g.cuda()
            og.step()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(pc, pg)):
                ws = og._ws[(b.device, "apollo", id(b))]["ws"].cpu().numpy()
                glows[id(a)] = torch.from_numpy(ws[:lows[i][0] * lows[i][1]].reshape(lows[i]).copy())
            oc.step()
    finally:
        F.set_exact_reductions(old)
    for i, (a, b) in enumerate(zip(pc, pg)):
        assert b.dtype == torch.float64
        ref, mine, p0 = a.detach().numpy(), b.detach().cpu().numpy(), init[i].numpy()
        disp = float(np.abs(ref - p0).max())
        assert disp > 0, f"{name} p{i}: no update"
        err = np.abs(mine - ref)
        ulp4 = 4 * np.spacing(np.abs(ref))
        frac_ok = float((err <= ulp4 + 1e-5 * disp).mean())
        print(f"  p{i} {tuple(a.shape)}: {frac_ok:.6f} within 4 ulps + 1e-5 disp, max err {err.max():.3e}, "
              f"disp {disp:.3e}", flush=True)
        assert frac_ok >= 0.95, f"{name} p{i}: only {frac_ok:.5f} within the double-precision bound"
        assert np.all(err <= ulp4 + 2e-4 * disp), f"{name} p{i}: max error {err.max():.3e} vs disp {disp:.3e}"
        sc, sg = oc.state[id(a)], og.state[b]
        for k, v in sc.items():
            if torch.is_tensor(v) and k.endswith("_q") and k.startswith(("v_low", "m_low")):
                frac, mx = gu.code_mismatch(v.reshape(-1).numpy(), sg[k].reshape(-1).cpu().numpy())
                print(f"  p{i} {k}: {frac:.2e} of codes differ, max {mx}", flush=True)
                assert frac <= 1e-4 + 1.0 / v.numel() and mx <= 1, f"{name} p{i} {k}: {frac:.2e} differ, max {mx}"


@pytest.mark.gpu
def test_fp64_apollo_scale_parameter_raises_as_the_reference():
    """APOLLO's alpha with scale_parameter is the same fp32 norm of the fp64
    parameter (optimizer.py:850-852): the oracle and this build both raise."""
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer
    kw = dict(APOLLO, scale_parameter=True)
    pc = torch.nn.Parameter(torch.ones(300, 200, dtype=torch.float64))
    pg = torch.nn.Parameter(torch.ones(300, 200, dtype=torch.float64, device="cuda"))
    pc.grad = torch.ones_like(pc)
    pg.grad = torch.ones_like(pg)
    with pytest.raises(RuntimeError) as ec:
        OracleOptimizer([pc], **kw).step()
    opt = Adafactor8Bit([pg], **kw)
    with pytest.raises(RuntimeError) as eg:
        opt.step()
    assert "Double" in str(ec.value) and "Double" in str(eg.value)
