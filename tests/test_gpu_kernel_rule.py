"""The fused 1-D step under the reference kernels' AL rule (al_refit_rule="kernel",
A8_AL_KERNEL_RULE) against the oracle's restatement of that rule
(oracle/fallback.py al_quantize_kernel / al_dequantize_kernel, pinned in
tests/test_oracle_kernel_rule.py).

Seeded AdamW / RMSprop-style trajectories with 5% exact-zero gradients (every
block holds a zero V at step 1, so every block takes the log_eps_sq floor, as
kernels.cu:772-774 does), over the unit layout's paths (one V block per
workgroup at B_V 2048, per-half blocks at B_V 256, a tensor's partial last unit),
the general-block kernel (B_V 384), AL16, no momentum, and multi-tensor against
per-tensor launches.  The bar is the north star's: step-1 codes bit-exact, later
steps <= 0.01% of codes one step apart, parameters within rtol 1e-5 except the
elements whose code differed.  The module's set_refit_rule("kernel") gives the
same codes, and the same inputs under the default rule refit differently.
"""
import math

import numpy as np
import pytest
import torch

from inputs import make_grad, make_param

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
             scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-4,
             min_8bit_size=1, al_refit_rule="kernel")

CASES = {
    "adamw_bv2048": (dict(ADAMW), [(1024, 1536), (5000,)]),
    "adamw_bv256_al16": (dict(ADAMW, block_size=256, m_block_size=64, v_quant_type="al16"), [(700, 300), (1000,)]),
    "rmsprop_nom_bv512": (dict(ADAMW, beta1=None, block_size=512), [(600, 512), (3000,)]),
    "adamw_bv384_gen": (dict(ADAMW, block_size=384, m_block_size=96), [(500, 384), (1000,)]),
    "adamw_uf4_single": (dict(ADAMW, m_quant_type="uf4", maximize=True), [(300, 700)]),
}


def _codes(a, b):
    a = a.reshape(-1).numpy().astype(np.int64) & 0xFFFF
    b = b.reshape(-1).cpu().numpy().astype(np.int64) & 0xFFFF
    d = np.abs(a - b)
    return float((d != 0).mean()), int(d.max()) if d.size else 0


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_kernel_rule_matches_oracle(name):
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer, kernel_floor
    kw, shapes = CASES[name]
    print(f"[kernel rule] {name}", flush=True)
    pc = [torch.nn.Parameter(make_param(s, i, 21)) for i, s in enumerate(shapes)]
    pg = [torch.nn.Parameter(p.detach().clone().cuda()) for p in pc]
    p0 = [p.detach().clone() for p in pc]
    oc, og = OracleOptimizer(pc, **kw), Adafactor8Bit(pg, **kw)
    touched = [np.zeros(p.numel(), dtype=bool) for p in pc]
    floor = kernel_floor(1e-8)
    for t in range(1, 5):
        for i, (a, b) in enumerate(zip(pc, pg)):
            g = make_grad(tuple(a.shape), i, t, 21, zero_frac=0.05)
            a.grad, b.grad = g, g.cuda()
        oc.step()
        og.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pc, pg)):
            sc, sg = oc.state[id(a)], og.state[b]
            ml = sg["variance_min_log"].reshape(-1).cpu().numpy()
            if t == 1:   # every block holds a zero V at step 1: the floor
                assert np.all(ml == np.float32(floor)), (i, ml[:4])
            keys = ("variance_q", "m_q") if kw.get("beta1") is not None else ("variance_q",)
            n = touched[i].size
            for k in keys:
                frac, mx = _codes(sc[k], sg[k])
                print(f"  step {t} tensor {i} {k}: {frac:.2e} differ, max {mx}", flush=True)
                if t == 1:
                    assert frac == 0.0, (t, i, k, frac)
                assert frac <= 1e-4 and mx <= 1, (t, i, k, frac, mx)
                a_, b_ = sc[k].reshape(-1).numpy(), sg[k].reshape(-1).cpu().numpy()
                if a_.size >= n:   # one code per element (UF4 packs two a byte: its stats above)
                    touched[i] |= (a_[:n].astype(np.int64) & 0xFFFF) != (b_[:n].astype(np.int64) & 0xFFFF)
            for k in ("variance_scale", "variance_min_log"):
                np.testing.assert_allclose(sg[k].reshape(-1).cpu().numpy(), sc[k].reshape(-1).numpy(),
                                           rtol=1e-5 if t > 1 else 3e-7)
    for i, (a, b) in enumerate(zip(pc, pg)):
        t_ = touched[i]
        assert t_.mean() <= 1e-4 + 1.0 / t_.size
        P, Q = b.detach().cpu().reshape(-1).numpy(), a.detach().reshape(-1).numpy()
        np.testing.assert_allclose(P[~t_], Q[~t_], rtol=1e-5, atol=1e-8)
        disp = float(np.abs(Q - p0[i].reshape(-1).numpy()).max())
        np.testing.assert_allclose(P[t_], Q[t_], rtol=2e-3, atol=1e-8 + 1e-2 * disp)


@pytest.mark.gpu
def test_kernel_rule_all_zero_block_and_default_rule_differs():
    """An all-zero-gradient tensor: every block gets the kernels' (1e-12, -1e30) and
    code 0, where the default rule writes (1, log2(1e-38) - 1); and on 5%-zero
    gradients the two rules refit different l_min."""
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import kernel_floor
    print("[kernel rule] all-zero block", flush=True)
    res = {}
    for rule in ("kernel", "fallback"):
        p = [torch.nn.Parameter(torch.ones(4096, device="cuda")), torch.nn.Parameter(torch.ones(4096, device="cuda"))]
        opt = Adafactor8Bit(p, **dict(ADAMW, al_refit_rule=rule))
        p[0].grad = torch.zeros(4096, device="cuda")
        p[1].grad = make_grad((4096,), 1, 1, 4, zero_frac=0.05).cuda()
        opt.step()
        torch.cuda.synchronize()
        res[rule] = [opt.state[q] for q in p]
    z = res["kernel"][0]
    assert torch.all(z["variance_q"] == 0)
    assert torch.all(z["variance_scale"] == np.float32(1e-12)) and torch.all(z["variance_min_log"] == -1e30)
    zf = res["fallback"][0]
    assert torch.all(zf["variance_scale"] == 1.0)
    assert abs(float(zf["variance_min_log"][0]) - (math.log2(1e-38) - 1.0)) < 1e-4
    mk = res["kernel"][1]["variance_min_log"].cpu().numpy()
    mf = res["fallback"][1]["variance_min_log"].cpu().numpy()
    assert np.all(mk == np.float32(kernel_floor(1e-8))) and np.all(mf != mk), (mk, mf)


@pytest.mark.gpu
def test_module_kernel_rule_matches_oracle():
    """fused_update_1d_noclip through the module with set_refit_rule("kernel"): the
    reference's own call (log_eps_sq as the floor argument, optimizer.py:1081-1096)
    refits by the kernels' rule; step-1 codes bit-exact against the oracle's."""
    from adafactor8bit import adafactor8bit_cuda as K
    from adafactor8bit import _state as S
    from oracle.fallback import OracleOptimizer
    print("[kernel rule] module", flush=True)
    shape, bs, mbs = (61, 1003), 2048, 256
    kw = dict(ADAMW, block_size=bs, m_block_size=mbs)
    pc = torch.nn.Parameter(make_param(shape, 0, 3))
    oc = OracleOptimizer([pc], **kw)
    g = make_grad(shape, 0, 1, 3, zero_frac=0.05)
    pc.grad = g
    pg = pc.detach().clone().cuda()
    oc.step()
    K.set_qmap(*[q.cuda() for q in K.qmaps()])
    st = {}
    S.new_al_slot(st, "variance", shape, bs, "al8", "cuda")
    S.new_momentum_codes(st, "m", pg.numel(), mbs, "uf8", "cuda")
    bc1, bc2 = 1.0 - 0.9, 1.0 - 0.999
    alpha = (torch.tensor(1e-4, dtype=torch.float32) * (math.sqrt(bc2) / bc1)).reshape(1).cuda()
    eps1 = 1e-8
    K.set_refit_rule("kernel")
    try:
        K.fused_update_1d_noclip(
            pg, g.cuda(), st["m_q"], st["m_scale"], st["variance_q"], st["variance_scale"],
            st["variance_min_log"], alpha, 0.9, 1.0 - 0.999, eps1 * math.sqrt(bc2), True,
            math.log2(max(eps1 * eps1, 1.17549435e-38)), 0.0, pg.numel(), bs, mbs, 8, 0, 8, False)
    finally:
        K.set_refit_rule("fallback")
    torch.cuda.synchronize()
    so = oc.state[id(pc)]
    for k in ("variance_q", "m_q"):
        a = so[k].reshape(-1).numpy()
        b = st[k].reshape(-1).cpu().numpy()
        assert np.array_equal(a, b), f"{k}: {(a != b).sum()} codes differ"
    for k in ("variance_scale", "variance_min_log", "m_scale"):
        np.testing.assert_allclose(st[k].cpu().numpy(), so[k].reshape(-1).numpy(), rtol=3e-7, atol=0)
    np.testing.assert_allclose(pg.cpu().numpy(), pc.detach().numpy(), rtol=1e-5, atol=0)
