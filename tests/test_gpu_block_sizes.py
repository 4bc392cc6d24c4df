"""Block sizes beyond powers of two.

The reference accepts any V block (B_V) that is a multiple of 128 and any momentum
block (B_M) that is a multiple of 4, at least 32 and a divisor of B_V
(optimizer.py:1395-1416).  Powers of two in [128, 2048] take the unit layout of
k_update1d; every other size (and B_V up to 65536) takes k_update1d_gen, one
workgroup per V block.  Against the oracle over 5 steps, to the parity bar of
the reference-written fixtures: codes equal at step 1, later at most 1e-4 of
codes (+1 per tensor) differ, by at most 2; block metadata within rtol 1e-5;
parameters within rtol 1e-5 except the elements whose codes differed at some
step, which stay within rtol 2e-3 plus 1% of the largest displacement.  The
modes: NOCLIP (AdamW, V-only), NORM/APPLY (RMS clip and Fira, batched) and
MNORM (momentum-only Fira).  Coded momentum on the SGD route and with fp32 V
takes k_sgd_gen at such blocks (one workgroup per whole number of M blocks).
"""
import numpy as np
import pytest
import torch

import golden_util as gu
from inputs import make_grad, make_param

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
             scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-3)
CASES = [
    ("adamw_bv384_bm96", dict(ADAMW, block_size=384, m_block_size=96)),
    ("adamw_bv1152_bm36_wd", dict(ADAMW, block_size=1152, m_block_size=36, weight_decay=0.1,
                                  scale_weight_decay=True)),
    ("adamw_bv6400_bm100_uf4_al16", dict(ADAMW, block_size=6400, m_block_size=100, m_quant_type="uf4",
                                         v_quant_type="al16")),
    ("adamw_bv640_bm160_d8", dict(ADAMW, block_size=640, m_block_size=160, m_quant_type="d8")),
    ("adamw_bv4096_bm256", dict(ADAMW, block_size=4096, m_block_size=256)),
    ("adamw_bv1536_bm48_d4", dict(ADAMW, block_size=1536, m_block_size=48, m_quant_type="d4")),
    ("rmsprop_bv384", dict(ADAMW, beta1=None, beta2=0.99, block_size=384)),
    ("adamw_bv384_bm96_clip_fira", dict(ADAMW, block_size=384, m_block_size=96, d=1.0,
                                        enable_fira_for_adafactor=True)),
    ("mom1d_bv640_bm160_fira", dict(beta1=0.9, beta2=None, beta2_decay=-0.8, factored=False, relative_step=False,
                                    scale_parameter=False, lr=1e-3, block_size=640, m_block_size=160,
                                    enable_fira_for_adafactor=True)),
]
SGD = dict(ADAMW, beta2=None, beta2_decay=None, lr=1e-2)
CASES += [
    # coded momentum outside the fused 1-D kernel: SGD (k_sgd) and fp32 V with the
    # stand-alone momentum EMA (a8_m_quantize_lerp), at blocks the unit layout cannot take
    ("sgd_bv1152_bm36", dict(SGD, block_size=1152, m_block_size=36, weight_decay=0.01)),
    ("sgd_bv6400_bm100_uf4_clip_fira", dict(SGD, block_size=6400, m_block_size=100, m_quant_type="uf4", d=1.0,
                                            enable_fira_for_adafactor=True)),
    ("sgd_bv4608_bm4608_d8", dict(SGD, block_size=4608, m_block_size=4608, m_quant_type="d8")),
    ("adamw_fp32v_bv6400_bm100", dict(ADAMW, v_quant_type="fp32", block_size=6400, m_block_size=100)),
    # quantised V with fp32 momentum: the stand-alone AL EMA (k_vema_gen) at such blocks
    ("adamw_fp32m_bv640_al8", dict(ADAMW, m_quant_type="fp32", block_size=640)),
    ("adamw_fp32m_bv3200_al16_clip", dict(ADAMW, m_quant_type="fp32", v_quant_type="al16", block_size=3200, d=1.0)),
    ("mom1d_fp32v_bv1152_bm36_fira", dict(beta1=0.9, beta2=None, beta2_decay=-0.8, factored=False,
                                          relative_step=False, scale_parameter=False, lr=1e-3, v_quant_type="fp32",
                                          block_size=1152, m_block_size=36, enable_fira_for_adafactor=True)),
]
SHAPES = [(300, 77), (5000,), (4096,), (9000,)]


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_general_block_sizes_match_oracle(name, kw):
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer
    print(f"[block sizes] {name}", flush=True)
    pc = [torch.nn.Parameter(make_param(s, i, 9)) for i, s in enumerate(SHAPES)]
    pg = [torch.nn.Parameter(p.detach().clone().cuda()) for p in pc]
    p0 = [p.detach().clone() for p in pc]
    oc, og = OracleOptimizer(pc, **kw), Adafactor8Bit(pg, **kw)
    touched = [np.zeros(p.numel(), dtype=bool) for p in pc]
    for t in range(1, 6):
        for i, (a, b) in enumerate(zip(pc, pg)):
            g = make_grad(tuple(a.shape), i, t, 9, kind="student_t")
            a.grad, b.grad = g, g.cuda()
        oc.step()
        og.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pc, pg)):
            sc, sg = oc.state[id(a)], og.state[b]
            assert sg["is_quantized"]
            n = touched[i].size
            for k in ("variance_q", "m_q"):
                if k not in sc:
                    continue
                x, y = sc[k].reshape(-1).numpy(), sg[k].reshape(-1).cpu().numpy()
                frac, mx = gu.code_mismatch(x, y)
                if t == 1:
                    assert frac == 0.0, f"{name} p{i} {k}: {frac:.2e} differ at step 1"
                assert frac <= 1e-4 + 1.0 / x.size and mx <= 2, f"{name} p{i} {k} step {t}: {frac:.2e}, max {mx}"
                if k == "variance_q":
                    touched[i] |= (x != y)[:n]
                elif x.size == y.size and sc[k].dtype == torch.uint8 and kw.get("m_quant_type", "uf8") in ("uf8", "d8"):
                    touched[i] |= (x != y)[:n]
                else:   # 4-bit codes: two elements per byte
                    d = np.repeat(x != y, 2)[:n]
                    touched[i] |= d
    for i, (a, b) in enumerate(zip(pc, pg)):
        sc, sg = oc.state[id(a)], og.state[b]
        for k in ("variance_scale", "variance_min_log", "m_scale"):
            if k in sc:
                np.testing.assert_allclose(sg[k].cpu().numpy().reshape(-1), sc[k].numpy().reshape(-1), rtol=1e-5,
                                           err_msg=f"{name} p{i} {k}")
        tm = touched[i]
        print(f"  p{i} {tuple(a.shape)}: {tm.mean():.2e} of elements ever had a differing code", flush=True)
        P, Q = b.detach().cpu().reshape(-1).numpy(), a.detach().reshape(-1).numpy()
        np.testing.assert_allclose(P[~tm], Q[~tm], rtol=1e-5, atol=1e-8, err_msg=f"{name} p{i} param")
        disp = float(np.abs(Q - p0[i].reshape(-1).numpy()).max())
        np.testing.assert_allclose(P[tm], Q[tm], rtol=2e-3, atol=1e-8 + 1e-2 * disp, err_msg=f"{name} p{i}")
