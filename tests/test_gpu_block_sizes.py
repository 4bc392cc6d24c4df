"""Block sizes beyond powers of two.

The reference accepts any V block (B_V) that is a multiple of 128 and any momentum
block (B_M) that is a multiple of 4, at least 32 and a divisor of B_V
(optimizer.py:1395-1416).  Powers of two in [128, 2048] take the unit layout of
k_update1d; every other size takes k_update1d_gen, one workgroup per V block.  Against the oracle over 5 steps, to the parity bar of
the reference-written fixtures: codes equal at step 1, later at most 1e-4 of
codes (+1 per tensor) differ, by at most 2; block metadata within rtol 1e-5;
parameters within rtol 1e-5 except the elements whose codes differed at some
step, which stay within rtol 2e-3 plus 1% of the largest displacement.  The
modes: NOCLIP (AdamW, V-only), NORM/APPLY (RMS clip and Fira, batched) and
MNORM (momentum-only Fira).  Coded momentum on the SGD route and with fp32 V
takes k_sgd_gen at such blocks (one workgroup per whole number of M blocks), and
the factored route's coded momentum k_fupdate_gen (compared as the factored
goldens are, against an exact-reduction oracle).
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


# Blocks beyond 65536 (the reference's rules put no bound on B_V): a V block of
# more than 2048 M blocks runs its M codes in segments of 2048 M blocks (B_V
# 131200 at B_M 32: 4100 M blocks, three segments, the last of four; a tensor of
# 70000 elements: one partial block of two segments), a power of two above 2048
# at AL16 / UF4, the clip + Fira NORM / APPLY passes, no momentum, SGD's momentum
# at B_M 70000, and the stand-alone AL EMA of fp32 momentum at B_V 131200.
BIG_SHAPES = [(300000,), (70000,)]
BIG_CASES = [
    ("adamw_bv131200_bm32", dict(ADAMW, block_size=131200, m_block_size=32)),
    ("adamw_bv262144_bm64_uf4_al16", dict(ADAMW, block_size=262144, m_block_size=64, m_quant_type="uf4",
                                          v_quant_type="al16")),
    ("adamw_bv131200_bm32_clip_fira", dict(ADAMW, block_size=131200, m_block_size=32, d=1.0,
                                           enable_fira_for_adafactor=True)),
    ("rmsprop_bv131200", dict(ADAMW, beta1=None, beta2=0.99, block_size=131200)),
    ("sgd_bv560000_bm70000", dict(SGD, block_size=560000, m_block_size=70000)),
    ("adamw_fp32m_bv131200", dict(ADAMW, m_quant_type="fp32", block_size=131200)),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_general_block_sizes_match_oracle(name, kw):
    _general_vs_oracle(name, kw, SHAPES)


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", BIG_CASES, ids=[c[0] for c in BIG_CASES])
def test_blocks_beyond_65536_match_oracle(name, kw):
    _general_vs_oracle(name, kw, BIG_SHAPES)


def _general_vs_oracle(name, kw, shapes):
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer
    print(f"[block sizes] {name}", flush=True)
    pc = [torch.nn.Parameter(make_param(s, i, 9)) for i, s in enumerate(shapes)]
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


# Factored route (row / column statistics, coded momentum): B_M outside the powers
# of two in [32, 2048] takes k_fupdate_gen, whole M blocks per workgroup, with the
# flat element walk of k_fupdate; CAME pass 1 decodes the old momentum by division.
# Shapes: ragged width (77), a width the tiles take at power-of-two blocks (384)
# and a batched 3-D tensor.  The oracle runs with exact reductions; the comparison
# is the factored golden one (tests/test_gpu_golden.py, _cmp_state) with the
# momentum-scale and parameter bounds of tests/test_gpu_factored_shapes.py.
FSHAPES = [(300, 77), (256, 384), (3, 100, 96)]
FACT = dict(beta1=0.9, beta2=None, beta2_decay=-0.8, beta3=None, factored=True, relative_step=False, lr=1e-3,
            scale_parameter=False)
CAME = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True, relative_step=False,
            scale_parameter=False, scale_weight_decay=False, eps_came=1e-16, lr=1e-4, v_quant_type="al8",
            c_quant_type="al8")
FCASES = [
    ("adafactor_factored_bm36", dict(FACT, block_size=1152, m_block_size=36, d=0.0)),
    ("adafactor_factored_bm100_uf4_clip_fira", dict(FACT, block_size=6400, m_block_size=100, m_quant_type="uf4",
                                                    d=1.0, enable_fira_for_adafactor=True)),
    ("adafactor_factored_bm4096_d4", dict(FACT, block_size=4096, m_block_size=4096, m_quant_type="d4", d=1.0,
                                          weight_decay=0.01)),
    ("came_bm96_d8_clip", dict(CAME, block_size=384, m_block_size=96, m_quant_type="d8", d=1.0)),
    ("came_bm160_uf8_fira", dict(CAME, block_size=640, m_block_size=160, d=1.0, enable_fira_for_adafactor=True,
                                 fira_margin=0.01)),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", FCASES, ids=[c[0] for c in FCASES])
def test_factored_general_m_block_matches_oracle(name, kw):
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    from test_gpu_factored_shapes import _cmp_m_scale, _state_np
    from test_gpu_golden import _cmp_state
    print(f"[block sizes] {name}", flush=True)
    pc = [torch.nn.Parameter(make_param(s, i, 13)) for i, s in enumerate(FSHAPES)]
    p0 = [p.detach().clone() for p in pc]
    pg = [torch.nn.Parameter(p.detach().clone().cuda()) for p in pc]
    oc, og = F.OracleOptimizer(pc, **kw), Adafactor8Bit(pg, **kw)
    for t in range(1, 6):
        for i, (a, b) in enumerate(zip(pc, pg)):
            g = make_grad(tuple(a.shape), i, t, 13, kind="student_t")
            a.grad, b.grad = g, g.cuda()
        old = F.set_exact_reductions(True)
        try:
            oc.step()
        finally:
            F.set_exact_reductions(old)
        og.step()
        torch.cuda.synchronize()
        report = []
        for i, (a, b) in enumerate(zip(pc, pg)):
            key = f"s{t}/p{i}"
            assert og.state[b]["is_quantized"]
            ref_p, mine_p = a.detach().numpy(), b.detach().cpu().numpy()
            disp = float(np.abs(ref_p - p0[i].numpy()).max())
            close = np.abs(mine_p - ref_p) <= 1e-5 * np.abs(ref_p) + 1e-8 + 1e-4 * disp
            assert (~close).mean() <= 1e-4 + 1.0 / close.size, f"{name} {key} param: {(~close).mean():.2e}"
            np.testing.assert_allclose(mine_p, ref_p, rtol=2e-3, atol=1e-8 + 1e-2 * disp,
                                       err_msg=f"{name} {key} param")
            ref_st = _state_np(oc.state[id(a)])
            assert "m_q" in ref_st, f"{name}: the oracle keeps no coded momentum"
            _cmp_m_scale(name, key, og.state[b]["m_scale"].cpu().numpy(), ref_st.pop("m_scale"))
            z = {f"{key}/{k}": v for k, v in ref_st.items()}
            _cmp_state(name, key, og.state[b], z, list(ref_st), report)
        print(report, flush=True)


# APOLLO route: a coded low-rank V block that is not a power of two in [128, 2048],
# or such a momentum block outside [32, 2048], takes the low-rank stage of
# a8_apollo_lowrank_x (the plain stage, or the factorised / CAME ones) with the
# general-block EMA kernels.  The last five cases keep power-of-two blocks: the
# factorised and CAME stages then end in the fused tails (k_fact_tail,
# k_came_tail), here in each state form (fp32 or coded momentum and residual,
# UF4 / D8 momentum, AL16 residual, with and without the RMS clip).  The oracle gets this library's projection output
# (glow_hook, as in the rank-256 test of tests/test_gpu_apollo.py) and reduces
# exactly.  Plain: V and M codes equal but for <= 0.01% (+1 per tensor), by one
# code; block metadata rtol 1e-5; the Fira norm rtol 1e-5; fp32 parameters rtol
# 1e-5 plus 2e-4 of the largest displacement.  Factorised / CAME: the bounds of
# the APOLLO golden comparison (tests/test_gpu_apollo.py, _cmp_state).
APOLLO_BASE = dict(lr=1e-3, beta1=0.9, beta2=0.999, relative_step=False, scale_parameter=False, apollo_rank=32,
                   apollo_update_proj_gap=200, apollo_cache_proj=True, enable_fira_for_apollo=True, d=0.0)
ACASES = [
    ("apollo_plain_bv384_bm96", dict(APOLLO_BASE, block_size=384, m_block_size=96)),
    ("apollo_plain_bv1152_bm36_uf4_al16_clip", dict(APOLLO_BASE, block_size=1152, m_block_size=36,
                                                    m_quant_type="uf4", v_quant_type="al16", d=1.0)),
    ("apollo_plain_bv4096_bm4096_d8_tensor", dict(APOLLO_BASE, block_size=4096, m_block_size=4096,
                                                  m_quant_type="d8", apollo_scale_type="tensor")),
    ("apollo_plain_bv6400_bm100_nofira", dict(APOLLO_BASE, block_size=6400, m_block_size=100,
                                              enable_fira_for_apollo=False, weight_decay=0.01)),
    ("apollo_plain_bv384_bm128", dict(APOLLO_BASE, block_size=384, m_block_size=128)),
    ("apollo_plain_bv640_nomom", dict(APOLLO_BASE, beta1=None, block_size=640)),
    ("apollo_came_bv640_bm160", dict(APOLLO_BASE, beta3=0.9999, d=1.0, eps_came=1e-16, block_size=640,
                                     m_block_size=160)),
    ("apollo_fact_bm36", dict(APOLLO_BASE, apollo_factorize=True, block_size=1152, m_block_size=36)),
    # a V block beyond 65536 (2188 M blocks each: the segmented general kernel) on the low-rank
    # state of a 3000 x 200 matrix (96,000 low-rank elements: one whole block and a ragged one)
    ("apollo_plain_bv70016_bm32", dict(APOLLO_BASE, block_size=70016, m_block_size=32)),
    # power-of-two blocks: the fused low-rank tails (k_fact_tail, k_came_tail) in each state form
    ("apollo_fact_fp32m", dict(APOLLO_BASE, apollo_factorize=True, m_quant_type="fp32")),
    ("apollo_fact_uf4", dict(APOLLO_BASE, apollo_factorize=True, m_quant_type="uf4", m_block_size=64)),
    ("apollo_came_res_fp32", dict(APOLLO_BASE, beta3=0.9999, d=1.0, eps_came=1e-16, c_quant_type="fp32")),
    ("apollo_came_d8_al16", dict(APOLLO_BASE, beta3=0.999, d=1.0, eps_came=1e-16, m_quant_type="d8",
                                 v_quant_type="al16", c_quant_type="al16", block_size=512, m_block_size=128)),
    ("apollo_came_fp32m_d0", dict(APOLLO_BASE, beta3=0.9999, d=0.0, eps_came=1e-16, m_quant_type="fp32")),
]
ASHAPES = [(300, 200), (160, 420)]
BIG_ASHAPES = [(3000, 200), (160, 420)]


class _Z(dict):
    """The oracle's state in the form the APOLLO golden comparison reads."""
    @property
    def files(self):
        return list(self.keys())


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw", ACASES, ids=[c[0] for c in ACASES])
def test_apollo_general_blocks_match_oracle(name, kw, monkeypatch):
    import adafactor8bit.optimizer as O
    import inputs
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    from test_gpu_apollo import _cmp_params, _t2np
    from test_gpu_apollo import _cmp_state as ap_cmp_state
    monkeypatch.setattr(O, "stable_randn", inputs.make_proj)
    monkeypatch.setattr(F, "stable_randn", inputs.make_proj)
    old = F.set_exact_reductions(True)
    plain = name.startswith("apollo_plain")
    shapes = BIG_ASHAPES if kw.get("block_size", 2048) > 65536 else ASHAPES
    try:
        print(f"[block sizes] {name}", flush=True)
        init = [inputs.make_param(s, i, 17) for i, s in enumerate(shapes)]
        pg = [torch.nn.Parameter(x.clone().cuda()) for x in init]
        pc = [torch.nn.Parameter(x.clone()) for x in init]
        og, oc = Adafactor8Bit(pg, **kw), F.OracleOptimizer(pc, **kw)
        lows = [(R, 32) if R >= C else (32, C) for R, C in shapes]
        glows = {}
        oc.glow_hook = lambda p, _g, _pt: glows[id(p)]
        for t in range(1, 6):
            for i, (a, b) in enumerate(zip(pc, pg)):
                g = inputs.make_grad(shapes[i], i, t, 17, zero_frac=0.0)
                a.grad, b.grad = g.clone(), g.cuda()
            og.step()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(pc, pg)):
                ws = og._ws[(b.device, "apollo", id(b))]["ws"].cpu().numpy()
                glows[id(a)] = torch.from_numpy(ws[:lows[i][0] * lows[i][1]].reshape(lows[i]).copy())
            oc.step()
            for i, (a, b) in enumerate(zip(pc, pg)):
                key = f"s{t}/p{i}"
                st, sr = og.state[b], oc.state[id(a)]
                if plain:
                    for k in ("v_low_q", "m_low_q"):
                        if k not in sr:
                            continue
                        x, y = st[k].cpu().numpy().reshape(-1), sr[k].numpy().reshape(-1)
                        frac, mx = gu.code_mismatch(x, y)
                        print(f"  {key} {k}: {frac:.2e} of codes differ, max {mx}", flush=True)
                        assert frac <= 1e-4 + 1.0 / x.size and mx <= 1, f"{name} {key} {k}: {frac:.2e}, max {mx}"
                    for k in ("v_low_scale", "v_low_min_log", "m_low_scale", "scaled_grad_norm_prev"):
                        if k in sr:
                            np.testing.assert_allclose(np.asarray(st[k].cpu()).reshape(-1),
                                                       np.asarray(sr[k]).reshape(-1), rtol=1e-5,
                                                       err_msg=f"{name} {key} {k}")
                    mine, want = b.detach().cpu().numpy(), a.detach().numpy()
                    disp = float(np.abs(want - init[i].numpy()).max())
                    np.testing.assert_allclose(mine, want, rtol=1e-5, atol=1e-8 + 2e-4 * disp,
                                               err_msg=f"{name} {key} param")
                else:
                    z = _Z({f"{key}/{k}": v.numpy() for k, v in sr.items() if torch.is_tensor(v)})
                    keys = [k[len(key) + 1:] for k in z.files]
                    _cmp_params(name, key, _t2np(b), a.detach().numpy(), init[i].numpy())
                    ap_cmp_state(name, key, st, z, keys)
            assert "m_low_q" in og.state[pg[0]] or "m_low" in og.state[pg[0]] or kw.get("beta1") is None
    finally:
        F.set_exact_reductions(old)


# SR writeback in the general-block kernels (k_update1d_gen, k_sgd_gen,
# k_fupdate_gen): the 16-bit result is the stochastic rounding, under the
# reference's stream (kernels.cu:48-131, oracle/sr.py), of the same step run on
# fp32 parameters; the two runs round (p - step * u) once apart, so at most 0.1% of
# the elements may land on the other neighbour (as in the unit-layout SR test,
# tests/test_gpu_apollo.py::test_1d_sr_writeback_stream).
SR_CASES = [
    ("adamw_bv384_bm96", dict(ADAMW, block_size=384, m_block_size=96), [(700, 300), (5000,)]),
    ("sgd_bm36_wd", dict(SGD, block_size=1152, m_block_size=36, weight_decay=0.01), [(700, 300), (5000,)]),
    ("factored_bm36", dict(FACT, block_size=1152, m_block_size=36, d=1.0), [(300, 77), (256, 384)]),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name,kw,shapes", SR_CASES, ids=[c[0] for c in SR_CASES])
def test_general_block_sr_writeback_stream(name, kw, shapes, dtype):
    from adafactor8bit import Adafactor8Bit
    from inputs import make_grad, make_param
    from oracle import sr
    print(f"[block sizes sr] {name} {dtype}", flush=True)
    p16 = [torch.nn.Parameter(make_param(s, i, 3).to("cuda", dtype)) for i, s in enumerate(shapes)]
    p32 = [torch.nn.Parameter(p.detach().float()) for p in p16]
    o16 = Adafactor8Bit(p16, **dict(kw, stochastic_round_writeback=True))
    o32 = Adafactor8Bit(p32, **kw)
    for i, s in enumerate(shapes):
        g = make_grad(s, i, 1, 3).to(dtype).cuda()
        p16[i].grad = g
        p32[i].grad = g.float()
    o16.step()
    o32.step()
    torch.cuda.synchronize()
    rnd = sr.sr_round_bf16 if dtype == torch.bfloat16 else sr.sr_round_fp16
    for p, q in zip(p16, p32):
        assert o16.state[p]["is_quantized"]
        x = q.detach().cpu().numpy().reshape(-1)
        want = rnd(x, seed=int(o16.state[p]["sr_seed"]), step=int(o16.state[p]["step"]))
        got = p.detach().cpu().view(torch.int16).numpy().reshape(-1).view(np.uint16)
        diff = got != want
        print(f"  {tuple(p.shape)}: {diff.mean():.2e} on the other neighbour", flush=True)
        assert diff.sum() <= max(1, 1e-3 * diff.size), diff.mean()
        x16 = x.astype(np.float16) if dtype == torch.float16 else None
        if dtype == torch.bfloat16:
            lo = (x.view(np.uint32) & np.uint32(0xFFFF0000)) >> np.uint32(16)
            assert np.all(np.isin(got[diff].astype(np.int64) - lo[diff].astype(np.int64), [0, 1]))
        else:
            xd, q16 = x[diff], x16[diff]
            other = np.nextafter(q16, np.where(q16.astype(np.float32) < xd, np.float16(np.inf),
                                               np.float16(-np.inf)).astype(np.float16))
            gv = got[diff].view(np.float16)
            assert np.all((gv == q16) | (gv == other))
