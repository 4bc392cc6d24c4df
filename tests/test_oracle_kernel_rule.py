"""The reference's fused 1-D CUDA kernels' AL rule, restated in the oracle
(oracle/fallback.py: al_quantize_kernel, al_dequantize_kernel, kernel_floor).

kernels.cu cannot be compiled or run here, so the restatement is pinned by what
kernels.cu:318-326, 686-687 and 772-791 fix in closed form, and by its relation
to the CPU rule (optimizer.py:299-353, itself pinned against reference-written
trajectories):
* a block holding a zero takes l_min = log2(max(eps1^2, FLT_MIN)), the floor;
* l_max is capped at 126 and codes above it clamp to 255;
* a block with no non-zero value gets scale 1e-12, min_log -1e30 and codes 0;
* equal values give l_min = l_max - 1, s = 1 and code 255;
* values below the floor take code 1;
* code 1 decodes to 2^l_min exactly, decode is monotone in the code, and
  quantize(decode(codes)) returns the codes;
* away from zeros, the floor and the cap, both rules fit the same [l_min, l_max]
  and their codes differ by at most one, only where the two operation orders
  round a near-tie differently.
A dropped cap, a zero-exclusive minimum, a swapped floor or a wrong operand in the
code formula fails one of these.
"""
import math

import numpy as np
import torch

from oracle import fallback as F

FLOOR = F.kernel_floor(1e-8)


def _block(vals, bs=None):
    v = torch.tensor(vals, dtype=torch.float32)
    return F.al_quantize_kernel(v, bs or v.numel(), FLOOR)


def test_kernel_floor_values():
    assert FLOOR == np.float32(math.log2(1e-16))
    assert abs(FLOOR - (-53.150849518197795)) < 1e-5
    # eps1^2 below FLT_MIN: the floor is log2(FLT_MIN) = -126 exactly
    assert F.kernel_floor(1e-30) == -126.0


def test_zero_in_block_takes_the_floor():
    q, s, ml, _ = _block([0.0, 1e-3, 2.0, 4.0])
    assert float(ml[0]) == FLOOR
    assert float(s[0]) == np.float32(np.float32(2.0) - np.float32(FLOOR))   # lmax = log2(4) = 2
    assert int(q[0]) == 0 and int(q[3]) == 255
    # the CPU rule ignores the zero: its l_min is log2(1e-3)
    q2, s2, ml2, _ = F.al_quantize(torch.tensor([0.0, 1e-3, 2.0, 4.0]), 4)
    assert abs(float(ml2[0]) - math.log2(1e-3)) < 1e-5


def test_codes_follow_the_kernel_formula():
    rng = np.random.default_rng(3)
    vals = np.concatenate([[0.0], rng.lognormal(-20, 6, 255)]).astype(np.float32)
    q, s, ml, _ = _block(vals)
    lm, sc = np.float32(ml[0]), np.float32(s[0])
    inv = np.float32(np.float32(254.0) / sc)
    logs = np.log2(vals[1:].astype(np.float64)).astype(np.float32)
    want = np.clip(np.rint(((logs - lm).astype(np.float32) * inv).astype(np.float32)) + 1, 1, 255)
    np.testing.assert_array_equal(q.numpy()[1:], want.astype(np.uint8))
    # values below the floor take code 1
    assert (q.numpy()[1:][vals[1:] < 2.0 ** FLOOR] == 1).all()
    assert (vals[1:] < 2.0 ** FLOOR).any()


def test_lmax_cap_126():
    q, s, ml, _ = _block([1.0, 2.0 ** 120, np.float32(2.0 ** 127), np.float32(3e38)])
    assert float(ml[0]) == 0.0                       # no zero: l_min = log2(1) = 0 > floor
    assert float(s[0]) == 126.0                      # l_max capped at 126
    assert q.tolist() == [1, round(120 / 126 * 254) + 1, 255, 255]


def test_all_zero_block_metadata():
    q, s, ml, _ = _block([0.0] * 8 + [1.0] * 8, bs=8)
    assert float(s[0]) == np.float32(1e-12) and float(ml[0]) == np.float32(-1e30)
    assert q[:8].tolist() == [0] * 8
    d = F.al_dequantize_kernel(q, s, ml, 16)
    assert d[:8].tolist() == [0.0] * 8
    # the CPU rule's all-zero block: s = 1, l_min = log2(1e-38) - 1
    _, s2, ml2, _ = F.al_quantize(torch.zeros(8), 8)
    assert float(s2[0]) == 1.0 and abs(float(ml2[0]) - (math.log2(1e-38) - 1)) < 1e-4


def test_equal_values():
    q, s, ml, _ = _block([0.5] * 6)
    assert float(ml[0]) == -2.0 and float(s[0]) == 1.0
    assert q.tolist() == [255] * 6


def test_decode_properties_and_round_trip():
    rng = np.random.default_rng(7)
    for levels in (256, 65536):
        v = torch.from_numpy(np.where(rng.random(4096) < 0.05, 0.0, rng.lognormal(-12, 4, 4096)).astype(np.float32))
        q, s, ml, _ = F.al_quantize_kernel(v, 1024, FLOOR, levels)
        d = F.al_dequantize_kernel(q, s, ml, v.numel())
        assert torch.equal(d == 0, v == 0)
        q2, s2, ml2, _ = F.al_quantize_kernel(d, 1024, FLOOR, levels)
        # decode -> encode returns the codes where the refit reproduces the block's
        # [l_min, l_max] (always here: each block keeps its zero, so l_min stays the
        # floor, and code L-1 decodes to within an ulp of 2^l_max)
        assert torch.equal(ml2, ml)
        qq = q.numpy().astype(np.int64) % levels
        qq2 = q2.numpy().astype(np.int64) % levels
        assert np.abs(qq - qq2).max() <= 1 and (qq != qq2).mean() < 1e-3
    # code 1 decodes to 2^l_min exactly; decode is monotone in the code
    codes = torch.arange(256, dtype=torch.int64).to(torch.uint8)
    d = F.al_dequantize_kernel(codes, torch.tensor([37.5]), torch.tensor([-20.25]), 256).numpy()
    assert d[1] == np.float32(2.0 ** -20.25)
    assert np.all(np.diff(d[1:].astype(np.float64)) > 0)


def test_agrees_with_cpu_rule_inside_the_range():
    """No zeros, nothing below the floor or above 2^126: both rules fit the same
    block range and code within one step of each other (different operation orders
    round near-ties differently)."""
    rng = np.random.default_rng(11)
    v = torch.from_numpy(rng.lognormal(-15, 5, 1 << 16).astype(np.float32))
    qk, sk, mk, _ = F.al_quantize_kernel(v, 2048, FLOOR)
    qc, sc, mc, _ = F.al_quantize(v, 2048, -126.0)
    np.testing.assert_allclose(mk.numpy(), mc.numpy(), rtol=0, atol=2e-6)
    np.testing.assert_allclose(sk.numpy(), sc.numpy(), rtol=1e-6)
    diff = np.abs(qk.numpy().astype(int) - qc.numpy().reshape(-1).astype(int))
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-3


def test_oracle_step_uses_the_rule_for_the_1d_path():
    """al_refit_rule="kernel" in the oracle's AdamW step: a block with an exact-zero
    gradient (v = 0 at step 1, Adam's eps_g = 0) takes the floor; without it, the
    CPU rule's l_min."""
    g = torch.ones(4096)
    g[7] = 0.0
    g[100:200] = 1e-3
    res = {}
    for rule in ("fallback", "kernel"):
        p = torch.nn.Parameter(torch.zeros(4096))
        opt = F.OracleOptimizer([p], lr=1e-3, beta1=0.9, beta2=0.999, beta2_decay=None, factored=False,
                                relative_step=False, scale_parameter=False, eps=(1e-8, 1e-3), block_size=2048,
                                al_refit_rule=rule)
        p.grad = g.clone()
        opt.step()
        res[rule] = opt.state[id(p)]
    assert float(res["kernel"]["variance_min_log"][0]) == FLOOR
    assert float(res["kernel"]["variance_min_log"][1]) != FLOOR   # block 1 holds no zero
    assert abs(float(res["fallback"]["variance_min_log"][0]) - math.log2(0.001 * 1e-3 * 1e-3)) < 0.1
