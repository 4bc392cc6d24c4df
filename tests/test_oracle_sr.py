"""Pins the CPU restatement of the stochastic-rounding stream (oracle/sr.py).

SplitMix64 against its published first output; the bf16 and fp16 roundings
against what defines them: the result is one of the two neighbours of x (fp16:
found by float16 nextafter, subnormals included), exact values and NaN keep
their class, no rounding to infinity (fp16 saturates at 65504), the threshold
u < (x - lo) / (hi - lo), and the rounding is unbiased (mean of many draws
equals x).
"""
import numpy as np
import torch

from oracle import sr


def _bf16_bits_to_f32(bits):
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def test_splitmix64_known_answer():
    # SplitMix64 (Steele, Lea, Flood 2014) seeded with 0: its first four outputs
    # (the state advances by the golden gamma, so output k mixes state k * gamma)
    published = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    g = np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        got = [int(sr.splitmix64(np.uint64(k) * g)) for k in range(4)]
    assert got == published


def test_counter_layout():
    # the counter is seed*gamma + step*K + idx (mod 2^64): idx and the counter add
    a = sr.sr_bits(3, 5, np.arange(4, dtype=np.uint64))
    with np.errstate(over="ignore"):
        c0 = np.uint64(3) * np.uint64(0x9E3779B97F4A7C15) + np.uint64(5) * np.uint64(0xD1B54A32D192ED03)
    b = (sr.splitmix64(c0 + np.arange(4, dtype=np.uint64)) >> np.uint64(32)).astype(np.uint32)
    assert np.array_equal(a, b)
    # different seeds / steps give different streams
    assert not np.array_equal(sr.sr_bits(3, 6, np.arange(64)), sr.sr_bits(3, 5, np.arange(64)))
    assert not np.array_equal(sr.sr_bits(4, 5, np.arange(64)), sr.sr_bits(3, 5, np.arange(64)))


def test_uniform_range():
    u = sr.sr_uniform(1, 1, np.arange(1 << 16))
    assert u.dtype == np.float32 and u.min() >= 0.0 and u.max() < 1.0
    assert abs(float(u.mean()) - 0.5) < 0.01


def test_bf16_neighbours_and_unbiased():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-6, 3, 4096)).astype(np.float32)
    down = (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    up = ((x.view(np.uint32) & np.uint32(0xFFFF0000)) + np.uint32(0x10000)).view(np.float32)
    acc = np.zeros(x.size, dtype=np.float64)
    n = 2000
    for step in range(n):
        r = _bf16_bits_to_f32(sr.sr_round_bf16(x, seed=7, step=step))
        assert np.all((r == down) | (r == up))
        acc += r
    mean = acc / n
    # unbiased: E[r] = x; the draw's standard error is |up - down| * 0.5 / sqrt(n)
    se = np.abs(up.astype(np.float64) - down) * 0.5 / np.sqrt(n)
    assert np.all(np.abs(mean - x) <= 5 * se + 1e-30)


def test_bf16_special_values():
    vals = np.array([0.0, -0.0, 1.0, -2.5, np.inf, -np.inf, np.nan,
                     np.float32(3.3895314e38),           # largest bf16: never rounds up to inf
                     np.finfo(np.float32).max], dtype=np.float32)
    u = np.zeros(vals.size, dtype=np.float32)            # u = 0 rounds up whenever allowed
    r = sr.sr_fp32_to_bf16_bits(vals, u)
    exact = torch.tensor(vals[:4]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(r[:4], exact)
    assert r[4] == 0x7F80 and r[5] == 0xFF80 and r[6] == 0x7FC0
    assert r[7] == 0x7F7F
    assert r[8] == 0x7F7F          # fp32 max: the round-up target would be infinity


def _fp16_bracket(x):
    """The two fp16 values around x (equal when fp16 holds x), by float16 nextafter."""
    q = x.astype(np.float16)
    qf = q.astype(np.float32)
    toward = np.where(qf < x, np.float16(np.inf), np.float16(-np.inf)).astype(np.float16)
    other = np.nextafter(q, toward).astype(np.float32)
    lo = np.where(qf <= x, qf, other)
    hi = np.where(qf <= x, np.where(qf == x, qf, other), qf)
    return lo, hi


def test_fp16_neighbours_and_unbiased():
    rng = np.random.default_rng(1)
    # normal, subnormal (< 6.1e-5) and near-saturation fp16 magnitudes, both signs
    x = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-7, 4.5, 4096)).astype(np.float32)
    x = x[np.abs(x) <= 65504.0]
    lo, hi = _fp16_bracket(x)
    acc = np.zeros(x.size, dtype=np.float64)
    n = 2000
    for step in range(n):
        r = sr.sr_round_fp16(x, seed=11, step=step).view(np.float16).astype(np.float32)
        assert np.all((r == lo) | (r == hi))
        acc += r
    se = np.abs(hi.astype(np.float64) - lo) * 0.5 / np.sqrt(n)
    assert np.all(np.abs(acc / n - x) <= 5 * se + 1e-30)


def test_fp16_threshold_and_exact_values():
    # x = lo + t (hi - lo) goes up exactly when u < t (t exact in fp32 here)
    lo, hi = np.float32(1.0), np.float32(1.0 + 2.0 ** -10)
    for t in (0.25, 0.5, 0.75):
        x = np.full(3, lo + np.float32(t) * (hi - lo), dtype=np.float32)
        u = np.array([t - 2.0 ** -24, t, t + 2.0 ** -24], dtype=np.float32)
        r = sr.sr_fp32_to_fp16_bits(x, u).view(np.float16).astype(np.float32)
        assert r.tolist() == [hi, lo, lo]
    # every finite fp16 value comes back unchanged whatever u is
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    fin = allh[np.isfinite(allh)]
    xs = fin.astype(np.float32)
    for uu in (0.0, 0.999):
        r = sr.sr_fp32_to_fp16_bits(xs, np.full(xs.size, uu, dtype=np.float32))
        same = (r == fin.view(np.uint16)) | ((xs == 0) & ((r & 0x7FFF) == 0))
        assert np.all(same)


def test_fp16_special_values():
    vals = np.array([np.inf, -np.inf, np.nan, 65504.0, 65505.0, -1e6, 3e-8, -3e-8], dtype=np.float32)
    r = sr.sr_fp32_to_fp16_bits(vals, np.zeros(vals.size, dtype=np.float32))
    assert r[0] == 0x7C00 and r[1] == 0xFC00 and (r[2] & 0x7FFF) == 0x7E00
    assert r[3] == 0x7BFF and r[4] == 0x7BFF and r[5] == 0xFBFF   # saturation, no infinity
    # 3e-8 lies between 0 and the smallest subnormal 2^-24 (5.96e-8): u = 0 takes
    # the upper neighbour (toward +inf), 2^-24 for 3e-8 and -0 for -3e-8
    assert r[6] == 0x0001 and r[7] == 0x8000
