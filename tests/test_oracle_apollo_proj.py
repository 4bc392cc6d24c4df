"""The CPU restatement of capturable APOLLO's projection schedule (oracle/apollo_proj.py).

* next_seed: the MT19937 restatement equals the reference's own next_seed
  (torch.randint on a CPU generator, optimizer.py:152-155, as this package's
  optimizer.next_seed keeps it) for 64-bit seeds, including seeds whose high
  32 bits are set (the generator keeps the low 32) and chains of seeds.
* the generator: its uniforms are SplitMix64 outputs 2k + 1 and 2k + 2 (pinned
  by the published first output, tests/test_oracle_sr.py), and its values are
  N(0, 1) / sqrt(r): mean, variance, tail mass and a Kolmogorov-Smirnov distance
  on 2^21 draws, pair independence, and the P / P^T orientation of both sides.
  A dropped factor (the 2 in -2 ln u1, the 2 pi), a swapped uniform or a wrong
  sign in the exponent fails one of these.
"""
import math

import numpy as np
import pytest
from scipy import stats

from oracle import apollo_proj as ap
from oracle.sr import splitmix64


def test_next_seed_matches_torch_generator():
    from adafactor8bit.optimizer import next_seed as ref_next_seed
    rng = np.random.default_rng(5)
    seeds = [0, 1, 2, 42, 921, 2 ** 31 - 1, 2 ** 32 - 1, 2 ** 32, 2 ** 32 + 5, 2 ** 40 + 17, 2 ** 63 - 2]
    seeds += [int(x) for x in rng.integers(0, 2 ** 63 - 1, size=120, dtype=np.int64)]
    for s in seeds:
        assert ap.next_seed(s) == ref_next_seed(s), s
    s = 7
    for _ in range(20):   # a chain, as successive refreshes walk it
        t = ref_next_seed(s)
        assert ap.next_seed(s) == t
        s = t


def test_generator_uses_splitmix64_outputs():
    # output i of SplitMix64 seeded with s is mix(s + i * gamma); oracle.sr.splitmix64(x) = mix(x + gamma)
    seed, k = 12345, np.arange(8, dtype=np.uint64)
    gold = np.uint64(0x9E3779B97F4A7C15)
    with np.errstate(over="ignore"):
        a = splitmix64(np.uint64(seed) + np.uint64(2) * k * gold)
        b = splitmix64(np.uint64(seed) + (np.uint64(2) * k + np.uint64(1)) * gold)
    u1 = ((a >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    z = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * math.pi * u2)).astype(np.float32)
    np.testing.assert_array_equal(ap.normals(seed, k), z)
    # SplitMix64 seeded with 0: first output (published) is 0xE220A8397B1DCDAF
    assert int(splitmix64(np.uint64(0))) == 0xE220A8397B1DCDAF


def test_generator_distribution_is_standard_normal():
    z = ap.normals(2024, np.arange(1 << 21, dtype=np.uint64)).astype(np.float64)
    n = z.size
    assert abs(z.mean()) < 5.0 / math.sqrt(n)
    assert abs(z.var() - 1.0) < 6.0 * math.sqrt(2.0 / n)
    assert abs((np.abs(z) > 2.0).mean() - 0.0455003) < 1e-3     # two-sided tail beyond 2 sigma
    assert abs((np.abs(z) > 3.0).mean() - 0.0026998) < 2.5e-4
    assert stats.kstest(z, "norm").statistic < 2e-3
    # neighbouring elements (consecutive SplitMix64 outputs) are uncorrelated
    assert abs(np.corrcoef(z[:-1], z[1:])[0, 1]) < 5.0 / math.sqrt(n)


@pytest.mark.parametrize("rows,cols,rank", [(40, 24, 8), (24, 40, 8), (33, 33, 5)])
def test_proj_t_orientation_and_scale(rows, cols, rank):
    pt = ap.proj_t(rows, cols, rank, 99)
    right = rows >= cols
    pshape = (rank, cols) if right else (rows, rank)
    assert pt.shape == (pshape[1], pshape[0]) and pt.dtype == np.float32
    z = ap.normals(99, np.arange(pshape[0] * pshape[1], dtype=np.uint64)).reshape(pshape)
    np.testing.assert_array_equal(pt, (z / np.float32(math.sqrt(rank))).T)
