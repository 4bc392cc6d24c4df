"""Seeded synthetic inputs shared by the golden-fixture generator and the tests.

Every tensor is drawn with numpy's PCG64 generator seeded per (config seed,
tensor index, step) and only IEEE-exact arithmetic (multiply, divide, sqrt) is
applied afterwards, so the same bits come out on every host.  (torch's CPU
``randn`` is not used: its vectorised normal sampler takes a different code
path per CPU instruction set, so two hosts can disagree in the last bits.)
Distributions follow the benchmark configurations: normal grads with exact
zeros, Student-t heavy tails, log-uniform per-tensor scales, sparse rows.
"""
import math

import numpy as np
import torch


def _rng(seed: int, idx: int, step: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed & 0xFFFFFFFF, idx, step, 0xA8]))


def _normal(rng, shape):
    return rng.standard_normal(size=tuple(shape), dtype=np.float32)


def make_param(shape, idx: int, seed: int = 0, dtype=torch.float32, kind: str = "normal"):
    """Initial parameter: N(0, 0.02^2) for matrices, ones for norm vectors."""
    if kind == "ones":
        return torch.ones(shape, dtype=torch.float32).to(dtype)
    x = _normal(_rng(seed, idx, 0), shape) * np.float32(0.02)
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype)


def make_grad(shape, idx: int, step: int, seed: int = 0, kind: str = "normal_zeros",
              dtype=torch.float32, zero_frac: float = 0.05, scale: float = 1e-3):
    """Gradient for tensor ``idx`` at optimizer step ``step`` (1-based).

    kinds:
      normal_zeros  scale*N(0,1) with a fraction ``zero_frac`` of exact zeros
      student_t     scale*t3 (t3 = z*sqrt(3/chi2_3) from four normals), 5% zeros
      logscale      N(0,1)*10^U(-5,-2) with the factor fixed per tensor
      sparse_rows   scale*t3 with 90% of the rows (dim 0) exactly zero
    """
    rng = _rng(seed, idx + 1000, step)
    shape = tuple(shape)
    f = np.float32
    if kind == "normal_zeros":
        x = _normal(rng, shape) * f(scale)
        if zero_frac > 0:
            x = x * (rng.random(size=shape, dtype=np.float32) >= f(zero_frac))
    elif kind in ("student_t", "sparse_rows"):
        z = _normal(rng, shape)
        c = _normal(rng, (3,) + shape)
        c = (c * c).sum(axis=0, dtype=np.float32)
        x = z * np.sqrt(f(3.0) / np.maximum(c, f(1e-12))) * f(scale)
        if kind == "sparse_rows":
            rows = shape[0]
            perm = _rng(seed, idx + 2000, 0).permutation(rows)
            x[perm[: int(math.floor(rows * 0.9))]] = 0.0
        elif zero_frac > 0:
            x = x * (rng.random(size=shape, dtype=np.float32) >= f(zero_frac))
    elif kind == "logscale":
        u = float(_rng(seed, idx + 3000, 0).random())
        s = f(10.0 ** (-5.0 + 3.0 * u))
        x = _normal(rng, shape) * s
    else:
        raise ValueError(kind)
    x = np.ascontiguousarray(x.astype(np.float32))
    return torch.from_numpy(x).to(dtype)


def make_proj(shape, seed: int, device=None, dtype=torch.float32):
    """Stand-in for the reference's ``stable_randn(shape, seed, device, dtype)``
    (optimizer.py:139-149) with a host-independent stream: N(0, 1) from PCG64
    keyed by the 64-bit seed.  The golden generator and the tests install it in
    place of the torch-generator version, whose CPU and GPU streams differ, so
    the reference's trajectories and this build's see the same projection."""
    s = int(seed) & 0xFFFFFFFFFFFFFFFF
    rng = np.random.Generator(np.random.PCG64([s & 0xFFFFFFFF, s >> 32, 0xA9]))
    x = np.ascontiguousarray(rng.standard_normal(size=tuple(shape), dtype=np.float32))
    t = torch.from_numpy(x).to(dtype)
    return t if device is None else t.to(device)
