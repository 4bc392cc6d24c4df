"""Seeded synthetic inputs shared by the golden-fixture generator and the tests.

Every tensor is drawn on the CPU from a ``torch.Generator`` seeded per
(config seed, tensor index, step), so the CPU oracle, the GPU path and the
fixture generator see identical bits.  Distributions follow the workload
descriptions of the benchmark configurations (normal grads with exact zeros,
Student-t heavy tails, log-uniform per-tensor scales, sparse embedding rows).
"""
import math

import torch


def _gen(seed: int, idx: int, step: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed((seed * 1_000_003 + idx * 7919 + step * 104_729) & ((1 << 62) - 1))
    return g


def make_param(shape, idx: int, seed: int = 0, dtype=torch.float32, kind: str = "normal"):
    """Initial parameter: N(0, 0.02^2) for matrices, ones for norm vectors."""
    if kind == "ones":
        return torch.ones(shape, dtype=torch.float32).to(dtype)
    g = _gen(seed, idx, 0)
    return (torch.randn(shape, generator=g) * 0.02).to(dtype)


def make_grad(shape, idx: int, step: int, seed: int = 0, kind: str = "normal_zeros",
              dtype=torch.float32, zero_frac: float = 0.05, scale: float = 1e-3):
    """Gradient for tensor ``idx`` at optimizer step ``step`` (1-based).

    kinds:
      normal_zeros  scale*N(0,1) with a fraction ``zero_frac`` of exact zeros
      student_t     scale*t3, t3 = z*sqrt(3/chi2_3) from four normals
      logscale      scale*N(0,1)*10^U(-5,-2) with the factor fixed per tensor
      sparse_rows   student_t with 90% of the rows (dim 0) exactly zero
    """
    g = _gen(seed, idx, step)
    if kind == "normal_zeros":
        x = torch.randn(shape, generator=g) * scale
        if zero_frac > 0:
            keep = torch.rand(shape, generator=g) >= zero_frac
            x = x * keep
    elif kind in ("student_t", "sparse_rows"):
        z = torch.randn(shape, generator=g)
        c = torch.randn((3,) + tuple(shape), generator=g).square().sum(0)
        x = z * torch.sqrt(3.0 / c.clamp(min=1e-12)) * scale
        if kind == "sparse_rows":
            gr = _gen(seed, idx, 0)
            rows = shape[0]
            perm = torch.randperm(rows, generator=gr)
            zero_rows = perm[: int(math.floor(rows * 0.9))]
            x[zero_rows] = 0.0
        if zero_frac > 0 and kind == "student_t":
            keep = torch.rand(shape, generator=g) >= zero_frac
            x = x * keep
    elif kind == "logscale":
        gs = _gen(seed, idx, 0)
        s = 10.0 ** (-5.0 + 3.0 * torch.rand((), generator=gs).item())
        x = torch.randn(shape, generator=g) * s
    else:
        raise ValueError(kind)
    return x.to(torch.float32).to(dtype)
