"""Factored Adafactor (C2) and CAME (C3) at matrix shapes like TinyLlama's, on the GPU,
against the CPU oracle.

The statistics pass tiles a matrix into strips of tr rows x 1024 columns: tr = 64
above 2048 rows, and a matrix wider than 1024 columns has several column chunks
whose row partial sums are reduced across chunks.  The update runs on the same
tiles when the width is a multiple of 4 (and, with quantised momentum, of the
momentum block), else as flat 2048-element units.  The shapes below reach each of
these:

  2304 x 2080      tr 64, 3 column chunks; C2 tiled update, C3 flat (2080 % 256 != 0)
  4160 x 1280      tr 64, 2 column chunks, 65 strips; tiled update in C2 and C3
  3 x 1100 x 2050  batched, tr 32, 3 column chunks; flat update (2050 % 4 != 0)

The oracle runs with exact reductions (float64 accumulation rounded once to float32,
oracle.fallback.set_exact_reductions).  The reference's own fallback reduces the row and
column means and the clip norms in float32 in torch's CPU order; over millions of terms
that order drifts from the exact value by up to ~1e-4 relative (the CAME clip factor of
a 2304 x 2080 matrix), which moves every momentum scale of the matrix by as much, and
it flips AL8 statistics codes near rounding boundaries at ~1e-4 of codes per step.
That drift belongs to the reference's summation order, not to the algorithm; the test
prints it (a second oracle in the reference's order runs alongside) and holds this
library to the exact values.

Tolerances are those of the factored golden comparison (tests/test_gpu_golden.py):
AL8 statistics codes at most 0.01% differ (plus one code per vector), by at most 2;
AL16 statistics on their decoded values, within three AL16 steps; block ranges to
4e-5 absolute (log2 units); momentum codes 0.01% and their block scales rtol 1e-5
(except blocks whose largest element flipped a code, see _cmp_m_scale); parameters within rtol 1e-5 plus
1e-4 of the largest displacement, except at most 0.01% of elements (a flipped code),
which stay within rtol 2e-3 plus 1% of it.
"""
import numpy as np
import pytest
import torch

from inputs import make_grad, make_param
from test_gpu_golden import _cmp_state

SHAPES = [(2304, 2080), (4160, 1280), (3, 1100, 2050)]

# C2: the adafactor preset (presets.py:42-49) with the defaults d = 1,
# scale_parameter, eps = (1e-30, 1e-3); B_V 256, AL8.
C2 = dict(beta1=None, beta2=None, beta2_decay=-0.8, beta3=None, factored=True, relative_step=False, lr=1e-3,
          block_size=256, v_quant_type="al8")
# C3: the came preset (presets.py:77-88) with Fira; UF8 M, AL16 V and confidence, B_V 2048.
C3 = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True, relative_step=False,
          scale_parameter=False, scale_weight_decay=False, d=1.0, eps_came=1e-16, lr=1e-4, block_size=2048,
          m_block_size=256, m_quant_type="uf8", v_quant_type="al16", c_quant_type="al16",
          enable_fira_for_adafactor=True, fira_margin=0.01)

CASES = [("adafactor_factored_c2", C2, "student_t"), ("came_c3", C3, "logscale")]


def _state_np(st):
    return {k: v.numpy() for k, v in st.items() if torch.is_tensor(v)}


def _code_report(oc_a, oc_b, pa, pb):
    """Fraction of statistics / momentum codes that differ between two oracle runs."""
    n = d = 0
    for x, y in zip(pa, pb):
        sa, sb = oc_a.state[id(x)], oc_b.state[id(y)]
        for k, v in sa.items():
            if torch.is_tensor(v) and k.endswith("_q"):
                a = v.reshape(-1).numpy().astype(np.int64) & 0xFFFF
                b = sb[k].reshape(-1).numpy().astype(np.int64) & 0xFFFF
                n += a.size
                d += int((a != b).sum())
    return d / max(n, 1)


def _cmp_m_scale(name, key, mine, ref):
    """Momentum block scales (absmax of M'): rtol 1e-5, except a block whose largest
    element had its code flipped at an earlier step (<= 0.01% of codes): its M' then
    moves by up to a code step, 1/128 of the scale for UF8.  At most 0.1% of blocks
    may take that room, and none more than two code steps."""
    rel = np.abs(mine.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)
    far = rel > 1e-5
    print(f"  {key}/m_scale: {far.mean():.2e} of blocks beyond rtol 1e-5, max {rel.max():.2e}", flush=True)
    assert far.mean() <= 1e-3 and rel.max() <= 2.0 / 128, f"{name} {key}/m_scale"


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,gkind", CASES, ids=[c[0] for c in CASES])
def test_factored_tinyllama_shapes_match_oracle(name, kw, gkind):
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    print(f"[factored shapes] {name}", flush=True)
    steps = 5
    pc = [torch.nn.Parameter(make_param(s, i, 31)) for i, s in enumerate(SHAPES)]
    pr = [torch.nn.Parameter(p.detach().clone()) for p in pc]   # the reference's reduction order
    p0 = [p.detach().clone() for p in pc]
    pg = [torch.nn.Parameter(p.detach().clone().cuda()) for p in pc]
    oc, orf, og = F.OracleOptimizer(pc, **kw), F.OracleOptimizer(pr, **kw), Adafactor8Bit(pg, **kw)
    for t in range(1, steps + 1):
        for i, (a, b) in enumerate(zip(pc, pg)):
            # the first matrix stands in for the embedding: 90% of its rows are zero (C2)
            kind = "sparse_rows" if (gkind == "student_t" and i == 0) else gkind
            g = make_grad(tuple(a.shape), i, t, 31, kind=kind)
            a.grad, b.grad, pr[i].grad = g, g.cuda(), g.clone()
        old = F.set_exact_reductions(True)
        try:
            oc.step()
        finally:
            F.set_exact_reductions(old)
        orf.step()
        og.step()
        if t not in (1, 2, steps):
            continue
        torch.cuda.synchronize()
        print(f"step {t}: reference-order oracle vs exact-reduction oracle: "
              f"{_code_report(oc, orf, pc, pr):.2e} of codes differ", flush=True)
        report = []
        for i, (a, b) in enumerate(zip(pc, pg)):
            key = f"s{t}/p{i}"
            ref_p, mine_p = a.detach().numpy(), b.detach().cpu().numpy()
            disp = float(np.abs(ref_p - p0[i].numpy()).max())
            close = np.abs(mine_p - ref_p) <= 1e-5 * np.abs(ref_p) + 1e-8 + 1e-4 * disp
            assert (~close).mean() <= 1e-4, f"{name} {key} param: {(~close).mean():.2e} beyond rtol 1e-5"
            np.testing.assert_allclose(mine_p, ref_p, rtol=2e-3, atol=1e-8 + 1e-2 * disp,
                                       err_msg=f"{name} {key} param")
            rdev = float(np.max(np.abs(pr[i].detach().numpy() - ref_p) / (np.abs(ref_p) + 1e-4 * disp + 1e-30)))
            ref_st = _state_np(oc.state[id(a)])
            if "m_scale" in ref_st:
                _cmp_m_scale(name, key, og.state[b]["m_scale"].cpu().numpy(), ref_st.pop("m_scale"))
            z = {f"{key}/{k}": v for k, v in ref_st.items()}
            _cmp_state(name, key, og.state[b], z, list(ref_st), report)
            print(f"  {key}: reference-order params deviate from exact by {rdev:.2e} (relative)", flush=True)
        print(report, flush=True)
