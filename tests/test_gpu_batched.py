"""Multi-tensor launches against per-tensor ones.

Quantised 1-D tensors (AL V, coded momentum) with an RMS clip (d > 0) or Fira
step as one group: NORM, MNORM (momentum-only Fira), one Fira launch for all
tensors, APPLY -- each one launch.  The per-tensor sequence (the reference's
_dispatch_1d_cuda per parameter, optimizer.py:1080-1170, with _apply_fira_cuda,
785-793) is what the optimizer runs for a parameter in a group of its own; both
agree.  They are not bit-identical: the NORM pass adds each wave's sum of u^2
into the tensor's norm buffer with a float atomic add (as the reference's
kernels do), so the last bit of the clip norm depends on the order the waves
finish, in either form.  Parameters therefore agree to rtol 1e-6 plus 1e-5 of
the tensor's largest displacement (bf16 parameters, where that last bit can move
a rounding decision: all but at most 1e-4 of them, the rest by one bf16 step),
and codes to the parity bar (at most 1e-4 of codes, by one).  The reference-written fixtures
adamw_clip_fira_wd and adafactor_mom1d_fira pin the arithmetic itself
(tests/test_gpu_golden.py), through this batched path.
"""
import numpy as np
import pytest
import torch

import golden_util as gu
import inputs

SHAPES = [(61, 1003), (5000,), (4096,), (300, 77), (9000,), (128, 2048)]
BASE = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False, relative_step=False,
            scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-3,
            block_size=2048, m_block_size=256)
CASES = {
    "clip": dict(d=1.0),
    "clip_fira_wd": dict(d=1.0, weight_decay=0.1, scale_weight_decay=True, enable_fira_for_adafactor=True),
    "fira_al16_uf4": dict(enable_fira_for_adafactor=True, v_quant_type="al16", m_quant_type="uf4",
                          block_size=256, m_block_size=64),
    "clip_d8_bf16": dict(d=0.5, m_quant_type="d8"),
    "vonly_clip_fira": dict(beta1=None, d=1.0, enable_fira_for_adafactor=True),
    "mom_only_fira": dict(beta2=None, beta2_decay=-0.8, enable_fira_for_adafactor=True, fira_margin=0.01,
                          eps=(1e-30, 1e-3)),
    "mom_only_clip_fira": dict(beta2=None, beta2_decay=-0.8, d=1.0, enable_fira_for_adafactor=True,
                               eps=(1e-30, 1e-3)),
}


@pytest.mark.gpu
@pytest.mark.parametrize("case", sorted(CASES))
def test_q1d_clip_batched_equals_per_tensor(case):
    from adafactor8bit import Adafactor8Bit
    kw = dict(BASE, **CASES[case])
    dtype = torch.bfloat16 if case.endswith("bf16") else torch.float32
    print(f"[q1d batched] {case}", flush=True)
    init = [inputs.make_param(s, i, 41) for i, s in enumerate(SHAPES)]
    runs = []
    for batched in (True, False):
        params = [torch.nn.Parameter(x.clone().to("cuda", dtype)) for x in init]
        opt = Adafactor8Bit(params if batched else [{"params": [p]} for p in params], **kw)
        for t in range(1, 5):
            for i, p in enumerate(params):
                p.grad = inputs.make_grad(SHAPES[i], i, t, 41, kind="logscale").to("cuda", dtype)
            opt.step()
        torch.cuda.synchronize()
        runs.append((params, opt))
    (pa, oa), (pb, ob) = runs
    for i, (a, b) in enumerate(zip(pa, pb)):
        disp = float((a.detach().float().cpu() - init[i].float()).abs().max())
        if dtype == torch.bfloat16:
            xa, xb = a.detach().cpu().view(torch.int16).reshape(-1), b.detach().cpu().view(torch.int16).reshape(-1)
            off = (xa.int() - xb.int()).abs()
            assert int(off.max()) <= 1 and int((off > 0).sum()) <= max(1, int(1e-4 * xa.numel())), \
                f"{case} p{i}: {int((off > 0).sum())} of {xa.numel()} bf16 values differ, by up to {int(off.max())} steps"
        else:
            torch.testing.assert_close(a.detach().float(), b.detach().float(), rtol=1e-6, atol=1e-5 * disp,
                                       msg=lambda m: f"{case} p{i}: {m}")
        sa, sb = oa.state[a], ob.state[b]
        assert "variance_q" in sa, f"{case} p{i}: expected quantised state"
        for k, v in sa.items():
            if not torch.is_tensor(v):
                continue
            x, y = v.reshape(-1).cpu().numpy(), sb[k].reshape(-1).cpu().numpy()
            if k.endswith("_q"):
                frac, mx = gu.code_mismatch(x, y)
                assert frac <= 1e-4 + 1.0 / x.size and mx <= 1, f"{case} p{i} {k}: {frac:.2e} differ, max {mx}"
            else:
                np.testing.assert_allclose(x, y, rtol=1e-5, atol=1e-30, err_msg=f"{case} p{i} {k}")
