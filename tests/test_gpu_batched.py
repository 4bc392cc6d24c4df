"""Multi-tensor launches against per-tensor ones, and run-to-run bit identity.

1-D tensors with an RMS clip (d > 0), Fira or scale_parameter step as one group:
NORM, MNORM (momentum-only Fira), one Fira launch for all tensors, APPLY -- each
one launch.  The per-tensor sequence (the reference's _dispatch_1d_cuda per
parameter, optimizer.py:1080-1170, with _apply_fira_cuda, 785-793) is what the
optimizer runs for a parameter in a group of its own.

Every sum of squares (the clip norm, Fira's norm, scale_parameter's sum of p^2)
is a fixed-order sum: each workgroup writes one partial and a second launch adds a
tensor's partials in index order (the reference adds into norm_buf with float
atomics, kernels.cu:297-316, whose order varies).  So the batched and per-tensor
forms give the same bits, and so do two runs of the same steps: both are asserted
with torch.equal on parameters and every state tensor, for quantised V with
coded momentum, fp32 state and SGD, on tensors that span hundreds of workgroups.
The reference-written fixtures adamw_clip_fira_wd and adafactor_mom1d_fira pin
the arithmetic itself (tests/test_gpu_golden.py), through this batched path.
"""
import pytest
import torch

import inputs

SHAPES = [(61, 1003), (5000,), (4096,), (300, 77), (9000,), (128, 2048), (700, 1100)]
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
    "gen_blocks_clip_fira": dict(d=1.0, enable_fira_for_adafactor=True, block_size=384, m_block_size=96),
    # fp32 state (quantize=False): NORM sums u^2 and, with scale_parameter, p^2
    "fp32_clip_scale_fira": dict(quantize=False, beta1=None, beta2=None, beta2_decay=-0.8, d=1.0,
                                 scale_parameter=True, enable_fira_for_adafactor=True, eps=(1e-30, 1e-3)),
    "fp32_mom_only_fira_bf16": dict(quantize=False, beta2=None, beta2_decay=-0.8, d=1.0,
                                    enable_fira_for_adafactor=True, eps=(1e-30, 1e-3)),
    # SGD (beta2 = beta2_decay = None): coded and fp32 momentum
    "sgd_uf8_clip_fira": dict(beta2=None, beta2_decay=None, d=1.0, enable_fira_for_adafactor=True),
    "sgd_fp32m_clip": dict(beta2=None, beta2_decay=None, d=0.5, m_quant_type="fp32"),
}


def _run(case, batched, seed=41, steps=4):
    from adafactor8bit import Adafactor8Bit
    kw = dict(BASE, **CASES[case])
    dtype = torch.bfloat16 if case.endswith("bf16") else torch.float32
    init = [inputs.make_param(s, i, seed) for i, s in enumerate(SHAPES)]
    params = [torch.nn.Parameter(x.clone().to("cuda", dtype)) for x in init]
    opt = Adafactor8Bit(params if batched else [{"params": [p]} for p in params], **kw)
    for t in range(1, steps + 1):
        for i, p in enumerate(params):
            p.grad = inputs.make_grad(SHAPES[i], i, t, seed, kind="logscale").to("cuda", dtype)
        opt.step()
    torch.cuda.synchronize()
    return params, opt


def _assert_same(case, ra, rb, what):
    (pa, oa), (pb, ob) = ra, rb
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a, b), f"{case} {what} p{i}: parameters differ"
        sa, sb = oa.state[a], ob.state[b]
        assert sorted(sa) == sorted(sb), f"{case} {what} p{i}"
        for k, v in sa.items():
            if torch.is_tensor(v):
                assert torch.equal(v, sb[k]), f"{case} {what} p{i} {k}"


@pytest.mark.gpu
@pytest.mark.parametrize("case", sorted(CASES))
def test_clip_batched_equals_per_tensor(case):
    print(f"[batched] {case}", flush=True)
    ra = _run(case, True)
    rb = _run(case, False)
    kw = CASES[case]
    want = None if kw.get("quantize") is False or kw.get("m_quant_type") == "fp32" else (
        "m_q" if case.startswith("sgd") else "variance_q")
    if want:
        assert all(want in ra[1].state[p] for p in ra[0]), f"{case}: expected {want} in every state"
    _assert_same(case, ra, rb, "batched vs per-tensor")


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["clip_fira_wd", "mom_only_clip_fira", "fp32_clip_scale_fira",
                                  "sgd_uf8_clip_fira", "clip_d8_bf16"])
def test_clip_runs_are_bit_identical(case):
    """The same clipped steps twice, batched: the same bits (a float-atomic norm
    would let the clip factor's last bit follow the workgroups' finishing order)."""
    print(f"[run twice] {case}", flush=True)
    _assert_same(case, _run(case, True), _run(case, True), "run 1 vs run 2")
