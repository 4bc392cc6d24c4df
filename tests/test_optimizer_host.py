"""Host-side optimizer logic that needs no GPU: constructor checks of block sizes
against the kernels' routes, and step-counter restore when a launch fails."""
import pytest
import torch


def _opt(shapes, **kw):
    from adafactor8bit import Adafactor8Bit
    ps = [torch.nn.Parameter(torch.zeros(s)) for s in shapes]
    return Adafactor8Bit(ps, **kw), ps


ADAMW = dict(lr=1e-3, beta1=0.9, beta2=0.999, factored=False, relative_step=False, scale_parameter=False)


@pytest.mark.parametrize("kw,shapes,ok", [
    (dict(ADAMW, block_size=2048, m_block_size=256), [(64, 64)], True),
    (dict(ADAMW, block_size=384, m_block_size=128), [(64, 64)], True),      # quantised 1-D V: any size
    (dict(ADAMW, block_size=1152, m_block_size=36), [(64, 64)], True),
    (dict(ADAMW, block_size=6400, m_block_size=100, m_quant_type="uf4"), [(64, 64)], True),
    (dict(ADAMW, block_size=131072, m_block_size=256), [(64, 64)], True),    # one workgroup per V block
    (dict(ADAMW, block_size=(1 << 30) + 128, m_block_size=128), [(64, 64)], False),   # beyond 2^30
    (dict(ADAMW, block_size=384, m_block_size=128, m_quant_type="fp32"), [(64, 64)], True),   # fp32 M: AL EMA
    (dict(ADAMW, apollo_rank=4, block_size=384, m_block_size=128), [(64, 64)], True),         # APOLLO low-rank V
    (dict(ADAMW, apollo_rank=4, block_size=131072, m_block_size=128), [(64, 64)], True),
    (dict(ADAMW, apollo_rank=4, block_size=(1 << 30) + 128, m_block_size=128), [(64, 64)], False),   # beyond 2^30
    (dict(ADAMW, block_size=384, m_block_size=128), [(63, 64)], True),      # below min_8bit_size
    (dict(ADAMW, block_size=384, m_block_size=128, quantize=False), [(64, 64)], True),
    (dict(ADAMW, block_size=384, m_block_size=128, v_quant_type="fp32", m_quant_type="fp32"), [(64, 64)], True),
    (dict(ADAMW, block_size=2048, m_block_size=36), [(64, 64)], False),      # 36 does not divide 2048
    (dict(ADAMW, block_size=4096, m_block_size=256), [(64, 64)], True),
    (dict(lr=1e-3, relative_step=False, block_size=384), [(64, 64)], True),  # factored, no momentum
    (dict(lr=1e-3, relative_step=False, beta1=0.9, block_size=384, m_block_size=128), [(64, 64)], True),
    (dict(lr=1e-3, relative_step=False, beta1=0.9, block_size=1024, m_block_size=100), [(64, 64)], False),
    (dict(lr=1e-3, relative_step=False, block_size=384), [(4096,)], True),   # 1-D vector of a factored group
    (dict(ADAMW, apollo_rank=8, block_size=640, m_block_size=160), [(64, 64)], True),
    (dict(lr=1e-3, relative_step=False, beta1=0.9, block_size=1152, m_block_size=36), [(64, 64)], True),
    (dict(ADAMW, apollo_rank=8, block_size=2048, m_block_size=256), [(64, 64)], True),
    (dict(lr=1e-2, beta1=0.9, beta2=None, beta2_decay=None, relative_step=False, block_size=1152,
          m_block_size=36), [(64, 64)], True),                                # SGD with coded momentum
    (dict(ADAMW, v_quant_type="fp32", block_size=6400, m_block_size=100), [(64, 64)], True),  # fp32 V, coded M
    (dict(ADAMW, v_quant_type="fp32", block_size=131072, m_block_size=131072), [(64, 64)], True),
    (dict(ADAMW, v_quant_type="fp32", block_size=(1 << 30) + 128, m_block_size=(1 << 30) + 128), [(64, 64)], False)
])
def test_block_sizes_checked_at_construction(kw, shapes, ok):
    if ok:
        _opt(shapes, **kw)
    else:
        with pytest.raises(ValueError, match="block_size"):
            _opt(shapes, **kw)


def test_add_param_group_rejects_and_leaves_groups_unchanged():
    opt, _ = _opt([(64, 64)], **dict(ADAMW))
    bad = {"params": [torch.nn.Parameter(torch.zeros(5000))], "block_size": (1 << 30) + 128, "m_block_size": 128}
    with pytest.raises(ValueError):
        opt.add_param_group(bad)
    assert len(opt.param_groups) == 1


def test_step_counter_restored_when_launch_fails(monkeypatch):
    from adafactor8bit import Adafactor8Bit
    opt, ps = _opt([(64, 64), (100,)], **dict(ADAMW))
    states = [opt.state[p] for p in ps]
    for st in states:
        st["step"] = 7

    def boom(self, group, params, grads, sts, dsc=None):
        for st in sts:
            st["step"] += 1
        raise RuntimeError("launch failed")

    monkeypatch.setattr(Adafactor8Bit, "_launch_group", boom)
    with pytest.raises(RuntimeError, match="launch failed"):
        opt._step_group(opt.param_groups[0], ps, [None, None], states)
    assert [st["step"] for st in states] == [7, 7]


def test_roctx_step_ranges_available():
    """step() pushes roctx ranges (adafactor8bit.step, adafactor8bit.group) that
    rocprofv3 --marker-trace records; the marker library is part of ROCm."""
    from adafactor8bit import _native as nat
    r = nat.roctx()
    assert r, "librocprofiler-sdk-roctx not loadable"
    depth = r.roctxRangePushA(b"adafactor8bit.test")
    assert depth >= 0
    assert r.roctxRangePop() >= 0
    with nat.range_marker(b"adafactor8bit.test"):
        pass
