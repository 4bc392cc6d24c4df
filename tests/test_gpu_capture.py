"""Graph-captured optimizer steps (capturable=True) on the GPU.

With ``capturable=True`` a group's step count lives on the device: each step
starts with a8_step_advance (count + 1, this step's scalars) and runs only
multi-tensor kernels that read those scalars, so ``step()`` captured once in a
graph replays as a real next step every time.  For the benchmark configurations
(C1 AdamW UF8/AL8, C2 factored Adafactor with its fp32-state vectors, C3 CAME with
Fira) and more (weight decay with bias correction; bf16 with stochastic
rounding; a clipped, Fira-limited quantised AdamW group and an fp32-state
Adafactor group with scale_parameter, clip and Fira, on tensors of hundreds of
workgroups, whose sums of squares are fixed-order sums; SGD; maximize):

* N graph replays leave parameters and every state tensor bit-identical to N
  eager steps of a second capturable optimizer on the same gradients, with eager
  work and synchronisations between the replays; ``state_dict()`` reports the
  replayed step count;
* eager capturable steps equal the default (host-scalar) path bit for bit.
"""
import numpy as np
import pytest
import torch

from inputs import make_grad, make_param

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False, scale_parameter=False,
             scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-4, block_size=2048, m_block_size=256)
C2 = dict(beta1=None, beta2=None, beta2_decay=-0.8, factored=True, relative_step=False, lr=1e-3, block_size=256)
C3 = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True, relative_step=False,
          scale_parameter=False, scale_weight_decay=False, d=1.0, eps_came=1e-16, lr=1e-4, block_size=2048,
          m_block_size=256, m_quant_type="uf8", v_quant_type="al16", c_quant_type="al16",
          enable_fira_for_adafactor=True, fira_margin=0.01)
SGD = dict(beta1=0.9, beta2=None, beta2_decay=None, factored=False, relative_step=False, scale_parameter=False,
           scale_weight_decay=True, weight_decay=0.01, d=0.0, lr=1e-2, block_size=2048, m_block_size=256,
           m_quant_type="uf8", stochastic_round_writeback=True)
FP32S = dict(beta1=None, beta2=None, beta2_decay=-0.8, factored=False, relative_step=False, scale_parameter=True,
             d=1.0, quantize=False, enable_fira_for_adafactor=True, eps=(1e-30, 1e-3), lr=1e-3)

CASES = [
    ("c1_adamw", ADAMW, [(300, 260), (2048,), (5000,), (64, 64)], torch.float32, "normal_zeros"),
    ("c2_adafactor", C2, [(300, 260), (130, 70), (2048,), (64,)], torch.float32, "student_t"),
    ("c3_came_fira", C3, [(256, 300), (300, 64), (2048,), (64,)], torch.float32, "logscale"),
    ("adamw_wd_bias", dict(ADAMW, weight_decay=0.1, scale_weight_decay=True, lr=1e-3), [(300, 260), (1000,)],
     torch.float32, "student_t"),
    ("adamw_bf16_sr", dict(ADAMW, stochastic_round_writeback=True, lr=1e-3), [(300, 260), (1000,)], torch.bfloat16,
     "normal_zeros"),
    # clipped / Fira / scale_parameter 1-D groups on tensors of hundreds of workgroups: their
    # sums of squares are fixed-order sums, so eager and replayed steps agree bit for bit
    ("adamw_clip_fira_q1d", dict(ADAMW, d=1.0, enable_fira_for_adafactor=True, lr=1e-3),
     [(700, 1100), (300, 260), (5000,)], torch.float32, "logscale"),
    ("adafactor1d_fp32_scale_clip_fira", FP32S, [(700, 1100), (2048,), (5000,)], torch.float32, "student_t"),
    # SGD (beta2 = beta2_decay = None): coded momentum with weight decay, bf16 with SR
    ("sgd_uf8_wd_bf16_sr", SGD, [(300, 260), (5000,), (2048,)], torch.bfloat16, "normal_zeros"),
    # SGD with an RMS clip and Fira (one NORM launch, one Fira launch and one APPLY launch for the
    # group), coded momentum with bf16 SR, and fp32 momentum with a clip only
    ("sgd_uf8_clip_fira_bf16_sr", dict(SGD, d=1.0, enable_fira_for_adafactor=True),
     [(700, 1100), (300, 260), (5000,)], torch.bfloat16, "logscale"),
    ("sgd_fp32m_clip", dict(SGD, d=0.5, m_quant_type="fp32", stochastic_round_writeback=False),
     [(700, 1100), (5000,)], torch.float32, "student_t"),
    # maximize: the kernels read a negated copy of the gradient kept per parameter, which the
    # captured step refills (bf16 SR quantised AdamW, and factored CAME with its vectors)
    ("adamw_bf16_sr_maximize", dict(ADAMW, stochastic_round_writeback=True, lr=1e-3, maximize=True),
     [(300, 260), (1000,), (5000,)], torch.bfloat16, "normal_zeros"),
    ("c3_came_fira_maximize", dict(C3, maximize=True), [(256, 300), (2048,)], torch.float32, "logscale"),
    # scale_parameter on quantised 1-D tensors (>= min_8bit_size): alpha = max(rms(p), eps2) * rho
    # per tensor, from the device block's rho and bias factor, with 1 - alpha * wd; AdamW with
    # bias correction, and Adafactor's defaults (relative step, scale_parameter) with a clip
    ("adamw_q1d_scale_param_wd", dict(ADAMW, scale_parameter=True, weight_decay=0.1, scale_weight_decay=True,
                                      lr=1e-3), [(300, 260), (5000,), (8192,)], torch.float32, "student_t"),
    ("adafactor_q1d_relative_scale_clip", dict(C2, factored=False, relative_step=True, scale_parameter=True,
                                               d=1.0, lr=1e-2), [(6000,), (8192,), (300, 260)], torch.float32,
     "student_t"),
]


def _setup(kw, shapes, dtype, **extra):
    from adafactor8bit import Adafactor8Bit
    ps = [torch.nn.Parameter(make_param(s, i, 17).to("cuda", dtype)) for i, s in enumerate(shapes)]
    for p in ps:
        p.grad = torch.zeros_like(p)   # static gradient buffers: the graph reads these addresses
    return ps, Adafactor8Bit(ps, **dict(kw, **extra))


def _load_grads(ps, t, gkind, dtype):
    for i, p in enumerate(ps):
        p.grad.copy_(make_grad(tuple(p.shape), i, t, 17, kind=gkind).to(dtype))


def _same_state(oa, ob, pa, pb, what):
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a, b), f"{what}: param {i}"
        sa, sb = oa.state[a], ob.state[b]
        assert sorted(sa) == sorted(sb), (what, i)
        for k, v in sa.items():
            if torch.is_tensor(v):
                assert torch.equal(v, sb[k]), f"{what}: param {i} {k}"


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,shapes,dtype,gkind", CASES, ids=[c[0] for c in CASES])
def test_graph_replays_equal_eager_steps(name, kw, shapes, dtype, gkind):
    print(f"[capture] {name}", flush=True)
    pa, oa = _setup(kw, shapes, dtype, capturable=True)   # replayed
    pb, ob = _setup(kw, shapes, dtype, capturable=True)   # eager
    for t in (1, 2):   # eager warm-up: state, tables and device step counts exist before capture
        for ps, o in ((pa, oa), (pb, ob)):
            _load_grads(ps, t, gkind, dtype)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load_grads(pa, 3, gkind, dtype)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _same_state(oa, ob, pa, pb, "after capture (nothing ran)")   # capture launches no kernel
    steps = 5
    for t in range(3, 3 + steps):
        _load_grads(pa, t, gkind, dtype)
        graph.replay()
        _load_grads(pb, t, gkind, dtype)
        ob.step()
        junk = torch.randn(1024, device="cuda").sum()   # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        _same_state(oa, ob, pa, pb, f"step {t}")
    sa = oa.state_dict()
    assert {st["step"] for st in sa["state"].values()} == {2 + steps}
    assert {st["step"] for st in ob.state_dict()["state"].values()} == {2 + steps}


@pytest.mark.gpu
@pytest.mark.parametrize("name,kw,shapes,dtype,gkind", CASES, ids=[c[0] for c in CASES])
def test_capturable_eager_equals_default_path(name, kw, shapes, dtype, gkind):
    print(f"[capturable eager] {name}", flush=True)
    pa, oa = _setup(kw, shapes, dtype, capturable=True)
    pb, ob = _setup(kw, shapes, dtype)
    for t in range(1, 6):
        for ps, o in ((pa, oa), (pb, ob)):
            _load_grads(ps, t, gkind, dtype)
            o.step()
    torch.cuda.synchronize()
    _same_state(oa, ob, pa, pb, "after 5 steps")


@pytest.mark.gpu
@pytest.mark.filterwarnings("ignore:Detected call of")
@pytest.mark.parametrize("name,kw,shapes", [("c1_adamw", ADAMW, [(300, 260), (2048,), (5000,)]),
                                            ("c2_adafactor", C2, [(300, 260), (2048,), (130, 70)])])
def test_tensor_lr_scheduled_between_replays(name, kw, shapes):
    """A one-element fp32 device tensor lr is read by every replay: a scheduler that
    fill_()s it between replays changes the step of the replayed graph exactly as
    it changes an eager capturable step."""
    print(f"[capture tensor lr] {name}", flush=True)
    lra = torch.tensor(1e-3, dtype=torch.float32, device="cuda")
    lrb = torch.tensor(1e-3, dtype=torch.float32, device="cuda")
    pa, oa = _setup(dict(kw, lr=lra), shapes, torch.float32, capturable=True)
    pb, ob = _setup(dict(kw, lr=lrb), shapes, torch.float32, capturable=True)
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob)):
            _load_grads(ps, t, "student_t", torch.float32)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    sched = torch.optim.lr_scheduler.LambdaLR(oa, lambda e: 0.5 ** e)
    schedb = torch.optim.lr_scheduler.LambdaLR(ob, lambda e: 0.5 ** e)
    before = [p.clone() for p in pa]
    for t in range(3, 7):
        _load_grads(pa, t, "student_t", torch.float32)
        graph.replay()
        _load_grads(pb, t, "student_t", torch.float32)
        ob.step()
        torch.cuda.synchronize()
        _same_state(oa, ob, pa, pb, f"step {t}")
        sched.step()
        schedb.step()
    assert abs(float(lra) - 1e-3 * 0.5 ** 4) < 1e-10 and float(lrb) == float(lra)
    assert not all(torch.equal(a, b) for a, b in zip(pa, before))


@pytest.mark.gpu
def test_lag_norm_clips_by_this_steps_norm():
    """lag_norm=True follows the PyTorch branches, which clip by this step's norm (the
    one-pass lagged clip is the CUDA branch's approximation, kept as the module's
    fused_update_*_lag): the same bits as lag_norm=False, in a captured step too."""
    print("[capture] lag_norm", flush=True)
    kw = dict(ADAMW, d=1.0, enable_fira_for_adafactor=True, lr=1e-3)
    shapes = [(700, 1100), (5000,), (2048,)]
    pa, oa = _setup(kw, shapes, torch.float32, lag_norm=True, capturable=True)
    pb, ob = _setup(kw, shapes, torch.float32, lag_norm=False)
    for t in range(1, 4):
        for ps, o in ((pa, oa), (pb, ob)):
            _load_grads(ps, t, "logscale", torch.float32)
            o.step()
    torch.cuda.synchronize()
    _same_state(oa, ob, pa, pb, "lag_norm")


@pytest.mark.gpu
def test_capturable_rejects_paths_with_host_scalars():
    """APOLLO without a projection gap refreshes P on the host schedule only: refused
    before the step touches the state."""
    print("[capturable] APOLLO with apollo_update_proj_gap=0 rejected", flush=True)
    ps, o = _setup(dict(ADAMW, apollo_rank=8, apollo_factorize=True, apollo_update_proj_gap=0, block_size=128,
                        m_block_size=32), [(64, 96)], torch.float32, capturable=True)
    ps[0].grad.copy_(make_grad((64, 96), 0, 1, 17))
    with pytest.raises(NotImplementedError, match="apollo_update_proj_gap"):
        o.step()
    assert o.state[ps[0]]["step"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c1_adamw", "c3_came_fira", "adamw_clip_fira_q1d", "sgd_uf8_clip_fira_bf16_sr"])
def test_checkpoint_of_replayed_steps_resumes(name):
    """state_dict() after graph replays (the step count lives on the device) loads
    into a fresh optimizer, default or capturable, and the next two eager steps
    give the bits of an uninterrupted default run (capturable steps equal default
    ones on these paths)."""
    _, kw, shapes, dtype, gkind = next(c for c in CASES if c[0] == name)
    print(f"[capture checkpoint] {name}", flush=True)
    pa, oa = _setup(kw, shapes, dtype, capturable=True)
    pr, orf = _setup(kw, shapes, dtype)   # uninterrupted default run
    for t in (1, 2):
        for ps, o in ((pa, oa), (pr, orf)):
            _load_grads(ps, t, gkind, dtype)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load_grads(pa, 3, gkind, dtype)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in (3, 4, 5):
        _load_grads(pa, t, gkind, dtype)
        graph.replay()
        _load_grads(pr, t, gkind, dtype)
        orf.step()
    torch.cuda.synchronize()
    sd = oa.state_dict()
    assert {st["step"] for st in sd["state"].values()} == {5}
    resumed = []
    for extra in ({}, {"capturable": True}):
        pb, ob = _setup(kw, shapes, dtype, **extra)
        with torch.no_grad():
            for a, b in zip(pa, pb):
                b.copy_(a)
        ob.load_state_dict(sd)
        resumed.append((pb, ob))
    for t in (6, 7):
        for ps, o in [(pr, orf)] + resumed:
            _load_grads(ps, t, gkind, dtype)
            o.step()
    torch.cuda.synchronize()
    for pb, ob in resumed:
        _same_state(orf, ob, pr, pb, f"{name}: resumed vs uninterrupted, step 7")


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c1_adamw", "c3_came_fira", "adamw_clip_fira_q1d"])
def test_replays_interleaved_with_eager_steps_and_checkpoints(name):
    """Replays of a captured step mixed with eager step() calls of the same optimizer,
    with state_dict() taken in between (it reads the device count back): every step
    advances the one device count, and the run equals six eager steps of a twin."""
    _, kw, shapes, dtype, gkind = next(c for c in CASES if c[0] == name)
    print(f"[capture interleaved] {name}", flush=True)
    pa, oa = _setup(kw, shapes, dtype, capturable=True)
    pb, ob = _setup(kw, shapes, dtype, capturable=True)
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob)):
            _load_grads(ps, t, gkind, dtype)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load_grads(pa, 3, gkind, dtype)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    for t in range(3, 7):
        _load_grads(pa, t, gkind, dtype)
        if t % 2:
            graph.replay()
        else:
            oa.step()
        if t == 4:
            assert {st["step"] for st in oa.state_dict()["state"].values()} == {4}
        _load_grads(pb, t, gkind, dtype)
        ob.step()
        torch.cuda.synchronize()
        _same_state(oa, ob, pa, pb, f"{name}: step {t}")


@pytest.mark.gpu
def test_two_optimizers_in_two_graphs():
    """Two capturable optimizers (AdamW quantised 1-D and CAME factored) captured in
    two graphs and replayed alternately: each equals the eager steps of its twin
    (the library's table staging, codebooks and step blocks are shared by none of
    their captured launches)."""
    print("[capture] two optimizers, two graphs", flush=True)
    c1 = next(c for c in CASES if c[0] == "c1_adamw")
    c3 = next(c for c in CASES if c[0] == "c3_came_fira")
    sets = []
    for _, kw, shapes, dtype, gkind in (c1, c3):
        pa, oa = _setup(kw, shapes, dtype, capturable=True)
        pb, ob = _setup(kw, shapes, dtype, capturable=True)
        sets.append((pa, oa, pb, ob, dtype, gkind))
    for t in (1, 2):
        for pa, oa, pb, ob, dtype, gkind in sets:
            for ps, o in ((pa, oa), (pb, ob)):
                _load_grads(ps, t, gkind, dtype)
                o.step()
    graphs = []
    for pa, oa, _, _, dtype, gkind in sets:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            _load_grads(pa, 3, gkind, dtype)
            with torch.cuda.graph(graph):
                oa.step()
        torch.cuda.current_stream().wait_stream(side)
        graphs.append(graph)
    for t in range(3, 7):
        for (pa, oa, pb, ob, dtype, gkind), graph in zip(sets, graphs):
            _load_grads(pa, t, gkind, dtype)
            graph.replay()
            _load_grads(pb, t, gkind, dtype)
            ob.step()
        torch.cuda.synchronize()
        for pa, oa, pb, ob, _, _ in sets:
            _same_state(oa, ob, pa, pb, f"step {t}")
