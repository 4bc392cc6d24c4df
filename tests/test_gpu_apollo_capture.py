"""Capturable APOLLO steps (capturable=True) at C4's settings on the GPU.

A capturable group keeps its step count on the device (a8_step_advance).  For
APOLLO matrices the per-step scalars (V lerp weight, lr, bias factor, SR step)
come from that block, and the projection schedule of _get_apollo_proj_matrix
(optimizer.py:2557-2584) runs on the device: the refresh decision, the
reference's seed chain next_seed (optimizer.py:152-155, restated on the device)
and a new P from the device generator.  The first step of a matrix takes P from
the host schedule (stable_randn); later refreshes use the device generator
(oracle/apollo_proj.py restates it).

* the device seed chain equals torch's next_seed bit for bit, and the device
  generator equals the oracle's restatement (all but a few elements bit-exact,
  those within one fp32 ulp: double log / cos of two libraries);
* at C4's settings (rank 256, B_V 2048, B_M 256, UF8 / AL8, channel scale, Fira,
  bf16 parameters with SR, one right-side and one left-side matrix plus an fp32-
  state vector, apollo_update_proj_gap=3; fp32 parameters too), graph replays across two projection
  refreshes equal eager capturable steps bit for bit, P^T after a device refresh
  is the generator's for the new seed, and the schedule's state (apollo_seed,
  current_proj_seed, last_proj_step) equals the default path's;
* before the first device refresh, capturable eager steps equal the default
  path's bit for bit;
* the same two properties for the low-rank stages that run between the phases
  of a8_apollo_step_multi_phase: factorised (with and without momentum, the
  latter with the step-dependent V weight t^-0.8), CAME (AL8, AL16 with UF4
  momentum, fp32), factorised CAME (AL8, fp32), and the plain stage at block
  sizes the fused kernel does not take (B_V 384, B_M 96).
"""
import numpy as np
import pytest
import torch

from inputs import make_grad, make_param
from oracle import apollo_proj as ap

C4_CAP = dict(lr=1e-3, beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False,
              relative_step=False, scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-6, 1e-3),
              apollo_eps=1e-6, apollo_factorize=False, apollo_update_proj_gap=3,
              apollo_scale_type="channel", apollo_scale=1.0, apollo_scale_front=False, apollo_cache_proj=True,
              enable_fira_for_apollo=True, apollo_rank=256, block_size=2048, m_block_size=256,
              m_quant_type="uf8", v_quant_type="al8", stochastic_round_writeback=True)
SHAPES = [(1024, 512), (512, 1536), (2048,)]


def _assert_ulp1(dev, ref, what):
    a = dev.view(np.int32).astype(np.int64)
    b = ref.view(np.int32).astype(np.int64)
    off = np.abs(a - b)
    nd = int((off > 0).sum())
    print(f"[apollo proj gen] {what}: {nd} of {a.size} differ (max {int(off.max())} ulp)", flush=True)
    assert int(off.max()) <= 1 and nd <= max(2, int(1e-5 * a.size)), (what, nd, int(off.max()))


@pytest.mark.gpu
def test_device_next_seed_matches_reference():
    from adafactor8bit import _native as nat
    from adafactor8bit.optimizer import next_seed
    rng = np.random.default_rng(11)
    seeds = [0, 1, 921, 2 ** 32 + 5, 2 ** 63 - 2] + [int(x) for x in rng.integers(0, 2 ** 63 - 1, 250)]
    dev = torch.device("cuda", 0)
    s = torch.tensor(seeds, dtype=torch.int64, device=dev)
    out = torch.empty_like(s)
    nat.check(nat.lib().a8_apollo_next_seed(s.data_ptr(), out.data_ptr(), s.numel(), nat.stream_of(dev)),
              "a8_apollo_next_seed")
    got = out.cpu().tolist()
    for x, y in zip(seeds, got):
        assert y == next_seed(x), x


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,rank", [(1024, 512, 256), (512, 1536, 256), (700, 384, 96), (300, 700, 64)])
def test_device_projection_generator_matches_oracle(rows, cols, rank):
    from adafactor8bit import _native as nat
    dev = torch.device("cuda", 0)
    seed = 0x5DEECE66D + rows
    k = rank * (cols if rows >= cols else rows)
    pt = torch.empty(k, dtype=torch.float32, device=dev)
    nat.check(nat.lib().a8_apollo_proj_gen(pt.data_ptr(), rows, cols, rank, seed, nat.stream_of(dev)),
              "a8_apollo_proj_gen")
    ref = ap.proj_t(rows, cols, rank, seed).reshape(-1)
    _assert_ulp1(pt.cpu().numpy(), ref, f"{rows}x{cols} r{rank}")


def _setup(capturable, dtype=torch.bfloat16, **extra):
    from adafactor8bit import Adafactor8Bit
    ps = [torch.nn.Parameter(make_param(s, i, 29).to("cuda", dtype)) for i, s in enumerate(SHAPES)]
    for p in ps:
        p.grad = torch.zeros_like(p)   # static gradient buffers
    return ps, Adafactor8Bit(ps, **dict(C4_CAP, capturable=capturable, **extra))


def _load(ps, t):
    for i, p in enumerate(ps):
        p.grad.copy_(make_grad(tuple(p.shape), i, t, 29, zero_frac=0.0).to(p.dtype))


def _same(oa, ob, pa, pb, what):
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a, b), f"{what}: param {i}"
        sa, sb = oa.state[a], ob.state[b]
        for k, v in sa.items():
            if torch.is_tensor(v) and k in sb:
                assert torch.equal(v, sb[k]), f"{what}: param {i} {k}"


SCHED = ("apollo_seed", "current_proj_seed", "last_proj_step")


def _schedule(opt, ps):
    sd = opt.state_dict()["state"]
    return [tuple(sd[i].get(k) for k in SCHED) for i in range(2)]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,maximize", [(torch.bfloat16, False), (torch.float32, False),
                                            (torch.float16, False), (torch.bfloat16, True)])
def test_apollo_graph_replays_equal_eager_steps_across_refreshes(dtype, maximize):
    """fp16 parameters project an fp32 copy of G, and maximize a negated one: both are
    refilled by the captured step in a buffer kept per parameter."""
    print(f"[apollo capture] C4 settings, gap 3, {dtype}, maximize={maximize}", flush=True)
    pa, oa = _setup(True, dtype, maximize=maximize)   # replayed
    pb, ob = _setup(True, dtype, maximize=maximize)   # eager
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob)):
            _load(ps, t)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load(pa, 3)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _same(oa, ob, pa, pb, "after capture (nothing ran)")
    for t in range(3, 10):   # device refreshes at steps 4 and 7
        _load(pa, t)
        graph.replay()
        _load(pb, t)
        ob.step()
        junk = torch.randn(4096, device="cuda").sum()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        _same(oa, ob, pa, pb, f"step {t}")
        print(f"[apollo capture] step {t} equal", flush=True)
    assert _schedule(oa, pa) == _schedule(ob, pb)
    sd = oa.state_dict()["state"]
    assert {sd[i]["step"] for i in range(3)} == {9}
    assert all(sd[i]["last_proj_step"] == 7 for i in range(2))


@pytest.mark.gpu
def test_apollo_capturable_schedule_matches_default_path():
    """Eager capturable steps against the default path: the same seed chain at every
    step; bit-identical parameters and states until the first device refresh
    (step 4), whose P is the device generator's for the new seed."""
    pa, oa = _setup(True)
    pb, ob = _setup(False)
    for t in range(1, 8):
        for ps, o in ((pa, oa), (pb, ob)):
            _load(ps, t)
            o.step()
        torch.cuda.synchronize()
        assert _schedule(oa, pa) == _schedule(ob, pb), t
        if t <= 3:
            _same(oa, ob, pa, pb, f"step {t}")
        if t == 4:
            for i, p in enumerate(pa[:2]):
                st = oa.state[p]
                pt = st["apollo_proj_matrix_T"].cpu().numpy().reshape(-1)
                ref = ap.proj_t(p.shape[0], p.shape[1], 256, int(st["current_proj_seed"])).reshape(-1)
                _assert_ulp1(pt, ref, f"step 4 refresh, matrix {i}")
        print(f"[apollo capturable eager] step {t}", flush=True)


# Low-rank stages between the projection and finish phases (a8_apollo_lowrank_x_multi)
X_CAP = {
    "fact_uf8": dict(apollo_factorize=True),
    "fact_nomom": dict(apollo_factorize=True, beta1=None, beta2=None, beta2_decay=-0.8, d=1.0),
    "came_al8_clip": dict(beta3=0.9999, d=1.0, eps_came=1e-16),
    "came_al16_uf4": dict(beta3=0.99, d=1.0, eps_came=1e-16, v_quant_type="al16", c_quant_type="al16",
                          m_quant_type="uf4"),
    "came_fp32": dict(beta3=0.9999, d=1.0, eps_came=1e-16, quantize=False),
    "fact_came_al8": dict(apollo_factorize=True, beta3=0.9999, d=1.0, eps_came=1e-16),
    "fact_came_fp32": dict(apollo_factorize=True, beta3=0.999, d=1.0, eps_came=1e-16, quantize=False),
    "plain_bv384_bm96": dict(block_size=384, m_block_size=96),
}


@pytest.mark.gpu
@pytest.mark.parametrize("variant", sorted(X_CAP))
def test_apollo_variant_graph_replays_equal_eager_steps(variant):
    """The variant's low-rank stage reads the V weight from the device block and
    uploads its tables only when a record changes (never under capture)."""
    print(f"[apollo capture] {variant}", flush=True)
    extra = X_CAP[variant]
    pa, oa = _setup(True, **extra)   # replayed
    pb, ob = _setup(True, **extra)   # eager
    pc, oc = _setup(False, **extra)  # default path
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob), (pc, oc)):
            _load(ps, t)
            o.step()
    torch.cuda.synchronize()
    _same(ob, oc, pb, pc, f"{variant}: capturable eager vs default, step 2")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load(pa, 3)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _same(oa, ob, pa, pb, f"{variant}: after capture (nothing ran)")
    for t in range(3, 9):   # device refreshes at steps 4 and 7
        _load(pa, t)
        graph.replay()
        _load(pb, t)
        ob.step()
        if t == 3:
            _load(pc, t)
            oc.step()
        junk = torch.randn(4096, device="cuda").sum()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        _same(oa, ob, pa, pb, f"{variant}: step {t}")
        if t == 3:
            _same(ob, oc, pb, pc, f"{variant}: capturable eager vs default, step 3")
    assert _schedule(oa, pa) == _schedule(ob, pb)
    print(f"[apollo capture] {variant}: 6 replays equal", flush=True)


@pytest.mark.gpu
def test_apollo_checkpoint_of_replayed_steps_resumes():
    """state_dict() after graph replays across a device projection refresh (steps 3-7,
    refresh at 4 and 7) carries the step, the schedule and the cached P^T: a fresh
    optimizer, capturable or default, that loads it continues (steps 8-9, no refresh)
    with the bits of the uninterrupted capturable run."""
    print("[apollo capture checkpoint]", flush=True)
    pa, oa = _setup(True)   # replayed, then checkpointed
    pr, orf = _setup(True)  # uninterrupted, eager
    for t in (1, 2):
        for ps, o in ((pa, oa), (pr, orf)):
            _load(ps, t)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load(pa, 3)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in range(3, 8):
        _load(pa, t)
        graph.replay()
        _load(pr, t)
        orf.step()
    torch.cuda.synchronize()
    _same(oa, orf, pa, pr, "before the checkpoint")
    sd = oa.state_dict()
    assert {s["step"] for s in sd["state"].values()} == {7}
    resumed = []
    for capturable in (False, True):
        pb, ob = _setup(capturable)
        with torch.no_grad():
            for a, b in zip(pa, pb):
                b.copy_(a)
        ob.load_state_dict(sd)
        resumed.append((pb, ob))
    for t in (8, 9):
        for ps, o in [(pr, orf)] + resumed:
            _load(ps, t)
            o.step()
    torch.cuda.synchronize()
    for pb, ob in resumed:
        _same(orf, ob, pr, pb, "resumed vs uninterrupted, step 9")
    assert _schedule(orf, pr) == _schedule(resumed[0][1], resumed[0][0])


@pytest.mark.gpu
def test_apollo_replays_interleaved_with_eager_steps_and_checkpoints():
    """C4 APOLLO replays mixed with eager steps and a state_dict() between them (it
    copies the device schedule back), across the device refreshes at steps 4 and 7:
    the run equals eager steps of a twin."""
    print("[apollo capture interleaved]", flush=True)
    pa, oa = _setup(True)
    pb, ob = _setup(True)
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob)):
            _load(ps, t)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load(pa, 3)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    for t in range(3, 10):
        _load(pa, t)
        if t % 2:
            graph.replay()
        else:
            oa.step()
        if t in (4, 7):
            sd = oa.state_dict()["state"]
            assert {s["step"] for s in sd.values()} == {t}
        _load(pb, t)
        ob.step()
        torch.cuda.synchronize()
        _same(oa, ob, pa, pb, f"step {t}")
    assert _schedule(oa, pa) == _schedule(ob, pb)
