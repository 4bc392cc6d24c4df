"""Benchmark: fused AL8/UF8 AdamW optimizer step over a TinyLlama-1.1B-shaped fp32 model.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload NAME]

One "step" is one ``Adafactor8Bit.step()`` (adamw preset: beta=(0.9, 0.999),
eps=(1e-8, 1e-3), d=0, lr=1e-4, UF8 momentum with 256-element blocks, AL8 second
moment with 2048-element blocks) over the 201 tensors of TinyLlama-1.1B
(1,100,048,384 fp32 params; the 45 RMSNorm vectors keep fp32 state).  Params,
grads and states are resident in HBM before timing; grads are synthetic
(1e-3*N(0,1), 5% exact zeros).

The optimizer runs with ``capturable=True``: after the warm-up, K eager ``step()``
calls are timed (``eager_ms_per_step``), then one ``step()`` is captured in a HIP
graph and K replays are timed; each replay is a whole step (device step count and
scalars, both multi-tensor launches), and ``value`` / ``ms_per_step`` are that.

Prints one JSON line: whole-step params/s, the dominant kernel's roofline
(algorithmic bytes per launch / average launch time from HIP events on the
launch stream) and a CPU baseline (the CPU oracle timed on the host cores).

``--workload`` also measures the other BASELINE configurations on the same
shapes (they are parity cases of the headline metric, reported for their own
kernels): ``adafactor`` (C2: factored AL8, B_V 256, no beta1, Student-t grads,
90% zero embedding rows), ``came`` (C3: UF8 M, AL16 V and confidence, B_V
2048, Fira on, per-tensor log-uniform gradient scales) and ``apollo`` (C4:
bf16 params and grads 1e-3*N(0,1), the reference's apollo preset at rank 256,
gap 200, channel scale, Fira, UF8 M / AL8 V low-rank states, SR writeback).
For those the roofline is the whole step's algorithmic bytes over its GPU time
(HIP events around each step); every workload is timed, like the headline,
eagerly and then as graph replays of one captured ``step()`` (``value`` from the
replays); apollo also reports the projection's flops.
``apollo_factorize`` and ``apollo_came`` time C4 with the factorised (row /
column low-rank second moment) and CAME (beta3 0.9999, RMS clip d=1) low-rank
stages; their roofline counts C4's bytes only (a lower bound).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "adafactor-8bit_amd"), os.path.join(ROOT, "tests", "golden")]

import torch  # noqa: E402

HBM_PEAK_GBPS = 8000.0
ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False,
             relative_step=False, scale_parameter=False, scale_weight_decay=False, d=0.0,
             eps=(1e-8, 1e-3), lr=1e-4, block_size=2048, m_block_size=256, m_quant_type="uf8",
             v_quant_type="al8")


ADAFACTOR = dict(beta1=None, beta2=None, beta2_decay=-0.8, beta3=None, factored=True,
                 relative_step=False, lr=1e-3, block_size=256, v_quant_type="al8")
CAME = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True,
            relative_step=False, scale_parameter=False, scale_weight_decay=False, d=1.0,
            eps_came=1e-16, lr=1e-4, block_size=2048, m_block_size=256, m_quant_type="uf8",
            v_quant_type="al16", c_quant_type="al16", enable_fira_for_adafactor=True,
            fira_margin=0.01)


def tinyllama_shapes():
    """TinyLlama-1.1B: 22 layers, hidden 2048, FFN 5632, 4 kv heads (k/v 256x2048), vocab 32000."""
    H, F, KV, V, L = 2048, 5632, 256, 32000, 22
    shapes = [(V, H)]
    for _ in range(L):
        shapes += [(H, H), (KV, H), (KV, H), (H, H), (F, H), (F, H), (H, F), (H,), (H,)]
    shapes += [(H,), (V, H)]
    return shapes


def llama3_8b_shapes():
    """Llama-3-8B: 32 layers, hidden 4096, FFN 14336, 8 kv heads of 128 (k/v 1024x4096),
    vocab 128256, untied embedding and head: 291 tensors, 8,030,261,248 params.  Its
    4096-element RMSNorm vectors reach min_8bit_size, so every tensor is quantised."""
    H, F, KV, V, L = 4096, 14336, 1024, 128256, 32
    shapes = [(V, H)]
    for _ in range(L):
        shapes += [(H, H), (KV, H), (KV, H), (H, H), (F, H), (F, H), (H, F), (H,), (H,)]
    shapes += [(H,), (V, H)]
    return shapes


def step_bytes(shapes, bv=2048, bm=256, min8=4096):
    """Algorithmic HBM bytes of one step: p r+w, g r, codes r+w, block metadata r+w;
    fp32-state tensors: p r+w, g r, v r+w, m r+w."""
    q = f = 0
    for s in shapes:
        n = 1
        for x in s:
            n *= x
        if n < min8:
            f += 28 * n
        else:
            q += 16 * n + 16 * (-(-n // bv)) + 8 * (-(-n // bm))
    return q, f


APOLLO = dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False, relative_step=False,
              scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-6, 1e-3), apollo_eps=1e-6,
              apollo_factorize=False, apollo_update_proj_gap=200, apollo_scale_type="channel", apollo_scale=1.0,
              apollo_scale_front=False, apollo_cache_proj=True, enable_fira_for_apollo=True, apollo_rank=256,
              lr=1e-3, block_size=2048, m_block_size=256, m_quant_type="uf8", v_quant_type="al8",
              stochastic_round_writeback=True)


APOLLO_VARIANTS = {"apollo": APOLLO, "apollo_factorize": dict(APOLLO, apollo_factorize=True),
                   "apollo_came": dict(APOLLO, beta3=0.9999, d=1.0, eps_came=1e-16),
                   "apollo_fp32": APOLLO}   # fp32 parameters (the reference's published APOLLO setting)


def apollo_step_bytes_flops(shapes, rank=256, bs=2048, mbs=256, pbytes=2):
    """Algorithmic bytes and projection flops of one APOLLO step (C4; pbytes 2 for
    bf16, 4 for fp32 parameters).  Per matrix element: g read by the projection
    and by the writeback, p read and written = 4 pbytes.  Per low-rank element
    (R*r or r*C): V code r+w and M code r+w = 4 B, plus their block scales; per
    matrix the fp32 P^T (4 r K B).  The projection is 2 R C r flops (three bf16
    terms of P, six products for fp32 G, on MFMA).  The 1-D vectors (p and g,
    fp32 V and M): 3 pbytes + 16 B."""
    nbytes = flops = 0.0
    for s in shapes:
        if len(s) < 2:
            nbytes += (3.0 * pbytes + 16.0) * s[0]
            continue
        R, C = s
        right = R >= C
        n_low = (R if right else C) * rank
        nbytes += 4.0 * pbytes * R * C + 4.0 * n_low + n_low * (8.0 / bs + 8.0 / mbs) + 4.0 * rank * (C if right else R)
        flops += 2.0 * R * C * rank
    return nbytes, flops


def factored_step_bytes(shapes, workload):
    """Algorithmic bytes of one factored step: per matrix element, adafactor (C2:
    scale_parameter, d = 1) reads g+p for the statistics, g for the norm pass and
    g+p and writes p in the update = 24 B; came with Fira (C3) reads g (statistics),
    g (U norm), g+M (pass 1), g+M (Fira norm), g+M+p and writes M+p (update) = 32 B,
    plus the M scale per 256 elements.  The 1-D vectors keep fp32 state: 28 B."""
    mat = vec = 0
    for s in shapes:
        n = 1
        for x in s:
            n *= x
        if len(s) >= 2:
            mat += n
        else:
            vec += n
    per = 24.0 if workload == "adafactor" else 32.0 + 3 * 4.0 / 256
    return mat * per + vec * 28.0


def make_grad(kind, shape, gen, dev, i, embed):
    if kind.startswith("apollo"):
        return torch.randn(shape, device=dev, generator=gen) * 1e-3
    if kind == "adamw":
        g = torch.randn(shape, device=dev, generator=gen) * 1e-3
        return g * (torch.rand(shape, device=dev, generator=gen) >= 0.05)
    if kind == "adamw_llama3_8b":   # Student-t df=3 scaled 1e-3 with 2% exact zeros
        z = torch.randn(shape, device=dev, generator=gen)
        chi = sum(torch.randn(shape, device=dev, generator=gen) ** 2 for _ in range(3))
        g = 1e-3 * z * torch.sqrt(3.0 / chi)
        return g * (torch.rand(shape, device=dev, generator=gen) >= 0.02)
    if kind == "adafactor":  # Student-t df=3 scaled 1e-3; embedding rows 90% zero
        z = torch.randn(shape, device=dev, generator=gen)
        chi = sum(torch.randn(shape, device=dev, generator=gen) ** 2 for _ in range(3))
        g = 1e-3 * z * torch.sqrt(3.0 / chi)
        if embed:
            keep = (torch.rand(shape[0], device=dev, generator=gen) >= 0.9).float()
            g = g * keep[:, None]
        return g
    # came: N(0, 1e-3) with a per-tensor scale 10^U(-5, -2)
    sc = 10.0 ** (-5.0 + 3.0 * torch.rand((), device=dev, generator=gen))
    return torch.randn(shape, device=dev, generator=gen) * 1e-3 * sc


def cpu_baseline(workload="adamw", seconds_budget=20.0):
    """The CPU oracle (torch CPU restatement of the reference's fallback) on a
    bounded sample of the workload, 2 warm-up + timed steps within the budget:
    adamw (C1): one 4096x4096 fp32 AdamW UF8/AL8 step; adafactor / came (C2, C3):
    one 2048x2048 fp32 matrix of the config; apollo (C4): one 2048x2048 bf16
    matrix at rank 256 (deterministic writeback: the reference's CPU stochastic
    rounding draws from torch's CPU generator, a different stream)."""
    from inputs import make_grad, make_param
    import oracle.fallback as F
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    shape, pdt, gk = (4096, 4096), torch.float32, "normal_zeros"
    kw = dict(ADAMW)
    if workload == "adamw_llama3_8b":
        shape, gk = (4096, 14336), "student_t"
    elif workload == "adafactor":
        shape, gk, kw = (2048, 2048), "student_t", dict(ADAFACTOR)
    elif workload == "came":
        shape, gk, kw = (2048, 2048), "logscale", dict(CAME)
    elif workload.startswith("apollo"):
        shape, pdt = (2048, 2048), (torch.float32 if workload == "apollo_fp32" else torch.bfloat16)
        kw = dict(APOLLO_VARIANTS[workload], stochastic_round_writeback=False)
    p = torch.nn.Parameter(make_param(shape, 0, 0).to(pdt))
    opt = F.OracleOptimizer([p], **kw)
    zf = 0.02 if workload == "adamw_llama3_8b" else 0.05
    grads = [make_grad(shape, 0, t, 0, kind=gk, zero_frac=zf).to(pdt) for t in (1, 2)]
    for w in range(2):   # two warm-up steps (the plan for the baseline)
        p.grad = grads[w]
        opt.step()
    times = []
    t_end = time.perf_counter() + seconds_budget
    i = 0
    while True:
        p.grad = grads[i % 2]
        t0 = time.perf_counter()
        opt.step()
        times.append(time.perf_counter() - t0)
        i += 1
        if time.perf_counter() > t_end or i >= 10:
            break
    times.sort()
    med = times[len(times) // 2]
    n = shape[0] * shape[1]
    what = {"adamw": "C1: one 4096x4096 fp32 AdamW UF8/AL8 step",
            "adamw_llama3_8b": "C5: one 4096x14336 fp32 AdamW UF8/AL8 step (Student-t grads)",
            "adafactor": "C2: one 2048x2048 fp32 factored Adafactor AL8 step",
            "came": "C3: one 2048x2048 fp32 CAME UF8/AL16/AL16+Fira step",
            "apollo": "C4: one 2048x2048 bf16 APOLLO r=256 UF8/AL8 step (deterministic writeback)",
            "apollo_factorize": "one 2048x2048 bf16 factorised APOLLO r=256 step (deterministic writeback)",
            "apollo_came": "one 2048x2048 bf16 CAME APOLLO r=256 step (deterministic writeback)",
            "apollo_fp32": "one 2048x2048 fp32 APOLLO r=256 UF8/AL8 step"}[workload]
    return {"value": n / med, "unit": "params/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{what}, median of {len(times)} after 2 warm-ups", "ms_per_step": med * 1e3}


def copy_ceiling(dev, stream, mib=1024, reps=10):
    """This box's streaming ceiling: a device-to-device copy of `mib` MiB (read +
    write counted), average of `reps` launches timed with HIP events."""
    src = torch.empty(mib << 18, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        dst.copy_(src)
    b.record(stream)
    torch.cuda.synchronize()
    return 2.0 * (mib << 20) * reps / (a.elapsed_time(b) * 1e-3) / 1e9


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib", action="store_true",
                    help="after timing, run a plain 256 MiB fp32 copy (for counter calibration)")
    ap.add_argument("--workload", default="adamw",
                    choices=["adamw", "adafactor", "came", "apollo", "adamw_llama3_8b", "apollo_factorize",
                             "apollo_came", "apollo_fp32"],
                    help="adamw (default, the headline metric), adafactor (C2), came (C3), apollo (C4) or "
                         "adamw_llama3_8b (C5)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (single-GPU boxes; no collectives); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from adafactor8bit import Adafactor8Bit
    from adafactor8bit import _native as nat
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    c5 = args.workload == "adamw_llama3_8b"
    shapes = llama3_8b_shapes() if c5 else tinyllama_shapes()
    params = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    pdt = torch.bfloat16 if (args.workload.startswith("apollo") and args.workload != "apollo_fp32") else torch.float32
    for i, s in enumerate(shapes):
        if len(s) == 1:
            p = torch.ones(s, device=dev)
        else:
            p = torch.randn(s, device=dev, generator=gen) * 0.02
        g = make_grad(args.workload, s, gen, dev, i, embed=(i == 0)).to(pdt)
        p = torch.nn.Parameter(p.to(pdt))
        p.grad = g
        params.append(p)
    nparams = sum(p.numel() for p in params)
    if args.workload not in ("adamw", "adamw_llama3_8b"):
        return bench_factored(args, params, nparams, shapes, Adafactor8Bit)
    opt = Adafactor8Bit(params, **dict(ADAMW, capturable=True))
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()

    # eager: K step() calls
    t0 = time.perf_counter()
    for _ in range(args.steps):
        opt.step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / args.steps * 1e3
    # graph: the same step captured once (capturable=True) and replayed K times; each
    # replay is a full step: device step count, scalars, both multi-tensor launches
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            opt.step()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()   # warm-up replay
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    qbytes, fbytes = step_bytes(shapes)

    # dominant kernel: the multi-tensor quantised launch, timed with HIP events on its stream
    stream = torch.cuda.current_stream(dev)
    big = [p for p in params if p.numel() >= 4096]
    ws = opt._ws[(dev, "tables")]
    ents = [v for k, v in ws.items() if k[0] == "q1d"]
    ent = ents[-1]
    arr, table, nbytes, _ = ent
    L = nat.lib()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        evs[i][0].record(stream)
        rc = L.a8_fused_update_1d_multi(0, 0, nat.F32, arr, len(big), table.data_ptr(), nbytes, 0.9,
                                        1.0 - 0.999, 1e-8 * (1.0 - 0.999 ** 1000) ** 0.5, 1, -126.0, 0.0, 1e-16, 2048, 256, 8, 0, 0.0,
                                        8, 0, 1, 1e-4, 1.0, 0, 0, None, stream.cuda_stream)
        nat.check(rc)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    kms = sorted(a.elapsed_time(b) for a, b in evs)
    k_avg = sum(kms) / len(kms)
    achieved = qbytes / (k_avg * 1e-3) / 1e9

    ceiling = copy_ceiling(dev, stream)
    if args.calib:  # known-size copy for the counters: 256 MiB read + 256 MiB written per launch
        src = torch.empty(64 << 20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()

    traffic = None   # counter-measured bytes exist for the TinyLlama launch only
    tpath = os.path.join(ROOT, "profiles", "traffic_adamw_uf8_al8_tinyllama.json")
    if not c5 and os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    out = {
        "metric": "fused step params/sec + achieved HBM GB/s (% of peak), AL8 AdamW @1.1B params",
        "value": nparams / (ms * 1e-3),
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "adamw_uf8_al8_llama3_8b_fp32" if c5 else "adamw_uf8_al8_tinyllama_1.1b_fp32",
                   "params": nparams,
                   "tensors": len(params), "block_size": 2048, "m_block_size": 256,
                   "step_bytes": qbytes + fbytes},
        "step_GBps": (qbytes + fbytes) / (ms * 1e-3) / 1e9,
        "step_mode": "graph replay of one captured step() (capturable=True)",
        "eager_ms_per_step": eager_ms,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "copy_ceiling_GBps": ceiling, "frac_of_copy": achieved / ceiling,
                     "kernel": f"k_update1d<float,8,0,false> (multi-tensor, {len(big)} tensors)",
                     "kernel_ms_avg": k_avg, "kernel_ms_min": kms[0], "bytes_per_launch": qbytes},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.workload),
    }
    if c5:
        out["metric"] = "fused step params/sec + achieved HBM GB/s (% of peak), AL8 AdamW @8.03B params"
    print(json.dumps(out), flush=True)


def bench_factored(args, params, nparams, shapes, Adafactor8Bit):
    apollo = args.workload.startswith("apollo")
    kw = APOLLO_VARIANTS[args.workload] if apollo else {"adafactor": ADAFACTOR, "came": CAME}[args.workload]
    # every workload runs capturable (device step count and, for APOLLO, the device
    # projection schedule): timed eagerly, then as replays of one captured step
    graphable = True
    opt = Adafactor8Bit(params, **(dict(kw, capturable=True) if graphable else kw))
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def timed(fn):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        t0 = time.perf_counter()
        for i in range(args.steps):
            evs[i][0].record(stream)
            fn()
            evs[i][1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return wall / args.steps * 1e3, sum(a.elapsed_time(b) for a, b in evs) / args.steps

    eager_ms, eager_gms = timed(opt.step)
    ms, gms, mode = eager_ms, eager_gms, "eager step()"
    if graphable:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph):
                opt.step()
        stream.wait_stream(side)
        graph.replay()   # warm-up replay
        torch.cuda.synchronize()
        ms, gms = timed(graph.replay)
        mode = "graph replay of one captured step() (capturable=True)"
    flops = None
    if apollo:
        nbytes, flops = apollo_step_bytes_flops(shapes, pbytes=4 if args.workload == "apollo_fp32" else 2)
    else:
        nbytes = factored_step_bytes(shapes, args.workload)
    achieved = nbytes / (gms * 1e-3) / 1e9
    name = {"adafactor": "adafactor_factored_al8_bv256", "came": "came_uf8_al16_al16_fira_bv2048",
            "apollo": "apollo_r256_uf8_al8_sr", "apollo_factorize": "apollo_factorize_r256_uf8_sr",
            "apollo_came": "apollo_came_r256_uf8_al8_sr", "apollo_fp32": "apollo_r256_uf8_al8"}[args.workload]
    dt = "bf16" if (apollo and args.workload != "apollo_fp32") else "fp32"
    out = {
        "metric": "fused step params/sec + achieved HBM GB/s (% of peak), " + args.workload + " @1.1B params",
        "value": nparams / (ms * 1e-3), "unit": "params/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": name + "_tinyllama_1.1b_" + dt, "params": nparams, "tensors": len(params),
                   "step_bytes": nbytes},
        "step_mode": mode, "eager_ms_per_step": eager_ms, "eager_gpu_ms_per_step": eager_gms,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": None,
                     "kernel": "whole step (all launches of one step, HIP events around each step)",
                     "gpu_ms_per_step": gms, "bytes_per_step": nbytes},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.workload),
    }
    if flops is not None:
        out["projection"] = {"flops_per_step": flops, "TFLOPs_at_step_time": flops / (gms * 1e-3) / 1e12}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
