"""APOLLO (low-rank projected Adafactor) on the GPU, against the reference.

Golden trajectories (apollo_* fixtures, made by the reference's own
``_update_param_apollo`` with the projection generator replaced by
``inputs.make_proj``, which the test installs in the same place).

The projection g_low = G P^T (right side, R >= C) or P^T G (left side) is a
GEMM: the HIP path sums its K products on MFMA (P^T, and fp32 G, split into
bf16 terms whose products are exact in the fp32 accumulator), the reference in
its CPU BLAS's order, so the two results differ at the ulp level.  That is why
the tolerances below are looser than the 1-D path's.  Where an element of g_low
is a cancelling sum, its relative error -- bounded by b / |g_low| with
b = 2 (3K + 2) u sum |g||p| for the two GEMMs -- passes into the states built on
it; those elements (and, at step 1, the V block ranges set by them) are held to
that bound (_GemmCond), everything else to the fixed tolerances:

* V codes (AL8, low rank): every decoded value within two code steps
  (2^(2 s / 254) - 1, relative) of the reference's decoded value, widened by
  the difference of the two block ranges (|dl_min| + |ds| in log2 units), and by
  4 rel for elements of an ill-conditioned g_low.  Codes differ by at most 2,
  and on at most 1% of the elements of blocks whose ranges agree to half a code
  step (a moved range shifts its block's codes together; measured: at most
  8.2e-3 on the bf16 fixtures, 9.8e-4 on the others).  The block's range is
  set by its smallest nonzero g_low^2, which can be a cancelling sum with a large
  relative error: block scale / min_log are held to 2e-2 absolute (log2 units),
  or, for a block beyond that, to the step-1 GEMM error envelope (at step 1) or
  its width (later steps, whose EMA remembers step 1).
* M codes: at most 1% differ, by at most 2 (measured: at most 6.3e-3, by 1).
  Block scales within rtol 1e-5.
* Parameters (fp32): within 1e-5 relative plus 2e-3 of the largest
  displacement the reference's own steps made.  A flipped code moves one
  element of the low-rank update by a code step.  That moves its channel's
  norm ratio, which scales the whole channel's update.
* Parameters (bf16, deterministic writeback): within two bf16 ulps of the
  larger of the two values plus the fp32 bound (for values small next to their
  update), and at most 1% of them not bit-equal.  An fp32 pre-rounding value a
  few ulps off lands on the neighbouring bf16 value when it sits next to a
  rounding midpoint.  Such a flip persists, and a later step can flip the
  same element again: after 4 steps 0.3% of the elements differ, at most by 2
  ulps.
* 16-bit vectors of an APOLLO group take the full-rank route.  Its kernel rounds
  p * decay - step * u once, as the reference's CUDA kernel does
  (kernels.cu:149-161).  The reference's CPU branch, which wrote the fixtures,
  rounds p * decay to 16 bits first (mul_ then add_).  With weight decay the two
  orders land on neighbouring values for a few percent of elements (6% of the
  fp16 vector here), so up to 10% may differ, each within two ulps.
* Norms (scaled_grad_norm_prev): rtol 3e-5; 1e-4 for the CAME, factorised and
  fp16 fixtures.  Their scale ||u|| / ||g_low|| sums every low-rank element.  A
  flipped V code moves one element of u by up to half a code step, which is
  ~1e-5 of ||u|| at n_low = 2560; a few flips over four steps reach 4e-5.  fp32 low-rank states: rtol 2e-6
  plus 1e-6 of the state's largest magnitude.  The projection matrix:
  bit-exact.

Factorised and CAME fixtures (apollo_came_*, apollo_fact_*):

* AL-coded low-rank statistics (V, the CAME residual, the confidence rows and
  columns) are compared on their decoded values: each within two code steps of
  its block plus 1e-3, relative.  The 1e-3 covers a block's smallest entries:
  on the left side they are cancelling GEMM sums, whose relative error (5e-4
  at most in these fixtures) passes to v = g^2 bv and to the residual.  Two
  AL16 code steps (2^(2 s / 65534) - 1, ~2e-4 here) are finer than that.  On the first CAME step every nonzero residual
  of a block is (0.9 U)^2 (1 - beta3) with |U| equal to the clip level, so the
  block's log range is at the rounding noise of U.  The reference may store
  lmin = lmax - 1 where this library stores a range of a few ulps; codes and
  block range then differ completely while the decoded values agree.
* The CAME momentum is an EMA of U = g / sqrt(v), so a V code that flipped
  moves U by half a V code step.  M block scales are then held to half of the
  widest V code step, 2^(s_max / L) - 1 for L = 254 (AL8) or 65534 (AL16).
* fp32 states of these paths (momentum, residual, confidence, row / column
  EMAs, V) are within rtol 1e-3 plus 1e-5 of the state's largest magnitude.
  The 1e-3 is the cancelling-sum bound above: where v < eps^2, U is g * 1/eps
  and the residual carries g's relative error.
  The momentum and residual are EMAs of U and (U - m)^2 whose elements cancel,
  and U carries the clip factor, a norm of the whole matrix reduced in another
  order.  An element therefore moves by ulps of the state's largest terms,
  not of its own value.  Left-side g_low entries that are cancelling GEMM sums
  carry the (K + 2) u sum |g||p| bound, K <= 160, into V.

The GEMM itself is pinned separately: g_low from the library is held to the
deterministic error bound of a K-term fp32 dot product, (K + 2) u sum |g||p|,
against an fp64 product.  For bf16 gradients the bound is three times that:
P^T is split into three bf16 terms, each a GEMM of its own.
"""
import math

import numpy as np
import pytest
import torch

import golden_util as gu
import inputs

APOLLO = ["apollo_uf8_al8", "apollo_tensor_clip_wd", "apollo_fp32_states", "apollo_bf16_det",
          "apollo_came_uf8_al8", "apollo_came_al16_tensor", "apollo_came_fp32", "apollo_came_bf16",
          "apollo_fact_uf8", "apollo_fact_nomom", "apollo_fact_came", "apollo_fact_came_fp32",
          "apollo_fp16_det", "apollo_fp16_tensor"]


@pytest.fixture
def det_proj(monkeypatch):
    import adafactor8bit.optimizer as O
    monkeypatch.setattr(O, "stable_randn", inputs.make_proj)


def _f32(a):
    a = np.asarray(a)
    if a.dtype == np.int16:   # bf16 stored as its bit pattern
        return (a.view(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
    return a


def _t2np(t):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


def _al_decode(q, scale, min_log):
    q = np.asarray(q)
    levels = 65536 if q.dtype == np.int16 else 256
    q = q.astype(np.int64).reshape(scale.size, -1) & (levels - 1)
    v = np.exp2((q - 1) * (scale.astype(np.float64)[:, None] / (levels - 2)) + min_log.astype(np.float64)[:, None])
    return np.where(q == 0, 0.0, v), levels


AL_STATS = ("v_low", "res_low", "conf_row_low", "conf_col_low")


class _GemmCond:
    """Per-element conditioning of g_low over a fixture's steps: for an APOLLO
    matrix with projection P^T and step-s gradient G, x = G P^T (or P^T G) in
    float64, b = 2 (3K + 2) u sum |g||p| (the HIP and the CPU GEMM each within
    (3K + 2) u sum |g||p|), and rel = min(b / |x|, 1), the largest relative error
    either GEMM can leave in an element.  ``cond`` keeps its maximum over the
    steps seen so far; ``v1_envelope`` gives, per AL block of g_low^2 * beta_v at
    step 1, the interval l_min and scale can take."""

    def __init__(self):
        self.cond, self.first = {}, {}

    def add(self, key, g, pt):
        G = _f32(_t2np(g)).astype(np.float64) if g.dtype == torch.bfloat16 else g.double().numpy()
        P = pt.double().cpu().numpy()
        R, C = G.shape
        right = R >= C
        K = C if right else R
        x = G @ P if right else P @ G
        b = 2 * (3 * K + 2) * 2.0 ** -24 * (np.abs(G) @ np.abs(P) if right else np.abs(P) @ np.abs(G))
        rel = np.minimum(b / np.maximum(np.abs(x), 1e-300), 1.0).reshape(-1)
        self.cond[key] = rel if key not in self.cond else np.maximum(self.cond[key], rel)
        if key not in self.first:
            self.first[key] = (np.abs(x).reshape(-1), b.reshape(-1))

    def v1_envelope(self, key, bs, bv):
        x, b = self.first[key]
        lo = (np.maximum(x - b, 0.0) ** 2 * bv).reshape(-1, bs)
        hi = ((x + b) ** 2 * bv).reshape(-1, bs)
        with np.errstate(divide="ignore"):
            lmin = (np.log2(lo.min(axis=1)), np.log2(hi.min(axis=1)))
            lmax = (np.log2(lo.max(axis=1)), np.log2(hi.max(axis=1)))
        return lmin, (lmax[0] - lmin[1], lmax[1] - lmin[0])


def _close(mine, ref, rtol, atol, msg, cond=None):
    """|mine - ref| <= rtol |ref| + atol (+ 4 cond |ref| for elements of an
    ill-conditioned g_low, cond from _GemmCond)."""
    m, r = np.asarray(mine, np.float64).reshape(-1), np.asarray(ref, np.float64).reshape(-1)
    tol = rtol * np.abs(r) + atol
    if cond is not None and cond.size == r.size:
        tol = tol + 4.0 * cond * np.abs(r)
    bad = ~(np.abs(m - r) <= tol)
    if bad.any():
        i = int(np.argmax(np.where(bad, np.abs(m - r) - tol, -np.inf)))
        raise AssertionError(f"{msg}: {int(bad.sum())} of {r.size} beyond tolerance, e.g. {m[i]!r} vs {r[i]!r}")


def _cmp_params(name, key, mine, ref, init, frac=1e-2):
    disp = float(np.abs(_f32(ref).astype(np.float64) - _f32(init)).max())
    if ref.dtype == np.int16:
        m, r = _f32(mine).astype(np.float64), _f32(ref).astype(np.float64)
        big = np.maximum(np.maximum(np.abs(m), np.abs(r)), 1e-38)
        ulp = np.exp2(np.floor(np.log2(big)) - 7)
        # two bf16 ulps, plus the fp32 bound for values small next to their update
        assert np.all(np.abs(m - r) <= 2 * ulp + 2e-3 * disp), f"{name} {key}: bf16 param beyond two ulps"
        assert (mine != ref).mean() <= frac, f"{name} {key}: {(mine != ref).mean():.2e} bf16 params differ"
    elif ref.dtype == np.float16:   # the same bound in fp16 ulps (11 significant bits)
        m, r = mine.astype(np.float64), ref.astype(np.float64)
        big = np.maximum(np.maximum(np.abs(m), np.abs(r)), 2.0 ** -24)
        ulp = np.maximum(np.exp2(np.floor(np.log2(big)) - 10), 2.0 ** -24)
        assert np.all(np.abs(m - r) <= 2 * ulp + 2e-3 * disp), f"{name} {key}: fp16 param beyond two ulps"
        assert (mine != ref).mean() <= frac, f"{name} {key}: {(mine != ref).mean():.2e} fp16 params differ"
    else:
        np.testing.assert_allclose(mine, ref, rtol=1e-5, atol=1e-8 + 2e-3 * disp, err_msg=f"{name} {key} param")


def _cmp_state(name, key, st, z, zkeys, norm_rtol=None, fp32_rtol=None, gc=None, pkey=None, step=None, bv1=None):
    extended = name.startswith(("apollo_came", "apollo_fact"))
    if norm_rtol is None:
        norm_rtol = 1e-4 if (extended or name.startswith("apollo_fp16")) else 3e-5
    fp32_rtol = fp32_rtol or {}
    m_scale_rtol = 1e-5
    if extended and f"{key}/v_low_scale" in z.files and f"{key}/res_low_q" in z.files:
        lv = 65534.0 if z[f"{key}/v_low_q"].dtype == np.int16 else 254.0
        m_scale_rtol = 0.5 * (2.0 ** (float(z[f"{key}/v_low_scale"].max()) / lv) - 1.0) + 1e-5
    for k in zkeys:
        ref = z[f"{key}/{k}"]
        assert k in st and st[k] is not None, f"{name} {key}: missing state {k}"
        mine = st[k]
        mine = mine.detach().cpu().numpy() if torch.is_tensor(mine) else np.asarray(mine)
        assert mine.dtype == ref.dtype and mine.shape == ref.shape, (name, key, k, mine.dtype, ref.dtype)
        msg = f"{name} {key}/{k}"
        if k == "apollo_proj_matrix_T":
            assert np.array_equal(mine, ref), msg
        elif k.endswith("_q") and k[:-2] in AL_STATS:
            pre = k[:-2]
            dm, levels = _al_decode(mine, st[pre + "_scale"].cpu().numpy(), st[pre + "_min_log"].cpu().numpy())
            dr, _ = _al_decode(ref, z[f"{key}/{pre}_scale"], z[f"{key}/{pre}_min_log"])
            # two code steps of the reference's block, widened by the difference of the two
            # block ranges (log2 v = l_min + (q - 1) s / L moves by at most |dl| + |ds|)
            sref = z[f"{key}/{pre}_scale"].astype(np.float64)
            drange = (np.abs(st[pre + "_scale"].cpu().numpy().astype(np.float64) - sref)
                      + np.abs(st[pre + "_min_log"].cpu().numpy().astype(np.float64)
                               - z[f"{key}/{pre}_min_log"].astype(np.float64)))
            step2 = np.exp2(2.0 * sref / (levels - 2) + drange)[:, None] - 1.0
            slack = 1e-3 if extended else 0.0
            if gc is not None and pkey in gc.cond and gc.cond[pkey].size == dr.size:
                slack = slack + 4.0 * gc.cond[pkey].reshape(dr.shape)   # V = EMA of g_low^2
            bad = ~(np.abs(dm - dr) <= (step2 + slack) * np.abs(dr) + 1e-37)
            if bad.any():
                i = np.argwhere(bad)[0]
                c = gc.cond[pkey].reshape(dr.shape)[tuple(i)] if (gc is not None and pkey in gc.cond) else None
                raise AssertionError(f"{msg}: decoded values: {int(bad.sum())} beyond, e.g. at {tuple(i)} "
                                     f"{dm[tuple(i)]!r} vs {dr[tuple(i)]!r} (codes {int(np.asarray(mine).reshape(dr.shape)[tuple(i)])} "
                                     f"vs {int(np.asarray(ref).reshape(dr.shape)[tuple(i)])}, cond {c})")
            if pre == "v_low" and levels == 256:
                # the share of differing codes counts blocks whose ranges agree to half a code
                # step; a block whose range moved shifts its codes together (decoded check above)
                _, mx = gu.code_mismatch(mine, ref)
                keep = drange < 0.5 * sref / 254.0
                qa, qb = np.asarray(mine).reshape(sref.size, -1), np.asarray(ref).reshape(sref.size, -1)
                frac = gu.code_mismatch(qa[keep], qb[keep])[0] if keep.any() else 0.0
                allf = gu.code_mismatch(mine, ref)[0]
                print(f"  {msg}: {allf:.2e} of codes differ ({frac:.2e} in blocks whose range agrees), max {mx}",
                      flush=True)
                assert mx <= 2 and frac <= 1e-2, f"{msg}: {frac:.2e} codes differ, max {mx}"
        elif k.endswith("_q"):
            frac, mx = gu.code_mismatch(mine, ref)
            low_rank = k.startswith(("v_low", "m_low"))
            allowed = 1e-2 if low_rank else 1e-4 + 1.0 / max(mine.size, 1)
            if low_rank:
                print(f"  {msg}: {frac:.2e} of codes differ, max {mx}", flush=True)
            assert mx <= 2 and frac <= allowed, f"{msg}: {frac:.2e} codes differ, max {mx}"
        elif k.startswith("v_low_") and (k.endswith("_scale") or k.endswith("_min_log")):
            off = np.abs(mine.astype(np.float64) - ref) > 2e-2
            if off.any() and gc is not None and pkey in gc.first:
                # a block whose range moved further: at step 1 both ranges lie in the GEMM
                # error envelope; later steps (an EMA that remembers step 1) stay within its width
                bs = ref.size and gc.first[pkey][0].size // ref.size
                env = gc.v1_envelope(pkey, bs, bv1)[0 if k.endswith("_min_log") else 1]
                if step == 1:
                    for v in (mine.astype(np.float64), ref.astype(np.float64)):
                        assert np.all((v[off] >= env[0][off] - 1e-5) & (v[off] <= env[1][off] + 1e-5)), \
                            f"{msg}: outside the GEMM error envelope"
                else:
                    width = (env[1] - env[0])[off]
                    assert np.all(np.abs(mine.astype(np.float64) - ref)[off] <= width + 1e-5), \
                        f"{msg}: beyond the step-1 GEMM envelope's width"
            else:
                np.testing.assert_allclose(mine, ref, rtol=0, atol=2e-2, err_msg=msg)
        elif k.startswith(AL_STATS[1:]) and (k.endswith("_scale") or k.endswith("_min_log")):
            pass   # a block of equal values: see the module doc (decoded values are checked)
        elif k == "m_low_scale":
            np.testing.assert_allclose(mine, ref, rtol=m_scale_rtol, atol=0, err_msg=msg)
        elif k.endswith("_scale") or k.endswith("_min_log"):
            np.testing.assert_allclose(mine, ref, rtol=1e-5, atol=0, err_msg=msg)
        elif "norm" in k:
            np.testing.assert_allclose(mine, ref, rtol=norm_rtol, atol=1e-30, err_msg=msg)
        elif k == "step":
            assert int(mine) == int(ref), msg
        elif extended:
            floor = 1e-5 * float(np.abs(ref).max()) if ref.size else 0.0
            _close(mine, ref, 1e-3, 1e-30 + floor, msg, gc.cond.get(pkey) if gc is not None else None)
        else:
            floor = 1e-6 * float(np.abs(ref).max()) if ref.size else 0.0
            np.testing.assert_allclose(mine, ref, rtol=fp32_rtol.get(k, 2e-6), atol=1e-30 + floor, err_msg=msg)


@pytest.mark.gpu
@pytest.mark.parametrize("name", APOLLO)
@pytest.mark.parametrize("multi", [True, False])
def test_apollo_matches_golden(name, multi, det_proj):
    from adafactor8bit import Adafactor8Bit
    meta, kw, z = gu.load(name)
    print(f"[apollo golden] {name} multi={multi}", flush=True)
    params = gu.init_params(meta, device="cuda")
    opt = Adafactor8Bit(params if multi else [{"params": [p]} for p in params], **kw)
    gc = _GemmCond()
    beta2, bdec = kw.get("beta2"), kw.get("beta2_decay", -0.8)
    bv1 = float(np.float32(1.0 - beta2)) if beta2 is not None else 1.0   # step 1: 1^beta2_decay
    for t in range(1, meta["steps"] + 1):
        grads = gu.grads_for(meta, params, t)
        for p, g in zip(params, grads):
            p.grad = g.cuda()
        opt.step()
        for i, (p, g) in enumerate(zip(params, grads)):
            pt = opt.state[p].get("apollo_proj_matrix_T")
            if p.dim() == 2 and pt is not None:
                gc.add(i, g.float() if g.dtype == torch.float16 else g, pt)
        if t not in meta["save_steps"]:
            continue
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            key = f"s{t}/p{i}"
            # a 16-bit vector under weight decay (full-rank route): see the module doc
            frac = 0.1 if (p.dim() == 1 and kw.get("weight_decay", 0.0)) else 1e-2
            _cmp_params(name, key, _t2np(p), z[f"{key}/param"], z[f"init/p{i}"], frac)
            zkeys = [k[len(key) + 1:] for k in z.files if k.startswith(key + "/") and not k.endswith("/param")]
            _cmp_state(name, key, opt.state[p], z, zkeys, gc=gc, pkey=i, step=t, bv1=bv1)


def _apollo_kw(**over):
    kw = dict(lr=1e-3, beta1=0.9, beta2=0.999, relative_step=False, scale_parameter=False, apollo_rank=32,
              apollo_update_proj_gap=200, apollo_cache_proj=True, block_size=128, m_block_size=32)
    kw.update(over)
    return kw


def _ws(opt, p):
    ent = opt._ws[(p.device, "apollo", id(p))]
    return ent["ws"].cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(300, 200), (96, 260), (513, 7), (5, 1030)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_apollo_projection_error_bound(shape, dtype, det_proj):
    """g_low from the library against an fp64 product of the same G and P^T."""
    from adafactor8bit import Adafactor8Bit
    print(f"[apollo gemm] {shape} {dtype}", flush=True)
    R, C = shape
    r = 32 if min(R, C) > 32 else 4
    p = torch.nn.Parameter(inputs.make_param(shape, 0, 11).to("cuda", dtype))
    g = inputs.make_grad(shape, 0, 1, 11, kind="student_t").to(dtype)
    opt = Adafactor8Bit([p], **_apollo_kw(apollo_rank=r))
    p.grad = g.cuda()
    opt.step()
    torch.cuda.synchronize()
    pt = opt.state[p]["apollo_proj_matrix_T"].double().cpu().numpy()
    G = g.double().numpy()
    right = R >= C
    exact = G @ pt if right else pt @ G
    absb = np.abs(G) @ np.abs(pt) if right else np.abs(pt) @ np.abs(G)
    K = C if right else R
    n_low = exact.size
    glow = _ws(opt, p)[:n_low].reshape(exact.shape).astype(np.float64)
    terms = 1 if dtype == torch.float32 else 3
    bound = terms * (K + 2) * 2.0 ** -24 * absb
    assert np.all(np.abs(glow - exact) <= bound + 1e-30), float(np.max(np.abs(glow - exact) / (absb + 1e-30)))


@pytest.mark.gpu
@pytest.mark.parametrize("shape,rank", [((128, 96), 16), ((64, 160), 16), ((600, 300), 256), ((300, 520), 256)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_apollo_nonfinite_grad_equals_scrubbed(shape, rank, dtype, det_proj):
    """NaN / +-Inf gradient entries count as zero (optimizer.py:2606): fp32 through
    the flag and recompute pass, bf16 scrubbed inside the projection kernel."""
    from adafactor8bit import Adafactor8Bit
    print(f"[apollo nonfinite] {shape} r={rank} {dtype}", flush=True)
    res = []
    for bad in (True, False):
        p = torch.nn.Parameter(inputs.make_param(shape, 0, 5).to("cuda", dtype))
        opt = Adafactor8Bit([p], **_apollo_kw(apollo_rank=rank))
        for t in range(1, 4):
            g = inputs.make_grad(shape, 0, t, 5).to(dtype)
            flat = g.view(-1)
            idx = torch.arange(t, flat.numel(), 97)
            if bad:
                flat[idx[0::3]] = float("nan")
                flat[idx[1::3]] = float("inf")
                flat[idx[2::3]] = float("-inf")
            else:
                flat[idx] = 0.0
            p.grad = g.cuda()
            opt.step()
        torch.cuda.synchronize()
        res.append((p.detach().float().cpu().numpy(), opt.state[p]["scaled_grad_norm_prev"].item()))
    (pb, nb), (pg, ng) = res
    assert np.all(np.isfinite(pb)) and math.isfinite(nb)
    if dtype == torch.bfloat16:   # the same kernels on equal scrubbed inputs: identical
        assert np.array_equal(pb, pg) and nb == ng
    else:   # g_low from the recompute pass vs the library GEMM: summation order differs
        init = inputs.make_param(shape, 0, 5).numpy()
        disp = float(np.abs(pg - init).max())
        np.testing.assert_allclose(pb, pg, rtol=1e-5, atol=1e-8 + 2e-3 * disp)
        np.testing.assert_allclose(nb, ng, rtol=3e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,channel", [((256, 64), True), ((48, 300), True), ((200, 100), False)])
def test_apollo_sr_writeback_bits(shape, channel, dtype, det_proj):
    """SR writeback (optimizer.py:3058-3063): x = (p * decay) + (G * f) * step in
    fp32, rounded with the stream of kernels.cu:48-87 (bf16) or 100-131 (fp16),
    bit for bit against the CPU restatement given the step's scalars from the
    library's workspace."""
    from adafactor8bit import Adafactor8Bit
    from oracle import sr
    print(f"[apollo sr] {shape} channel={channel} {dtype}", flush=True)
    R, C = shape
    p = torch.nn.Parameter(inputs.make_param(shape, 0, 9).to("cuda", dtype))
    opt = Adafactor8Bit([p], **_apollo_kw(apollo_rank=16, weight_decay=0.1, stochastic_round_writeback=True,
                                          apollo_scale_type="channel" if channel else "tensor"))
    for t in range(1, 3):
        p_old = _f32(_t2np(p)).reshape(-1).astype(np.float32)
        g = inputs.make_grad(shape, 0, t, 9).to(dtype)
        p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        st = opt.state[p]
        ws = _ws(opt, p)
        # workspace: g_low [n_low], u [n_low], ||G_ch||^2 [nch], s_ch [nch], scalars
        n_low = (R * 16) if R >= C else (16 * C)
        nch = R if R >= C else C
        fin = 2 * n_low + nch
        scal = fin + nch
        step_s, dec, fs = np.float32(ws[scal]), np.float32(ws[scal + 1]), np.float32(ws[scal + 6])
        gf = _f32(_t2np(g)).reshape(R, C).astype(np.float32)
        if channel:   # f = (s * fira) * sqrt(apollo_scale) (apollo_scale 1 here)
            f = ws[fin:fin + nch].astype(np.float32) * fs
            fm = np.broadcast_to(f[:, None] if R >= C else f[None, :], (R, C))
        else:
            fm = np.full((R, C), np.float32(ws[scal + 3]), dtype=np.float32)
        x = (p_old * dec) + ((gf * fm) * step_s).reshape(-1)
        rnd = sr.sr_round_bf16 if dtype == torch.bfloat16 else sr.sr_round_fp16
        want = rnd(x.astype(np.float32), seed=int(st["sr_seed"]), step=int(st["step"]))
        got = _t2np(p).reshape(-1).view(np.uint16)
        assert np.array_equal(got, want), f"step {t}: {(got != want).mean():.2e} differ"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_1d_sr_writeback_stream(dtype):
    """1-D fused steps with SR writeback (quantised and fp32 state): the 16-bit
    result is the stochastic rounding of the fp32 result under the reference's
    stream (bf16: kernels.cu:67-87, fp16: 100-131).  The fp32 run writes
    fma(-step, u, p) and the SR path rounds (p - step * u), one fp32 rounding
    apart, which moves the round-up probability by 2^-16 (bf16) or 2^-13 (fp16):
    at most 0.1% of the elements may land on the other neighbour."""
    from adafactor8bit import Adafactor8Bit
    from oracle import sr
    meta, kw, _ = gu.load("adamw_uf8_al8")
    # quantised-state tensors and, below min_8bit_size (4096), fp32-state ones
    shapes = [(700, 300), (4097,), (64, 64), (2048,), (1000,), (3,)]
    print(f"[1d sr] {dtype}", flush=True)
    p16 = [torch.nn.Parameter(inputs.make_param(s, i, 3).to("cuda", dtype)) for i, s in enumerate(shapes)]
    p32 = [torch.nn.Parameter(p.detach().float()) for p in p16]
    o16 = Adafactor8Bit(p16, **dict(kw, stochastic_round_writeback=True))
    o32 = Adafactor8Bit(p32, **kw)
    for i, s in enumerate(shapes):
        g = inputs.make_grad(s, i, 1, 3).to(dtype).cuda()
        p16[i].grad = g
        p32[i].grad = g.float()
    o16.step()
    o32.step()
    torch.cuda.synchronize()
    rnd = sr.sr_round_bf16 if dtype == torch.bfloat16 else sr.sr_round_fp16
    for p, q in zip(p16, p32):
        x = q.detach().cpu().numpy().reshape(-1)
        want = rnd(x, seed=int(o16.state[p]["sr_seed"]), step=int(o16.state[p]["step"]))
        got = _t2np(p).reshape(-1).view(np.uint16)
        diff = got != want
        assert diff.sum() <= max(1, 1e-3 * diff.size), diff.mean()
        # where they differ, both are neighbours of x
        if dtype == torch.bfloat16:
            lo = (x.view(np.uint32) & np.uint32(0xFFFF0000)) >> np.uint32(16)
            assert np.all(np.isin(got[diff].astype(np.int64) - lo[diff].astype(np.int64), [0, 1]))
        else:
            xd = x[diff]
            q16 = xd.astype(np.float16)
            other = np.nextafter(q16, np.where(q16.astype(np.float32) < xd, np.float16(np.inf),
                                               np.float16(-np.inf)).astype(np.float16))
            gv = got[diff].view(np.float16)
            assert np.all((gv == q16) | (gv == other))


@pytest.mark.gpu
@pytest.mark.parametrize("shape,rank", [((200, 12), 4), ((40, 260), 8)])
def test_apollo_fp32_width_4_mod_8_matches_oracle(shape, rank, det_proj, monkeypatch):
    """fp32 matrices whose width is 4 mod 8: an 8-element writeback unit spans two
    rows, so each element takes its own row's (right side) or column's (left
    side) channel scale.  Three steps against the CPU oracle, parameters to the
    fp32 bound of the golden comparison."""
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    monkeypatch.setattr(F, "stable_randn", inputs.make_proj)
    print(f"[apollo width] {shape} r={rank}", flush=True)
    kw = _apollo_kw(apollo_rank=rank, weight_decay=0.05)
    init = inputs.make_param(shape, 0, 4)
    p = torch.nn.Parameter(init.clone().cuda())
    q = torch.nn.Parameter(init.clone())
    opt = Adafactor8Bit([p], **kw)
    ref = F.OracleOptimizer([q], **kw)
    for t in range(1, 4):
        g = inputs.make_grad(shape, 0, t, 4)
        p.grad, q.grad = g.cuda(), g.clone()
        opt.step()
        ref.step()
    torch.cuda.synchronize()
    _cmp_params("width", "s3", p.detach().cpu().numpy(), q.detach().numpy(), init.numpy())


# C4's configuration: the reference's apollo preset (presets.py:106-125) at rank
# 256 with 2048-element V blocks and 256-element M blocks.  At rank >= 64 the
# projection tiles run their second accumulator pair, and AL8 V blocks of 2048
# elements take the low-rank stage's LDS decode table.
C4_KW = dict(lr=1e-3, beta1=0.9, beta2=0.999, beta2_decay=None, beta3=None, factored=False,
             relative_step=False, scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-6, 1e-3),
             apollo_eps=1e-6, apollo_factorize=False, apollo_update_proj_gap=200,
             apollo_scale_type="channel", apollo_scale=1.0, apollo_scale_front=False, apollo_cache_proj=True,
             enable_fira_for_apollo=True, apollo_rank=256, block_size=2048, m_block_size=256,
             m_quant_type="uf8", v_quant_type="al8")

# (shape, rank): right side (R >= C, K = C) and left side (K = R).  Rank 320 takes
# two 256-wide output passes.  bf16 G at ranks 256 and 512 takes the wide tiles
# (256 channels x 256 outputs): whole tiles (1024 x 512, 512 x 1536), a partial
# last tile with K % 32 != 0 and rows that are not 16-byte aligned (700 x 390,
# 390 x 1100: C % 8 == 6 and 4), and two passes (1100 x 600, 600 x 1300).
GEMM_RANKS = [((1024, 512), 64), ((700, 384), 96), ((1024, 512), 256), ((700, 384), 320),
              ((512, 1536), 256), ((384, 900), 320), ((300, 700), 64), ((200, 900), 96),
              ((700, 390), 256), ((390, 1100), 256), ((1100, 600), 512), ((600, 1300), 512)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape,rank", GEMM_RANKS, ids=[f"{s[0]}x{s[1]}_r{r}" for s, r in GEMM_RANKS])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_apollo_projection_error_bound_large_rank(shape, rank, dtype, det_proj):
    """g_low at ranks 64-320 on both sides against an fp64 product of the same G
    and P^T, to the K-term fp32 dot-product bound (three times it for bf16 G,
    whose P^T is split into three bf16 terms)."""
    from adafactor8bit import Adafactor8Bit
    print(f"[apollo gemm large rank] {shape} r={rank} {dtype}", flush=True)
    R, C = shape
    p = torch.nn.Parameter(inputs.make_param(shape, 0, 12).to("cuda", dtype))
    g = inputs.make_grad(shape, 0, 1, 12, kind="student_t").to(dtype)
    opt = Adafactor8Bit([p], **dict(C4_KW, apollo_rank=rank))
    p.grad = g.cuda()
    opt.step()
    torch.cuda.synchronize()
    pt = opt.state[p]["apollo_proj_matrix_T"].double().cpu().numpy()
    G = g.double().numpy()
    right = R >= C
    exact = G @ pt if right else pt @ G
    assert exact.shape == ((R, rank) if right else (rank, C))
    absb = np.abs(G) @ np.abs(pt) if right else np.abs(pt) @ np.abs(G)
    K = C if right else R
    glow = _ws(opt, p)[:exact.size].reshape(exact.shape).astype(np.float64)
    terms = 1 if dtype == torch.float32 else 3
    bound = terms * (K + 2) * 2.0 ** -24 * absb
    err = np.abs(glow - exact)
    assert np.all(err <= bound + 1e-30), float(np.max(err / (absb + 1e-30)))


def _oracle_state_view(st):
    """The oracle's per-parameter state as a flat mapping of numpy arrays (and the
    step), for the golden comparison helpers."""
    out = {}
    for k, v in st.items():
        if torch.is_tensor(v):
            out[k] = (v.view(torch.int16) if v.dtype == torch.bfloat16 else v).numpy()
        elif k == "step":
            out[k] = np.asarray(v)
    return out


C4_SHAPES = [(1024, 512), (512, 1536)]


def _c4_codes(name, mine, ref, step):
    frac, mx = gu.code_mismatch(mine.reshape(-1), ref.reshape(-1))
    print(f"  {name}: {frac:.2e} of codes differ, max {mx}", flush=True)
    if step == 1:
        assert frac <= 1e-5 and mx <= 1, (name, frac, mx)
    assert frac <= 1e-4 and mx <= 1, (name, frac, mx)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", C4_SHAPES, ids=["right_1024x512", "left_512x1536"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_apollo_c4_rank256_matches_oracle(shape, dtype, det_proj, monkeypatch):
    """Four APOLLO steps at C4's configuration (rank 256, B_V 2048, B_M 256,
    UF8 M / AL8 V, channel scale, Fira), deterministic writeback, against the CPU
    oracle given this library's projection output.

    The projection itself is held to its error bound above.  Here g_low is read
    from the library's workspace after each step and handed to the oracle
    (OracleOptimizer.glow_hook): at K = 512 a block's smallest g_low can be a
    cancelling sum whose last bits depend on the GEMM's summation order, and the
    AL8 block range follows that smallest value.  With the same g_low, and the
    oracle's reductions (channel norms, ||G_ch||, the Fira norm) accumulated
    exactly, the rest of the step is held to the north star's bar: low-rank V
    and M codes equal except <= 0.01% (by one code; step 1: <= 1e-5, where the
    CPU log2 is not correctly rounded), block metadata rtol 1e-5, the Fira norm
    rtol 1e-5, fp32 parameters rtol 1e-5 plus 2e-4 of the largest displacement
    (a flipped V code moves one element of a 256-element channel norm), bf16
    parameters within two ulps (of the largest magnitude the element has had) plus
    1e-5 of the largest displacement, <= 0.1% of them not bit-equal."""
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    monkeypatch.setattr(F, "stable_randn", inputs.make_proj)
    old = F.set_exact_reductions(True)
    try:
        print(f"[apollo c4] {shape} {dtype}", flush=True)
        R, C = shape
        low = (R, 256) if R >= C else (256, C)
        init = inputs.make_param(shape, 0, 21).to(dtype)
        p = torch.nn.Parameter(init.clone().cuda())
        q = torch.nn.Parameter(init.clone())
        opt = Adafactor8Bit([p], **C4_KW)
        ref = F.OracleOptimizer([q], **C4_KW)
        mag = np.abs(_f32(_t2np(init)).astype(np.float64))
        for t in range(1, 5):
            g = inputs.make_grad(shape, 0, t, 21, zero_frac=0.0).to(dtype)
            p.grad, q.grad = g.cuda(), g.clone()
            opt.step()
            torch.cuda.synchronize()
            glow = torch.from_numpy(_ws(opt, p)[:low[0] * low[1]].reshape(low).copy())
            ref.glow_hook = lambda _p, _g, _pt, x=glow: x
            ref.step()
            st, sr = opt.state[p], ref.state[id(q)]
            print(f"[apollo c4] step {t}", flush=True)
            _c4_codes("v_low_q", st["v_low_q"].cpu().numpy(), sr["v_low_q"].numpy(), t)
            _c4_codes("m_low_q", st["m_low_q"].cpu().numpy(), sr["m_low_q"].numpy(), t)
            for k in ("v_low_scale", "v_low_min_log", "m_low_scale"):
                np.testing.assert_allclose(st[k].cpu().numpy(), sr[k].numpy(), rtol=3e-7 if t == 1 else 1e-5,
                                           err_msg=f"step {t} {k}")
            np.testing.assert_allclose(float(st["scaled_grad_norm_prev"]), float(sr["scaled_grad_norm_prev"]),
                                       rtol=1e-5, err_msg=f"step {t} scaled_grad_norm_prev")
            assert np.array_equal(st["apollo_proj_matrix_T"].cpu().numpy(), sr["apollo_proj_matrix_T"].numpy())
            mine, want = _t2np(p), _t2np(q)
            disp = float(np.abs(_f32(want).astype(np.float64) - _f32(_t2np(init))).max())
            if dtype == torch.bfloat16:
                m64, r64 = _f32(mine).astype(np.float64), _f32(want).astype(np.float64)
                # largest magnitude each element has had: a one-ulp flip made there keeps its size
                # in absolute terms when the value later shrinks into a finer binade
                mag = np.maximum(mag, np.maximum(np.abs(m64), np.abs(r64)))
                ulp = np.exp2(np.floor(np.log2(np.maximum(mag, 1e-38))) - 7)
                diff = mine != want
                print(f"  bf16 params not bit-equal: {diff.mean():.2e}", flush=True)
                # an element whose fp32 value sat on a bf16 midpoint keeps the one-ulp flip, and a
                # later step may flip it once more; next to zero the fp32 bound of the update applies
                err = np.abs(m64 - r64) - (2 * ulp + 1e-5 * disp)
                k = int(np.argmax(err))
                assert err.flat[k] <= 0, (f"step {t}: bf16 param beyond two ulps: {m64.flat[k]:.6e} vs "
                                          f"{r64.flat[k]:.6e} (displacement {disp:.3e})")
                assert diff.mean() <= 1e-3, f"step {t}: {diff.mean():.2e} bf16 params differ"
            else:
                np.testing.assert_allclose(mine, want, rtol=1e-5, atol=1e-8 + 2e-4 * disp, err_msg=f"step {t} param")
        assert st["v_low_q"].numel() == low[0] * low[1] and st["v_low_scale"].numel() == low[0] * low[1] // 2048
    finally:
        F.set_exact_reductions(old)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", C4_SHAPES, ids=["right_1024x512", "left_512x1536"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_apollo_c4_rank256_end_to_end_against_oracle(shape, dtype, monkeypatch):
    """C4's configuration end to end against the CPU oracle in its default mode:
    nothing injected (the oracle runs its own fp32 CPU GEMM on the same P and sums
    in the reference's order), 4 steps, deterministic writeback.  Both sides use
    the same host-independent stand-in for stable_randn, as the reference
    fixtures do.

    An AL8 block's range is set by its smallest nonzero g_low^2, which at K = 512
    can be a cancelling sum: two correct fp32 GEMMs may give it several percent
    apart (the rank-16 fixtures, with K = 48..96, move it far less).  So at step 1
    (v = g_low^2 * beta_v) every block's l_min and scale are held to the envelope
    the GEMM error bound allows -- from g_low in float64 and each element's bound
    b = (3K + 2) 2^-24 sum|g||p| for either side.  A block whose range moved by
    (dl, ds) moves its codes by up to 254 (|dl| + |ds|) / s, so at step 1 each
    block's code difference is held to 2 + ceil(254 (|dl| + |ds|) / s) (rounding,
    and one more for the near-minimum elements whose own value is ill-conditioned).
    Later steps decode the previous step's differing codes, so there the decoded V
    of each side stays within its accumulated half code steps of exact arithmetic:
    |log2 V_hip - log2 V_oracle| <= sum over steps of (s_hip + s_oracle) / 508 on all
    but 1e-3 of elements (those near a block minimum at step 1).  The share of
    differing low-rank V codes (measured 0.7-2.7%, by up to 6) has only a sanity
    cap of 5%; M codes keep the golden bound (at most 2%, by at most 2).  The
    measured figures are printed."""
    import oracle.fallback as F
    from adafactor8bit import Adafactor8Bit
    import adafactor8bit.optimizer as O
    monkeypatch.setattr(O, "stable_randn", inputs.make_proj)
    monkeypatch.setattr(F, "stable_randn", inputs.make_proj)
    R, C = shape
    rank, bs = 256, 2048
    init = inputs.make_param(shape, 0, 23).to(dtype)
    p = torch.nn.Parameter(init.clone().cuda())
    q = torch.nn.Parameter(init.clone())
    opt = Adafactor8Bit([p], **C4_KW)
    ref = F.OracleOptimizer([q], **C4_KW)
    worst = {}
    budget = 0.0   # accumulated half code steps, log2 units, per block
    for t in range(1, 5):
        g = inputs.make_grad(shape, 0, t, 23, zero_frac=0.0).to(dtype)
        p.grad, q.grad = g.cuda(), g.clone()
        opt.step()
        ref.step()
        torch.cuda.synchronize()
        st, sr = opt.state[p], ref.state[id(q)]
        line = [f"[apollo c4 e2e] {shape} {str(dtype)[6:]} step {t}:"]
        lm, lr_ = st["v_low_min_log"].cpu().numpy().astype(np.float64), sr["v_low_min_log"].numpy().astype(np.float64)
        sm, sr_s = st["v_low_scale"].cpu().numpy().astype(np.float64), sr["v_low_scale"].numpy().astype(np.float64)
        for k in ("v_low_q", "m_low_q"):
            a, b_ = st[k].cpu().numpy().reshape(-1), sr[k].numpy().reshape(-1)
            frac, mx = gu.code_mismatch(a, b_)
            worst[k] = max(worst.get(k, 0.0), frac)
            line.append(f"{k} {frac:.2e} differ (max {mx})")
            if k == "m_low_q":
                assert mx <= 2 and frac <= 2e-2, f"step {t} {k}: {frac:.2e} codes differ, max {mx}"
            else:
                # the bounds are the range envelope and the decoded budget; the share of
                # differing codes (measured 0.7-2.7%) only has a sanity cap
                assert frac <= 5e-2, f"step {t} {k}: {frac:.2e} codes differ"
                budget = budget + (sm + sr_s) / 508.0
                if t == 1:
                    d = np.abs(a.astype(np.int64) - b_.astype(np.int64)).reshape(-1, bs).max(axis=1)
                    allowed = 2 + np.ceil(254.0 * (np.abs(lm - lr_) + np.abs(sm - sr_s)) / np.minimum(sm, sr_s))
                    assert np.all(d <= allowed), f"step {t} {k}: a block's codes moved beyond its range change"
                else:
                    dm, _ = _al_decode(a, sm, lm)
                    dr, _ = _al_decode(b_, sr_s, lr_)
                    both = (dm > 0) & (dr > 0)
                    with np.errstate(divide="ignore"):
                        gap = np.abs(np.log2(np.where(both, dm, 1.0)) - np.log2(np.where(both, dr, 1.0)))
                    over = (gap > budget[:, None] + 1e-4) | ((dm > 0) != (dr > 0))
                    line.append(f"decoded V beyond budget {over.mean():.2e}")
                    assert over.mean() <= 1e-3, f"step {t} {k}: {over.mean():.2e} of decoded V beyond budget"
        dr = float(max(np.abs(lm - lr_).max(), np.abs(sm - sr_s).max()))
        worst["range"] = max(worst.get("range", 0.0), dr)
        line.append(f"block range max diff {dr:.3e} (log2)")
        if t == 1:
            gd = _f32(_t2np(g)).astype(np.float64).reshape(R, C)
            pt = st["apollo_proj_matrix_T"].cpu().numpy().astype(np.float64)
            right = R >= C
            K = C if right else R
            x = gd @ pt if right else pt @ gd
            ab = np.abs(gd) @ np.abs(pt) if right else np.abs(pt) @ np.abs(gd)
            b = (3 * K + 2) * 2.0 ** -24 * ab
            bv = np.float64(np.float32(1.0 - 0.999))
            lo = (np.maximum(np.abs(x) - b, 0.0) ** 2 * bv).reshape(-1, bs)
            hi = ((np.abs(x) + b) ** 2 * bv).reshape(-1, bs)
            with np.errstate(divide="ignore"):
                lmin_lo, lmin_hi = np.log2(lo.min(axis=1)), np.log2(hi.min(axis=1))
                lmax_lo, lmax_hi = np.log2(lo.max(axis=1)), np.log2(hi.max(axis=1))
            slack = 1e-5
            for name, lmin, sc in (("hip", lm, sm), ("oracle", lr_, sr_s)):
                assert np.all((lmin >= lmin_lo - slack) & (lmin <= lmin_hi + slack)), f"{name}: l_min outside bound"
                assert np.all((sc >= lmax_lo - lmin_hi - slack) & (sc <= lmax_hi - lmin_lo + slack)), \
                    f"{name}: block scale outside bound"
        mine, want = _t2np(p), _t2np(q)
        line.append(f"params not bit-equal {(mine != want).mean():.2e}")
        print("  ".join(line), flush=True)
        _cmp_params("c4 e2e", f"step {t}", mine, want, _t2np(init))
    print(f"[apollo c4 e2e] {shape} {str(dtype)[6:]} worst over 4 steps: "
          + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()), flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", C4_SHAPES, ids=["right_1024x512", "left_512x1536"])
def test_apollo_c4_rank256_sr_writeback_bits(shape, det_proj):
    """C4's SR writeback at rank 256: x = (p * decay) + (G * f) * step in fp32,
    rounded with the reference's stream (kernels.cu:48-87), bit for bit against
    the CPU restatement given the step's scalars from the library's workspace."""
    from adafactor8bit import Adafactor8Bit
    from oracle import sr
    print(f"[apollo c4 sr] {shape}", flush=True)
    R, C = shape
    rank = 256
    p = torch.nn.Parameter(inputs.make_param(shape, 0, 22).to("cuda", torch.bfloat16))
    opt = Adafactor8Bit([p], **dict(C4_KW, weight_decay=0.1, stochastic_round_writeback=True))
    right = R >= C
    n_low = R * rank if right else rank * C
    nch = R if right else C
    fin = 2 * n_low + nch
    scal = fin + nch
    for t in range(1, 4):
        p_old = _f32(_t2np(p)).reshape(-1).astype(np.float32)
        g = inputs.make_grad(shape, 0, t, 22, zero_frac=0.0).to(torch.bfloat16)
        p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        st = opt.state[p]
        ws = _ws(opt, p)
        step_s, dec, fs = np.float32(ws[scal]), np.float32(ws[scal + 1]), np.float32(ws[scal + 6])
        gf = _f32(_t2np(g)).reshape(R, C).astype(np.float32)
        f = ws[fin:fin + nch].astype(np.float32) * fs
        fm = np.broadcast_to(f[:, None] if right else f[None, :], (R, C))
        x = (p_old * dec) + ((gf * fm) * step_s).reshape(-1)
        want = sr.sr_round_bf16(x.astype(np.float32), seed=int(st["sr_seed"]), step=int(st["step"]))
        got = _t2np(p).reshape(-1).view(np.uint16)
        assert np.array_equal(got, want), f"step {t}: {(got != want).mean():.2e} differ"


# Factorised and CAME APOLLO over a group of matrices of several shapes (right
# and left side, ragged widths).  The optimizer runs the low-rank stage of the
# whole group as one launch per pass (a8_apollo_lowrank_x_multi); the same steps
# through the one-matrix entry point (a8_apollo_lowrank_x, per matrix, in
# order) must give the same bits, since every reduction stays inside its matrix.
X_SHAPES = [(300, 200), (96, 260), (513, 40), (64, 1030), (200, 300), (700, 129)]
X_VARIANTS = {
    "fact_uf8": dict(apollo_factorize=True),
    "fact_nomom": dict(apollo_factorize=True, beta1=None, beta2=None, beta2_decay=-0.8, d=1.0),
    "came_al8_clip": dict(beta3=0.9999, d=1.0, eps_came=1e-16),
    "came_al16_uf4": dict(beta3=0.99, d=1.0, eps_came=1e-16, v_quant_type="al16", c_quant_type="al16",
                          m_quant_type="uf4"),
    "came_fp32": dict(beta3=0.9999, d=1.0, eps_came=1e-16, quantize=False),
    "fact_came_al8": dict(apollo_factorize=True, beta3=0.9999, d=1.0, eps_came=1e-16),
    "fact_came_fp32": dict(apollo_factorize=True, beta3=0.999, d=1.0, eps_came=1e-16, quantize=False),
}


def _per_matrix_stage(L):
    import ctypes
    from adafactor8bit import _native as nat

    def run(xarr, n, tab, nbytes, upload, dsc, stream):
        recs = ctypes.cast(xarr, ctypes.POINTER(nat.ApolloXArgs))
        for i in range(n):
            rc = L.a8_apollo_lowrank_x(ctypes.byref(recs[i]), stream)
            if rc:
                return rc
        return 0
    return run


@pytest.mark.gpu
@pytest.mark.parametrize("variant", sorted(X_VARIANTS))
@pytest.mark.parametrize("rank", [32, 5])
def test_apollo_x_batched_equals_per_matrix(variant, rank, det_proj):
    from adafactor8bit import Adafactor8Bit
    from adafactor8bit import _native as nat
    print(f"[apollo x batched] {variant} rank={rank}", flush=True)
    kw = dict(_apollo_kw(apollo_rank=rank, apollo_scale_type="channel"), **X_VARIANTS[variant])
    init = [inputs.make_param(s, i, 31) for i, s in enumerate(X_SHAPES)]
    runs = []
    for batched in (True, False):
        with pytest.MonkeyPatch.context() as mp:
            L = nat.lib()
            if not batched:
                mp.setattr(L, "a8_apollo_lowrank_x_multi", _per_matrix_stage(L))
            params = [torch.nn.Parameter(x.clone().cuda()) for x in init]
            opt = Adafactor8Bit(params, **kw)
            for t in range(1, 4):
                for i, p in enumerate(params):
                    p.grad = inputs.make_grad(X_SHAPES[i], i, t, 31, kind="student_t").cuda()
                opt.step()
            torch.cuda.synchronize()
        runs.append((params, opt))
    (pa, oa), (pb, ob) = runs
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a.detach(), b.detach()), f"{variant} p{i}: parameters differ"
        sa, sb = oa.state[a], ob.state[b]
        for k, v in sa.items():
            if torch.is_tensor(v):
                assert torch.equal(v, sb[k]), f"{variant} p{i}: state {k} differs"


@pytest.mark.gpu
@pytest.mark.parametrize("shape,big", [((1024, 512), (4096, 2048)), ((512, 1536), (2048, 4096))],
                         ids=["right", "left"])
def test_apollo_step_is_the_same_alone_or_batched(shape, big):
    """A matrix's APOLLO step does not depend on what else its group holds: the
    wide projection's XCD ranges, the batched low-rank stage and the finish put
    a 4-tile matrix stepped alone (each tile the only one of its XCD range) and
    beside a 16-tile matrix (its tiles sharing a range with the big one's) on
    different workgroups, but every output sums its K terms in the same order,
    so the parameters and every state come out bit for bit the same (C4 settings,
    bf16 SR, three steps)."""
    from adafactor8bit import Adafactor8Bit
    print(f"[apollo alone vs batched] {shape} beside {big}", flush=True)
    kw = dict(C4_KW, stochastic_round_writeback=True)
    runs = []
    for with_big in (False, True):
        shapes = [shape, big] if with_big else [shape]
        ps = [torch.nn.Parameter(inputs.make_param(s, i, 23).to("cuda", torch.bfloat16)) for i, s in enumerate(shapes)]
        opt = Adafactor8Bit(ps, **kw)
        for t in range(1, 4):
            for i, p in enumerate(ps):
                p.grad = inputs.make_grad(shapes[i], i, t, 23, zero_frac=0.0).to("cuda", torch.bfloat16)
            opt.step()
        torch.cuda.synchronize()
        runs.append((ps[0], opt))
    (pa, oa), (pb, ob) = runs
    assert torch.equal(pa, pb), "parameters differ"
    sa, sb = oa.state[pa], ob.state[pb]
    for k, v in sa.items():
        if torch.is_tensor(v):
            assert torch.equal(v, sb[k]), k
