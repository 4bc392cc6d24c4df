// Device helpers shared by the adafactor8bit MI355X kernels (gfx950, wave64).
//
// Numerics contract ("reference numerics"): every value that is stored as a
// quantised code is decided exactly as the reference's PyTorch path decides it
// (adafactor8bit/optimizer.py:299-353, 504-532, 690-700):
//   * EMA      lerp(s, e, w) = fma(w, e - s, s) for |w| < 0.5, else fma(w - 1, e - s, e)
//   * AL code  q = clamp(rint(((log2(max(v,1e-38)) - lmin) / s) * (L-2)) + 1, 1, L-1), q=0 <=> v=0
//   * UF code  q = clamp(rint((m / absmax) * 2^(b-1)), -2^(b-1), 2^(b-1)-1) + 2^(b-1)
// with IEEE float32 division and correctly rounded log2 / exp2.  A fast path
// (hardware v_log_f32 / v_rcp_f32) decides a code whenever the rounding
// argument lies farther from a half-integer than a proven error margin; the
// rare remaining elements are recomputed exactly (double-precision log2, IEEE
// division).  Parameters are not re-quantised, so the update direction may use
// the hardware sqrt/rcp (<= 2 ulp) without changing any code.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/adafactor8bit_amd.h"

namespace a8 {

// Global-memory (address space 1) view of a pointer: descriptor-table pointers
// would otherwise be generic (flat), costing flat_load/flat_store and combined
// vmcnt/lgkmcnt waits against LDS traffic.
#define A8_G __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ A8_G T* gp(T* p) { return (A8_G T*)p; }
template <typename T>
__device__ __forceinline__ const A8_G T* gp(const T* p) { return (const A8_G T*)p; }

// Constant-address-space (address space 4) view for data that is uniform across
// a workgroup and not written during the launch: loads go through the scalar
// cache into SGPRs.
#define A8_C __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ const A8_C T* cp(const T* p) { return (const A8_C T*)p; }

// This step's scalars from the block a8_step_advance wrote (uniform, written
// before the launch): read through the scalar cache as 64-bit words.
__device__ __forceinline__ a8_step_scalars load_step_scalars(const a8_step_scalars* p) {
  const A8_C uint64_t* w = (const A8_C uint64_t*)cp(p);
  uint64_t buf[sizeof(a8_step_scalars) / 8];
#pragma unroll
  for (int i = 0; i < (int)(sizeof(a8_step_scalars) / 8); ++i) buf[i] = w[i];
  a8_step_scalars s;
  __builtin_memcpy(&s, buf, sizeof(s));
  return s;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kFltMin = 1.17549435e-38f;   // FP32 smallest normal
constexpr float kLogClampIn = 1e-38f;        // clamp(min=1e-38) before log2 (optimizer.py:309)

// ---------------------------------------------------------------- numerics
__device__ __forceinline__ float lerp_ref(float s, float e, float w) {
  // torch.lerp on CPU (vectorised): fma(coeff, e - s, base)
  return (fabsf(w) < 0.5f) ? __builtin_fmaf(w, e - s, s) : __builtin_fmaf(w - 1.0f, e - s, e);
}

// lerp_ref with a weight shared by every lane: the weight's branch is settled
// once (lerp_weight), so each element costs one subtraction, one select and one
// fma.  lerp_u(s, e, lerp_weight(w)) == lerp_ref(s, e, w) bit for bit.
struct LerpW {
  float wc;     // w, or w - 1 for |w| >= 0.5
  bool small;   // |w| < 0.5: base s, else base e
};

__device__ __forceinline__ LerpW lerp_weight(float w) {
  const bool small = fabsf(w) < 0.5f;
  return LerpW{small ? w : w - 1.0f, small};
}

__device__ __forceinline__ float lerp_u(float s, float e, LerpW L) {
  return __builtin_fmaf(L.wc, e - s, L.small ? s : e);
}

// q[i] = x[i] / d, correctly rounded, for a divisor d >= 1 shared by every lane
// and its IEEE reciprocal rd = 1.0f / d: one Markstein correction of x * rd (rd
// the correctly rounded reciprocal and q0 within an ulp of x / d, so the
// remainder x - q0 d is exact in one fma and q0 + r rd rounds to the correctly
// rounded quotient).  The theorem needs quotient and remainder in the normal
// range: when any lane holds a value with |q0| < 2^-100, zero or non-finite, the
// wave redoes those elements with the IEEE division (a uniform branch, so the
// division is not executed otherwise).  Three operations in place of ten.
__device__ __forceinline__ bool div_fast_ok(float q0) {
  const float a = fabsf(q0);
  return a >= 0x1p-100f && a <= 0x1.fffffep127f;   // false for NaN
}

template <int N>
__device__ __forceinline__ void div_by(float* q, const float* x, float d, float rd) {
  bool bad = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float q0 = x[i] * rd;
    const float r = __builtin_fmaf(-q0, d, x[i]);
    q[i] = __builtin_fmaf(r, rd, q0);
    bad = bad || !div_fast_ok(q0);
  }
  if (__builtin_amdgcn_ballot_w64(bad)) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (!div_fast_ok(x[i] * rd)) q[i] = x[i] / d;
  }
}

__device__ __forceinline__ float log2_exact(float x) {   // x > 0, correctly rounded to fp32
  return (float)::log2((double)x);
}

__device__ __forceinline__ float exp2_exact(float x) {
  return (float)::exp2((double)x);
}

__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }

// Non-finite gradients are treated as zero (the reference's GPU kernels do the
// same, kernels.cu:43-46; its CPU path has no defined result for them).
__device__ __forceinline__ float scrub(float g) {
  return (__builtin_isfinite(g)) ? g : 0.0f;
}

// Per-block constants of the AL refit.
struct ALFit {
  float lmin;     // new min_log
  float s;        // new scale
  float k;        // ~ (L-2)/s
  float c1;       // 1 - lmin*k: t1 = fma(log2 v, k, c1) ~ ((log2 v - lmin)/s)*(L-2) + 1
  float kmar;     // fast-path margin: kmar*|log2 v| + cmar
  float cmar;
};

__device__ __forceinline__ void al_fit_consts(ALFit& f, float levels_m2) {
  f.k = levels_m2 * fast_rcp(f.s);
  f.c1 = 1.0f - f.lmin * f.k;
  f.kmar = f.k * 0x1p-22f;
  f.cmar = __builtin_fmaf(fabsf(f.lmin), f.kmar, 2e-4f);
}

// Refit from the block's max v and min non-zero v (optimizer.py:308-318):
// l = log2(max(v, 1e-38)); lmax over all, lmin over v != 0, floored, lmin := lmax-1
// if lmin >= lmax, scale = max(lmax - lmin, 1e-12).
__device__ __forceinline__ ALFit al_refit(float vmax, float vmin_nz, float floor_, float levels_m2) {
  ALFit f;
  const float lmax = log2_exact(fmaxf(vmax, kLogClampIn));
  float lmin = (vmin_nz == __builtin_inff()) ? __builtin_inff()
                                              : log2_exact(fmaxf(vmin_nz, kLogClampIn));
  lmin = fmaxf(lmin, floor_);
  if (lmin >= lmax) lmin = lmax - 1.0f;
  const float s = fmaxf(lmax - lmin, 1e-12f);
  f.lmin = lmin;
  f.s = s;
  al_fit_consts(f, levels_m2);
  return f;
}

// Same refit, with the two correctly rounded logarithms of a block computed in
// one call per wave: even lanes take log2 of the block max, odd lanes of the
// block min, and every lane reads its block's pair back.  Requires that the
// block's lanes hold the same (vmax, vmin_nz) and span at least two lanes.
// ---- the reference's fused-kernel AL rule (kernels.cu:318-326, 686-687, 772-791)
// The fused 1-D CUDA kernels refit differently from the CPU quantiser above:
// l = log2(v) with log2(0) = -inf (no 1e-38 clamp); lmax = min(max l, 126), -1e30
// for a block without a non-zero v; lmin = max(min(126, min l), floor) where the
// minimum includes zeros, so a block holding a zero takes the floor (the caller's
// log2(max(eps1^2, FLT_MIN))); lmin := lmax - 1 if lmin >= lmax; s = max(lmax -
// lmin, 1e-12).  Codes: 0 for v == 0, else clamp(rint((l - lmin) * RN((L-2)/s)) + 1,
// 1, L-1); decode 2^(((q-1) * RN(1/(L-2))) * s + lmin).  A call selects it with
// krule; the default is the CPU rule.
__device__ __forceinline__ float al_klog(float x, float lo) { return x > 0.0f ? log2_exact(x) : lo; }
__device__ __forceinline__ void al_kfit(float lmax_raw, float lmin_raw, float floor_, float levels_m2, ALFit& f) {
  const float lmax = fminf(lmax_raw, 126.0f);
  float lmin = fmaxf(fminf(lmin_raw, 126.0f), floor_);
  if (lmin >= lmax) lmin = lmax - 1.0f;
  f.lmin = lmin;
  f.s = fmaxf(lmax - lmin, 1e-12f);
  al_fit_consts(f, levels_m2);
}
// The decode exponent of code c >= 1 (c1 = c - 1) under either rule.
template <int LM2>
__device__ __forceinline__ float al_dec_log(float c1, float s, float lm, bool krule) {
  return krule ? (c1 * (1.0f / (float)LM2)) * s + lm : (c1 * s) / (float)LM2 + lm;
}

// krule: vmin_nz is the block minimum including zeros, and the fit is al_kfit's.
__device__ __forceinline__ ALFit al_refit_pair(float vmax, float vmin_nz, float floor_, float levels_m2,
                                               int lane, bool krule = false) {
  const float x = (lane & 1) ? vmin_nz : vmax;   // inf (no non-zero entry) stays inf
  const float l = krule ? al_klog(x, (lane & 1) ? -__builtin_inff() : -1e30f) : log2_exact(fmaxf(x, kLogClampIn));
  const float lmax = __shfl(l, lane & ~1, 64);
  float lmin = __shfl(l, lane | 1, 64);
  ALFit f;
  if (krule) {
    al_kfit(lmax, lmin, floor_, levels_m2, f);
    return f;
  }
  lmin = fmaxf(lmin, floor_);
  if (lmin >= lmax) lmin = lmax - 1.0f;
  const float s = fmaxf(lmax - lmin, 1e-12f);
  f.lmin = lmin;
  f.s = s;
  al_fit_consts(f, levels_m2);
  return f;
}

// Exact AL code argument (before clamping): rint(((log2(max(v,1e-38)) - lmin) / s)
// * (L-2)) + 1 with a correctly rounded log2 and IEEE division, in the
// reference's operation order (optimizer.py:310-321).
template <int LM2>
__device__ __forceinline__ float al_round_exact(float v, const ALFit& f) {
  const float le = log2_exact(fmaxf(v, kLogClampIn));
  return rintf(((le - f.lmin) / f.s) * (float)LM2) + 1.0f;
}
// The same under the kernels' rule (kernels.cu:322-326, 783-787): (l - lmin) times
// the rounded (L-2)/s, no clamp of v (v > 0; v == 0 is code 0 before this matters).
template <int LM2>
__device__ __forceinline__ float al_round_exact_k(float v, const ALFit& f) {
  const float le = log2_exact(v);
  return rintf((le - f.lmin) * ((float)LM2 / f.s)) + 1.0f;
}
template <int LM2>
__device__ __forceinline__ float al_round_exact(float v, const ALFit& f, bool krule) {
  return krule ? al_round_exact_k<LM2>(v, f) : al_round_exact<LM2>(v, f);
}

// Fast AL8 code argument from the hardware log2 (faithful: |error| <= |l|*2^-23,
// measured on gfx950): t1 = fma(lf, k, 1 - lmin*k).  Against the exact argument
// t* + 1 the error is at most (|l| + |lmin|)*k*2^-23 (log error, rounding of
// lmin*k and of c1) + 1.3e-4 (reciprocal, the fma, and t*'s own three roundings,
// t <= 255), so rint(t1) is exact whenever t1 lies farther than
// (|l| + |lmin|)*k*2^-22 + 2e-4 from a half-integer.  bad=true flags the rest
// (and subnormal inputs) for al_round_exact; v == 0 needs no rounding (code 0).
__device__ __forceinline__ float al8_round_fast(float v, const ALFit& f, bool& bad) {
  const float lf = __builtin_amdgcn_logf(v);
  const float t1 = __builtin_fmaf(lf, f.k, f.c1);
  const float r = rintf(t1);
  const float e = fabsf(fabsf(t1 - r) - 0.5f);
  const bool good = (v == 0.0f) | ((v >= kFltMin) & (e > __builtin_fmaf(fabsf(lf), f.kmar, f.cmar)));
  bad = !good;
  return r;
}

// Code value from the argument: 0 for v == 0, else clamp to [1, L-1].
template <int LM2>
__device__ __forceinline__ float al_clamp(float v, float r1) {
  return (v == 0.0f) ? 0.0f : __builtin_amdgcn_fmed3f(r1, 1.0f, (float)(LM2 + 1));
}

template <int LM2>
__device__ __forceinline__ uint32_t al_finish(float v, float r1) {
  return (uint32_t)al_clamp<LM2>(v, r1);
}

// AL codes of N values under one block fit, equal to al_round_exact's: AL8 takes
// the fast argument and re-decides only the values inside its margin; AL16,
// whose margin would cover most values, always rounds exactly.
// The fast argument approximates the real (l - lmin) * (L-2)/s + 1 of both rules;
// each rule's own roundings stay inside the margin, so krule changes only the
// exact re-decision.
template <int LM2, int N>
__device__ __forceinline__ void al_codes(const float* v, const ALFit& f, uint32_t* q, bool krule = false) {
  float r[N];
  if constexpr (LM2 == 254) {
    bool bad[N];
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = al8_round_fast(v[i], f, bad[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (bad[i]) r[i] = al_round_exact<254>(v[i], f, krule);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = al_round_exact<LM2>(v[i], f, krule);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) q[i] = al_finish<LM2>(v[i], r[i]);
}

// Fast UF code argument: t' = fma(m, H/absmax, H) ~ (m/absmax)*H + H with a
// faithful reciprocal; against the exact argument the error is at most
// H*3*2^-24 + ulp(2H)/2 (< 4e-5 for H = 128), margin 1e-4.
template <int H>
__device__ __forceinline__ float uf_round_fast(float m, float kam, bool& bad) {
  const float t = __builtin_fmaf(m, kam, (float)H);
  const float r = rintf(t);
  bad = !(fabsf(fabsf(t - r) - 0.5f) > 1e-4f);
  return r;
}

// Exact UF code argument: rint((m / absmax) * H) + H (optimizer.py:516-518).
template <int H>
__device__ __forceinline__ float uf_round_exact(float m, float amax) {
  return rintf((m / amax) * (float)H) + (float)H;
}

template <int H>
__device__ __forceinline__ float uf_clamp(float r) {
  return __builtin_amdgcn_fmed3f(r, 0.0f, (float)(2 * H - 1));
}

template <int H>
__device__ __forceinline__ uint32_t uf_finish(float r) {
  return (uint32_t)uf_clamp<H>(r);
}

template <int H>
__device__ __forceinline__ uint32_t uf_code(float m, float amax, float ramax) {
  bool bad;
  float r = uf_round_fast<H>(m, (float)H * ramax, bad);
  if (bad) r = uf_round_exact<H>(m, amax);
  return uf_finish<H>(r);
}

// Pack four integer-valued floats in [0, 255] into one dword, byte k from x[k].
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
  uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(a, 0, 0u);
  w = __builtin_amdgcn_cvt_pk_u8_f32(b, 1, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(c, 2, w);
  return __builtin_amdgcn_cvt_pk_u8_f32(d, 3, w);
}

// ---------------------------------------------------------------- dtypes
template <typename T> __device__ __forceinline__ float to_f(T x);
template <> __device__ __forceinline__ float to_f<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f<__hip_bfloat16>(__hip_bfloat16 x) {
  return __bfloat162float(x);
}
template <> __device__ __forceinline__ float to_f<__half>(__half x) { return __half2float(x); }

template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f<__hip_bfloat16>(float x) {
  return __float2bfloat16(x);
}
// x as a materialised fp32 value: the empty asm stops instruction selection from
// fusing the conversion that follows with the multiply or fma that produced x
// into one v_fma_mix*_f16, which rounds the exact result to fp16 once instead of
// rounding to fp32 first, as the reference and its PyTorch path do.
__device__ __forceinline__ float f32_value(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
template <> __device__ __forceinline__ __half from_f<__half>(float x) { return __float2half(f32_value(x)); }

// fp64 parameters: gradients are read as fp32 (torch's grad.float(), round to
// nearest), parameters stay double and take their update in double -- what
// p.mul_(decay) and p.add_(u, alpha=-step) do on a float64 tensor.  pval_t<T> is
// the register type of a parameter value: double for fp64, fp32 otherwise.
template <> __device__ __forceinline__ float to_f<double>(double x) { return (float)x; }
template <> __device__ __forceinline__ double from_f<double>(float x) { return (double)x; }
template <typename T> struct PVal { using type = float; };
template <> struct PVal<double> { using type = double; };
template <typename T> using pval_t = typename PVal<T>::type;

// p * decay and fma(-step, u, p) in the parameter's register type.  With fp64
// the product step * u of two floats is exact in double, so the fma rounds once,
// as the double add of torch does.
__device__ __forceinline__ float pdec(float p, float d) { return p * d; }
__device__ __forceinline__ double pdec(double p, float d) { return p * (double)d; }
__device__ __forceinline__ float pupd(float step, float u, float p) { return __builtin_fmaf(-step, u, p); }
__device__ __forceinline__ double pupd(float step, float u, double p) {
  return __builtin_fma(-(double)step, (double)u, p);
}

typedef double f64x2 __attribute__((ext_vector_type(2)));

// A parameter element to / from its register type.
template <typename T>
__device__ __forceinline__ pval_t<T> pv_of(T x) {
  if constexpr (sizeof(T) == 8) return x; else return to_f<T>(x);
}
template <typename T>
__device__ __forceinline__ T pv_to(pval_t<T> x) {
  if constexpr (sizeof(T) == 8) return x; else return from_f<T>(x);
}

// Single-element global load / store of a param-typed value (16-bit types go
// through their bit pattern: class types cannot be bound in address space 1).
// V: the register type (fp32, or double for fp64 parameters).
template <typename T, typename V = float>
__device__ __forceinline__ V ld1(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 8) {
    return (V)gp(reinterpret_cast<const double*>(p))[i];
  } else if constexpr (sizeof(T) == 4) {
    return gp(reinterpret_cast<const float*>(p))[i];
  } else {
    const uint16_t b = gp(reinterpret_cast<const uint16_t*>(p))[i];
    T t;
    __builtin_memcpy(&t, &b, 2);
    return to_f<T>(t);
  }
}
template <typename T, typename V>
__device__ __forceinline__ void st1(T* p, int64_t i, V v) {
  if constexpr (sizeof(T) == 8) {
    gp(reinterpret_cast<double*>(p))[i] = (double)v;
  } else if constexpr (sizeof(T) == 4) {
    gp(reinterpret_cast<float*>(p))[i] = v;
  } else {
    const T t = from_f<T>(v);
    uint16_t b;
    __builtin_memcpy(&b, &t, 2);
    gp(reinterpret_cast<uint16_t*>(p))[i] = b;
  }
}

// Four fp64 values from 32 aligned bytes.
template <typename V>
__device__ __forceinline__ void ld4d(const double* p, V* out) {
  const f64x2 a = __builtin_nontemporal_load(gp(reinterpret_cast<const f64x2*>(p)));
  const f64x2 b = __builtin_nontemporal_load(gp(reinterpret_cast<const f64x2*>(p)) + 1);
  out[0] = (V)a.x; out[1] = (V)a.y; out[2] = (V)b.x; out[3] = (V)b.y;
}
template <typename V>
__device__ __forceinline__ void st4d(double* p, const V* v) {
  const f64x2 a = {(double)v[0], (double)v[1]};
  const f64x2 b = {(double)v[2], (double)v[3]};
  __builtin_nontemporal_store(a, gp(reinterpret_cast<f64x2*>(p)));
  __builtin_nontemporal_store(b, gp(reinterpret_cast<f64x2*>(p)) + 1);
}

// Load / store 8 consecutive elements (aligned fast path when fully in range).
template <typename T, typename V>
__device__ __forceinline__ void load8(const T* base, int64_t i0, int64_t n, V* out) {
  if (i0 + 8 <= n) {
    if constexpr (sizeof(T) == 8) {
      ld4d<V>(reinterpret_cast<const double*>(base) + i0, out);
      ld4d<V>(reinterpret_cast<const double*>(base) + i0 + 4, out + 4);
    } else if constexpr (sizeof(T) == 4) {
      const A8_G f32x4* p = gp(reinterpret_cast<const f32x4*>(base + i0));
      f32x4 a = __builtin_nontemporal_load(p);
      f32x4 b = __builtin_nontemporal_load(p + 1);
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
      u32x4 a = __builtin_nontemporal_load(gp(reinterpret_cast<const u32x4*>(base + i0)));
      const T* h = reinterpret_cast<const T*>(&a);
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = to_f<T>(h[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = (i0 + k < n) ? ld1<T, V>(base, i0 + k) : (V)0;
  }
}

template <typename T, typename V>
__device__ __forceinline__ void store8(T* base, int64_t i0, int64_t n, const V* v) {
  if (i0 + 8 <= n) {
    if constexpr (sizeof(T) == 8) {
      st4d<V>(reinterpret_cast<double*>(base) + i0, v);
      st4d<V>(reinterpret_cast<double*>(base) + i0 + 4, v + 4);
    } else if constexpr (sizeof(T) == 4) {
      A8_G f32x4* p = gp(reinterpret_cast<f32x4*>(base + i0));
      f32x4 a = {v[0], v[1], v[2], v[3]};
      f32x4 b = {v[4], v[5], v[6], v[7]};
      __builtin_nontemporal_store(a, p);
      __builtin_nontemporal_store(b, p + 1);
    } else {
      u32x4 a;
      T* h = reinterpret_cast<T*>(&a);
#pragma unroll
      for (int k = 0; k < 8; ++k) h[k] = from_f<T>(v[k]);
      __builtin_nontemporal_store(a, gp(reinterpret_cast<u32x4*>(base + i0)));
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + k < n) st1<T, V>(base, i0 + k, v[k]);
  }
}

// Load / store 4 consecutive elements (one 16-byte fp32 or 8-byte 16-bit
// access per lane when fully in range; two 16-byte accesses for fp64).
template <typename T, typename V>
__device__ __forceinline__ void load4n(const T* base, int64_t i0, int64_t n, V* out) {
  if (i0 + 4 <= n) {
    if constexpr (sizeof(T) == 8) {
      ld4d<V>(reinterpret_cast<const double*>(base) + i0, out);
    } else if constexpr (sizeof(T) == 4) {
      const f32x4 a = __builtin_nontemporal_load(gp(reinterpret_cast<const f32x4*>(base + i0)));
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    } else {
      const u32x2 a = __builtin_nontemporal_load(gp(reinterpret_cast<const u32x2*>(base + i0)));
      const T* h = reinterpret_cast<const T*>(&a);
#pragma unroll
      for (int k = 0; k < 4; ++k) out[k] = to_f<T>(h[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = (i0 + k < n) ? ld1<T, V>(base, i0 + k) : (V)0;
  }
}

// Unchecked form of load4n for a window known to lie inside the tensor.
template <typename T, typename V>
__device__ __forceinline__ void load4v(const T* base, int64_t i0, V* out) {
  if constexpr (sizeof(T) == 8) {
    ld4d<V>(reinterpret_cast<const double*>(base) + i0, out);
  } else if constexpr (sizeof(T) == 4) {
    const f32x4 a = __builtin_nontemporal_load(gp(reinterpret_cast<const f32x4*>(base + i0)));
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  } else {
    const u32x2 a = __builtin_nontemporal_load(gp(reinterpret_cast<const u32x2*>(base + i0)));
    const T* h = reinterpret_cast<const T*>(&a);
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = to_f<T>(h[k]);
  }
}

template <typename T, typename V>
__device__ __forceinline__ void store4n(T* base, int64_t i0, int64_t n, const V* v) {
  if (i0 + 4 <= n) {
    if constexpr (sizeof(T) == 8) {
      st4d<V>(reinterpret_cast<double*>(base) + i0, v);
    } else if constexpr (sizeof(T) == 4) {
      const f32x4 a = {v[0], v[1], v[2], v[3]};
      __builtin_nontemporal_store(a, gp(reinterpret_cast<f32x4*>(base + i0)));
    } else {
      u32x2 a;
      T* h = reinterpret_cast<T*>(&a);
#pragma unroll
      for (int k = 0; k < 4; ++k) h[k] = from_f<T>(v[k]);
      __builtin_nontemporal_store(a, gp(reinterpret_cast<u32x2*>(base + i0)));
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (i0 + k < n) st1<T, V>(base, i0 + k, v[k]);
  }
}

// ---------------------------------------------------------------- reductions
// Max / min over aligned groups of G lanes (G a power of two <= 64, uniform),
// with no LDS traffic: DPP moves inside 16-lane rows (quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror -- each pairs every lane with one of
// its own group, so after them every lane of a row holds the row's result),
// ds_swizzle in bit mode (xor 16) across the two rows of a 32-lane half, and
// v_readlane of lanes 0 and 32 across the halves (the result is then uniform).
// Max and min are exact, so the order of the steps does not matter.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __uint_as_float(dpp_u<CTRL>(__float_as_uint(x)));
}

template <typename Op>
__device__ __forceinline__ uint32_t grp_red_u(uint32_t x, int G, Op op) {
  if (G >= 2) x = op(x, dpp_u<0xB1>(x));    // quad_perm [1,0,3,2]
  if (G >= 4) x = op(x, dpp_u<0x4E>(x));    // quad_perm [2,3,0,1]
  if (G >= 8) x = op(x, dpp_u<0x141>(x));   // row_half_mirror
  if (G >= 16) x = op(x, dpp_u<0x140>(x));  // row_mirror
  if (G >= 32) x = op(x, (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, 0x401F));   // xor 16 within 32
  if (G >= 64) x = op((uint32_t)__builtin_amdgcn_readlane((int)x, 0), (uint32_t)__builtin_amdgcn_readlane((int)x, 32));
  return x;
}

__device__ __forceinline__ float grp_max(float x, int G) {
  return __uint_as_float(grp_red_u(__float_as_uint(x), G, [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ float grp_min(float x, int G) {
  return __uint_as_float(grp_red_u(__float_as_uint(x), G, [](uint32_t a, uint32_t b) {
    return __float_as_uint(fminf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ uint32_t grp_umin(uint32_t x, int G) {
  return grp_red_u(x, G, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ float grp_max_dpp(float x, int G) { return grp_max(x, G); }

// Sums over the same groups: every step adds two equal-ordered partial sums
// (within a quad the xor-1 / xor-2 partners, then whole quads, rows and halves
// whose lanes already agree), so each lane's result is the butterfly's, bit for
// bit, whatever the pairing inside a step.
__device__ __forceinline__ float grp_sum(float x, int G) {
  return __uint_as_float(grp_red_u(__float_as_uint(x), G, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}

template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = dpp_u<CTRL>((uint32_t)u), hi = dpp_u<CTRL>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double swz16_d(double x) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)u, 0x401F);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)(u >> 32), 0x401F);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double lane_d(double x, int l) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double grp_sum_d(double x, int G) {
  if (G >= 2) x += dpp_d<0xB1>(x);
  if (G >= 4) x += dpp_d<0x4E>(x);
  if (G >= 8) x += dpp_d<0x141>(x);
  if (G >= 16) x += dpp_d<0x140>(x);
  if (G >= 32) x += swz16_d(x);
  if (G >= 64) x = lane_d(x, 0) + lane_d(x, 32);
  return x;
}

// ---------------------------------------------------------------- fixed-order sums
// A norm pass writes one partial sum per workgroup, and a finishing launch adds
// a tensor's partials in index order, so a sum of squares has the same bits
// whatever order the workgroups ran in (float atomics would not), and a tensor
// gives the same sum in a batched launch as on its own.
//
// wg_partial: the workgroup's sum of one float per lane -- each wave's butterfly
// sum (grp_sum), then the NW wave sums added in wave order in double.  Every lane
// calls it (one barrier); lane 0 receives the sum.  s_w: NW floats of LDS that
// nothing else uses.
template <int NW>
__device__ __forceinline__ double wg_partial(float v, float* s_w) {
  const float t = grp_sum(v, 64);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = t;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < NW; ++w) s += (double)s_w[w];
  }
  return s;
}

// sum_parts: the sum of p[0..n) by one 256-lane workgroup in a fixed order --
// lane l adds p[l], p[l + 256], ... in turn, then each wave's butterfly and the
// four wave sums in wave order.  Every lane calls it; lane 0 receives the sum.
// s_w: 4 doubles of LDS.
__device__ __forceinline__ double sum_parts(const double* p, int64_t n, double* s_w) {
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 256) s += p[i];
  s = grp_sum_d(s, 64);
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = s;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0) t = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
  return t;
}

}  // namespace a8
