// APOLLO optimizer step for MI355X (gfx950): one full-rank matrix per call.
//
// Follows _update_param_apollo (optimizer.py:2587-3084) on its non-factorised
// path without CAME (apollo_factorize=False, beta3=None):
//   G (R x C) is projected to rank r: right side (R >= C) g_low = G P^T (R x r),
//   left side g_low = P^T G (r x C), P the seeded Gaussian / sqrt(r);
//   low-rank V: first step v = g_low^2 * beta_v (AL floor -126), later
//   v = lerp(v, g_low^2, beta_v) (floor log2(eps^2)); low-rank M: lerp(m, g_low, 1-beta1);
//   u = m / (sqrt(v) + eps) (or g_low / (...) without beta1);
//   channel scale s = ||u_ch|| / (||g_low_ch|| + 1e-8) over rows (right) or
//   columns (left), or one tensor scale; Fira on sqrt(sum ||G_ch||^2 s^2) (or
//   ||G|| s); p <- p * decay + (step * G) * final_scale, step = -alpha / denom
//   with bias correction.
// Launches: [split of P^T into three bf16 terms when P changed] -> projection
// GEMM (rocBLAS gemm_ex: bf16 G times the three terms, accumulated in fp32,
// which carries P's 24 bits; fp32 G: one fp32 GEMM) -> k_ap_gnorm (norms of G)
// -> k_ap_low (low-rank V/M EMA, re-encode, u) -> k_ap_scale (channel norms of
// u and g_low) -> k_ap_scalars (Fira, step, final scales) -> k_ap_apply.
#include <rocblas/rocblas.h>
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

constexpr int kApUnit = 2048;   // low-rank elements per k_ap_low workgroup (8 per lane)
constexpr int kApNP = 1024;     // maximum workgroups of the partial-sum passes
constexpr int kApSc = 16;       // per-tensor scalars

// Workspace of one tensor (offsets in floats; partial arrays are doubles).
struct ApWs {
  int64_t glow;      // [n_low]   projected gradient
  int64_t u;         // [n_low]   low-rank update direction
  int64_t ngsq;      // [nch]     ||G_ch||^2
  int64_t fin;       // [nch]     s, then the final scale
  int64_t gpart;     // double[kApNP]   ||G||^2 per k_ap_gnorm workgroup
  int64_t ppart;     // double[kApNP]   sum p^2 per k_ap_gnorm workgroup
  int64_t spart;     // double[2 kApNP] scale pass: sum ngsq s^2 | sum u^2, sum g_low^2
  int64_t nfpart;    // int[kApNP]      k_ap_gnorm workgroup saw a non-finite gradient
  int64_t gcol;      // double[nrc C]   left side: column sums of G^2 per row chunk
  int64_t split;     // bf16[3 r K]     P^T in three terms
  int64_t scal;      // [16]
  int64_t total;
  int64_t n_low, nch, K;
  int64_t rcr, nrc, ncc;   // left side: rows per chunk, row chunks, 2048-column chunks
};

__host__ __device__ inline ApWs ap_layout(int64_t R, int64_t C, int64_t r, int channel) {
  ApWs w;
  const bool right = R >= C;
  w.n_low = right ? R * r : r * C;
  w.nch = channel ? (right ? R : C) : 1;
  w.K = right ? C : R;
  w.glow = 0;
  w.u = w.glow + w.n_low;
  w.ngsq = w.u + w.n_low;
  w.fin = w.ngsq + w.nch;
  w.gpart = (w.fin + w.nch + 1) / 2 * 2;
  w.ppart = w.gpart + 2 * kApNP;
  w.spart = w.ppart + 2 * kApNP;
  w.ncc = (C + 2047) / 2048;
  w.rcr = 64;
  while (w.ncc * ((R + w.rcr - 1) / w.rcr) > kApNP) w.rcr *= 2;
  w.nrc = (R + w.rcr - 1) / w.rcr;
  w.nfpart = w.spart + 4 * kApNP;
  w.gcol = w.nfpart + kApNP;
  w.split = (w.gcol + (right ? 0 : 2 * w.nrc * C) + 63) / 64 * 64;
  w.scal = w.split + (3 * r * w.K + 1) / 2;
  w.total = w.scal + kApSc;
  return w;
}

// Scalars: [0] step (-alpha/denom, bias-corrected), [1] decay, [2] has decay,
// [3] tensor final scale, [4] alpha, [5] norm_unscaled, [6] fira scale.
struct ApArgs {
  void* param;
  const void* grad;
  int64_t R, C, r;
  void* v_q;
  float* v_scale;
  float* v_min_log;
  float* v_fp32;
  uint8_t* m_q;
  float* m_scale;
  float* m_fp32;
  float* fira_prev;
  const float* lr;
  float* ws;
  uint64_t sr_seed;
  float bv, w_m, aeps, floor_, lr_val, eps2, bias_factor, wd, d, margin, sv;
  int has_fira_prev, first, has_m, mk, vb, lbv, lbm, channel, front, fira, scale_param, bias_mode, wd_mode;
  int ngn, nsc;   // workgroups of k_ap_gnorm and k_ap_scale
  int valign;     // rows of G start 16-byte aligned (C % 8 == 0, or C % 4 == 0 for fp32)
  uint64_t sr_step;
};

__device__ __forceinline__ double ws_d(float* ws, int64_t off, int64_t i) {
  return gp(reinterpret_cast<double*>(ws + off))[i];
}
__device__ __forceinline__ void ws_d_set(float* ws, int64_t off, int64_t i, double v) {
  gp(reinterpret_cast<double*>(ws + off))[i] = v;
}

// Eight consecutive elements of one row (16-byte vector loads when rows start
// aligned, i.e. C % 8 == 0; element loads otherwise or at the row's end).
template <typename T>
__device__ __forceinline__ void ld8_row(const T* rowp, int64_t c, int64_t C, int aligned, float* out) {
  if (aligned) {
    load8<T>(rowp, c, C, out);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = (c + k < C) ? ld1<T>(rowp, c + k) : 0.0f;
  }
}

// Workgroup sum of a double (256 lanes), fixed order; every lane gets it.
__device__ __forceinline__ double ap_wg_sum(double x, double* s4) {
  x = grp_sum_d(x, 64);
  const int lane = threadIdx.x;
  __syncthreads();
  if ((lane & 63) == 0) s4[lane >> 6] = x;
  __syncthreads();
  return ((s4[0] + s4[1]) + s4[2]) + s4[3];
}

// ------------------------------------------------------------ P^T split
// P^T = hi + mid + lo, each term rounded to bf16: 3 x 8 significand bits carry
// fp32's 24, so bf16 products of an exact bf16 G with the three terms, summed
// in fp32, give the fp32 GEMM to fp32 rounding.
__global__ __launch_bounds__(256) void k_ap_split(const float* __restrict__ pt, int64_t n,
                                                 __hip_bfloat16* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float x = gp(pt)[i];
    const __hip_bfloat16 h = __float2bfloat16(x);
    const float r1 = x - __bfloat162float(h);
    const __hip_bfloat16 m = __float2bfloat16(r1);
    const float r2 = r1 - __bfloat162float(m);
    out[i] = h;
    out[n + i] = m;
    out[2 * n + i] = __float2bfloat16(r2);
  }
}

// ------------------------------------------------------------ norms of G (and p^2)
// Channel norms: right side one wave per row of G, left side lanes over
// columns walking the rows; sums of fp32 squares in double, fixed order;
// ngsq = (sqrt(sum))^2 as torch.linalg.vector_norm(...).square().  Per
// workgroup partials of ||G||^2 (tensor scale) and p^2 (scale_parameter).
template <typename T>
__global__ __launch_bounds__(256) void k_ap_gnorm(ApArgs a) {
  __shared__ double sd[4];
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  const int64_t R = a.R, C = a.C;
  const bool right = R >= C;
  const T* G = reinterpret_cast<const T*>(a.grad);
  const T* P = reinterpret_cast<const T*>(a.param);
  float* ws = a.ws;
  const int lane = threadIdx.x, wave = lane >> 6, wl = lane & 63;
  double psq = 0.0, gsq = 0.0;
  bool nonfin = false;
  if (right) {
    // one wave per row, 8 elements per lane per step
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < R; row += (int64_t)gridDim.x * 4) {
      double s = 0.0, sp = 0.0;
      for (int64_t c = (int64_t)wl * 8; c < C; c += 512) {
        float g[8];
        ld8_row<T>(G + row * C, c, C, a.valign, g);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          nonfin |= !__builtin_isfinite(g[k]);
          const float gk = scrub(g[k]);
          s += (double)(gk * gk);
        }
        if (a.scale_param) {
          float p[8];
          ld8_row<T>(P + row * C, c, C, a.valign, p);
#pragma unroll
          for (int k = 0; k < 8; ++k) sp += (double)(p[k] * p[k]);
        }
      }
      s = grp_sum_d(s, 64);
      sp = grp_sum_d(sp, 64);
      if (a.channel && wl == 0) {
        const float nrm = sqrtf((float)s);
        gp(ws)[W.ngsq + row] = nrm * nrm;
      }
      if (wl == 0) { gsq += s; psq += sp; }
    }
  } else {
    // 2-D grid: x = 2048-column chunk, y = chunk of rcr rows; column partials in double
    const int64_t c0 = (int64_t)blockIdx.x * 2048 + (int64_t)lane * 8;
    const int64_t r0 = (int64_t)blockIdx.y * W.rcr;
    const int64_t r1 = (r0 + W.rcr < R) ? r0 + W.rcr : R;
    double s[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) s[k] = 0.0;
    if (c0 < C) {
      for (int64_t row = r0; row < r1; ++row) {
        float g[8];
        ld8_row<T>(G + row * C, c0, C, a.valign, g);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          nonfin |= !__builtin_isfinite(g[k]);
          const float gk = scrub(g[k]);
          s[k] += (double)(gk * gk);
        }
        if (a.scale_param) {
          float p[8];
          ld8_row<T>(P + row * C, c0, C, a.valign, p);
#pragma unroll
          for (int k = 0; k < 8; ++k) psq += (double)(p[k] * p[k]);
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (c0 + k < C) {
          ws_d_set(ws, W.gcol, (int64_t)blockIdx.y * C + c0 + k, s[k]);
          gsq += s[k];
        }
      }
    }
  }
  const double tg = ap_wg_sum(gsq, sd);
  const double tp = ap_wg_sum(psq, sd);
  const int nf = __syncthreads_or(nonfin ? 1 : 0);
  if (lane == 0) {
    const int64_t wg = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    ws_d_set(ws, W.gpart, wg, tg);
    ws_d_set(ws, W.ppart, wg, tp);
    gp(reinterpret_cast<int*>(ws + W.nfpart))[wg] = nf ? 1 : 0;
  }
}

// ------------------------------------------------------------ non-finite gradients
// The reference zeroes NaN / Inf gradient entries before the projection
// (optimizer.py:2606); the library GEMM reads G as given, so when k_ap_gnorm
// flagged a non-finite entry this pass recomputes g_low from the scrubbed G with
// plain fp32 dot products (one element per lane).  With a finite G every
// workgroup returns after reading the flags.
template <typename T>
__global__ __launch_bounds__(256) void k_ap_fixlow(ApArgs a, const float* __restrict__ pt) {
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  const int lane = threadIdx.x;
  int f = 0;
  for (int k = lane; k < a.ngn; k += 256) f |= gp(reinterpret_cast<const int*>(a.ws + W.nfpart))[k];
  if (!__syncthreads_or(f)) return;
  const int64_t R = a.R, C = a.C, r = a.r;
  const T* G = reinterpret_cast<const T*>(a.grad);
  for (int64_t i = (int64_t)blockIdx.x * 256 + lane; i < W.n_low; i += (int64_t)gridDim.x * 256) {
    float acc = 0.0f;
    if (R >= C) {
      const int64_t row = i / r, k = i - row * r;
      for (int64_t c = 0; c < C; ++c) acc = __builtin_fmaf(scrub(ld1<T>(G, row * C + c)), gp(pt)[c * r + k], acc);
    } else {
      const int64_t k = i / C, j = i - k * C;
      for (int64_t q = 0; q < R; ++q) acc = __builtin_fmaf(gp(pt)[k * R + q], scrub(ld1<T>(G, q * C + j)), acc);
    }
    gp(a.ws)[W.glow + i] = acc;
  }
}

// ------------------------------------------------------------ low-rank V / M and u
// Flat 2048-element units of g_low (8 contiguous per lane).  V block B_V and M
// block B_M are powers of two (B_V in [128, 2048], B_M in [32, B_V]), so a
// block is B/8 consecutive lanes.  Arithmetic as optimizer.py:2765-2790, 2911-2951
// (quantised states through _quant_v / _m_ema_pytorch, fp32 states through
// lerp_): v = first ? g^2 * bv : lerp(v, g^2, bv); m = lerp(m, g, 1 - beta1);
// u = m / (sqrt(v) + eps) with IEEE sqrt and division.
template <int VB, int MK>
__global__ __launch_bounds__(256) void k_ap_low(ApArgs a) {
  __shared__ float xw[16];
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  const int64_t n = W.n_low;
  float* ws = a.ws;
  const int lane = threadIdx.x, wave = lane >> 6;
  const int64_t e0 = (int64_t)blockIdx.x * kApUnit + (int64_t)lane * 8;
  const int lbv = a.lbv, lbm = a.lbm;
  const int VL = (1 << lbv) >> 3, ML = (1 << lbm) >> 3;
  const int64_t nvb = VB ? (n + (1 << lbv) - 1) >> lbv : 0;
  const int64_t nmb = (n + (1 << lbm) - 1) >> lbm;
  const int64_t vb = e0 >> lbv, mb = e0 >> lbm;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);
  const bool v_ok = VB ? vb < nvb : cnt > 0;
  const bool m_ok = (MK == 1 || MK == 2) && mb < nmb;   // codes padded to whole M blocks
  const int mk = MK == 1 ? 1 : a.mk;
  float g[8], v[8], m[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) { g[k] = 0.0f; v[k] = 0.0f; m[k] = 0.0f; }
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < cnt) g[k] = gp(ws)[W.glow + e0 + k];
  // ---- V
  float vo[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) vo[k] = 0.0f;
  if (!a.first) {
    if constexpr (VB == 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < cnt) vo[k] = gp(a.v_fp32)[e0 + k];
    } else if (v_ok) {
      const float s_old = gp(a.v_scale)[vb], lm_old = gp(a.v_min_log)[vb];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        uint32_t c;
        if constexpr (VB == 8) c = gp(reinterpret_cast<const uint8_t*>(a.v_q))[e0 + k];
        else c = gp(reinterpret_cast<const uint16_t*>(a.v_q))[e0 + k];
        const float lm2 = VB == 8 ? 254.0f : 65534.0f;
        vo[k] = c ? exp2_exact(((float)(c - 1) * s_old) / lm2 + lm_old) : 0.0f;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float g2 = g[k] * g[k];
    v[k] = a.first ? g2 * a.bv : lerp_ref(vo[k], g2, a.bv);
    if (k >= cnt) v[k] = 0.0f;
  }
  // ---- M
  if constexpr (MK != 0) {
    float mo[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) mo[k] = 0.0f;
    if (MK == 3) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < cnt) mo[k] = gp(a.m_fp32)[e0 + k];
    } else if (m_ok) {
      const float ms = gp(a.m_scale)[mb];
      if (mk == 2 || mk == 4) {
        const uint32_t qw = *gp(reinterpret_cast<const uint32_t*>(a.m_q + (e0 >> 1)));
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t byte = (qw >> (8 * (k >> 1))) & 0xFFu;
          mo[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
        }
      } else {
        const u32x2 qv = *gp(reinterpret_cast<const u32x2*>(a.m_q + e0));
#pragma unroll
        for (int k = 0; k < 8; ++k) mo[k] = m_decode(mk, ((k < 4 ? qv.x : qv.y) >> (8 * (k & 3))) & 0xFFu, ms);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], g[k], a.w_m) : 0.0f;
  }
  // ---- u
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < cnt) {
      const float x = MK != 0 ? m[k] : g[k];
      gp(ws)[W.u + e0 + k] = x / (sqrtf(v[k]) + a.aeps);
    }
  }
  // ---- V state
  if constexpr (VB == 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) gp(a.v_fp32)[e0 + k] = v[k];
  } else {
    uint32_t vmaxb = 0u, vkey = 0xFFFFFFFFu;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      vmaxb = max(vmaxb, __float_as_uint(v[k]));
      vkey = min(vkey, __float_as_uint(v[k]) - 1u);
    }
    float bmax = grp_max(__uint_as_float(vmaxb), VL < 64 ? VL : 64);
    uint32_t bkey = vkey;
    for (int o = 1; o < (VL < 64 ? VL : 64); o <<= 1) bkey = min(bkey, (uint32_t)__shfl_xor((int)bkey, o, 64));
    if (VL > 64) {
      if ((lane & 63) == 0) { xw[wave * 2] = bmax; xw[wave * 2 + 1] = __uint_as_float(bkey); }
      __syncthreads();
      const int wpb = VL >> 6, w0 = (wave / wpb) * wpb;
      bmax = xw[w0 * 2];
      bkey = __float_as_uint(xw[w0 * 2 + 1]);
      for (int w = 1; w < wpb; ++w) {
        bmax = fmaxf(bmax, xw[(w0 + w) * 2]);
        bkey = min(bkey, __float_as_uint(xw[(w0 + w) * 2 + 1]));
      }
    }
    const float mnz = (bkey == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey + 1u);
    constexpr int LM2 = VB == 8 ? 254 : 65534;
    const ALFit f = al_refit(bmax, mnz, a.floor_, (float)LM2);
    if (v_ok) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t code = al_finish<LM2>(v[k], al_round_exact<LM2>(v[k], f));
        if constexpr (VB == 8) gp(reinterpret_cast<uint8_t*>(a.v_q))[e0 + k] = (uint8_t)code;
        else gp(reinterpret_cast<uint16_t*>(a.v_q))[e0 + k] = (uint16_t)code;
      }
      if ((lane & (VL - 1)) == 0) { gp(a.v_scale)[vb] = f.s; gp(a.v_min_log)[vb] = f.lmin; }
    }
  }
  // ---- M state
  if constexpr (MK == 3) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) gp(a.m_fp32)[e0 + k] = m[k];
  } else if constexpr (MK != 0) {
    uint32_t ab = 0u;
#pragma unroll
    for (int k = 0; k < 8; ++k) ab = max(ab, __float_as_uint(m[k]) & 0x7FFFFFFFu);
    float bam = grp_max(__uint_as_float(ab), ML < 64 ? ML : 64);
    if (ML > 64) {
      __syncthreads();
      if ((lane & 63) == 0) xw[8 + wave] = bam;
      __syncthreads();
      const int wpb = ML >> 6, w0 = (wave / wpb) * wpb;
      bam = xw[8 + w0];
      for (int w = 1; w < wpb; ++w) bam = fmaxf(bam, xw[8 + w0 + w]);
    }
    if (m_ok) {
      const float am = fmaxf(bam, 1e-12f);
      const float ram = fast_rcp(am);
      if (mk == 2 || mk == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t hi = m_encode(mk, m[2 * j], am, ram);
          const uint32_t lo = m_encode(mk, m[2 * j + 1], am, ram);
          w |= ((hi << 4) | lo) << (8 * j);
        }
        *gp(reinterpret_cast<uint32_t*>(a.m_q + (e0 >> 1))) = w;
      } else {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w0 |= m_encode(mk, m[k], am, ram) << (8 * k);
#pragma unroll
        for (int k = 0; k < 4; ++k) w1 |= m_encode(mk, m[k + 4], am, ram) << (8 * k);
        *gp(reinterpret_cast<u32x2*>(a.m_q + e0)) = u32x2{w0, w1};
      }
      if ((lane & (ML - 1)) == 0) gp(a.m_scale)[mb] = am;
    }
  }
}

// ------------------------------------------------------------ scale
// s_ch = ||u_ch|| / (||g_low_ch|| + 1e-8) (optimizer.py:2997-3001): right side one
// wave per row of g_low, left side one lane per column walking the r rows;
// norms as sqrt of fp32 sums accumulated in double.  Partials per workgroup:
// channel sum(ngsq * s^2); tensor sum(u^2), sum(g_low^2).
__global__ __launch_bounds__(256) void k_ap_scale(ApArgs a) {
  __shared__ double sd[4];
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  const int64_t R = a.R, C = a.C, r = a.r;
  const bool right = R >= C;
  float* ws = a.ws;
  const int lane = threadIdx.x, wave = lane >> 6, wl = lane & 63;
  double acc0 = 0.0, acc1 = 0.0;
  if (!a.channel) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + lane; i < W.n_low; i += (int64_t)gridDim.x * 256) {
      const float u = gp(ws)[W.u + i], g = gp(ws)[W.glow + i];
      acc0 += (double)(u * u);
      acc1 += (double)(g * g);
    }
  } else if (right) {
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < R; row += (int64_t)gridDim.x * 4) {
      double su = 0.0, sg = 0.0;
      for (int64_t k = wl; k < r; k += 64) {
        const float u = gp(ws)[W.u + row * r + k], g = gp(ws)[W.glow + row * r + k];
        su += (double)(u * u);
        sg += (double)(g * g);
      }
      su = grp_sum_d(su, 64);
      sg = grp_sum_d(sg, 64);
      if (wl == 0) {
        float s = sqrtf((float)su) / (sqrtf((float)sg) + 1e-8f);
        if (a.front) s = s * a.sv;
        gp(ws)[W.fin + row] = s;
        const float ng = gp(ws)[W.ngsq + row];
        acc0 += (double)(ng * (s * s));
      }
    }
  } else {
    for (int64_t c = (int64_t)blockIdx.x * 256 + lane; c < C; c += (int64_t)gridDim.x * 256) {
      double gc = 0.0;
      for (int64_t q = 0; q < W.nrc; ++q) gc += ws_d(ws, W.gcol, q * C + c);
      const float gn = sqrtf((float)gc);
      gp(ws)[W.ngsq + c] = gn * gn;
      double su = 0.0, sg = 0.0;
      for (int64_t k = 0; k < r; ++k) {
        const float u = gp(ws)[W.u + k * C + c], g = gp(ws)[W.glow + k * C + c];
        su += (double)(u * u);
        sg += (double)(g * g);
      }
      float s = sqrtf((float)su) / (sqrtf((float)sg) + 1e-8f);
      if (a.front) s = s * a.sv;
      gp(ws)[W.fin + c] = s;
      const float ng = gp(ws)[W.ngsq + c];
      acc0 += (double)(ng * (s * s));
    }
  }
  const double t0 = ap_wg_sum(acc0, sd);
  const double t1 = ap_wg_sum(acc1, sd);
  if (lane == 0) {
    ws_d_set(ws, W.spart, blockIdx.x, t0);
    ws_d_set(ws, W.spart, kApNP + blockIdx.x, t1);
  }
}

// ------------------------------------------------------------ per-tensor scalars
// One workgroup: alpha (optimizer.py:832-856), norm_unscaled and Fira on it
// (optimizer.py:3003-3024, 760-782 with the key scaled_grad_norm_prev), the
// final channel scales s * fira (* sqrt(apollo_scale) at the back), the RMS
// denominator, the step -alpha/denom with bias correction, and the decay.
__global__ __launch_bounds__(256) void k_ap_scalars(ApArgs a) {
  __shared__ double sd[4];
  __shared__ float sh[2];
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  float* ws = a.ws;
  const int lane = threadIdx.x;
  double pg = 0.0, pp = 0.0, s0 = 0.0, s1 = 0.0;
  for (int k = lane; k < a.ngn; k += 256) { pg += ws_d(ws, W.gpart, k); pp += ws_d(ws, W.ppart, k); }
  for (int k = lane; k < a.nsc; k += 256) { s0 += ws_d(ws, W.spart, k); s1 += ws_d(ws, W.spart, kApNP + k); }
  pg = ap_wg_sum(pg, sd);
  pp = ap_wg_sum(pp, sd);
  s0 = ap_wg_sum(s0, sd);
  s1 = ap_wg_sum(s1, sd);
  const int64_t numel = a.R * a.C;
  if (lane == 0) {
    const float rho = a.lr ? *gp(a.lr) : a.lr_val;
    float alpha = rho;
    if (a.scale_param) {
      const float rms = sqrtf((float)pp) / (float)sqrt((double)numel);
      alpha = fmaxf(rms, a.eps2) * rho;
    }
    float s_t = 1.0f;                 // tensor scale
    float nun;                        // norm_unscaled
    if (a.channel) {
      nun = sqrtf((float)s0);
    } else {
      s_t = sqrtf((float)s0) / (sqrtf((float)s1) + 1e-8f);
      if (a.front) s_t = s_t * a.sv;
      nun = sqrtf((float)pg) * s_t;
    }
    float fs = 1.0f;
    if (a.fira) {
      const float curr = __builtin_isfinite(nun) ? nun : 0.0f;
      float next = curr;
      if (a.has_fira_prev) {
        const float p = *gp(a.fira_prev);
        const float ratio = curr / (p + 1e-8f);
        const float lim = (ratio != ratio ? ratio : fmaxf(ratio, a.margin)) / a.margin;
        const bool reset = p < 1e-6f;
        fs = reset ? 1.0f : 1.0f / lim;
        next = reset ? curr : curr * fs;
      }
      *gp(a.fira_prev) = next;
    }
    float denom = 1.0f;
    if (a.d > 0.0f) denom = fmaxf(nun / (float)(sqrt((double)numel) * (double)a.d), 1.0f);
    float step = -alpha / denom;
    if (a.bias_mode == 1) step = step * a.bias_factor;
    else if (a.bias_mode == 2) step = step / a.bias_factor;
    float dec = 1.0f;
    if (a.wd_mode == 1) dec = 1.0f - alpha * a.wd;
    else if (a.wd_mode == 2) dec = 1.0f - rho * a.wd;
    float fin_t = s_t;
    if (a.fira) fin_t = fin_t * fs;
    if (!a.front) fin_t = fin_t * a.sv;
    float* sl = ws + W.scal;
    gp(sl)[0] = step;
    gp(sl)[1] = dec;
    gp(sl)[3] = fin_t;
    gp(sl)[4] = alpha;
    gp(sl)[5] = nun;
    gp(sl)[6] = fs;
    sh[0] = fs;
  }
  __syncthreads();
  if (a.channel) {
    const float fs = sh[0];
    for (int64_t c = lane; c < W.nch; c += 256) {
      float f = gp(ws)[W.fin + c];
      if (a.fira) f = f * fs;
      if (!a.front) f = f * a.sv;
      gp(ws)[W.fin + c] = f;
    }
  }
}

// ------------------------------------------------------------ full-rank writeback
// Deterministic (optimizer.py:3071-3077): p := p * decay (rounded to T), then
// channel p + (step * G) * f_ch (addcmul) or tensor fma(step * f, G, p) (add_),
// rounded to T.  SR (optimizer.py:3058-3063 with the stream of kernels.cu:48-87):
// x = (p * decay) + (G * f) * step in fp32, stochastically rounded.
template <typename T, bool SR>
__global__ __launch_bounds__(256) void k_ap_apply(ApArgs a) {
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  const int64_t R = a.R, C = a.C, n = R * C;
  const bool right = R >= C;
  const float* ws = a.ws;
  const float* sl = ws + W.scal;
  const float step = gp(sl)[0], dec = gp(sl)[1], fin_t = gp(sl)[3];
  const bool has_dec = a.wd_mode != 0;
  T* P = reinterpret_cast<T*>(a.param);
  const T* G = reinterpret_cast<const T*>(a.grad);
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= n) return;
  float g[8], p[8];
  load8<T>(G, e0, n, g);
  if constexpr (!SR) load8<T>(P, e0, n, p);
  int64_t row = e0 / C;
  int64_t col = e0 - row * C;
  const float ts = step * fin_t;   // tensor: alpha = step * final_scale
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (e0 + k < n) {
      const float gk = scrub(g[k]);
      const float f = a.channel ? gp(ws)[W.fin + (right ? row : col)] : fin_t;
      if constexpr (SR) {
        float x = ld1<T>(P, e0 + k);
        if (has_dec) x = x * dec;
        x = x + (gk * f) * step;
        const T rr = sr_round<T>(x, a.sr_seed, a.sr_step, (uint64_t)(e0 + k));
        uint16_t bits;
        __builtin_memcpy(&bits, &rr, 2);
        gp(reinterpret_cast<uint16_t*>(P))[e0 + k] = bits;
      } else {
        float x = p[k];
        if (has_dec) x = to_f<T>(from_f<T>(x * dec));
        if (a.channel) x = x + (step * gk) * f;
        else x = __builtin_fmaf(ts, gk, x);
        p[k] = x;
      }
    }
    if (++col == C) { col = 0; ++row; }
  }
  if constexpr (!SR) store8<T>(P, e0, n, p);
}

hipError_t apollo_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

// ------------------------------------------------------------ rocBLAS
static rocblas_handle g_blas[64];

static int blas_handle(rocblas_handle* out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(A8_ERR_HIP, "hipGetDevice");
  if (!g_blas[dev]) {
    if (rocblas_create_handle(&g_blas[dev]) != rocblas_status_success)
      return set_error(A8_ERR_HIP, "rocblas_create_handle failed");
    rocblas_set_pointer_mode(g_blas[dev], rocblas_pointer_mode_host);
  }
  *out = g_blas[dev];
  return 0;
}

// g_low = G P^T (right) or P^T G (left), row-major, through column-major GEMMs:
// right: g_low^T (r x R) = PT^T (r x C) . G^T (C x R); left: g_low^T (C x r) = G^T . PT^T.
static int ap_gemm(rocblas_handle hb, int dtype, const ApArgs& a, const ApWs& W, const float* pt,
                   int split_fresh, hipStream_t st) {
  const bool right = a.R >= a.C;
  const int64_t R = a.R, C = a.C, r = a.r;
  float* glow = a.ws + W.glow;
  const float one = 1.0f, zero = 0.0f;
  rocblas_set_stream(hb, st);
  if (dtype == A8_F32) {
    rocblas_status s;
    if (right)
      s = rocblas_sgemm(hb, rocblas_operation_none, rocblas_operation_none, (rocblas_int)r, (rocblas_int)R,
                        (rocblas_int)C, &one, pt, (rocblas_int)r, reinterpret_cast<const float*>(a.grad),
                        (rocblas_int)C, &zero, glow, (rocblas_int)r);
    else
      s = rocblas_sgemm(hb, rocblas_operation_none, rocblas_operation_none, (rocblas_int)C, (rocblas_int)r,
                        (rocblas_int)R, &one, reinterpret_cast<const float*>(a.grad), (rocblas_int)C, pt,
                        (rocblas_int)R, &zero, glow, (rocblas_int)C);
    return s == rocblas_status_success ? 0 : set_error(A8_ERR_HIP, "rocblas_sgemm failed");
  }
  // bf16 G: three bf16 GEMMs against the split P^T, accumulated in fp32
  __hip_bfloat16* sp = reinterpret_cast<__hip_bfloat16*>(a.ws + W.split);
  const int64_t np = r * W.K;
  if (split_fresh) {
    const int64_t nb = (np + 255) / 256;
    hipLaunchKernelGGL(k_ap_split, dim3((unsigned)(nb < 4096 ? nb : 4096)), dim3(256), 0, st, pt, np, sp);
    int rc = check_launch("k_ap_split");
    if (rc) return rc;
  }
  for (int t = 0; t < 3; ++t) {
    const void* pterm = sp + t * np;
    const float* beta = t == 0 ? &zero : &one;
    rocblas_status s;
    if (right)
      s = rocblas_gemm_ex(hb, rocblas_operation_none, rocblas_operation_none, (rocblas_int)r, (rocblas_int)R,
                          (rocblas_int)C, &one, pterm, rocblas_datatype_bf16_r, (rocblas_int)r, a.grad,
                          rocblas_datatype_bf16_r, (rocblas_int)C, beta, glow, rocblas_datatype_f32_r,
                          (rocblas_int)r, glow, rocblas_datatype_f32_r, (rocblas_int)r, rocblas_datatype_f32_r,
                          rocblas_gemm_algo_standard, 0, 0);
    else
      s = rocblas_gemm_ex(hb, rocblas_operation_none, rocblas_operation_none, (rocblas_int)C, (rocblas_int)r,
                          (rocblas_int)R, &one, a.grad, rocblas_datatype_bf16_r, (rocblas_int)C, pterm,
                          rocblas_datatype_bf16_r, (rocblas_int)R, beta, glow, rocblas_datatype_f32_r,
                          (rocblas_int)C, glow, rocblas_datatype_f32_r, (rocblas_int)C, rocblas_datatype_f32_r,
                          rocblas_gemm_algo_standard, 0, 0);
    if (s != rocblas_status_success) return set_error(A8_ERR_HIP, "rocblas_gemm_ex (bf16) failed");
  }
  return 0;
}

template <int VB>
static void launch_low(int mkt, unsigned nb, const ApArgs& a, hipStream_t st) {
  switch (mkt) {
    case 0: hipLaunchKernelGGL((k_ap_low<VB, 0>), dim3(nb), dim3(256), 0, st, a); break;
    case 1: hipLaunchKernelGGL((k_ap_low<VB, 1>), dim3(nb), dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL((k_ap_low<VB, 3>), dim3(nb), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((k_ap_low<VB, 2>), dim3(nb), dim3(256), 0, st, a); break;
  }
}

}  // namespace a8

using namespace a8;

extern "C" {

int64_t a8_apollo_workspace_floats(int64_t rows, int64_t cols, int64_t rank, int channel) {
  if (rows <= 0 || cols <= 0 || rank <= 0) return 0;
  return ap_layout(rows, cols, rank, channel ? 1 : 0).total;
}

int a8_apollo_step(int dtype, int stochastic, const a8_apollo_tensor* t, int first_step, int proj_fresh,
                   double beta_val, double beta1, int has_m, float apollo_eps, float log_floor, int v_bits,
                   int block_size, int m_bits, int m_mode, int m_fp32, int m_block_size, int channel,
                   float apollo_scale, int scale_front, int fira, float fira_margin, float d, float lr_val,
                   float eps2, int scale_parameter, int bias_mode, float bias_factor, float weight_decay,
                   int wd_mode, uint64_t sr_step, void* stream) {
  if (!t || !t->param || !t->grad || !t->proj_t || !t->workspace) return set_error(A8_ERR_ARG, "null pointer");
  if (dtype != A8_F32 && dtype != A8_BF16) return set_error(A8_ERR_DTYPE, "APOLLO supports fp32 and bf16 params");
  if (t->rows <= 0 || t->cols <= 0 || t->rank <= 0) return set_error(A8_ERR_SIZE, "empty APOLLO tensor");
  if (t->rows * t->cols >= ((int64_t)1 << 31)) return set_error(A8_ERR_SIZE, "APOLLO tensor too large");
  if (v_bits != 0 && v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 0, 8 or 16");
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  if (v_bits && !(pow2(block_size) && block_size >= 128 && block_size <= 2048))
    return set_error(A8_ERR_BLOCK, "APOLLO V block_size must be a power of two in [128, 2048]");
  if (has_m && !m_fp32 && !(pow2(m_block_size) && m_block_size >= 32 && m_block_size <= 2048))
    return set_error(A8_ERR_BLOCK, "APOLLO m_block_size must be a power of two in [32, 2048]");
  if (v_bits ? !(t->v_q && t->v_scale && t->v_min_log) : !t->v_fp32)
    return set_error(A8_ERR_ARG, "APOLLO V state missing");
  if (has_m && (m_fp32 ? !t->m_fp32 : !(t->m_q && t->m_scale))) return set_error(A8_ERR_ARG, "APOLLO M state missing");
  if (fira && !t->fira_prev) return set_error(A8_ERR_ARG, "APOLLO Fira needs scaled_grad_norm_prev");
  if ((reinterpret_cast<uintptr_t>(t->param) | reinterpret_cast<uintptr_t>(t->grad)) & 15)
    return set_error(A8_ERR_ARG, "APOLLO param and grad must be 16-byte aligned");
  if (stochastic && dtype == A8_F32) stochastic = 0;
  hipStream_t st = (hipStream_t)stream;
  ApArgs a{};
  a.param = t->param; a.grad = t->grad; a.R = t->rows; a.C = t->cols; a.r = t->rank;
  a.v_q = t->v_q; a.v_scale = t->v_scale; a.v_min_log = t->v_min_log; a.v_fp32 = t->v_fp32;
  a.m_q = t->m_q; a.m_scale = t->m_scale; a.m_fp32 = t->m_fp32;
  a.fira_prev = t->fira_prev; a.has_fira_prev = t->has_fira_prev; a.lr = t->lr; a.ws = t->workspace;
  a.sr_seed = t->sr_seed; a.sr_step = sr_step;
  a.bv = (float)beta_val; a.w_m = (float)(1.0 - beta1); a.aeps = apollo_eps;
  a.floor_ = first_step ? -126.0f : log_floor;
  a.lr_val = lr_val; a.eps2 = eps2; a.bias_factor = bias_factor; a.bias_mode = bias_mode;
  a.wd = weight_decay; a.wd_mode = wd_mode; a.d = d; a.margin = (float)(1.0 + (double)fira_margin);
  a.sv = (float)sqrt((double)apollo_scale);
  a.first = first_step; a.has_m = has_m; a.vb = v_bits; a.channel = channel ? 1 : 0; a.front = scale_front;
  a.fira = fira; a.scale_param = scale_parameter;
  int lbv = 0, lbm = 0;
  while ((1 << lbv) < (v_bits ? block_size : 2048)) ++lbv;
  while ((1 << lbm) < ((has_m && !m_fp32) ? m_block_size : 32)) ++lbm;
  a.lbv = lbv; a.lbm = lbm;
  a.mk = has_m && !m_fp32 ? (m_mode == 0 ? (m_bits == 8 ? 1 : 2) : (m_bits == 8 ? 3 : 4)) : 0;
  const ApWs W = ap_layout(a.R, a.C, a.r, a.channel);
  const bool right = a.R >= a.C;
  int64_t ngn = right ? (a.R + 3) / 4 : W.ncc * W.nrc;
  ngn = ngn < kApNP ? ngn : kApNP;
  int64_t nsc = !a.channel ? (W.n_low + 255) / 256 : (right ? (a.R + 3) / 4 : (a.C + 255) / 256);
  nsc = nsc < kApNP ? nsc : kApNP;
  a.ngn = (int)ngn; a.nsc = (int)nsc;
  a.valign = (a.C % (dtype == A8_F32 ? 4 : 8)) == 0 ? 1 : 0;

  rocblas_handle hb;
  int rc = blas_handle(&hb);
  if (rc) return rc;
  if ((rc = ap_gemm(hb, dtype, a, W, t->proj_t, proj_fresh, st))) return rc;
  const dim3 ggn = right ? dim3((unsigned)ngn) : dim3((unsigned)W.ncc, (unsigned)W.nrc);
  if (dtype == A8_F32) hipLaunchKernelGGL((k_ap_gnorm<float>), ggn, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((k_ap_gnorm<__hip_bfloat16>), ggn, dim3(256), 0, st, a);
  if ((rc = check_launch("k_ap_gnorm"))) return rc;
  {
    const int64_t nf = (W.n_low + 255) / 256;
    const unsigned nfb = (unsigned)(nf < 1024 ? nf : 1024);
    if (dtype == A8_F32) hipLaunchKernelGGL((k_ap_fixlow<float>), dim3(nfb), dim3(256), 0, st, a, t->proj_t);
    else hipLaunchKernelGGL((k_ap_fixlow<__hip_bfloat16>), dim3(nfb), dim3(256), 0, st, a, t->proj_t);
    if ((rc = check_launch("k_ap_fixlow"))) return rc;
  }
  const unsigned nlow = (unsigned)((W.n_low + kApUnit - 1) / kApUnit);
  const int mkt = !has_m ? 0 : (m_fp32 ? 3 : (a.mk == 1 ? 1 : 2));
  if (v_bits == 8) launch_low<8>(mkt, nlow, a, st);
  else if (v_bits == 16) launch_low<16>(mkt, nlow, a, st);
  else launch_low<0>(mkt, nlow, a, st);
  if ((rc = check_launch("k_ap_low"))) return rc;
  hipLaunchKernelGGL(k_ap_scale, dim3((unsigned)nsc), dim3(256), 0, st, a);
  if ((rc = check_launch("k_ap_scale"))) return rc;
  hipLaunchKernelGGL(k_ap_scalars, dim3(1), dim3(256), 0, st, a);
  if ((rc = check_launch("k_ap_scalars"))) return rc;
  const unsigned napp = (unsigned)((a.R * a.C + 2047) / 2048);
  if (dtype == A8_F32) hipLaunchKernelGGL((k_ap_apply<float, false>), dim3(napp), dim3(256), 0, st, a);
  else if (stochastic) hipLaunchKernelGGL((k_ap_apply<__hip_bfloat16, true>), dim3(napp), dim3(256), 0, st, a);
  else hipLaunchKernelGGL((k_ap_apply<__hip_bfloat16, false>), dim3(napp), dim3(256), 0, st, a);
  return check_launch("k_ap_apply");
}

}  // extern "C"
