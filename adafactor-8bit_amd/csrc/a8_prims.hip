// Stand-alone step primitives of the reference's module (gfx950).
//
// The reference's optimizer drives its factored, CAME and APOLLO steps as
// sequences of small kernels (kernels.cu:340-480, 1523-2440, 2638-3000).  This
// build's own optimizer fuses those sequences (a8_factored.hip, a8_apollo.hip);
// the kernels here give the same primitives one by one, so the reference's
// optimizer can run on this library through the reference-named module.
//
// Arithmetic follows the reference's PyTorch twins of each primitive:
//   V EMA        lerp(deq(v), x, beta) with x = g^2 + eps1 when squared, AL codes
//                refit per block from the non-zero values (optimizer.py:2232-2238)
//   2-D update   inv_row = 1/sqrt(row / row_mean), inv_col = 1/sqrt(col),
//                u = (x * inv_row) * inv_col with x = lerp(m, g, 1 - beta1) or g,
//                p = fma(-step, u, p)                (optimizer.py:818-821, 958-970)
//   CAME         U = ((g * inv_row) * inv_col) / clip, M = lerp(M, U, 1 - beta1),
//                res = (U - M)^2 + eps_came; update (M * inv_crow) * inv_ccol with
//                the confidence factors              (optimizer.py:929-956)
// and the reference's kernels where no twin exists (APOLLO norms and writeback,
// kernels.cu:2410-2570, 2638-3000).
//
// Layout: the element kernels give each lane 8 consecutive elements and a
// 256-lane workgroup 2048, a whole number of momentum blocks; the row / column
// of each element is stepped from the lane's first element.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

constexpr int kPElems = 2048;

// ============================================================ V EMA
// One 2048-element unit (unit index bid) of the EMA; xw: 8 floats and dtab:
// 4 * 256 floats of LDS.  dec, when given, receives the decoded new codes (what
// dequantize_log_nonneg would read back).  AL8 blocks of >= 512 elements decode
// through a table of their 255 values (one correctly rounded exp2 per lane and
// block instead of one per element); the new codes take the fast AL8 argument
// with exact re-decision near rounding boundaries.
// XREG: the lane's eight inputs come in registers (xreg) instead of from x, and
// the decoded new codes are returned in dvr (every lane reaches the barriers).
template <int VB, typename T, bool XREG = false>
__device__ __forceinline__ void vema_unit(void* __restrict__ q, float* __restrict__ scale,
                                          float* __restrict__ min_log, const T* __restrict__ x,
                                          float* __restrict__ out, float* __restrict__ dec, int64_t n, int64_t nblk,
                                          int64_t bid, int lbv, float w, int square, float eps1, float floor_,
                                          float* xw, float* dtab, const float* xreg = nullptr,
                                          float* dvr = nullptr) {
  const int lane = threadIdx.x, wave = lane >> 6;
  const int64_t e0 = bid * kPElems + (int64_t)lane * 8;
  const int VL = (1 << lbv) >> 3;
  const int64_t vb = e0 >> lbv;
  const bool v_ok = vb < nblk;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);
  constexpr float LM2 = VB == 8 ? 254.0f : 65534.0f;
  float xv[8];
  if constexpr (XREG) {
#pragma unroll
    for (int k = 0; k < 8; ++k) xv[k] = xreg[k];
  } else {
    load8<T>(x, e0, n, xv);
  }
  float v[8];
  const float s_old = v_ok ? gp(scale)[vb] : 0.0f, lm_old = v_ok ? gp(min_log)[vb] : 0.0f;
  // The lane's eight codes in one 8- or 16-byte access, issued with the loads
  // above (before the decode table's barrier).  Codes are padded to whole blocks,
  // so a lane of an existing block reads all eight.
  const bool cvec = v_ok && ((reinterpret_cast<uintptr_t>(q) & 15) == 0);
  uint32_t cq[VB == 8 ? 2 : 4];
#pragma unroll
  for (int i = 0; i < (VB == 8 ? 2 : 4); ++i) cq[i] = 0u;
  if (cvec) {
    if constexpr (VB == 8) {
      const u32x2 t = *gp(reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(q) + e0));
      cq[0] = t.x; cq[1] = t.y;
    } else {
      const u32x4 t = *gp(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(q) + e0));
      cq[0] = t.x; cq[1] = t.y; cq[2] = t.z; cq[3] = t.w;
    }
  }
  const bool tab8 = VB == 8 && VL >= 64;   // uniform
  const int bw = tab8 ? lane / VL : 0;     // block slot of this lane in the unit
  if (tab8) {
    for (int c = lane % VL; c < 256; c += VL)
      dtab[bw * 256 + c] = c ? exp2_exact(((float)(c - 1) * s_old) / LM2 + lm_old) : 0.0f;
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float xi = xv[k];
    if (square) xi = xi * xi + eps1;
    xi = scrub(xi);
    float vo = 0.0f;
    if (k < cnt) {
      uint32_t c;
      if (cvec) c = VB == 8 ? (cq[k >> 2] >> (8 * (k & 3))) & 0xFFu : (cq[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
      else if constexpr (VB == 8) c = gp(reinterpret_cast<const uint8_t*>(q))[e0 + k];
      else c = gp(reinterpret_cast<const uint16_t*>(q))[e0 + k];
      vo = tab8 ? dtab[bw * 256 + c] : (c ? exp2_exact(((float)(c - 1) * s_old) / LM2 + lm_old) : 0.0f);
    }
    v[k] = (k < cnt) ? lerp_ref(vo, xi, w) : 0.0f;   // padding quantises as zero
  }
  if (out) store8<float>(out, e0, n, v);
  uint32_t vmaxb = 0u, vkey = 0xFFFFFFFFu;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    vmaxb = max(vmaxb, __float_as_uint(v[k]));
    vkey = min(vkey, __float_as_uint(v[k]) - 1u);   // zero wraps to the largest key
  }
  const int G = VL < 64 ? VL : 64;
  float bmax = grp_max(__uint_as_float(vmaxb), G);
  uint32_t bkey = vkey;
  bkey = grp_umin(bkey, G);
  if (VL > 64) {
    if ((lane & 63) == 0) { xw[wave * 2] = bmax; xw[wave * 2 + 1] = __uint_as_float(bkey); }
    __syncthreads();
    const int wpb = VL >> 6, w0 = (wave / wpb) * wpb;
    bmax = xw[w0 * 2];
    bkey = __float_as_uint(xw[w0 * 2 + 1]);
    for (int ww = 1; ww < wpb; ++ww) {
      bmax = fmaxf(bmax, xw[(w0 + ww) * 2]);
      bkey = min(bkey, __float_as_uint(xw[(w0 + ww) * 2 + 1]));
    }
  }
  // every lane stays to the end (the read-back table below has barriers); lanes
  // past the last block store nothing
  const float mnz = (bkey == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey + 1u);
  constexpr int L2 = VB == 8 ? 254 : 65534;
  const ALFit f = al_refit_pair(bmax, mnz, floor_, (float)L2, lane);   // a block spans >= 16 lanes
  uint32_t code[8];
  al_codes<L2, 8>(v, f, code);
  if (cvec) {
    if constexpr (VB == 8) {
      *gp(reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(q) + e0)) =
          u32x2{code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24),
                code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24)};
    } else {
      *gp(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(q) + e0)) =
          u32x4{code[0] | (code[1] << 16), code[2] | (code[3] << 16), code[4] | (code[5] << 16),
                code[6] | (code[7] << 16)};
    }
  } else if (v_ok) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (VB == 8) gp(reinterpret_cast<uint8_t*>(q))[e0 + k] = (uint8_t)code[k];
      else gp(reinterpret_cast<uint16_t*>(q))[e0 + k] = (uint16_t)code[k];
    }
  }
  if (dec || XREG) {   // uniform
    float dv[8];
    if (tab8) {   // the new fit's table, after every lane has read the old one
      __syncthreads();
      for (int c = lane % VL; c < 256; c += VL)
        dtab[bw * 256 + c] = c ? exp2_exact(((float)(c - 1) * f.s) / LM2 + f.lmin) : 0.0f;
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 8; ++k) dv[k] = dtab[bw * 256 + code[k]];
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        dv[k] = code[k] ? exp2_exact(((float)(code[k] - 1) * f.s) / LM2 + f.lmin) : 0.0f;
    }
    if (dec && v_ok) store8<float>(dec, e0, n, dv);
    if constexpr (XREG) {
#pragma unroll
      for (int k = 0; k < 8; ++k) dvr[k] = dv[k];
    }
  }
  if (v_ok && (lane & (VL - 1)) == 0) { gp(scale)[vb] = f.s; gp(min_log)[vb] = f.lmin; }
}

template <int VB, typename T>
__global__ __launch_bounds__(256) void k_vema(void* __restrict__ q, float* __restrict__ scale,
                                              float* __restrict__ min_log, const T* __restrict__ x,
                                              float* __restrict__ out, int64_t n, int64_t nblk, int lbv, float w,
                                              int square, float eps1, float floor_) {
  __shared__ float xw[8];
  __shared__ float dtab[4 * 256];
  vema_unit<VB, T>(q, scale, min_log, x, out, nullptr, n, nblk, (int64_t)blockIdx.x, lbv, w, square, eps1, floor_,
                   xw, dtab);
}

// Table form: one launch over several tensors, each a run of whole units.
struct VemaDesc {
  void* q;
  float* scale;
  float* min_log;
  const float* x;
  float* out;
  float* dec;
  int64_t n, nblk, wg_begin;
};

template <int VB>
__global__ __launch_bounds__(256) void k_vema_multi(VemaDesc one, const VemaDesc* __restrict__ tab, int ntab,
                                                    int lbv, float w, int square, float eps1, float floor_,
                                                    const a8_step_scalars* w_dev) {
  if (w_dev) w = (float)load_step_scalars(w_dev).beta_val;   // the device step's V weight
  __shared__ float xw[8];
  __shared__ float dtab[4 * 256];
  const int64_t wg = blockIdx.x;
  int lo = 0;
  if (tab) {
    int hi = ntab - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tab[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
    }
  }
  const VemaDesc d = tab ? tab[lo] : one;
  vema_unit<VB, float>(d.q, d.scale, d.min_log, d.x, d.out, d.dec, d.n, d.nblk, wg - d.wg_begin, lbv, w, square,
                       eps1, floor_, xw, dtab);
}

// ============================================================ factored element kernel
enum { F_NOCLIP = 0, F_NORM = 1, F_APPLY = 2, F_LAG = 3, F_SUMS = 4, F_CAME1 = 5, F_CAME2N = 6, F_CAME2 = 7 };

struct F2 {
  void* param;
  const void* grad;
  uint8_t* m_q;
  float* m_scale;
  float* m;
  const float* row;       // b*R + r
  const float* col;       // b*C + c
  const float* rmean;     // b
  const float* crow;
  const float* ccol;
  const float* crmean;
  float* row_sum;
  float* col_sum;
  float* norm_buf;
  const float* alpha;
  const float* prev_norm;
  const float* decay;
  const float* clip;
  int64_t R, C, n;
  uint64_t sr_seed, sr_step;
  float w_m;        // (float)(1 - beta1)
  float eps_came;
  float d;
  float sqrt_nd;    // (float)(sqrt(n) * d)
  float sqrt_nf;    // sqrtf((float)n): the CUDA kernels' sqrt_numel (the lagged clip)
  int mq;           // momentum: 0 none, 1 quantised, 2 fp32
  int mk;           // codec of quantised momentum (1 UF8, 2 UF4, 3 D8, 4 D4)
  int lbm;          // log2 of the momentum block
  int sr;
};

template <typename T>
__device__ __forceinline__ void f2_write(const F2& a, int64_t e0, int cnt, float step, const float* u) {
  float p[8];
  load8<T>(reinterpret_cast<const T*>(a.param), e0, a.n, p);
  if (a.sr) {
    const float dec = a.decay ? *a.decay : 1.0f;
    T* P = reinterpret_cast<T*>(a.param);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) P[e0 + k] = sr_round<T>(__builtin_fmaf(-step, u[k], p[k] * dec), a.sr_seed, a.sr_step,
                                           (uint64_t)(e0 + k));
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) p[k] = __builtin_fmaf(-step, u[k], p[k]);
    store8<T>(reinterpret_cast<T*>(a.param), e0, a.n, p);
  }
}

__device__ __forceinline__ void f2_sum_add(float* buf, float v) {
  const float t = grp_sum(v, 64);
  if ((threadIdx.x & 63) == 0 && t != 0.0f) atomicAdd(buf, t);
}

// Row sums: one atomic per row segment of the lane; column sums: one per element.
__device__ __forceinline__ void f2_rowcol_add(const F2& a, int cnt, const int64_t* ri, const int64_t* ci,
                                              const float* val) {
  float acc = 0.0f;
  int64_t cur = ri[0];
  for (int k = 0; k < cnt; ++k) {
    if (ri[k] != cur) {
      atomicAdd(a.row_sum + cur, acc);
      acc = 0.0f;
      cur = ri[k];
    }
    acc += val[k];
    atomicAdd(a.col_sum + ci[k], val[k]);
  }
  if (cnt > 0) atomicAdd(a.row_sum + cur, acc);
}

template <typename T, int OP>
__global__ __launch_bounds__(256) void k_f2d(F2 a) {
  __shared__ float xw[4];
  const int lane = threadIdx.x;
  const int64_t n = a.n;
  const int64_t e0 = (int64_t)blockIdx.x * kPElems + (int64_t)lane * 8;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);

  // row (b*R + r), column (b*C + c) and batch of each element
  int64_t ri[8], ci[8], bi[8];
  {
    const int64_t RC = a.R * a.C;
    const int64_t s = e0 < n ? e0 : 0;
    int64_t b = s / RC, r = (s - b * RC) / a.C, c = s - b * RC - r * a.C;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      ri[k] = b * a.R + r; ci[k] = b * a.C + c; bi[k] = b;
      if (++c == a.C) { c = 0; if (++r == a.R) { r = 0; ++b; } }
    }
  }
  const bool need_g = !((OP == F_CAME2N || OP == F_CAME2) && a.mq == 2);
  float g[8];
  if (need_g) {
    load8<T>(reinterpret_cast<const T*>(a.grad), e0, n, g);
#pragma unroll
    for (int k = 0; k < 8; ++k) g[k] = scrub(g[k]);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) g[k] = 0.0f;
  }

  if constexpr (OP == F_SUMS) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = g[k] * g[k];
    f2_rowcol_add(a, cnt, ri, ci, v);
    return;
  }

  // x: what the momentum averages (g, or U = ((g * inv_row) * inv_col) / clip for CAME)
  float x[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = g[k];
  if constexpr (OP == F_CAME1 || OP == F_CAME2N || OP == F_CAME2) {
    if (need_g) {
      const float clip = a.clip ? *a.clip : 1.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k < cnt) {
          const float ir = 1.0f / sqrtf(gp(a.row)[ri[k]] / gp(a.rmean)[bi[k]]);
          const float ic = 1.0f / sqrtf(gp(a.col)[ci[k]]);
          x[k] = ((g[k] * ir) * ic) / clip;
        }
      }
    }
  }

  // momentum
  const int ML = (1 << a.lbm) >> 3;
  const int64_t mb = e0 >> a.lbm;
  const bool m_ok = a.mq == 1 && mb < ((n + (1 << a.lbm) - 1) >> a.lbm);
  float m[8];
  const bool fresh_m = a.mq == 1 || (a.mq == 2 && OP != F_CAME2N && OP != F_CAME2);
  if (a.mq == 1) {
    mq_decode8(a.mk, a.m_q, a.m_scale, e0, mb, m_ok, m);
  } else if (a.mq == 2) {
    load8<float>(a.m, e0, n, m);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = 0.0f;
  }
  if (fresh_m) {
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(m[k], x[k], a.w_m) : 0.0f;
  }

  if constexpr (OP == F_CAME1) {
    float res[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float dd = x[k] - m[k];
      res[k] = dd * dd + a.eps_came;
    }
    f2_rowcol_add(a, cnt, ri, ci, res);
    if (a.mq == 2) store8<float>(a.m, e0, n, m);
    return;
  }

  // update
  float u[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    u[k] = 0.0f;
    if (k < cnt) {
      const float y = a.mq ? m[k] : x[k];
      if constexpr (OP == F_CAME2N || OP == F_CAME2) {
        const float icr = 1.0f / sqrtf(gp(a.crow)[ri[k]] / gp(a.crmean)[bi[k]]);
        const float icc = 1.0f / sqrtf(gp(a.ccol)[ci[k]]);
        u[k] = (y * icr) * icc;
      } else {
        const float ir = 1.0f / sqrtf(gp(a.row)[ri[k]] / gp(a.rmean)[bi[k]]);
        const float ic = 1.0f / sqrtf(gp(a.col)[ci[k]]);
        u[k] = (y * ir) * ic;
      }
    }
  }
  if constexpr (OP == F_NORM || OP == F_LAG || OP == F_CAME2N) {
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) sq += u[k] * u[k];
    f2_sum_add(a.norm_buf, sq);
  }
  if constexpr (OP == F_NOCLIP || OP == F_APPLY || OP == F_LAG || OP == F_CAME2) {
    const float al = *a.alpha;
    float step = al;
    if constexpr (OP == F_APPLY) {
      if (a.d > 0.0f) step = al / fmaxf(1.0f, sqrtf(*a.norm_buf) / a.sqrt_nd);
    } else if constexpr (OP == F_LAG) {
      // LAG has no CPU branch: the CUDA kernels' pn / (sqrt_numel * d) in fp32 (kernels.cu:1562-1565)
      if (a.d > 0.0f) step = al / fmaxf(1.0f, *a.prev_norm / (a.sqrt_nf * a.d));
    }
    f2_write<T>(a, e0, cnt, step, u);
    if (a.mq == 2 && OP != F_CAME2) store8<float>(a.m, e0, n, m);
  }
  const bool writes_m = OP == F_NOCLIP || OP == F_APPLY || OP == F_LAG || OP == F_CAME2;
  if (writes_m && a.mq == 1) mq_encode8(a.mk, a.m_q, a.m_scale, e0, mb, m_ok, m, ML, xw);
}

// ============================================================ APOLLO primitives
// Channel norms of u = m / (sqrt(v) + eps) (or m * rsqrt(max(res, eps_sq)) for
// CAME) and of the low-rank gradient, one workgroup per channel.
template <bool CAME>
__global__ __launch_bounds__(256) void k_apnorm(const float* __restrict__ m, const float* __restrict__ v,
                                                const float* __restrict__ gl, float* __restrict__ nu,
                                                float* __restrict__ ng, int64_t N, int64_t D, int64_t sN,
                                                int64_t sD, int64_t numel, float eps) {
  __shared__ double sd[8];
  const int64_t row = blockIdx.x;
  double su = 0.0, sg = 0.0;
  for (int64_t i = threadIdx.x; i < D; i += 256) {
    const int64_t gi = row * sN + i * sD;
    if (CAME && gi >= numel) break;
    float uu;
    if constexpr (CAME) uu = gp(m)[gi] * (1.0f / sqrtf(fmaxf(gp(v)[gi], eps)));
    else uu = gp(m)[gi] / (sqrtf(gp(v)[gi]) + eps);
    const float gg = CAME ? scrub(gp(gl)[gi]) : gp(gl)[gi];
    su += (double)(uu * uu);
    sg += (double)(gg * gg);
  }
  su = grp_sum_d(su, 64);
  sg = grp_sum_d(sg, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sd[wave] = su; sd[4 + wave] = sg; }
  __syncthreads();
  if (threadIdx.x == 0) {
    nu[row] = sqrtf((float)(sd[0] + sd[1] + sd[2] + sd[3]));
    ng[row] = sqrtf((float)(sd[4] + sd[5] + sd[6] + sd[7]));
  }
}

__global__ __launch_bounds__(256) void k_apcrms(const float* __restrict__ gl, const float* __restrict__ v,
                                                float* __restrict__ out, int64_t n, float eps_sq) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  float sq = 0.0f;
  if (i < n) {
    const float u = scrub(gp(gl)[i]) * (1.0f / sqrtf(fmaxf(gp(v)[i], eps_sq)));
    sq = u * u;
  }
  f2_sum_add(out, sq);
}

__global__ __launch_bounds__(256) void k_apres(const float* __restrict__ gl, const float* __restrict__ v,
                                               const uint8_t* __restrict__ mq, const float* __restrict__ ms,
                                               const float* __restrict__ res_old, float* __restrict__ m_out,
                                               float* __restrict__ res_out, const float* __restrict__ clip,
                                               float w1, float w3, float eps_came, float eps_sq, int64_t bs,
                                               int64_t n, int mk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float ut = (scrub(gp(gl)[i]) * (1.0f / sqrtf(fmaxf(gp(v)[i], eps_sq)))) / *clip;
  uint32_t c;
  if (mk == 2 || mk == 4) {
    const uint32_t byte = gp(mq)[i >> 1];
    c = (i & 1) ? (byte & 0x0Fu) : (byte >> 4);
  } else {
    c = gp(mq)[i];
  }
  const float mo = m_decode(mk, c, gp(ms)[i / bs]);
  const float mn = lerp_ref(mo, ut, w1);
  gp(m_out)[i] = mn;
  const float dd = ut - mn;
  gp(res_out)[i] = fmaxf(lerp_ref(gp(res_old)[i], dd * dd + eps_came, w3), kFltMin);
}

// Writeback p <- p * decay + (g * scale) * update_scale (kernels.cu:2638-3000).
// DET: the decayed value and the sum are each rounded to the parameter type;
// SR: the fp32 sum is rounded with the kernels.cu:48-87 stream.  GT: the
// gradient's element type (fp32, or the parameter's for the native forms, whose
// gradient is scrubbed and optionally negated).
template <typename T, typename GT, bool SR>
__global__ __launch_bounds__(256) void k_apwb(T* __restrict__ param, const GT* __restrict__ grad,
                                              const float* __restrict__ fs, const float* __restrict__ decay,
                                              const float* __restrict__ us, int side_right, int is_channel,
                                              int maximize, int native, uint64_t sr_seed, uint64_t sr_step,
                                              int64_t R, int64_t C) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= R * C) return;
  const int64_t r = i / C, c = i - r * C;
  const float sc = is_channel ? gp(fs)[side_right ? r : c] : gp(fs)[0];
  const float dec = decay ? *decay : 1.0f;
  const float usv = *us;
  float g = ld1<GT>(grad, i);
  if (native) {
    g = scrub(g);
    if (maximize) g = -g;
  }
  const float p = ld1<T>(param, i);
  if constexpr (SR) {
    const float nw = p * dec + (g * sc) * usv;
    param[i] = sr_round<T>(nw, sr_seed, sr_step, (uint64_t)i);
  } else {
    const float dcy = to_f<T>(from_f<T>(p * dec));
    st1<T>(param, i, dcy + (usv * g) * sc);
  }
}

// fp32 second moment of the reference's PyTorch branch (optimizer.py:2185-2188):
// v = v * (1 - bv) + (bv * g) * g, then + bv * eps_g when eps_g > 0; g scrubbed.
template <typename GT>
__global__ __launch_bounds__(256) void k_vema32(float* __restrict__ v, const GT* __restrict__ g, float omb, float bv,
                                                float add, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float gi = scrub(ld1<GT>(g, i));
  float x = gp(v)[i] * omb;
  x = x + (bv * gi) * gi;
  if (add > 0.0f) x = x + add;
  gp(v)[i] = x;
}

hipError_t prims_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

// AL EMA at a block size the unit layout cannot take (a multiple of 128 that is
// not a power of two in [128, 2048], up to 65536): one workgroup per block,
// lanes over its quads.  Pass 1 forms v' (and out), the block max and non-zero
// minimum meet in LDS (exact); pass 2 forms v' again from the same inputs and
// writes the codes (and dec).  vema_unit's arithmetic, element for element.
template <int VB, typename T>
__global__ __launch_bounds__(256) void k_vema_gen(VemaDesc one, const VemaDesc* __restrict__ tab, int ntab, int bs,
                                                  float w, int square, float eps1, float floor_,
                                                  const a8_step_scalars* w_dev) {
  if (w_dev) w = (float)load_step_scalars(w_dev).beta_val;   // the device step's V weight
  __shared__ float s_tab[256];   // decode table of the old fit (both passes read it)
  __shared__ float s_new[256];   // decode table of the new fit (dec)
  __shared__ uint32_t s_st[2];
  __shared__ float s_fit[2];
  const int64_t wg = blockIdx.x;
  int lo = 0;
  if (tab) {
    int hi = ntab - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tab[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
    }
  }
  const VemaDesc d = tab ? tab[lo] : one;
  const int lane = threadIdx.x;
  const int64_t blk = wg - d.wg_begin, base = blk * bs, n = d.n;
  constexpr float LM2 = VB == 8 ? 254.0f : 65534.0f;
  const T* X = reinterpret_cast<const T*>(d.x);
  const float s_old = gp(d.scale)[blk], lm_old = gp(d.min_log)[blk];
  if (lane == 0) { s_st[0] = 0u; s_st[1] = 0xFFFFFFFFu; }
  if (VB == 8) s_tab[lane] = lane ? exp2_exact(((float)(lane - 1) * s_old) / 254.0f + lm_old) : 0.0f;
  __syncthreads();
  auto quad = [&](int q, float* v) {
    const int64_t i0 = base + 4 * q;
    float xv[4];
    load4n<T>(X, i0, n, xv);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float xi = xv[k];
      if (square) xi = xi * xi + eps1;
      xi = scrub(xi);
      float vo = 0.0f;
      if (i0 + k < n) {
        uint32_t c;
        if constexpr (VB == 8) c = gp(reinterpret_cast<const uint8_t*>(d.q))[i0 + k];
        else c = gp(reinterpret_cast<const uint16_t*>(d.q))[i0 + k];
        vo = VB == 8 ? s_tab[c] : (c ? exp2_exact(((float)(c - 1) * s_old) / LM2 + lm_old) : 0.0f);
      }
      v[k] = (i0 + k < n) ? lerp_ref(vo, xi, w) : 0.0f;   // padding quantises as zero
    }
  };
  uint32_t vmax = 0u, vkey = 0xFFFFFFFFu;
  for (int q = lane; q < (bs >> 2); q += 256) {
    float v[4];
    quad(q, v);
    if (d.out) store4n<float>(d.out, base + 4 * q, n, v);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      vmax = max(vmax, __float_as_uint(v[k]));
      vkey = min(vkey, __float_as_uint(v[k]) - 1u);
    }
  }
  vmax = grp_red_u(vmax, 64, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
  vkey = grp_umin(vkey, 64);
  if ((lane & 63) == 0) {
    atomicMax(&s_st[0], vmax);
    atomicMin(&s_st[1], vkey);
  }
  __syncthreads();
  if (lane < 64) {
    const uint32_t key = s_st[1];
    const float mnz = key == 0xFFFFFFFFu ? __builtin_inff() : __uint_as_float(key + 1u);
    const ALFit ft = al_refit_pair(__uint_as_float(s_st[0]), mnz, floor_, LM2, lane);
    if (lane == 0) { s_fit[0] = ft.lmin; s_fit[1] = ft.s; }
  }
  __syncthreads();
  ALFit f{};
  f.lmin = s_fit[0];
  f.s = s_fit[1];
  al_fit_consts(f, LM2);
  if (d.dec && VB == 8) s_new[lane] = lane ? exp2_exact(((float)(lane - 1) * f.s) / 254.0f + f.lmin) : 0.0f;
  __syncthreads();
  for (int q = lane; q < (bs >> 2); q += 256) {
    float v[4];
    quad(q, v);
    uint32_t code[4];
    al_codes<(int)LM2, 4>(v, f, code);
    const int64_t i0 = base + 4 * q;
    if constexpr (VB == 8) {
      *gp(reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(d.q) + i0)) =
          code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
    } else {
      *gp(reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(d.q) + i0)) =
          u32x2{code[0] | (code[1] << 16), code[2] | (code[3] << 16)};
    }
    if (d.dec) {
      float dv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        dv[k] = VB == 8 ? s_new[code[k]]
                        : (code[k] ? exp2_exact(((float)(code[k] - 1) * f.s) / LM2 + f.lmin) : 0.0f);
      store4n<float>(d.dec, i0, n, dv);
    }
  }
  __syncthreads();   // every lane has read the old metadata
  if (lane == 0) { gp(d.scale)[blk] = f.s; gp(d.min_log)[blk] = f.lmin; }
}

// AL block sizes: powers of two in [128, 2048] take the unit layout; other
// multiples of 128 (up to 2^30: block_size is a 32-bit int) take k_vema_gen.
static bool al_gen_ok(int64_t bs) { return bs >= 128 && bs % 128 == 0 && bs <= (1 << 30); }

static int lb_of(int64_t bs, int lo, int hi, int& lb, const char* what) {
  if (bs < lo || bs > hi || (bs & (bs - 1)) != 0) {
    static char msg[128];
    snprintf(msg, sizeof msg, "%s must be a power of two in [%d, %d]", what, lo, hi);
    return set_error(A8_ERR_BLOCK, msg);
  }
  lb = 0;
  while ((1LL << lb) < bs) ++lb;
  return 0;
}

template <typename T>
static void launch_f2d_t(int op, unsigned nwg, hipStream_t st, const F2& a) {
  switch (op) {
    case F_NOCLIP: hipLaunchKernelGGL((k_f2d<T, F_NOCLIP>), dim3(nwg), dim3(256), 0, st, a); break;
    case F_NORM: hipLaunchKernelGGL((k_f2d<T, F_NORM>), dim3(nwg), dim3(256), 0, st, a); break;
    case F_APPLY: hipLaunchKernelGGL((k_f2d<T, F_APPLY>), dim3(nwg), dim3(256), 0, st, a); break;
    case F_LAG: hipLaunchKernelGGL((k_f2d<T, F_LAG>), dim3(nwg), dim3(256), 0, st, a); break;
    case F_SUMS: hipLaunchKernelGGL((k_f2d<T, F_SUMS>), dim3(nwg), dim3(256), 0, st, a); break;
    case F_CAME1: hipLaunchKernelGGL((k_f2d<T, F_CAME1>), dim3(nwg), dim3(256), 0, st, a); break;
    case F_CAME2N: hipLaunchKernelGGL((k_f2d<T, F_CAME2N>), dim3(nwg), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((k_f2d<T, F_CAME2>), dim3(nwg), dim3(256), 0, st, a); break;
  }
}

int64_t v_ema_table_bytes(int n) { return (int64_t)sizeof(VemaDesc) * (int64_t)n; }

int v_ema_multi(const VEmaItem* it, int n, void* table_dev, double w, int block_size, int square, float eps1,
                float log_floor, int v_bits, hipStream_t st, int upload, const a8_step_scalars* w_dev) {
  if (n <= 0) return 0;
  if (!table_dev && n > 1) {   // no table: one launch per tensor
    for (int i = 0; i < n; ++i) {
      const int rc = v_ema_multi(it + i, 1, nullptr, w, block_size, square, eps1, log_floor, v_bits, st, 1, w_dev);
      if (rc) return rc;
    }
    return 0;
  }
  if (v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  int lbv = 0;
  const bool gen = lb_of(block_size, 128, kPElems, lbv, "block_size") != 0;
  if (gen && !al_gen_ok(block_size))
    return set_error(A8_ERR_BLOCK, "block_size must be a multiple of 128 in [128, 2^30]");
  std::vector<VemaDesc> tab((size_t)n);
  int64_t wg = 0;
  for (int i = 0; i < n; ++i) {
    const VEmaItem& t = it[i];
    if (!t.q || !t.scale || !t.min_log || !t.x) return set_error(A8_ERR_ARG, "null AL state");
    if (!aligned16(t.x) || (t.out && !aligned16(t.out)) || (t.dec && !aligned16(t.dec)))
      return set_error(A8_ERR_ALIGN, "AL EMA input and outputs must be 16-byte aligned");
    VemaDesc& D = tab[(size_t)i];
    D.q = t.q; D.scale = t.scale; D.min_log = t.min_log; D.x = t.x; D.out = t.out; D.dec = t.dec; D.n = t.n;
    D.nblk = (t.n + block_size - 1) / block_size;
    D.wg_begin = wg;
    wg += gen ? D.nblk : (D.nblk * block_size + kPElems - 1) / kPElems;
  }
  if (wg == 0) return 0;
  if (wg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "AL EMA: too many elements");
  const VemaDesc* dt = nullptr;
  if (table_dev) {
    if (upload && upload_table(table_dev, tab.data(), sizeof(VemaDesc) * (size_t)n, st) != hipSuccess)
      return set_error(A8_ERR_HIP, "table upload failed");
    dt = reinterpret_cast<const VemaDesc*>(table_dev);
  }
  const VemaDesc one = tab[0];
  if (gen) {
    if (v_bits == 8)
      hipLaunchKernelGGL((k_vema_gen<8, float>), dim3((unsigned)wg), dim3(256), 0, st, one, dt, n, block_size,
                         (float)w, square, eps1, log_floor, w_dev);
    else
      hipLaunchKernelGGL((k_vema_gen<16, float>), dim3((unsigned)wg), dim3(256), 0, st, one, dt, n, block_size,
                         (float)w, square, eps1, log_floor, w_dev);
    return check_launch("k_vema_gen");
  }
  if (v_bits == 8)
    hipLaunchKernelGGL(k_vema_multi<8>, dim3((unsigned)wg), dim3(256), 0, st, one, dt, n, lbv, (float)w, square,
                       eps1, log_floor, w_dev);
  else
    hipLaunchKernelGGL(k_vema_multi<16>, dim3((unsigned)wg), dim3(256), 0, st, one, dt, n, lbv, (float)w, square,
                       eps1, log_floor, w_dev);
  return check_launch("k_vema_multi");
}

// Row sums for the finish phase of APOLLO: the squares of a lane's eight
// elements summed in double, then over the C / 8 lanes of its row (C a power
// of two in [8, 512], so a row lies inside one wave and starts on a lane that
// is a multiple of C / 8), stored as two doubles per row.  Every lane of the
// wave must take part.
__device__ __forceinline__ void rowsum_store(const float* u, const float* g, int cnt, int64_t e0, int64_t n,
                                             int64_t C, double* out) {
  double su = 0.0, sg = 0.0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < cnt) {
      su += (double)(u[k] * u[k]);
      sg += (double)(g[k] * g[k]);
    }
  }
  const int G = (int)(C >> 3);
  su = grp_sum_d(su, G);
  sg = grp_sum_d(sg, G);
  if ((threadIdx.x & (G - 1)) == 0 && e0 < n) {
    const int64_t row = e0 / C;
    gp(out)[2 * row] = su;
    gp(out)[2 * row + 1] = sg;
  }
}

__global__ __launch_bounds__(256) void k_rowsum_sq(const float* u, const float* g, int64_t n, int64_t C,
                                                   double* out) {
  const int64_t e0 = (int64_t)blockIdx.x * kPElems + (int64_t)threadIdx.x * 8;
  const int cnt = e0 >= n ? 0 : 8;   // n is a multiple of C >= 8
  float uv[8], gv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uv[k] = k < cnt ? gp(u)[e0 + k] : 0.0f;
    gv[k] = k < cnt ? gp(g)[e0 + k] : 0.0f;
  }
  rowsum_store(uv, gv, cnt, e0, n, C, out);
}

bool rowsum_len_ok(int64_t C) { return C >= 8 && C <= 512 && (C & (C - 1)) == 0; }

int rowsum_sq(const float* u, const float* g, int64_t n, int64_t C, double* out, hipStream_t st) {
  if (!u || !g || !out) return set_error(A8_ERR_ARG, "row sums: null pointer");
  if (!rowsum_len_ok(C) || n <= 0 || n % C) return set_error(A8_ERR_SIZE, "row sums: rows must be 8..512 (2^k)");
  if (reinterpret_cast<uintptr_t>(out) & 7) return set_error(A8_ERR_ALIGN, "row sums: output must be 8-byte aligned");
  const int64_t wg = (n + kPElems - 1) / kPElems;
  if (wg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "row sums: too many elements");
  hipLaunchKernelGGL(k_rowsum_sq, dim3((unsigned)wg), dim3(256), 0, st, u, g, n, C, out);
  return check_launch("k_rowsum_sq");
}

// ------------------------------------------------------------ CAME APOLLO tail
// The low-rank passes of non-factorised CAME APOLLO after the RMS clip, in one
// kernel (optimizer.py:2846-2896): U /= clip; m' = lerp(m, U, 1 - beta1)
// re-encoded per M block (or fp32 m); res = (U - m')^2 + eps_came; its EMA with
// beta3 (AL codes re-fitted per block and read back decoded, or fp32);
// u = m' / sqrt(max(res, eps^2)).  One workgroup per 2048-element unit, eight
// consecutive elements per lane (the units of k_sgd and k_vema), element for
// element the arithmetic of the passes it replaces: the division of the clip
// pass, k_sgd's momentum EMA (U scrubbed, as k_sgd scrubs its input) or the
// fp32 lerp, the residual of the element pass, vema_unit for the residual EMA,
// and the update's 1 / sqrt.  MK: 1 coded M, 3 fp32 M; VB: 8 / 16 coded
// residual, 0 fp32.
struct CameTailDesc {
  const float* U;
  const float* clip;
  uint8_t* m_q;
  float* m_scale;
  float* m_fp32;
  void* r_q;
  float* r_scale;
  float* r_min_log;
  float* r_fp32;
  float* u;
  const float* g;
  int64_t n, nmb, nvb, wg_begin, rs_C;
};

struct CameTailHyp {
  float w1, w3, eps_came, eps_sq;
  int mk, lbm, lbv;
};

template <int VB, int MK>
__global__ __launch_bounds__(256) void k_came_tail(CameTailDesc one, const CameTailDesc* __restrict__ tab, int ntab,
                                                   CameTailHyp h) {
  __shared__ float xw[8];
  __shared__ float xm[4];
  __shared__ float dtab[4 * 256];
  const int64_t wg = blockIdx.x;
  CameTailDesc D = one;
  if (tab) {
    int lo = 0, hi = ntab - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tab[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
    }
    D = tab[lo];
  }
  const int64_t bid = wg - D.wg_begin;
  const int64_t n = D.n;
  const int64_t e0 = bid * kPElems + (int64_t)threadIdx.x * 8;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);
  float U[8];
  load8<float>(D.U, e0, n, U);
  if (D.clip) {   // uniform
    const float clip = *gp(D.clip);
#pragma unroll
    for (int k = 0; k < 8; ++k) U[k] = U[k] / clip;
  }
  // ---- momentum
  float m[8];
  if constexpr (MK == 3) {
    float mo[8];
    load8<float>(D.m_fp32, e0, n, mo);
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = lerp_ref(mo[k], U[k], h.w1);
    store8<float>(D.m_fp32, e0, n, m);
  } else {
    const int64_t mb = e0 >> h.lbm;
    const bool m_ok = mb < D.nmb;   // codes are padded to whole blocks
    float mo[8];
    mq_decode8(h.mk, D.m_q, D.m_scale, e0, mb, m_ok, mo);
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], scrub(U[k]), h.w1) : 0.0f;
    mq_encode8(h.mk, D.m_q, D.m_scale, e0, mb, m_ok, m, (1 << h.lbm) >> 3, xm);
  }
  // ---- residual and its EMA
  float rin[8], res[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float r = U[k] - m[k];
    r = r * r;
    rin[k] = r + h.eps_came;
  }
  if constexpr (VB == 0) {
    float ro[8];
    load8<float>(D.r_fp32, e0, n, ro);
#pragma unroll
    for (int k = 0; k < 8; ++k) res[k] = lerp_ref(ro[k], rin[k], h.w3);
    store8<float>(D.r_fp32, e0, n, res);
  } else {
    vema_unit<VB, float, true>(D.r_q, D.r_scale, D.r_min_log, nullptr, nullptr, nullptr, n, D.nvb, bid, h.lbv, h.w3,
                               0, 0.0f, -126.0f, xw, dtab, rin, res);
  }
  // ---- update
  float uo[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) uo[k] = m[k] * (1.0f / sqrtf(fmaxf(res[k], h.eps_sq)));
  if (D.rs_C) {   // uniform
    float g[8];
    load8<float>(D.g, e0, n, g);
    rowsum_store(uo, g, cnt, e0, n, D.rs_C, reinterpret_cast<double*>(D.u));
  } else {
    store8<float>(D.u, e0, n, uo);
  }
}

// Factorised APOLLO with momentum, after the row / column EMAs and their clamped
// row mean (optimizer.py:2689-2758): m' = lerp(m, g_low, 1 - beta1) re-encoded
// per M block (or fp32 m), u = m' / (sqrt((r_i c_j) / rmean) + eps), in one pass
// (k_sgd's momentum EMA, g scrubbed as k_sgd scrubs it, then the update pass's
// arithmetic), for the same units as k_came_tail.
struct FactTailDesc {
  const float* g;
  uint8_t* m_q;
  float* m_scale;
  float* m_fp32;
  const float* rv;
  const float* cv;
  const float* rmean;
  float* u;
  int64_t n, C, nmb, wg_begin, rs;
};

struct FactTailHyp {
  float w1, aeps;
  int mk, lbm;
};

template <int MK>
__global__ __launch_bounds__(256) void k_fact_tail(FactTailDesc one, const FactTailDesc* __restrict__ tab, int ntab,
                                                   FactTailHyp h) {
  __shared__ float xm[4];
  const int64_t wg = blockIdx.x;
  FactTailDesc D = one;
  if (tab) {
    int lo = 0, hi = ntab - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tab[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
    }
    D = tab[lo];
  }
  const int64_t n = D.n;
  const int64_t e0 = (wg - D.wg_begin) * kPElems + (int64_t)threadIdx.x * 8;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);
  float g[8], m[8];
  load8<float>(D.g, e0, n, g);
  if constexpr (MK == 3) {
    float mo[8];
    load8<float>(D.m_fp32, e0, n, mo);
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = lerp_ref(mo[k], g[k], h.w1);
    store8<float>(D.m_fp32, e0, n, m);
  } else {
    const int64_t mb = e0 >> h.lbm;
    const bool m_ok = mb < D.nmb;   // codes are padded to whole blocks
    float mo[8];
    mq_decode8(h.mk, D.m_q, D.m_scale, e0, mb, m_ok, mo);
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], scrub(g[k]), h.w1) : 0.0f;
    mq_encode8(h.mk, D.m_q, D.m_scale, e0, mb, m_ok, m, (1 << h.lbm) >> 3, xm);
  }
  const float rmean = *gp(D.rmean);
  float uo[8];
  int64_t r = e0 / D.C, c = e0 - r * D.C;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uo[k] = 0.0f;
    if (k < cnt) {
      const float ve = (gp(D.rv)[r] * gp(D.cv)[c]) / rmean;
      uo[k] = m[k] / (sqrtf(ve) + h.aeps);
    }
    if (++c == D.C) { c = 0; ++r; }
  }
  if (D.rs) rowsum_store(uo, g, cnt, e0, n, D.C, reinterpret_cast<double*>(D.u));   // uniform
  else store8<float>(D.u, e0, n, uo);
}

int64_t fact_tail_table_bytes(int n) { return (int64_t)sizeof(FactTailDesc) * (int64_t)n; }

int fact_tail_multi(const FactTailItem* it, int n, void* table_dev, double beta1, float apollo_eps, int m_fp32,
                    int m_bits, int m_mode, int m_block_size, hipStream_t st, int upload) {
  if (n <= 0) return 0;
  if (!m_fp32 && !(m_block_size >= 32 && m_block_size <= 2048 && (m_block_size & (m_block_size - 1)) == 0))
    return set_error(A8_ERR_BLOCK, "factorised tail: m_block_size must be a power of two in [32, 2048]");
  FactTailHyp h{};
  h.w1 = (float)(1.0 - beta1);
  h.aeps = apollo_eps;
  if (!m_fp32) {
    if (!((m_bits == 8 || m_bits == 4) && (m_mode == 0 || m_mode == 1)))
      return set_error(A8_ERR_ARG, "m_bits must be 4/8 and m_mode 0/1");
    h.mk = m_mode == 0 ? (m_bits == 8 ? 1 : 2) : (m_bits == 8 ? 3 : 4);
  }
  while ((1 << h.lbm) < (m_fp32 ? 32 : m_block_size)) ++h.lbm;
  std::vector<FactTailDesc> tab((size_t)n);
  int64_t wg = 0;
  for (int i = 0; i < n; ++i) {
    const FactTailItem& t = it[i];
    if (!t.g || !t.u || !t.rv || !t.cv || !t.rmean || t.C <= 0 || (m_fp32 ? !t.m_fp32 : !(t.m_q && t.m_scale)))
      return set_error(A8_ERR_ARG, "factorised tail: state missing");
    if (!aligned16(t.g) || !aligned16(t.u) || (m_fp32 ? !aligned16(t.m_fp32) : !aligned16(t.m_q)))
      return set_error(A8_ERR_ALIGN, "factorised tail: streams must be 16-byte aligned");
    FactTailDesc& D = tab[(size_t)i];
    D.g = t.g; D.m_q = t.m_q; D.m_scale = t.m_scale; D.m_fp32 = t.m_fp32;
    D.rv = t.rv; D.cv = t.cv; D.rmean = t.rmean; D.u = t.u;
    D.n = t.n; D.C = t.C;
    if (t.rs && !(rowsum_len_ok(t.C) && t.n % t.C == 0))
      return set_error(A8_ERR_SIZE, "factorised tail: row sums need rows of 8..512 (2^k) elements");
    D.rs = t.rs ? 1 : 0;
    D.nmb = (t.n + (1 << h.lbm) - 1) >> h.lbm;
    D.wg_begin = wg;
    wg += (t.n + kPElems - 1) / kPElems;   // M blocks are powers of two up to a unit
  }
  if (wg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "factorised tail: too many elements");
  const FactTailDesc* dt = nullptr;
  if (n > 1) {
    if (!table_dev) return set_error(A8_ERR_ARG, "factorised tail: a table is needed for several matrices");
    if (upload && upload_table(table_dev, tab.data(), sizeof(FactTailDesc) * (size_t)n, st) != hipSuccess)
      return set_error(A8_ERR_HIP, "table upload failed");
    dt = reinterpret_cast<const FactTailDesc*>(table_dev);
  }
  const dim3 g((unsigned)wg), b(256);
  if (m_fp32) hipLaunchKernelGGL((k_fact_tail<3>), g, b, 0, st, tab[0], dt, n, h);
  else hipLaunchKernelGGL((k_fact_tail<1>), g, b, 0, st, tab[0], dt, n, h);
  return check_launch("k_fact_tail");
}

static bool pow2_in(int x, int lo, int hi) { return x >= lo && x <= hi && (x & (x - 1)) == 0; }

bool came_tail_ok(int m_fp32, int m_block_size, int c_bits, int block_size) {
  return (m_fp32 || pow2_in(m_block_size, 32, 2048)) && (c_bits == 0 || pow2_in(block_size, 128, 2048));
}

int64_t came_tail_table_bytes(int n) { return (int64_t)sizeof(CameTailDesc) * (int64_t)n; }

int came_tail_multi(const CameTailItem* it, int n, void* table_dev, double beta1, double beta3, float eps_came,
                    float eps_sq, int m_fp32, int m_bits, int m_mode, int m_block_size, int c_bits, int block_size,
                    hipStream_t st, int upload) {
  if (n <= 0) return 0;
  if (!came_tail_ok(m_fp32, m_block_size, c_bits, block_size))
    return set_error(A8_ERR_BLOCK, "CAME tail: block sizes must be powers of two");
  CameTailHyp h{};
  h.w1 = (float)(1.0 - beta1);
  h.w3 = (float)(1.0 - beta3);
  h.eps_came = eps_came;
  h.eps_sq = eps_sq;
  if (!m_fp32) {
    if (!((m_bits == 8 || m_bits == 4) && (m_mode == 0 || m_mode == 1)))
      return set_error(A8_ERR_ARG, "m_bits must be 4/8 and m_mode 0/1");
    h.mk = m_mode == 0 ? (m_bits == 8 ? 1 : 2) : (m_bits == 8 ? 3 : 4);
  }
  while ((1 << h.lbm) < (m_fp32 ? 32 : m_block_size)) ++h.lbm;
  while ((1 << h.lbv) < (c_bits ? block_size : 128)) ++h.lbv;
  std::vector<CameTailDesc> tab((size_t)n);
  int64_t wg = 0;
  for (int i = 0; i < n; ++i) {
    const CameTailItem& t = it[i];
    if (!t.U || !t.u || (m_fp32 ? !t.m_fp32 : !(t.m_q && t.m_scale)) ||
        (c_bits ? !(t.r_q && t.r_scale && t.r_min_log) : !t.r_fp32))
      return set_error(A8_ERR_ARG, "CAME tail: state missing");
    if (!aligned16(t.U) || !aligned16(t.u) || (m_fp32 ? !aligned16(t.m_fp32) : !aligned16(t.m_q)) ||
        (!c_bits && !aligned16(t.r_fp32)))
      return set_error(A8_ERR_ALIGN, "CAME tail: streams must be 16-byte aligned");
    CameTailDesc& D = tab[(size_t)i];
    D.U = t.U; D.clip = t.clip; D.m_q = t.m_q; D.m_scale = t.m_scale; D.m_fp32 = t.m_fp32;
    D.r_q = t.r_q; D.r_scale = t.r_scale; D.r_min_log = t.r_min_log; D.r_fp32 = t.r_fp32; D.u = t.u;
    D.n = t.n;
    if (t.rs_C && !(t.g && aligned16(t.g) && rowsum_len_ok(t.rs_C) && t.n % t.rs_C == 0))
      return set_error(A8_ERR_SIZE, "CAME tail: row sums need an aligned g_low and rows of 8..512 (2^k) elements");
    D.g = t.g;
    D.rs_C = t.rs_C;
    D.nmb = (t.n + (1 << h.lbm) - 1) >> h.lbm;
    D.nvb = (t.n + (1 << h.lbv) - 1) >> h.lbv;
    D.wg_begin = wg;
    wg += (t.n + kPElems - 1) / kPElems;   // blocks are powers of two up to a unit: padding stays inside
  }
  if (wg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "CAME tail: too many elements");
  const CameTailDesc* dt = nullptr;
  if (n > 1) {
    if (!table_dev) return set_error(A8_ERR_ARG, "CAME tail: a table is needed for several matrices");
    if (upload && upload_table(table_dev, tab.data(), sizeof(CameTailDesc) * (size_t)n, st) != hipSuccess)
      return set_error(A8_ERR_HIP, "table upload failed");
    dt = reinterpret_cast<const CameTailDesc*>(table_dev);
  }
  const dim3 g((unsigned)wg), b(256);
  const CameTailDesc& one = tab[0];
  if (m_fp32) {
    if (c_bits == 8) hipLaunchKernelGGL((k_came_tail<8, 3>), g, b, 0, st, one, dt, n, h);
    else if (c_bits == 16) hipLaunchKernelGGL((k_came_tail<16, 3>), g, b, 0, st, one, dt, n, h);
    else hipLaunchKernelGGL((k_came_tail<0, 3>), g, b, 0, st, one, dt, n, h);
  } else {
    if (c_bits == 8) hipLaunchKernelGGL((k_came_tail<8, 1>), g, b, 0, st, one, dt, n, h);
    else if (c_bits == 16) hipLaunchKernelGGL((k_came_tail<16, 1>), g, b, 0, st, one, dt, n, h);
    else hipLaunchKernelGGL((k_came_tail<0, 1>), g, b, 0, st, one, dt, n, h);
  }
  return check_launch("k_came_tail");
}

}  // namespace a8

using namespace a8;

extern "C" {

int a8_log_quantize_lerp(void* q, float* scale, float* min_log, const void* x, int x_dtype, float* fp32_out,
                         double beta, int block_size, int square_input, float eps1, int64_t numel, float log_floor,
                         int v_bits, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!q || !scale || !min_log || !x) return set_error(A8_ERR_ARG, "null pointer");
  if (v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  if (!aligned16(x) || (fp32_out && !aligned16(fp32_out)))
    return set_error(A8_ERR_ALIGN, "new_val and fp32_out must be 16-byte aligned");
  int lbv = 0;
  const bool gen = lb_of(block_size, 128, kPElems, lbv, "block_size") != 0;
  if (gen && !al_gen_ok(block_size))
    return set_error(A8_ERR_BLOCK, "block_size must be a multiple of 128 in [128, 2^30]");
  const int64_t nblk = (numel + block_size - 1) / block_size;
  const int64_t nwg = gen ? nblk : (nblk * block_size + kPElems - 1) / kPElems;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  hipStream_t st = (hipStream_t)stream;
  const float w = (float)beta;
  if (gen) {
    VemaDesc one{};
    one.q = q; one.scale = scale; one.min_log = min_log; one.x = reinterpret_cast<const float*>(x);
    one.out = fp32_out; one.n = numel; one.nblk = nblk;
#define A8_VEMAG(VB, T)                                                                                        \
  hipLaunchKernelGGL((k_vema_gen<VB, T>), dim3((unsigned)nwg), dim3(256), 0, st, one, nullptr, 1, block_size, w, \
                     square_input, eps1, log_floor, nullptr)
    switch (x_dtype) {
      case A8_F32: if (v_bits == 8) A8_VEMAG(8, float); else A8_VEMAG(16, float); break;
      case A8_BF16: if (v_bits == 8) A8_VEMAG(8, __hip_bfloat16); else A8_VEMAG(16, __hip_bfloat16); break;
      case A8_F16: if (v_bits == 8) A8_VEMAG(8, __half); else A8_VEMAG(16, __half); break;
      default: return set_error(A8_ERR_DTYPE, "unsupported new_val dtype");
    }
#undef A8_VEMAG
    return check_launch("k_vema_gen");
  }
#define A8_VEMA(VB, T)                                                                                      \
  hipLaunchKernelGGL((k_vema<VB, T>), dim3((unsigned)nwg), dim3(256), 0, st, q, scale, min_log,             \
                     reinterpret_cast<const T*>(x), fp32_out, numel, nblk, lbv, w, square_input, eps1, log_floor)
  switch (x_dtype) {
    case A8_F32: if (v_bits == 8) A8_VEMA(8, float); else A8_VEMA(16, float); break;
    case A8_BF16: if (v_bits == 8) A8_VEMA(8, __hip_bfloat16); else A8_VEMA(16, __hip_bfloat16); break;
    case A8_F16: if (v_bits == 8) A8_VEMA(8, __half); else A8_VEMA(16, __half); break;
    default: return set_error(A8_ERR_DTYPE, "unsupported new_val dtype");
  }
#undef A8_VEMA
  return check_launch("k_vema");
}

int a8_factored_prim(int op, int dtype, int stochastic, const a8_factored_prim_args* args, void* stream) {
  const a8_factored_prim_args& p = *args;
  if (op < 0 || op > 7) return set_error(A8_ERR_ARG, "op must be 0..7");
  if (p.numel < 0 || p.rows <= 0 || p.cols <= 0) return set_error(A8_ERR_SIZE, "bad numel/rows/cols");
  if (p.numel == 0) return 0;
  if (p.numel % (p.rows * p.cols) != 0) return set_error(A8_ERR_SIZE, "numel must be a multiple of rows*cols");
  F2 a{};
  a.param = p.param; a.grad = p.grad; a.m_q = p.m_q; a.m_scale = p.m_scale; a.m = p.m;
  a.row = p.row; a.col = p.col; a.rmean = p.row_mean; a.crow = p.conf_row; a.ccol = p.conf_col;
  a.crmean = p.conf_row_mean; a.row_sum = p.row_sum; a.col_sum = p.col_sum; a.norm_buf = p.norm_buf;
  a.alpha = p.alpha; a.prev_norm = p.prev_norm; a.decay = p.decay; a.clip = p.clip;
  a.R = p.rows; a.C = p.cols; a.n = p.numel; a.sr_seed = p.sr_seed; a.sr_step = p.sr_step;
  a.w_m = (float)(1.0 - p.beta1); a.eps_came = p.eps_came; a.d = p.d;
  a.sqrt_nd = (float)(sqrt((double)p.numel) * (double)p.d);
  a.sqrt_nf = sqrtf((float)p.numel);
  a.sr = stochastic && dtype != A8_F32;
  a.lbm = 5;
  const bool writes_p = op == F_NOCLIP || op == F_APPLY || op == F_LAG || op == F_CAME2;
  const bool uses_g = !((op == F_CAME2N || op == F_CAME2) && p.m && !p.m_q);
  if (uses_g && !p.grad) return set_error(A8_ERR_ARG, "null grad");
  if (writes_p && (!p.param || !p.alpha)) return set_error(A8_ERR_ARG, "null param/alpha");
  if (op != F_SUMS && uses_g && (!p.row || !p.col || !p.row_mean)) return set_error(A8_ERR_ARG, "null row/col/row_mean");
  if ((op == F_CAME2N || op == F_CAME2) && (!p.conf_row || !p.conf_col || !p.conf_row_mean))
    return set_error(A8_ERR_ARG, "null confidence vectors");
  if ((op == F_SUMS || op == F_CAME1) && (!p.row_sum || !p.col_sum)) return set_error(A8_ERR_ARG, "null row/col sums");
  if ((op == F_NORM || op == F_LAG || op == F_CAME2N || op == F_APPLY) && !p.norm_buf)
    return set_error(A8_ERR_ARG, "null norm_buf");
  if (op == F_LAG && !p.prev_norm) return set_error(A8_ERR_ARG, "null prev_norm");
  if (p.m_q && p.m) return set_error(A8_ERR_ARG, "give quantised (m_q) or fp32 (m) momentum, not both");
  if (op == F_CAME1 || op == F_CAME2N || op == F_CAME2) {
    if (!p.m_q && !p.m) return set_error(A8_ERR_ARG, "CAME needs momentum");
  }
  if (p.m_q) {
    a.mq = 1;
    if (!p.m_scale) return set_error(A8_ERR_ARG, "null m_scale");
    if (p.m_bits == 8) a.mk = p.m_mode ? 3 : 1;
    else if (p.m_bits == 4) a.mk = p.m_mode ? 4 : 2;
    else return set_error(A8_ERR_ARG, "m_bits must be 8 or 4");
    int rc = lb_of(p.m_block_size, 32, kPElems, a.lbm, "m_block_size");
    if (rc) return rc;
  } else if (p.m) {
    a.mq = 2;
  }
  if ((uses_g && !aligned16(p.grad)) || (p.param && !aligned16(p.param)) || (p.m && !aligned16(p.m)) ||
      (p.m_q && !aligned16(p.m_q)))
    return set_error(A8_ERR_ALIGN, "param, grad and momentum must be 16-byte aligned");
  const int64_t nwg = (p.numel + kPElems - 1) / kPElems;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case A8_F32: launch_f2d_t<float>(op, (unsigned)nwg, st, a); break;
    case A8_BF16: launch_f2d_t<__hip_bfloat16>(op, (unsigned)nwg, st, a); break;
    case A8_F16: launch_f2d_t<__half>(op, (unsigned)nwg, st, a); break;
    default: return set_error(A8_ERR_DTYPE, "unsupported dtype");
  }
  return check_launch("k_f2d");
}

int a8_apollo_norms(const float* m, const float* v, const float* grad_low, float* norm_update, float* norm_grad,
                    int64_t n_channels, int64_t d, int64_t stride_n, int64_t stride_d, int64_t numel, float eps,
                    int came, void* stream) {
  if (n_channels < 0 || d < 0) return set_error(A8_ERR_SIZE, "bad sizes");
  if (n_channels == 0) return 0;
  if (!m || !v || !grad_low || !norm_update || !norm_grad) return set_error(A8_ERR_ARG, "null pointer");
  if (n_channels > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "too many channels");
  hipStream_t st = (hipStream_t)stream;
  if (came)
    hipLaunchKernelGGL(k_apnorm<true>, dim3((unsigned)n_channels), dim3(256), 0, st, m, v, grad_low, norm_update,
                       norm_grad, n_channels, d, stride_n, stride_d, numel, eps);
  else
    hipLaunchKernelGGL(k_apnorm<false>, dim3((unsigned)n_channels), dim3(256), 0, st, m, v, grad_low, norm_update,
                       norm_grad, n_channels, d, stride_n, stride_d, numel, eps);
  return check_launch("k_apnorm");
}

int a8_apollo_came_rms(const float* grad_low, const float* v, float* sum_u2, float eps_sq, int64_t numel,
                       void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!grad_low || !v || !sum_u2) return set_error(A8_ERR_ARG, "null pointer");
  const int64_t nwg = (numel + 255) / 256;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  hipLaunchKernelGGL(k_apcrms, dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream, grad_low, v, sum_u2, numel,
                     eps_sq);
  return check_launch("k_apcrms");
}

int a8_apollo_came_m_res(const float* grad_low, const float* v, const uint8_t* m_q_old, const float* m_scale_old,
                         const float* res_old, float* m_out, float* res_out, const float* clip_factor, double beta1,
                         double beta3, float eps_came, float eps_sq, int m_block_size, int64_t numel, int m_bits,
                         int m_mode, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!grad_low || !v || !m_q_old || !m_scale_old || !res_old || !m_out || !res_out || !clip_factor)
    return set_error(A8_ERR_ARG, "null pointer");
  if (m_block_size <= 0) return set_error(A8_ERR_BLOCK, "m_block_size must be positive");
  int mk;
  if (m_bits == 8) mk = m_mode ? 3 : 1;
  else if (m_bits == 4) mk = m_mode ? 4 : 2;
  else return set_error(A8_ERR_ARG, "m_bits must be 8 or 4");
  const int64_t nwg = (numel + 255) / 256;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  hipLaunchKernelGGL(k_apres, dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream, grad_low, v, m_q_old,
                     m_scale_old, res_old, m_out, res_out, clip_factor, (float)(1.0 - beta1), (float)(1.0 - beta3),
                     eps_came, eps_sq, (int64_t)m_block_size, numel, mk);
  return check_launch("k_apres");
}

int a8_vema_fp32(float* v, const void* grad, int grad_dtype, double beta_val, float eps_g, int64_t numel,
                 void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!v || !grad) return set_error(A8_ERR_ARG, "null pointer");
  const int64_t nwg = (numel + 255) / 256;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  const float omb = (float)(1.0 - beta_val), bv = (float)beta_val;
  const float add = eps_g > 0.0f ? (float)(beta_val * (double)eps_g) : 0.0f;
  hipStream_t st = (hipStream_t)stream;
  if (grad_dtype == A8_F32)
    hipLaunchKernelGGL(k_vema32<float>, dim3((unsigned)nwg), dim3(256), 0, st, v, (const float*)grad, omb, bv, add,
                       numel);
  else if (grad_dtype == A8_BF16)
    hipLaunchKernelGGL(k_vema32<__hip_bfloat16>, dim3((unsigned)nwg), dim3(256), 0, st, v,
                       (const __hip_bfloat16*)grad, omb, bv, add, numel);
  else if (grad_dtype == A8_F16)
    hipLaunchKernelGGL(k_vema32<__half>, dim3((unsigned)nwg), dim3(256), 0, st, v, (const __half*)grad, omb, bv, add,
                       numel);
  else
    return set_error(A8_ERR_DTYPE, "grad_dtype must be A8_F32, A8_BF16 or A8_F16");
  return check_launch("k_vema32");
}

int a8_apollo_writeback(int dtype, int grad_native, int stochastic, void* param, const void* grad,
                        const float* final_scale, const float* decay, const float* update_scale, int side_right,
                        int is_channel, int maximize, uint64_t sr_seed, uint64_t sr_step, int64_t rows, int64_t cols,
                        void* stream) {
  if (rows < 0 || cols < 0) return set_error(A8_ERR_SIZE, "bad shape");
  if (rows == 0 || cols == 0) return 0;
  if (!param || !grad || !final_scale || !update_scale) return set_error(A8_ERR_ARG, "null pointer");
  const int64_t nwg = (rows * cols + 255) / 256;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "tensor too large");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)nwg), blk(256);
#define A8_APWB(T, GT, SR)                                                                                  \
  hipLaunchKernelGGL((k_apwb<T, GT, SR>), grid, blk, 0, st, reinterpret_cast<T*>(param),                    \
                     reinterpret_cast<const GT*>(grad), final_scale, decay, update_scale, side_right,          \
                     is_channel, maximize, grad_native, sr_seed, sr_step, rows, cols)
  if (dtype == A8_BF16) {
    if (grad_native) { if (stochastic) A8_APWB(__hip_bfloat16, __hip_bfloat16, true); else A8_APWB(__hip_bfloat16, __hip_bfloat16, false); }
    else { if (stochastic) A8_APWB(__hip_bfloat16, float, true); else A8_APWB(__hip_bfloat16, float, false); }
  } else if (dtype == A8_F16) {
    if (grad_native) { if (stochastic) A8_APWB(__half, __half, true); else A8_APWB(__half, __half, false); }
    else { if (stochastic) A8_APWB(__half, float, true); else A8_APWB(__half, float, false); }
  } else {
    return set_error(A8_ERR_DTYPE, "param must be bfloat16 or float16");
  }
#undef A8_APWB
  return check_launch("k_apwb");
}

}  // extern "C"
