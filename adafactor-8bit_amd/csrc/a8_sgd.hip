// SGD step (beta2 = beta2_decay = None) and the standalone momentum EMA (gfx950).
//
// SGD follows the SGD branch of _update_param_8bit (optimizer.py:2045-2077) with
// the fallback's arithmetic:
//   m' = lerp(deq(m), g, 1 - beta1)       (optimizer.py:2056-2059; fp32 m: 2065-2068)
//   u  = m' / (1 - beta1)  or  u = g       (optimizer.py:2069-2072)
//   p  = fma(-alpha / denom, u * fira_scale, p * decay)   (_apply_update_pytorch,
//        optimizer.py:866-881; denom = max(1, |u| / (sqrt(n) d)) when d > 0)
// and M is requantised from the fp32 m' (the value the update used), one
// absmax per B_M block (optimizer.py:504-519, 454-480).
// The standalone EMA replaces fused_m_quantize_lerp (kernels.cu:523-588) with
// the arithmetic of its twin _m_ema_pytorch (optimizer.py:690-701):
// m' = lerp(deq(m), x, 1 - beta), requantised, with an optional fp32 copy.
//
// Layout: one workgroup covers 2048 consecutive elements of one tensor, 8 per
// lane, which is a whole number of M blocks (B_M a power of two in [32, 2048]).
// Tensor tables let one launch cover a parameter group.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

constexpr int kSLanes = 256;
constexpr int kSElems = kSLanes * 8;

struct SgdDesc {
  void* param;
  const void* grad;     // g, or x of the standalone EMA
  uint8_t* m_q;
  float* m_scale;
  float* m;             // fp32 momentum
  float* m_out;         // optional fp32 copy of m' (standalone EMA)
  float* norm_buf;      // sum of u^2 (NORM), read by APPLY
  const float* fira;    // Fira's scale (the first of its [scale, prev', finite sum]), or null
  const float* fira_sum;   // Fira's finite sum of u^2 (with fira)
  const float* alpha;
  const float* decay;
  int64_t numel;
  int64_t wg_begin;
  uint64_t sr_seed;
  double* norm_part;    // NORM: one partial sum of u^2 per workgroup (added in order by k_sgd_fin)
};

struct SgdHyp {
  float w_m;        // (float)(1 - beta1): lerp weight
  float mdiv;       // (float)(1 - beta1): bias divisor of the update
  float d;
  float alpha_val;
  float decay_val;
  int has_decay;
  int lbm;          // log2(B_M)
  int mk;           // 1 UF8, 2 UF4, 3 D8, 4 D4
  uint64_t sr_step;
  int gen;          // B_M not a power of two in [32, 2048]: k_sgd_gen over units of `unit` elements
  int bm;           // B_M (gen)
  int unit;         // elements per workgroup (gen): a whole number of M blocks
  const a8_step_scalars* dsc;   // if set: alpha, decay (when has_decay) and the SR step of this step
};

// A captured step reads its scalars from the device block of a8_step_advance.
__device__ __forceinline__ void sgd_step_scalars(SgdHyp& h) {
  if (!h.dsc) return;
  const a8_step_scalars sc = load_step_scalars(h.dsc);
  h.alpha_val = sc.alpha;
  h.decay_val = sc.decay;
  h.sr_step = sc.step;
}

__device__ __forceinline__ const SgdDesc* find_sgd(const SgdDesc* tab, int n, int64_t wg) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tab[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
  }
  return tab + lo;
}

// MK: 0 no momentum, 1 quantised momentum, 2 fp32 momentum.
// MODE: 0 single pass (update without clipping), 1 NORM (sum of u^2 only, no
// writes), 2 APPLY (clip from the NORM sum, optional Fira scale; writes p and
// M), 3 EMA (standalone momentum EMA: writes M and m_out, no parameter).
// SR: the parameter write is fma(-step, u, p * decay) stochastically rounded to
// T with the stream of kernels.cu:48-87, element index within the tensor.
template <typename T, int MK, int MODE, bool SR>
__global__ __launch_bounds__(kSLanes) void k_sgd(SgdDesc one, const SgdDesc* __restrict__ table, int ntab,
                                                 SgdHyp h) {
  __shared__ float xw[4];
  sgd_step_scalars(h);
  const SgdDesc D = table ? *find_sgd(table, ntab, (int64_t)blockIdx.x) : one;
  const int lane = threadIdx.x, wave = lane >> 6;
  const int64_t n = D.numel;
  const int64_t e0 = ((int64_t)blockIdx.x - D.wg_begin) * kSElems + (int64_t)lane * 8;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);

  float g[8];
  load8<T>(reinterpret_cast<const T*>(D.grad), e0, n, g);
#pragma unroll
  for (int k = 0; k < 8; ++k) g[k] = scrub(g[k]);

  // ---- momentum
  float m[8];
  const int ML = (1 << h.lbm) >> 3;   // lanes per M block
  const int64_t mb = e0 >> h.lbm;
  const int64_t nmb = (n + (1 << h.lbm) - 1) >> h.lbm;
  const bool m_ok = MK == 1 && mb < nmb;   // codes are padded to whole blocks
  if constexpr (MK == 1) {
    float mo[8];
    mq_decode8(h.mk, D.m_q, D.m_scale, e0, mb, m_ok, mo);
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], g[k], h.w_m) : 0.0f;
  } else if constexpr (MK == 2) {
    float mo[8];
    load8<float>(D.m, e0, n, mo);
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], g[k], h.w_m) : 0.0f;
  }

  // ---- update and parameter
  if constexpr (MODE != 3) {
    float u[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) u[k] = (MK != 0) ? m[k] / h.mdiv : g[k];
    if constexpr (MODE == 1) {
      float sq = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) sq += u[k] * u[k];
      __shared__ float s_nw[4];
      const double t = wg_partial<4>(sq, s_nw);
      if (lane == 0) gp(D.norm_part)[(int64_t)blockIdx.x - D.wg_begin] = t;
    } else {
      const float a = D.alpha ? *D.alpha : h.alpha_val;
      float step = a;
      if constexpr (MODE == 2) {
        float sum = *D.norm_buf;
        if (D.fira) {
          // a non-finite norm zeroes the update (optimizer.py:797-800)
          const bool fin = __builtin_isfinite(sqrtf(sum));
          const float sc = fin ? D.fira[0] : 0.0f;
          sum = *D.fira_sum;
#pragma unroll
          for (int k = 0; k < 8; ++k) u[k] = u[k] * sc;
        }
        if (h.d > 0.0f) step = a / fmaxf(1.0f, sqrtf(sum) / (float)(sqrt((double)n) * (double)h.d));
      }
      const float dec = D.decay ? *D.decay : (h.has_decay ? h.decay_val : 1.0f);
      const bool use_dec = D.decay != nullptr || h.has_decay;
      pval_t<T> p[8];   // double for fp64 parameters
      load8<T>(reinterpret_cast<const T*>(D.param), e0, n, p);
      if constexpr (SR) {
        T* P = reinterpret_cast<T*>(D.param);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (k < cnt) P[e0 + k] = sr_round<T>(__builtin_fmaf(-step, u[k], p[k] * dec), D.sr_seed, h.sr_step,
                                               (uint64_t)(e0 + k));
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = pupd(step, u[k], use_dec ? pdec(p[k], dec) : p[k]);
        store8<T>(reinterpret_cast<T*>(D.param), e0, n, p);
      }
    }
  }

  // ---- momentum state
  if constexpr (MODE != 1 && MK == 2) {
    store8<float>(D.m, e0, n, m);
  }
  if constexpr (MODE == 3) {
    if (D.m_out) store8<float>(D.m_out, e0, n, m);
  }
  if constexpr (MODE != 1 && MK == 1) mq_encode8(h.mk, D.m_q, D.m_scale, e0, mb, m_ok, m, ML, xw);
}

// Coded momentum with a block size the reference accepts but the unit layout
// cannot take (B_M a multiple of 4, at least 32, not a power of two in
// [32, 2048]; up to 2^30).  One workgroup covers `unit` elements: floor(2048 /
// B_M) whole M blocks (one block when B_M > 2048).  Lanes take quads (a quad never
// straddles a block, B_M % 4 == 0); each block's absmax meets in LDS (an exact
// max).  Pass 1 forms m' and u and writes p (or m_out); pass 2, after the
// absmaxes, forms m' again from the same inputs and writes the codes.  The
// arithmetic is k_sgd's, element for element.
constexpr int kSGenMaxMB = 64;

template <typename T, int MODE, bool SR>
__global__ __launch_bounds__(kSLanes) void k_sgd_gen(SgdDesc one, const SgdDesc* __restrict__ table, int ntab,
                                                     SgdHyp h) {
  __shared__ uint32_t s_mab[kSGenMaxMB];
  sgd_step_scalars(h);
  const SgdDesc D = table ? *find_sgd(table, ntab, (int64_t)blockIdx.x) : one;
  const int lane = threadIdx.x;
  const int BM = h.bm, U = h.unit, mpu = U / BM;
  const int64_t n = D.numel;
  const int64_t base = ((int64_t)blockIdx.x - D.wg_begin) * U;
  const int64_t mb0 = base / BM, nmb = (n + BM - 1) / BM;
  const T* G = reinterpret_cast<const T*>(D.grad);
  T* P = reinterpret_cast<T*>(D.param);
  for (int i = lane; i < mpu; i += kSLanes) s_mab[i] = 0u;
  __syncthreads();

  auto quad = [&](int q, float* g, float* m, int& cnt, int& mb, bool& m_ok) {
    const int64_t i0 = base + 4 * q;
    cnt = i0 >= n ? 0 : (n - i0 >= 4 ? 4 : (int)(n - i0));
    load4n<T>(G, i0, n, g);
#pragma unroll
    for (int k = 0; k < 4; ++k) g[k] = scrub(g[k]);
    mb = (4 * q) / BM;
    m_ok = mb0 + mb < nmb;
    float mo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (m_ok) {
      const float ms = gp(D.m_scale)[mb0 + mb];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t e = i0 + k;
        uint32_t c;
        if (h.mk == 2 || h.mk == 4) {
          const uint32_t byte = gp(D.m_q)[e >> 1];
          c = (e & 1) ? (byte & 0x0Fu) : (byte >> 4);
        } else {
          c = gp(D.m_q)[e];
        }
        mo[k] = m_decode(h.mk, c, ms);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], g[k], h.w_m) : 0.0f;
  };

  float step = 0.0f, dec = 1.0f, fsc = 1.0f;   // fsc: the Fira scale of APPLY
  bool use_dec = false;
  if constexpr (MODE == 0 || MODE == 2) {
    const float a = D.alpha ? *D.alpha : h.alpha_val;
    step = a;
    if constexpr (MODE == 2) {
      float sum = *D.norm_buf;
      if (D.fira) {
        const bool fin = __builtin_isfinite(sqrtf(sum));   // a non-finite norm zeroes the update
        fsc = fin ? D.fira[0] : 0.0f;
        sum = *D.fira_sum;
      }
      if (h.d > 0.0f) step = a / fmaxf(1.0f, sqrtf(sum) / (float)(sqrt((double)n) * (double)h.d));
    }
    dec = D.decay ? *D.decay : (h.has_decay ? h.decay_val : 1.0f);
    use_dec = D.decay != nullptr || h.has_decay;
  }

  // ---- pass 1
  float sq = 0.0f;
  for (int q = lane; q < (U >> 2); q += kSLanes) {
    float g[4], m[4];
    int cnt, mb;
    bool m_ok;
    quad(q, g, m, cnt, mb, m_ok);
    const int64_t i0 = base + 4 * q;
    if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float u = m[k] / h.mdiv;
        sq += u * u;
      }
    } else if constexpr (MODE == 3) {
      if (D.m_out) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (k < cnt) gp(D.m_out)[i0 + k] = m[k];
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (k >= cnt) continue;
        float u = m[k] / h.mdiv;
        if constexpr (MODE == 2) {
          if (D.fira) u = u * fsc;
        }
        if constexpr (SR) {
          const float pv = ld1<T>(P, i0 + k);
          const T r = sr_round<T>(__builtin_fmaf(-step, u, pv * dec), D.sr_seed, h.sr_step, (uint64_t)(i0 + k));
          uint16_t bits;
          __builtin_memcpy(&bits, &r, 2);
          gp(reinterpret_cast<uint16_t*>(P))[i0 + k] = bits;
        } else {
          const pval_t<T> pv = ld1<T, pval_t<T>>(P, i0 + k);
          st1<T>(P, i0 + k, pupd(step, u, use_dec ? pdec(pv, dec) : pv));
        }
      }
    }
    if constexpr (MODE != 1) {
      uint32_t ab = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) ab = max(ab, __float_as_uint(m[k]) & 0x7FFFFFFFu);
      if (m_ok) atomicMax(&s_mab[mb], ab);
    }
  }
  if constexpr (MODE == 1) {
    __shared__ float s_nw[4];
    const double t = wg_partial<4>(sq, s_nw);
    if (lane == 0) gp(D.norm_part)[(int64_t)blockIdx.x - D.wg_begin] = t;
    return;
  }
  __syncthreads();

  // ---- pass 2: codes
  for (int q = lane; q < (U >> 2); q += kSLanes) {
    float g[4], m[4];
    int cnt, mb;
    bool m_ok;
    quad(q, g, m, cnt, mb, m_ok);
    if (!m_ok) continue;
    const int64_t i0 = base + 4 * q;
    const float am = fmaxf(__uint_as_float(s_mab[mb]), 1e-12f);
    const float ram = __builtin_amdgcn_rcpf(am);
    if (h.mk == 2 || h.mk == 4) {
      const uint32_t w = ((m_encode(h.mk, m[0], am, ram) << 4) | m_encode(h.mk, m[1], am, ram)) |
                         (((m_encode(h.mk, m[2], am, ram) << 4) | m_encode(h.mk, m[3], am, ram)) << 8);
      *gp(reinterpret_cast<uint16_t*>(D.m_q + (i0 >> 1))) = (uint16_t)w;
    } else {
      uint32_t w = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) w |= m_encode(h.mk, m[k], am, ram) << (8 * k);
      *gp(reinterpret_cast<uint32_t*>(D.m_q + i0)) = w;
    }
  }
  __syncthreads();   // every lane has read the old scales
  for (int i = lane; i < mpu; i += kSLanes)
    if (mb0 + i < nmb) gp(D.m_scale)[mb0 + i] = fmaxf(__uint_as_float(s_mab[i]), 1e-12f);
}

template <typename T, int MK, bool SR>
static void launch_mode(int mode, dim3 grid, hipStream_t st, const SgdDesc& one, const SgdDesc* tab, int ntab,
                        const SgdHyp& h) {
  if (MK == 1 && h.gen) {
    switch (mode) {
      case 0: hipLaunchKernelGGL((k_sgd_gen<T, 0, SR>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
      case 1: hipLaunchKernelGGL((k_sgd_gen<T, 1, SR>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
      case 2: hipLaunchKernelGGL((k_sgd_gen<T, 2, SR>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
      default: hipLaunchKernelGGL((k_sgd_gen<T, 3, false>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
    }
    return;
  }
  switch (mode) {
    case 0: hipLaunchKernelGGL((k_sgd<T, MK, 0, SR>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
    case 1: hipLaunchKernelGGL((k_sgd<T, MK, 1, SR>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
    case 2: hipLaunchKernelGGL((k_sgd<T, MK, 2, SR>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
    default: hipLaunchKernelGGL((k_sgd<T, MK, 3, false>), grid, dim3(kSLanes), 0, st, one, tab, ntab, h); break;
  }
}

template <typename T, bool SR>
static int launch_t(int mode, int mk, int64_t nwg, hipStream_t st, const SgdDesc& one, const SgdDesc* tab,
                    int ntab, const SgdHyp& h) {
  const dim3 grid((unsigned)nwg);
  if (mk == 0) launch_mode<T, 0, SR>(mode, grid, st, one, tab, ntab, h);
  else if (mk == 1) launch_mode<T, 1, SR>(mode, grid, st, one, tab, ntab, h);
  else launch_mode<T, 2, SR>(mode, grid, st, one, tab, ntab, h);
  return check_launch("k_sgd");
}

// Second launch of a NORM pass: one workgroup per tensor adds the tensor's
// partials in index order (sum_parts) to its norm_buf, which the caller zeroed.
__global__ __launch_bounds__(kSLanes) void k_sgd_fin(SgdDesc one, const SgdDesc* __restrict__ table, int ntab,
                                                    int64_t nwg) {
  __shared__ double s_w[4];
  const int i = (int)blockIdx.x;
  const SgdDesc D = table ? table[i] : one;
  const int64_t end = table ? (i + 1 < ntab ? table[i + 1].wg_begin : nwg) : nwg;
  const double s = sum_parts(D.norm_part, end - D.wg_begin, s_w);
  if (threadIdx.x == 0) *gp(D.norm_buf) += (float)s;
}

static int launch_sgd_body(int dtype, int stochastic, int mode, int kind, int64_t nwg, hipStream_t st,
                           const SgdDesc& one, const SgdDesc* tab, int ntab, const SgdHyp& h);

// kind: 0 no momentum, 1 quantised, 2 fp32 momentum.  NORM adds its finishing launch.
static int launch_sgd(int dtype, int stochastic, int mode, int kind, int64_t nwg, hipStream_t st,
                      const SgdDesc& one, const SgdDesc* tab, int ntab, const SgdHyp& h) {
  const int rc = launch_sgd_body(dtype, stochastic, mode, kind, nwg, st, one, tab, ntab, h);
  if (rc || mode != 1 || nwg <= 0) return rc;
  hipLaunchKernelGGL(k_sgd_fin, dim3(tab ? (unsigned)ntab : 1u), dim3(kSLanes), 0, st, one, tab, ntab, nwg);
  return check_launch("k_sgd_fin");
}

static int launch_sgd_body(int dtype, int stochastic, int mode, int kind, int64_t nwg, hipStream_t st,
                      const SgdDesc& one, const SgdDesc* tab, int ntab, const SgdHyp& h) {
  if (nwg <= 0) return 0;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "tensor too large");
  if (mode == 3) stochastic = 0;
  switch (dtype) {
    case A8_F32: return launch_t<float, false>(mode, kind, nwg, st, one, tab, ntab, h);
    case A8_BF16:
      return stochastic ? launch_t<__hip_bfloat16, true>(mode, kind, nwg, st, one, tab, ntab, h)
                        : launch_t<__hip_bfloat16, false>(mode, kind, nwg, st, one, tab, ntab, h);
    case A8_F16:
      return stochastic ? launch_t<__half, true>(mode, kind, nwg, st, one, tab, ntab, h)
                        : launch_t<__half, false>(mode, kind, nwg, st, one, tab, ntab, h);
    case A8_F64:
      if (mode == 3) return set_error(A8_ERR_DTYPE, "the momentum EMA input must be fp32, bf16 or fp16");
      return launch_t<double, false>(mode, kind, nwg, st, one, tab, ntab, h);
    default: return set_error(A8_ERR_DTYPE, "unsupported dtype");
  }
}

static int m_codec(int m_bits, int m_mode, int& mk) {
  if (m_bits == 8) mk = m_mode ? 3 : 1;
  else if (m_bits == 4) mk = m_mode ? 4 : 2;
  else return set_error(A8_ERR_ARG, "m_bits must be 8 or 4");
  return 0;
}

// The momentum block: a power of two in [32, 2048] takes the unit layout (lbm);
// any other multiple of 4 from 32 to 2^30 takes k_sgd_gen (gen, bm, unit).
static int block_log2(int bs, SgdHyp& h) {
  const bool pow2 = bs >= 32 && bs <= kSElems && (bs & (bs - 1)) == 0;
  if (!pow2 && !(bs >= 32 && bs % 4 == 0 && bs <= (1 << 30)))
    return set_error(A8_ERR_BLOCK, "m_block_size must be a multiple of 4 in [32, 2^30]");
  h.gen = pow2 ? 0 : 1;
  h.bm = bs;
  h.unit = pow2 ? kSElems : bs * (bs < kSElems ? kSElems / bs : 1);
  h.lbm = 0;
  while (pow2 && (1 << h.lbm) < bs) ++h.lbm;
  return 0;
}
static int64_t units_of(int64_t numel, const SgdHyp& h) {
  const int64_t u = h.gen ? h.unit : kSElems;
  return (numel + u - 1) / u;
}

hipError_t sgd_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

int64_t m_ema_table_bytes(int n) { return (int64_t)sizeof(SgdDesc) * (int64_t)n; }

// The standalone momentum EMA over n tensors in one launch (the table form of
// a8_m_quantize_lerp).  table_dev: m_ema_table_bytes(n) of device memory, or null
// for one launch per tensor (the descriptor then travels as a kernel argument).
int m_ema_multi(const MEmaItem* it, int n, void* table_dev, double beta, int block_size, int m_bits, int m_mode,
                hipStream_t st, int upload) {
  if (n <= 0) return 0;
  if (!table_dev && n > 1) {   // no table: one launch per tensor
    for (int i = 0; i < n; ++i) {
      const int rc = m_ema_multi(it + i, 1, nullptr, beta, block_size, m_bits, m_mode, st);
      if (rc) return rc;
    }
    return 0;
  }
  SgdHyp h{};
  int rc = m_codec(m_bits, m_mode, h.mk);
  if (rc) return rc;
  if ((rc = block_log2(block_size, h))) return rc;
  h.w_m = (float)(1.0 - beta);
  std::vector<SgdDesc> tab((size_t)n);
  int64_t wg = 0;
  for (int i = 0; i < n; ++i) {
    if (!it[i].m_q || !it[i].m_scale || !it[i].x) return set_error(A8_ERR_ARG, "null momentum state");
    if (!aligned16(it[i].x) || !aligned16(it[i].m_q) || (it[i].out && !aligned16(it[i].out)))
      return set_error(A8_ERR_ALIGN, "momentum codes, input and output must be 16-byte aligned");
    SgdDesc& D = tab[(size_t)i];
    D.grad = it[i].x; D.m_q = it[i].m_q; D.m_scale = it[i].m_scale; D.m_out = it[i].out; D.numel = it[i].n;
    D.wg_begin = wg;
    wg += units_of(it[i].n, h);
  }
  if (!table_dev) return launch_sgd(A8_F32, 0, 3, 1, wg, st, tab[0], nullptr, 0, h);
  if (upload && upload_table(table_dev, tab.data(), sizeof(SgdDesc) * (size_t)n, st) != hipSuccess)
    return set_error(A8_ERR_HIP, "table upload failed");
  SgdDesc none{};
  return launch_sgd(A8_F32, 0, 3, 1, wg, st, none, reinterpret_cast<const SgdDesc*>(table_dev), n, h);
}

}  // namespace a8

using namespace a8;

extern "C" {

int a8_sgd_step(int mode, int dtype, int stochastic, void* param, const void* grad, uint8_t* m_q, float* m_scale,
                float* m, float* norm_buf, double* norm_parts, const float* fira, const float* alpha, const float* decay, int64_t numel,
                double beta1, int m_bits, int m_mode, int m_block_size, float d, float alpha_val, float decay_val,
                int has_decay, uint64_t sr_seed, uint64_t sr_step, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (mode < 0 || mode > 2) return set_error(A8_ERR_ARG, "mode must be 0 (single), 1 (NORM) or 2 (APPLY)");
  if (numel == 0) return 0;
  if (!grad || (mode != 1 && !param)) return set_error(A8_ERR_ARG, "null param/grad");
  if (mode != 0 && !norm_buf) return set_error(A8_ERR_ARG, "null norm_buf");
  if (mode == 1 && !norm_parts) return set_error(A8_ERR_ARG, "NORM needs norm_parts (a8_norm_parts_sgd doubles)");
  if (m_q && m) return set_error(A8_ERR_ARG, "give quantised (m_q) or fp32 (m) momentum, not both");
  if (m_q && !m_scale) return set_error(A8_ERR_ARG, "null m_scale");
  if (!aligned16(grad) || (param && !aligned16(param)) || (m && !aligned16(m)) || (m_q && !aligned16(m_q)))
    return set_error(A8_ERR_ALIGN, "param, grad and momentum must be 16-byte aligned");
  SgdHyp h{};
  h.w_m = (float)(1.0 - beta1);
  h.mdiv = (float)(1.0 - beta1);
  h.d = d; h.alpha_val = alpha_val; h.decay_val = decay_val; h.has_decay = has_decay; h.sr_step = sr_step;
  int kind = 0;
  if (m_q) {
    kind = 1;
    int rc = m_codec(m_bits, m_mode, h.mk);
    if (rc) return rc;
    if ((rc = block_log2(m_block_size, h))) return rc;
  } else if (m) {
    kind = 2;
    h.lbm = 5;
  } else {
    h.lbm = 5;
  }
  SgdDesc D{};
  D.param = param; D.grad = grad; D.m_q = m_q; D.m_scale = m_scale; D.m = m; D.norm_buf = norm_buf;
  D.fira = fira; D.fira_sum = fira ? fira + 2 : nullptr;
  D.alpha = alpha; D.decay = decay; D.numel = numel; D.sr_seed = sr_seed;
  D.norm_part = norm_parts;
  return launch_sgd(dtype, stochastic, mode, kind, units_of(numel, h), (hipStream_t)stream, D,
                    nullptr, 0, h);
}

int a8_sgd_step_multi(int mode, int dtype, int stochastic, const a8_tensor_sgd* tensors, int ntensors,
                      void* table_dev, int64_t table_bytes, double beta1, int m_kind, int m_bits, int m_mode,
                      int m_block_size, float d, float alpha_val, float decay_val, int has_decay, uint64_t sr_step,
                      int upload, const void* step_scalars, void* stream) {
  if (ntensors <= 0) return 0;
  if (mode < 0 || mode > 2) return set_error(A8_ERR_ARG, "mode must be 0 (single), 1 (NORM) or 2 (APPLY)");
  if ((int64_t)sizeof(SgdDesc) * ntensors > table_bytes)
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_table_bytes_sgd(ntensors)");
  if (m_kind < 0 || m_kind > 2) return set_error(A8_ERR_ARG, "m_kind must be 0 (none), 1 (quantised), 2 (fp32)");
  SgdHyp h{};
  h.w_m = (float)(1.0 - beta1);
  h.mdiv = (float)(1.0 - beta1);
  h.d = d; h.alpha_val = alpha_val; h.decay_val = decay_val; h.has_decay = has_decay; h.sr_step = sr_step;
  h.dsc = reinterpret_cast<const a8_step_scalars*>(step_scalars);
  h.lbm = 5;
  if (m_kind == 1) {
    int rc = m_codec(m_bits, m_mode, h.mk);
    if (rc) return rc;
    if ((rc = block_log2(m_block_size, h))) return rc;
  }
  std::vector<SgdDesc> tab((size_t)ntensors);
  int64_t wg = 0;
  for (int i = 0; i < ntensors; ++i) {
    const a8_tensor_sgd& t = tensors[i];
    if (t.numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
    if (!t.grad || (mode != 1 && !t.param)) return set_error(A8_ERR_ARG, "null param/grad");
    if (mode != 0 && !t.norm_buf) return set_error(A8_ERR_ARG, "null norm_buf");
    if (mode == 1 && !t.norm_parts) return set_error(A8_ERR_ARG, "NORM needs norm_parts (a8_norm_parts_sgd doubles)");
    if (m_kind == 1 && (!t.m_q || !t.m_scale)) return set_error(A8_ERR_ARG, "null m_q/m_scale");
    if (m_kind == 2 && !t.m) return set_error(A8_ERR_ARG, "null m");
    if (!aligned16(t.grad) || (t.param && !aligned16(t.param)) || (m_kind == 2 && !aligned16(t.m)) ||
        (m_kind == 1 && !aligned16(t.m_q)))
      return set_error(A8_ERR_ALIGN, "param, grad and momentum must be 16-byte aligned");
    SgdDesc& D = tab[(size_t)i];
    D.param = t.param; D.grad = t.grad; D.norm_buf = t.norm_buf; D.fira = t.fira; D.norm_part = t.norm_parts;
    D.fira_sum = t.fira ? (t.fira_sum ? t.fira_sum : t.fira + 2) : nullptr;
    D.alpha = t.alpha; D.decay = t.decay; D.numel = t.numel; D.sr_seed = t.sr_seed;
    if (m_kind == 1) { D.m_q = t.m_q; D.m_scale = t.m_scale; }
    if (m_kind == 2) D.m = t.m;
    D.wg_begin = wg;
    wg += units_of(t.numel, h);
  }
  hipStream_t st = (hipStream_t)stream;
  if (upload && upload_table(table_dev, tab.data(), sizeof(SgdDesc) * (size_t)ntensors, st) != hipSuccess)
    return set_error(A8_ERR_HIP, "table upload failed");
  SgdDesc none{};
  return launch_sgd(dtype, stochastic, mode, m_kind, wg, st, none, reinterpret_cast<const SgdDesc*>(table_dev),
                    ntensors, h);
}

int64_t a8_table_bytes_sgd(int ntensors) { return (int64_t)sizeof(SgdDesc) * (int64_t)ntensors; }

int64_t a8_norm_parts_sgd(int64_t numel, int m_block_size) {
  SgdHyp h{};
  if (m_block_size > 0 && block_log2(m_block_size, h)) return -1;
  if (numel <= 0) return 0;
  return units_of(numel, h);
}

int a8_m_quantize_lerp(uint8_t* m_q, float* m_scale, const void* x, int x_dtype, float* fp32_out, double beta,
                       int block_size, int64_t numel, int m_bits, int m_mode, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!m_q || !m_scale || !x) return set_error(A8_ERR_ARG, "null pointer");
  if (!aligned16(x) || !aligned16(m_q) || (fp32_out && !aligned16(fp32_out)))
    return set_error(A8_ERR_ALIGN, "q, new_val and fp32_out must be 16-byte aligned");
  SgdHyp h{};
  int rc = m_codec(m_bits, m_mode, h.mk);
  if (rc) return rc;
  if ((rc = block_log2(block_size, h))) return rc;
  h.w_m = (float)(1.0 - beta);   // lerp weight of _m_ema_pytorch (optimizer.py:699)
  SgdDesc D{};
  D.grad = x; D.m_q = m_q; D.m_scale = m_scale; D.m_out = fp32_out; D.numel = numel;
  return launch_sgd(x_dtype, 0, 3, 1, units_of(numel, h), (hipStream_t)stream, D, nullptr, 0, h);
}

}  // extern "C"
