// Fused full-rank (1-D) optimizer step for MI355X (gfx950).
//
// One launch streams every element once: decode V (AL8/AL16) and M (UF8/UF4/
// D8/D4), EMA both, compute the update, write the parameter, refit the V block
// [l_min, l_max] and the M block absmax, and write the new codes.  Follows the
// reference's fused_update_1d kernels (kernels.cu:594-822 with M,
// kernels.cu:998-1098 without M) and, for the numbers it produces, the CPU
// path of _update_param_8bit (optimizer.py:2115-2123, 886-917).
//
// Layout: a 256-lane workgroup owns 2048 consecutive elements, 8 per lane held
// in VGPRs (two 16-byte loads of fp32 p/g, one 8-byte load of each code
// stream).  A V block of B_V elements is B_V/8 consecutive lanes and an M block
// of B_M elements is B_M/8 lanes, so both block reductions are butterfly
// shuffles inside a wave, plus one LDS exchange when B_V/8 > 64.  AL8 decode is
// a per-block 256-entry table in LDS (one exp2 per code instead of one per
// element).  A tensor table lets one launch cover many tensors.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

struct Desc1D {
  void* param;
  const void* grad;
  uint8_t* m_q;
  float* m_scale;
  void* v_q;
  float* v_scale;
  float* v_min_log;
  float* v_buf;
  float* norm_buf;
  const float* alpha;
  const float* prev_norm;
  const float* decay;
  int64_t numel;
  int64_t wg_begin;
  uint64_t sr_seed;
};

struct Hyper1D {
  float beta1;     // M EMA decay (kernel-rule arithmetic)
  float w_m;       // lerp weight of M: (float)(1 - beta1)
  float bv;        // lerp weight of V
  float eps_d;     // Adam denominator epsilon
  float eps_g;     // added to g^2
  float eps_sq;    // rsqrt floor
  float floor_;    // AL l_min floor
  float d;         // RMS clip threshold (APPLY/LAG)
  int block_size;
  int m_block_size;
  int mk;          // momentum codec
  int adam_denom;
  int momentum_only;
  int lbv;          // log2(block_size)
  int lbm;          // log2(m_block_size)
  float alpha_val;  // used when a tensor's alpha pointer is NULL
  float decay_val;  // used when a tensor's decay pointer is NULL and has_decay
  int has_decay;
  uint64_t sr_step;
};

// ------------------------------------------------------------ main kernel
constexpr int kLanes = 256;
constexpr int kEPT = 8;
constexpr int kWGElems = kLanes * kEPT;

// Tensor table in device memory: ntab descriptors, then one int32 first
// workgroup per tensor.  It is uniform per workgroup and read-only during the
// launch, so it is read through the scalar cache (constant address space): the
// search probes a compact 4-byte array and the descriptor arrives in SGPRs.
__device__ __forceinline__ Desc1D load_desc(const Desc1D* tab, int n, int wg) {
  const A8_C Desc1D* ct = cp(tab);
  const A8_C int32_t* wb = (const A8_C int32_t*)(ct + n);
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (wb[mid] <= wg) lo = mid; else hi = mid - 1;
  }
  static_assert(sizeof(Desc1D) % 8 == 0, "descriptor is loaded as 64-bit words");
  const A8_C uint64_t* w = (const A8_C uint64_t*)(ct + lo);
  uint64_t buf[sizeof(Desc1D) / 8];
#pragma unroll
  for (int i = 0; i < (int)(sizeof(Desc1D) / 8); ++i) buf[i] = w[i];
  Desc1D d;
  __builtin_memcpy(&d, buf, sizeof(Desc1D));
  return d;
}

// Integer view of a non-negative float minus one: for v >= 0 the unsigned
// order of these keys is the float order, and v == 0 maps to 0xFFFFFFFF, so an
// unsigned min over keys is the minimum over the non-zero entries.
__device__ __forceinline__ uint32_t nz_key(float v) { return __float_as_uint(v) - 1u; }
__device__ __forceinline__ uint32_t grp_umin(uint32_t x, int G) {
  for (int o = 1; o < G; o <<= 1) x = min(x, (uint32_t)__shfl_xor((int)x, o, 64));
  return x;
}

// MK: 0 no momentum, 1 UF8 (specialised), 2 UF4/D8/D4 (codec chosen by h.mk).
// MODE: 0 single pass, 1 NORM (V codes + v_buf, sum of squares), 2 APPLY (reads
// v_buf, writes M and p), 3 LAG (single pass clipped by the previous norm),
// 4 MNORM (momentum-only: reads v_buf, clips U by the NORM pass's sum of U^2 in
// prev_norm, and sums M'^2 for Fira; writes no state).
template <typename T, int VB, int MODE, bool SR, int MK>
__global__ __launch_bounds__(kLanes) void k_update1d(Desc1D one, const Desc1D* __restrict__ table,
                                                   int ntab, Hyper1D h) {
  extern __shared__ float s_lds[];  // [nv_wg * 256] AL8 tables | [16] cross-wave partials
  constexpr bool kHasM = MK != 0;
  constexpr bool kVbuf = MODE == 2 || MODE == 4;     // V comes from the NORM pass
  constexpr bool kSq = MODE == 1 || MODE == 3 || MODE == 4;
  constexpr bool kWrite = MODE == 0 || MODE == 2 || MODE == 3;   // p and M
  Desc1D D;
  if (table != nullptr) D = load_desc(table, ntab, (int)blockIdx.x);
  else D = one;
  const int64_t wl = (int64_t)blockIdx.x - D.wg_begin;
  const int lane = threadIdx.x;
  const int64_t n = D.numel;
  // block sizes are powers of two: all block arithmetic is shifts and masks
  const int lbv = h.lbv, lbm = h.lbm;
  const int BV = 1 << lbv, BM = 1 << lbm;
  const int VL = BV >> 3;                        // lanes per V block (16..256)
  const int ML = BM >> 3;                        // lanes per M block (4..256)
  const int nv_wg = kWGElems >> lbv;             // V blocks per workgroup
  const int64_t e0 = wl * kWGElems + (int64_t)lane * kEPT;
  const int64_t nvb = (n + BV - 1) >> lbv;
  const int64_t nmb = (n + BM - 1) >> lbm;
  const int64_t vb = e0 >> lbv;
  const int64_t mb = e0 >> lbm;
  const bool v_ok = vb < nvb;
  const bool m_ok = kHasM && (mb < nmb);
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= kEPT ? kEPT : (int)rem);   // valid elements of this lane
  const int vloc = lane >> (lbv - 3);
  const int mk = (MK == 1) ? 1 : h.mk;
  float* tabs = s_lds;
  float* xw = s_lds + ((VB == 8 && !kVbuf) ? nv_wg * 256 : 0);  // 4 waves x 4 | 4 fits x 4

  // ---- stream loads, issued before the decode table and its barrier so that
  // their latency overlaps the table build
  float g[kEPT], pin[kEPT];
  u32x2 vq8 = {0u, 0u}, mq8 = {0u, 0u};
  u32x4 vq16 = {0u, 0u, 0u, 0u};
  uint32_t mq4 = 0u;
  float ms = 0.0f;
#pragma unroll
  for (int k = 0; k < kEPT; ++k) { g[k] = 0.0f; pin[k] = 0.0f; }
  if (v_ok) {
    load8<T>(reinterpret_cast<const T*>(D.grad), e0, n, g);
    if constexpr (!kVbuf) {
      if constexpr (VB == 8) vq8 = *gp(reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(D.v_q) + e0));
      else vq16 = *gp(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(D.v_q) + e0));
    }
    if (m_ok) {
      ms = gp(D.m_scale)[mb];
      if (MK == 1 || !(mk == 2 || mk == 4)) mq8 = *gp(reinterpret_cast<const u32x2*>(D.m_q + e0));
      else mq4 = *gp(reinterpret_cast<const uint32_t*>(D.m_q + (e0 >> 1)));
    }
    if constexpr (kWrite && !SR) load8<T>(reinterpret_cast<const T*>(D.param), e0, n, pin);
  }

  // ---- AL8 decode tables for this workgroup's V blocks
  if constexpr (VB == 8 && !kVbuf) {
    const int64_t vb0 = wl * nv_wg;
    if (nv_wg == 1) {
      // one block per workgroup: its scale and min_log are uniform, read
      // through the scalar cache (each block's metadata is read here once and
      // rewritten at the end of this workgroup only)
      const int c = lane;
      float val = 0.0f;
      if (vb0 < nvb && c != 0) {
        const float sc = cp(D.v_scale)[vb0];
        const float lm = cp(D.v_min_log)[vb0];
        val = exp2_exact(((float)(c - 1) * sc) / 254.0f + lm);
      }
      tabs[c] = val;
    } else {
      for (int k = lane; k < nv_wg * 256; k += kLanes) {
        const int64_t b = vb0 + (k >> 8);
        const int c = k & 255;
        float val = 0.0f;
        if (b < nvb && c != 0) {
          const float sc = gp(D.v_scale)[b], lm = gp(D.v_min_log)[b];
          val = exp2_exact(((float)(c - 1) * sc) / 254.0f + lm);
        }
        tabs[k] = val;
      }
    }
    __syncthreads();
  }

  // ---- step scale
  float step = 0.0f, ut_clip = 1.0f;
  if constexpr (MODE != 1) {
    const float a = D.alpha ? *gp(D.alpha) : h.alpha_val;
    if constexpr (MODE == 0) {
      step = a;
    } else {
      float denom = 1.0f;
      if (h.d > 0.0f) {
        const float nrm = (MODE == 2) ? sqrtf(*gp(D.norm_buf))
                          : (MODE == 4 ? sqrtf(*gp(D.prev_norm)) : *gp(D.prev_norm));
        // U-clip of momentum_only divides by sqrt(n) then d (optimizer.py:894-895);
        // the update clip divides by sqrt(n)*d (optimizer.py:859-863)
        if (h.momentum_only && kHasM)
          denom = fmaxf(1.0f, (nrm / (float)sqrt((double)n)) / h.d);
        else
          denom = fmaxf(1.0f, nrm / (float)(sqrt((double)n) * (double)h.d));
      }
      if (h.momentum_only && kHasM) { step = a; ut_clip = denom; }
      else { step = a / denom; }
    }
  }

  float vn[kEPT], mn[kEPT];
  float sq = 0.0f;
  uint32_t vmaxb = 0u, amaxb = 0u;   // max of non-negative floats as integer bit patterns
  uint32_t vkey = 0xFFFFFFFFu;

  if (v_ok) {
    {  // non-finite gradients become 0 (kernels.cu:43-46); one test per lane
      float t = ((g[0] + g[1]) + (g[2] + g[3])) + ((g[4] + g[5]) + (g[6] + g[7]));
      if (!__builtin_isfinite(t)) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) g[k] = scrub(g[k]);
      }
    }

    // ---- V: decode + EMA (APPLY reads the exact V of the NORM pass)
    if constexpr (kVbuf) {
#pragma unroll
      for (int k = 0; k < kEPT; ++k) vn[k] = (k < cnt) ? gp(D.v_buf)[e0 + k] : 0.0f;
    } else {
      float vo[kEPT];
      if constexpr (VB == 8) {
        const u32x2 qv = vq8;
        const float* tb = tabs + vloc * 256;
#pragma unroll
        for (int k = 0; k < kEPT; ++k) vo[k] = tb[((k < 4 ? qv.x : qv.y) >> (8 * (k & 3))) & 0xFFu];
      } else {
        const float s_old = gp(D.v_scale)[vb], lm_old = gp(D.v_min_log)[vb];
        const u32x4 qv = vq16;
        const uint32_t w4[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int k = 0; k < kEPT; ++k) {
          const uint32_t c = (w4[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
          vo[k] = c ? exp2_exact(((float)(c - 1) * s_old) / 65534.0f + lm_old) : 0.0f;
        }
      }
      float gsq[kEPT];
#pragma unroll
      for (int k = 0; k < kEPT; ++k) gsq[k] = g[k] * g[k];
      if (h.eps_g != 0.0f) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) gsq[k] = gsq[k] + h.eps_g;
      }
      // torch.lerp: fma(w, e - s, s) for |w| < 0.5, else fma(w - 1, e - s, e)
      if (fabsf(h.bv) < 0.5f) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) vn[k] = __builtin_fmaf(h.bv, gsq[k] - vo[k], vo[k]);
      } else {
        const float c = h.bv - 1.0f;
#pragma unroll
        for (int k = 0; k < kEPT; ++k) vn[k] = __builtin_fmaf(c, gsq[k] - vo[k], gsq[k]);
      }
    }

    // ---- M decode
    float mo[kEPT];
#pragma unroll
    for (int k = 0; k < kEPT; ++k) mo[k] = 0.0f;
    if (m_ok) {
      if (MK == 1) {
        const u32x2 q = mq8;
        const float s128 = ms / 128.0f, b128 = -128.0f * s128;   // (q-128)*s128 == fma(q, s128, -128*s128)
#pragma unroll
        for (int k = 0; k < kEPT; ++k)
          mo[k] = __builtin_fmaf((float)(((k < 4 ? q.x : q.y) >> (8 * (k & 3))) & 0xFFu), s128, b128);
      } else if (mk == 2 || mk == 4) {
        const uint32_t qw = mq4;
#pragma unroll
        for (int k = 0; k < kEPT; ++k) {
          const uint32_t byte = (qw >> (8 * (k >> 1))) & 0xFFu;
          mo[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
        }
      } else {
        const u32x2 q = mq8;
#pragma unroll
        for (int k = 0; k < kEPT; ++k)
          mo[k] = m_decode(mk, ((k < 4 ? q.x : q.y) >> (8 * (k & 3))) & 0xFFu, ms);
      }
    }

    // ---- inverse second-moment denominators (uniform choice, hoisted)
    const bool mom = kHasM && h.momentum_only;
    float inv[kEPT];
    if (mom) {
      // feeds the momentum codes: IEEE sqrt then division, as torch's
      // variance.clamp(min=eps_sq).rsqrt() on the CPU (optimizer.py:893)
#pragma unroll
      for (int k = 0; k < kEPT; ++k) inv[k] = 1.0f / sqrtf(fmaxf(vn[k], h.eps_sq));
    } else if (h.adam_denom) {
#pragma unroll
      for (int k = 0; k < kEPT; ++k) inv[k] = fast_rcp(fast_sqrt(vn[k]) + h.eps_d);
    } else {
#pragma unroll
      for (int k = 0; k < kEPT; ++k) inv[k] = __builtin_amdgcn_rsqf(fmaxf(vn[k], h.eps_sq));
    }

    // ---- M EMA and update direction
    float uu[kEPT];
    if constexpr (kHasM) {
      float x[kEPT];
      if (mom) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) {
          const float ut = g[k] * inv[k];
          if (MODE == 1 || MODE == 3) sq = __builtin_fmaf(ut, ut, sq);
          x[k] = ut;
        }
        if (ut_clip != 1.0f) {
#pragma unroll
          for (int k = 0; k < kEPT; ++k) x[k] = x[k] / ut_clip;
        }
      } else {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) x[k] = g[k];
      }
      if (fabsf(h.w_m) < 0.5f) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) mn[k] = __builtin_fmaf(h.w_m, x[k] - mo[k], mo[k]);
      } else {
        const float c = h.w_m - 1.0f;
#pragma unroll
        for (int k = 0; k < kEPT; ++k) mn[k] = __builtin_fmaf(c, x[k] - mo[k], x[k]);
      }
      if (mom) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) {
          uu[k] = mn[k];
          if (MODE == 4) sq = __builtin_fmaf(mn[k], mn[k], sq);
        }
      } else {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) {
          uu[k] = mn[k] * inv[k];
          if (MODE == 1 || MODE == 3) sq = __builtin_fmaf(uu[k], uu[k], sq);
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < kEPT; ++k) {
        mn[k] = 0.0f;
        uu[k] = g[k] * inv[k];
        if (MODE == 1 || MODE == 3) sq = __builtin_fmaf(uu[k], uu[k], sq);
      }
    }
    if (cnt < kEPT) {  // the last lane of a tensor: padding elements hold zero state
      sq = 0.0f;
#pragma unroll
      for (int k = 0; k < kEPT; ++k) {
        if (k >= cnt) { vn[k] = 0.0f; mn[k] = 0.0f; uu[k] = 0.0f; }
        const float ut = (MODE == 4) ? mn[k] : (mom ? g[k] * inv[k] : uu[k]);
        if (kSq && k < cnt) sq = __builtin_fmaf(ut, ut, sq);
      }
    }
    if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < kEPT; ++k)
        if (k < cnt) gp(D.v_buf)[e0 + k] = vn[k];
    }
#pragma unroll
    for (int k = 0; k < kEPT; ++k) {
      vmaxb = max(vmaxb, __float_as_uint(vn[k]));
      vkey = min(vkey, nz_key(vn[k]));
      amaxb = max(amaxb, __float_as_uint(mn[k]) & 0x7FFFFFFFu);
    }

    // ---- parameter write
    if constexpr (kWrite) {
      T* P = reinterpret_cast<T*>(D.param);
      const bool has_dec = D.decay || h.has_decay;
      const float dec = D.decay ? *gp(D.decay) : (h.has_decay ? h.decay_val : 1.0f);
      if constexpr (SR) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) {
          if (k < cnt) {
            const float pv = ld1<T>(P, e0 + k);
            const T r = sr_round<T>(pv * dec - step * uu[k], D.sr_seed, h.sr_step, (uint64_t)(e0 + k));
            uint16_t bits;
            __builtin_memcpy(&bits, &r, 2);
            gp(reinterpret_cast<uint16_t*>(P))[e0 + k] = bits;
          }
        }
      } else {
        float p[kEPT];
#pragma unroll
        for (int k = 0; k < kEPT; ++k) p[k] = pin[k];
        if (has_dec) {  // decoupled weight decay: p*decay rounded, then the update (optimizer.py:2039)
#pragma unroll
          for (int k = 0; k < kEPT; ++k) p[k] = p[k] * dec;
        }
#pragma unroll
        for (int k = 0; k < kEPT; ++k) p[k] = __builtin_fmaf(-step, uu[k], p[k]);
        store8<T>(P, e0, n, p);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < kEPT; ++k) { vn[k] = 0.0f; mn[k] = 0.0f; }
  }
  const float vmax = __uint_as_float(vmaxb);
  const float amax = __uint_as_float(amaxb);

  const int wave = lane >> 6;

  // ---- V refit + codes
  if constexpr (!kVbuf) {
    float bmax = grp_max(vmax, VL < 64 ? VL : 64);
    uint32_t bkey = grp_umin(vkey, VL < 64 ? VL : 64);
    const float lm2 = VB == 8 ? 254.0f : 65534.0f;
    ALFit f;
    if (VL > 64) {
      // a V block spans VL/64 waves: wave 0 refits every block of the workgroup
      // (lane pair 2j, 2j+1 for block j) and shares the fit through LDS, so
      // the other waves do not repeat the correctly rounded logarithms.
      if ((lane & 63) == 0) { xw[wave * 4 + 0] = bmax; xw[wave * 4 + 1] = __uint_as_float(bkey); }
      __syncthreads();
      if (wave == 0) {
        const int j = (lane >> 1) < nv_wg ? (lane >> 1) : 0;
        const int wpb = VL >> 6;   // waves per block
        float mx = xw[(j * wpb) * 4];
        uint32_t ky = __float_as_uint(xw[(j * wpb) * 4 + 1]);
        for (int w = 1; w < wpb; ++w) {
          mx = fmaxf(mx, xw[(j * wpb + w) * 4]);
          ky = min(ky, __float_as_uint(xw[(j * wpb + w) * 4 + 1]));
        }
        const float mn_ = (ky == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(ky + 1u);
        const ALFit g = al_refit_pair(mx, mn_, h.floor_, lm2, lane);
        if ((lane & 1) == 0 && (lane >> 1) < nv_wg) {
          float* xf = xw + 16 + (lane >> 1) * 8;
          xf[0] = g.lmin; xf[1] = g.s; xf[2] = g.k; xf[3] = g.c1; xf[4] = g.kmar; xf[5] = g.cmar;
        }
      }
      __syncthreads();
      const float* xf = xw + 16 + vloc * 8;
      f.lmin = xf[0]; f.s = xf[1]; f.k = xf[2]; f.c1 = xf[3]; f.kmar = xf[4]; f.cmar = xf[5];
    } else {
      const float bmin = (bkey == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey + 1u);
      f = al_refit_pair(bmax, bmin, h.floor_, lm2, lane);
    }
    {
      if (v_ok) {
      if constexpr (VB == 8) {
        float r[kEPT];
        bool bad[kEPT];
#pragma unroll
        for (int k = 0; k < kEPT; ++k) r[k] = al8_round_fast(vn[k], f, bad[k]);
#pragma unroll
        for (int k = 0; k < kEPT; ++k)
          if (bad[k]) r[k] = al_round_exact<254>(vn[k], f);
#pragma unroll
        for (int k = 0; k < kEPT; ++k) r[k] = al_clamp<254>(vn[k], r[k]);
        *gp(reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(D.v_q) + e0)) =
            u32x2{pack4(r[0], r[1], r[2], r[3]), pack4(r[4], r[5], r[6], r[7])};
      } else {
        uint32_t q[kEPT];
#pragma unroll
        for (int k = 0; k < kEPT; ++k) q[k] = al_finish<65534>(vn[k], al_round_exact<65534>(vn[k], f));
        *gp(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(D.v_q) + e0)) =
            u32x4{q[0] | (q[1] << 16), q[2] | (q[3] << 16), q[4] | (q[5] << 16), q[6] | (q[7] << 16)};
      }
      if ((lane & (VL - 1)) == 0) { gp(D.v_scale)[vb] = f.s; gp(D.v_min_log)[vb] = f.lmin; }
      }
    }
  }

  // ---- M refit + codes
  if constexpr (kWrite && kHasM) {
    float bam = grp_max(amax, ML < 64 ? ML : 64);
    if (ML > 64) {
      __syncthreads();
      if ((lane & 63) == 0) xw[wave * 4 + 2] = bam;
      __syncthreads();
      const int w0 = (lane >> (lbm - 3)) * (ML >> 6);
      bam = xw[w0 * 4 + 2];
      for (int w = 1; w < (ML >> 6); ++w) bam = fmaxf(bam, xw[(w0 + w) * 4 + 2]);
    }
    if (m_ok) {
      const float am = fmaxf(bam, 1e-12f);
      const float ram = fast_rcp(am);
      if (MK == 1) {
        const float kam = 128.0f * ram;
        float r[kEPT];
        bool bad[kEPT];
#pragma unroll
        for (int k = 0; k < kEPT; ++k) r[k] = uf_round_fast<128>(mn[k], kam, bad[k]);
#pragma unroll
        for (int k = 0; k < kEPT; ++k)
          if (bad[k]) r[k] = uf_round_exact<128>(mn[k], am);
#pragma unroll
        for (int k = 0; k < kEPT; ++k) r[k] = uf_clamp<128>(r[k]);
        *gp(reinterpret_cast<u32x2*>(D.m_q + e0)) =
            u32x2{pack4(r[0], r[1], r[2], r[3]), pack4(r[4], r[5], r[6], r[7])};
      } else if (mk == 2 || mk == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t hi = m_encode(mk, mn[2 * j], am, ram);
          const uint32_t lo = m_encode(mk, mn[2 * j + 1], am, ram);
          w |= ((hi << 4) | lo) << (8 * j);
        }
        *gp(reinterpret_cast<uint32_t*>(D.m_q + (e0 >> 1))) = w;
      } else {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w0 |= m_encode(mk, mn[k], am, ram) << (8 * k);
#pragma unroll
        for (int k = 0; k < 4; ++k) w1 |= m_encode(mk, mn[k + 4], am, ram) << (8 * k);
        *gp(reinterpret_cast<u32x2*>(D.m_q + e0)) = u32x2{w0, w1};
      }
      if ((lane & (ML - 1)) == 0) gp(D.m_scale)[mb] = am;
    }
  }

  // ---- sum of squares for NORM / LAG / MNORM
  if constexpr (kSq) {
    const float t = grp_sum(sq, 64);
    if ((lane & 63) == 0 && t != 0.0f) atomicAdd(D.norm_buf, t);
  }
}

// ------------------------------------------------------------ launch glue
static bool fast_shape_ok(int bv, int bm) {
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  return pow2(bv) && bv >= 128 && bv <= 2048 && pow2(bm) && bm >= 32 && bm <= bv;
}

template <typename T, int VB, int MODE, bool SR, int MK>
static int launch_t(const Desc1D& one, const Desc1D* table, int ntab, int64_t nwg, const Hyper1D& h,
                    hipStream_t st) {
  const int nv_wg = kWGElems / h.block_size;
  size_t lds = ((VB == 8 && MODE != 2 && MODE != 4) ? (size_t)nv_wg * 256 : 0) * sizeof(float) +
               48 * sizeof(float);
  if (nwg <= 0) return 0;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "too many workgroups");
  hipLaunchKernelGGL((k_update1d<T, VB, MODE, SR, MK>), dim3((unsigned)nwg), dim3(kLanes), lds, st, one,
                     table, ntab, h);
  return check_launch("k_update1d");
}

template <typename T, bool SR, int MK>
static int launch_mode(int vbits, int mode, const Desc1D& one, const Desc1D* table, int ntab,
                       int64_t nwg, const Hyper1D& h, hipStream_t st) {
#define A8_L(VB, MO) return launch_t<T, VB, MO, SR, MK>(one, table, ntab, nwg, h, st)
  if (mode == 4) {
    if constexpr (MK == 0 || SR) {
      return set_error(A8_ERR_ARG, "MNORM needs momentum codes");
    } else {
      if (vbits == 8) A8_L(8, 4);
      A8_L(16, 4);
    }
  }
  if (vbits == 8) {
    switch (mode) { case 0: A8_L(8, 0); case 1: A8_L(8, 1); case 2: A8_L(8, 2); default: A8_L(8, 3); }
  } else {
    switch (mode) { case 0: A8_L(16, 0); case 1: A8_L(16, 1); case 2: A8_L(16, 2); default: A8_L(16, 3); }
  }
#undef A8_L
}

template <typename T, bool SR>
static int launch_dispatch(int vbits, int mode, const Desc1D& one, const Desc1D* table, int ntab,
                           int64_t nwg, const Hyper1D& h, hipStream_t st) {
  switch (h.mk) {
    case 0: return launch_mode<T, SR, 0>(vbits, mode, one, table, ntab, nwg, h, st);
    case 1: return launch_mode<T, SR, 1>(vbits, mode, one, table, ntab, nwg, h, st);
    default: return launch_mode<T, SR, 2>(vbits, mode, one, table, ntab, nwg, h, st);
  }
}

static int launch_any(int dtype, int sr, int vbits, int mode, const Desc1D& one, const Desc1D* table,
                      int ntab, int64_t nwg, const Hyper1D& h, hipStream_t st) {
  if ((mode == 1 || mode == 4) && sr) sr = 0;
  switch (dtype) {
    case A8_F32: return launch_dispatch<float, false>(vbits, mode, one, table, ntab, nwg, h, st);
    case A8_BF16:
      return sr ? launch_dispatch<__hip_bfloat16, true>(vbits, mode, one, table, ntab, nwg, h, st)
                : launch_dispatch<__hip_bfloat16, false>(vbits, mode, one, table, ntab, nwg, h, st);
    case A8_F16:
      return sr ? launch_dispatch<__half, true>(vbits, mode, one, table, ntab, nwg, h, st)
                : launch_dispatch<__half, false>(vbits, mode, one, table, ntab, nwg, h, st);
    default: return set_error(A8_ERR_DTYPE, "unsupported param dtype");
  }
}

static int check_common(int dtype, int64_t numel, int bv, int bm, int mbits, int mmode, int vbits,
                        bool has_m) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (vbits != 8 && vbits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  if (!has_m) bm = bv;
  if (!fast_shape_ok(bv, bm))
    return set_error(A8_ERR_BLOCK, "block_size must be a power of two in [128, 2048] and "
                                   "m_block_size a power of two in [32, block_size]");
  if (has_m && !((mbits == 8 || mbits == 4) && (mmode == 0 || mmode == 1)))
    return set_error(A8_ERR_ARG, "m_bits must be 4/8 and m_mode 0/1");
  if (dtype != A8_F32 && dtype != A8_BF16 && dtype != A8_F16) return set_error(A8_ERR_DTYPE, "dtype");
  return 0;
}

static int ilog2(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

static int mk_of(int mbits, int mmode) {
  if (mmode == 0) return mbits == 8 ? 1 : 2;
  return mbits == 8 ? 3 : 4;
}

}  // namespace a8

using namespace a8;

// ============================================================== C-ABI
static int update1d_entry(int mode, int sr, int dtype, void* param, const void* grad, uint8_t* m_q,
                          float* m_scale, void* v_q, float* v_scale, float* v_min_log, float* v_buf,
                          float* norm_buf, const float* alpha, const float* prev_norm,
                          const float* decay, uint64_t sr_seed, uint64_t sr_step, double beta1,
                          double beta_val, float eps_for_denom, int use_adam_denom, float log_floor,
                          float eps_for_grad_sq, float eps_sq, int64_t numel, int block_size,
                          int m_block_size, int m_bits, int m_mode, float d, int v_bits,
                          int momentum_only, float alpha_val, float decay_val, int has_decay,
                          void* stream) {
  const bool has_m = m_q != nullptr;
  int rc = check_common(dtype, numel, block_size, m_block_size, m_bits, m_mode, v_bits, has_m);
  if (rc) return rc;
  if (!v_q || !v_scale || !v_min_log || !grad || (has_m && !m_scale))
    return set_error(A8_ERR_ARG, "null state pointer");
  if (mode < 0 || mode > 4) return set_error(A8_ERR_ARG, "mode must be 0..4");
  if (mode != 1 && mode != 4 && !param) return set_error(A8_ERR_ARG, "null param");
  if ((mode == 1 || mode == 2 || mode == 4) && !v_buf) return set_error(A8_ERR_ARG, "NORM/APPLY/MNORM need v_buf");
  if (mode == 4 && !(norm_buf && prev_norm && has_m && momentum_only))
    return set_error(A8_ERR_ARG, "MNORM needs momentum codes, momentum_only, norm_buf and prev_norm");
  if ((mode == 1 || mode == 3) && !norm_buf) return set_error(A8_ERR_ARG, "NORM/LAG need norm_buf");
  if (mode == 2 && !norm_buf) return set_error(A8_ERR_ARG, "APPLY needs norm_buf");
  if (mode == 3 && !prev_norm) return set_error(A8_ERR_ARG, "LAG needs prev_norm");
  if (!aligned16(param) || !aligned16(grad) || !aligned16(v_q) || (has_m && !aligned16(m_q)))
    return set_error(A8_ERR_ALIGN, "param/grad/code buffers must be 16-byte aligned");
  Desc1D D{};
  D.param = param; D.grad = grad; D.m_q = m_q; D.m_scale = m_scale;
  D.v_q = v_q; D.v_scale = v_scale; D.v_min_log = v_min_log; D.v_buf = v_buf;
  D.norm_buf = norm_buf; D.alpha = alpha; D.prev_norm = prev_norm; D.decay = decay;
  D.numel = numel; D.wg_begin = 0; D.sr_seed = sr_seed;
  Hyper1D h{};
  h.beta1 = (float)beta1;
  h.w_m = (float)(1.0 - beta1);
  h.bv = (float)beta_val;
  h.eps_d = eps_for_denom; h.eps_g = eps_for_grad_sq; h.eps_sq = eps_sq;
  h.floor_ = log_floor; h.d = d;
  h.block_size = block_size; h.m_block_size = has_m ? m_block_size : block_size;
  h.lbv = ilog2(h.block_size); h.lbm = ilog2(h.m_block_size);
  h.mk = has_m ? mk_of(m_bits, m_mode) : 0;
  h.adam_denom = use_adam_denom; h.momentum_only = momentum_only;
  h.alpha_val = alpha_val; h.decay_val = decay_val; h.has_decay = has_decay;
  h.sr_step = sr_step;
  const int64_t nwg = (numel + kWGElems - 1) / kWGElems;
  return launch_any(dtype, sr, v_bits, mode, D, nullptr, 0, nwg, h, (hipStream_t)stream);
}

extern "C" {

int a8_fused_update_1d(int mode, int stochastic, int dtype, void* param, const void* grad,
                       uint8_t* m_q, float* m_scale, void* v_q, float* v_scale, float* v_min_log,
                       float* v_buf, float* norm_buf, const float* alpha, const float* prev_norm,
                       const float* decay, uint64_t sr_seed, uint64_t sr_step, double beta1,
                       double beta_val, float eps_for_denom, int use_adam_denom, float log_floor,
                       float eps_for_grad_sq, float eps_sq, int64_t numel, int block_size,
                       int m_block_size, int m_bits, int m_mode, float d, int v_bits,
                       int momentum_only, float alpha_val, float decay_val, int has_decay,
                       void* stream) {
  return update1d_entry(mode, stochastic, dtype, param, grad, m_q, m_scale, v_q, v_scale, v_min_log,
                        v_buf, norm_buf, alpha, prev_norm, decay, sr_seed, sr_step, beta1, beta_val,
                        eps_for_denom, use_adam_denom, log_floor, eps_for_grad_sq, eps_sq, numel,
                        block_size, m_block_size, m_bits, m_mode, d, v_bits, momentum_only, alpha_val,
                        decay_val, has_decay, stream);
}

int a8_fused_update_1d_multi(int mode, int stochastic, int dtype, const a8_tensor1d* tensors,
                             int ntensors, void* table_dev, int64_t table_bytes, double beta1,
                             double beta_val, float eps_for_denom, int use_adam_denom,
                             float log_floor, float eps_for_grad_sq, float eps_sq, int block_size,
                             int m_block_size, int m_bits, int m_mode, float d, int v_bits,
                             int momentum_only, uint64_t sr_step, float alpha_val,
                             float decay_val, int has_decay, int upload, void* stream) {
  if (ntensors <= 0) return 0;
  const bool has_m = tensors[0].m_q != nullptr;
  int rc = check_common(dtype, 0, block_size, m_block_size, m_bits, m_mode, v_bits, has_m);
  if (rc) return rc;
  if (a8_table_bytes_1d(ntensors) > table_bytes)
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_table_bytes_1d(ntensors)");
  if (mode < 0 || mode > 4) return set_error(A8_ERR_ARG, "mode must be 0..4");
  if (mode == 4 && !momentum_only) return set_error(A8_ERR_ARG, "MNORM needs momentum_only");
  std::vector<Desc1D> tab((size_t)ntensors);
  std::vector<int32_t> first((size_t)ntensors);
  int64_t wg = 0;
  for (int i = 0; i < ntensors; ++i) {
    const a8_tensor1d& t = tensors[i];
    if ((t.m_q != nullptr) != has_m) return set_error(A8_ERR_ARG, "mixed M / no-M tensors in one launch");
    if (!t.grad || !t.v_q || !t.v_scale || !t.v_min_log || (has_m && !t.m_scale))
      return set_error(A8_ERR_ARG, "null state pointer");
    if (mode != 1 && mode != 4 && !t.param) return set_error(A8_ERR_ARG, "null param");
    if ((mode == 1 || mode == 2 || mode == 4) && !t.v_buf)
      return set_error(A8_ERR_ARG, "NORM/APPLY/MNORM need v_buf");
    if (mode != 0 && !t.norm_buf) return set_error(A8_ERR_ARG, "NORM/APPLY/LAG/MNORM need norm_buf");
    if ((mode == 3 || mode == 4) && !t.prev_norm) return set_error(A8_ERR_ARG, "LAG/MNORM need prev_norm");
    if (mode == 4 && !has_m) return set_error(A8_ERR_ARG, "MNORM needs momentum codes");
    if (!aligned16(t.param) || !aligned16(t.grad) || !aligned16(t.v_q) || (has_m && !aligned16(t.m_q)))
      return set_error(A8_ERR_ALIGN, "param/grad/code buffers must be 16-byte aligned");
    if (t.numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
    Desc1D& D = tab[(size_t)i];
    D.param = t.param; D.grad = t.grad; D.m_q = t.m_q; D.m_scale = t.m_scale;
    D.v_q = t.v_q; D.v_scale = t.v_scale; D.v_min_log = t.v_min_log; D.v_buf = t.v_buf;
    D.norm_buf = t.norm_buf; D.alpha = t.alpha; D.prev_norm = t.prev_norm; D.decay = t.decay;
    D.numel = t.numel; D.wg_begin = wg; D.sr_seed = t.sr_seed;
    first[(size_t)i] = (int32_t)(wg < 0x7FFFFFFF ? wg : 0x7FFFFFFF);
    wg += (t.numel + kWGElems - 1) / kWGElems;
  }
  if (wg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "too many workgroups");
  hipStream_t st = (hipStream_t)stream;
  if (upload) {
    // one staging copy: descriptors followed by the first-workgroup array
    std::vector<char> blob((size_t)a8_table_bytes_1d(ntensors));
    std::memcpy(blob.data(), tab.data(), sizeof(Desc1D) * (size_t)ntensors);
    std::memcpy(blob.data() + sizeof(Desc1D) * (size_t)ntensors, first.data(), sizeof(int32_t) * (size_t)ntensors);
    if (hipMemcpyAsync(table_dev, blob.data(), blob.size(), hipMemcpyHostToDevice, st) != hipSuccess)
      return set_error(A8_ERR_HIP, "table upload failed");
  }
  Hyper1D h{};
  h.beta1 = (float)beta1;
  h.w_m = (float)(1.0 - beta1);
  h.bv = (float)beta_val;
  h.eps_d = eps_for_denom; h.eps_g = eps_for_grad_sq; h.eps_sq = eps_sq;
  h.floor_ = log_floor; h.d = d;
  h.block_size = block_size; h.m_block_size = has_m ? m_block_size : block_size;
  h.lbv = ilog2(h.block_size); h.lbm = ilog2(h.m_block_size);
  h.mk = has_m ? mk_of(m_bits, m_mode) : 0;
  h.adam_denom = use_adam_denom; h.momentum_only = momentum_only;
  h.alpha_val = alpha_val; h.decay_val = decay_val; h.has_decay = has_decay;
  h.sr_step = sr_step;
  Desc1D none{};
  return launch_any(dtype, stochastic, v_bits, mode, none, reinterpret_cast<const Desc1D*>(table_dev),
                    ntensors, wg, h, st);
}

int64_t a8_table_bytes_1d(int ntensors) {
  return ((int64_t)sizeof(Desc1D) + (int64_t)sizeof(int32_t)) * (int64_t)ntensors;
}

int a8_set_qmap(const float* qmap8_host, const float* qmap4_host) {
  if (!qmap8_host || !qmap4_host) return set_error(A8_ERR_ARG, "null codebook");
  if (upload_qmap_tu(qmap8_host, qmap4_host) != hipSuccess ||
      a8::factored_upload_qmap(qmap8_host, qmap4_host) != hipSuccess)
    return set_error(A8_ERR_HIP, "codebook upload failed");
  return 0;
}

}  // extern "C"
