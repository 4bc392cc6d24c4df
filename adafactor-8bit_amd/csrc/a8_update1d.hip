// Fused full-rank (1-D) optimizer step for MI355X (gfx950).
//
// One launch streams every element once: decode V (AL8/AL16) and M (UF8/UF4/
// D8/D4), EMA both, compute the update, write the parameter, refit the V block
// [l_min, l_max] and the M block absmax, and write the new codes.  Follows the
// reference's fused_update_1d kernels (kernels.cu:594-822 with M,
// kernels.cu:998-1098 without M) and, for the numbers it produces, the CPU
// path of _update_param_8bit (optimizer.py:2115-2123, 886-917).
//
// Layout: a 256-lane workgroup owns 2048 consecutive elements as two halves of
// 1024; lane t holds elements 4t..4t+3 of each half in VGPRs, so every
// wave-wide access (16 bytes of fp32 p/g, 4 bytes of each code stream per lane)
// covers one contiguous span.  A V block of B_V <= 1024 elements is B_V/4
// consecutive lanes of a half and an M block B_M/4 lanes, so block reductions
// are butterfly shuffles inside a wave, plus one LDS exchange when a block
// spans several waves.  AL8 decode is a per-block 256-entry table in LDS (one
// exp2 per code instead of one per element).  A tensor table lets one launch
// cover many tensors.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

#include <mutex>

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
  const float* fira_scale;   // APPLY: Fira limiter scale multiplied into the step, or null
  double* norm_part;         // NORM / LAG / MNORM: one partial sum of squares per workgroup
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
  const a8_step_scalars* dsc;   // if set: bv, eps_d, alpha_val, decay_val and sr_step come from here
  int gen;          // block sizes the unit layout cannot take: k_update1d_gen, one V block per workgroup
};

// ------------------------------------------------------------ main kernel
constexpr int kLanes = 256;
constexpr int kEPT = 8;
constexpr int kWGElems = kLanes * kEPT;
constexpr int kHalf = kWGElems / 2;

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

// MK: 0 no momentum, 1 UF8 (specialised), 2 UF4/D8/D4 (codec chosen by h.mk).
// MODE: 0 single pass, 1 NORM (V codes + v_buf, sum of squares), 2 APPLY (reads
// v_buf, writes M and p), 3 LAG (single pass clipped by the previous norm),
// 4 MNORM (momentum-only: reads v_buf, clips U by the NORM pass's sum of U^2 in
// prev_norm, and sums M'^2 for Fira; writes no state).
//
// Lane t of a workgroup holds elements j*1024 + 4t + i of its 2048-element
// unit (half j = 0, 1; i = 0..3), at register index k = 4j + i: every
// wave-wide 16-byte access covers 1 KB of contiguous memory.  A V block of
// B_V <= 1024 elements is B_V/4 consecutive lanes in each half (so a lane holds
// two blocks, one per half); B_V = 2048 is the whole workgroup.  M blocks map
// the same way with B_M.
//
// FULL: the unit lies entirely inside the tensor (every unit but a tensor's
// last): no lane is partial or outside the tensor's blocks, so every load is
// unconditional; the workgroup chooses its body once, and the two bodies never
// rejoin.
template <typename T, int VB, int MODE, bool SR, int MK, bool FULL>
__device__ __forceinline__ void unit_step(const Desc1D& D, const Hyper1D& h, int64_t wl, float* s_lds) {
  constexpr bool kHasM = MK != 0;
  constexpr bool kVbuf = MODE == 2 || MODE == 4;     // V comes from the NORM pass
  constexpr bool kSq = MODE == 1 || MODE == 3 || MODE == 4;
  constexpr bool kWrite = MODE == 0 || MODE == 2 || MODE == 3;   // p and M
  const int lane = threadIdx.x;
  const int wave = lane >> 6;
  const int64_t n = D.numel;
  // block sizes are powers of two: all block arithmetic is shifts and masks
  const int lbv = h.lbv, lbm = h.lbm;
  const int BV = 1 << lbv, BM = 1 << lbm;
  const bool vwhole = BV == kWGElems;            // one V block spans the workgroup
  const bool mwhole = BM == kWGElems;
  const int VLh = vwhole ? kLanes : (BV >> 2);   // lanes per V block in one half
  const int MLh = mwhole ? kLanes : (BM >> 2);   // lanes per M block in one half
  const int nv_wg = kWGElems >> lbv;             // V blocks per workgroup
  // Addresses are a uniform (SGPR) base of this unit plus a 32-bit lane offset,
  // so the loads and stores use SGPR-based addressing and no 64-bit VGPR pairs.
  const int64_t ub = wl * kWGElems;              // first element of the unit
  const int64_t nvb = (n + BV - 1) >> lbv;
  const int64_t nmb = (n + BM - 1) >> lbm;
  const int64_t vb_u = ub >> lbv, mb_u = ub >> lbm;
  const int64_t rem64 = n - ub;
  const uint32_t nrem = FULL ? (uint32_t)kWGElems
                             : (rem64 <= 0 ? 0u : (rem64 >= kWGElems ? (uint32_t)kWGElems : (uint32_t)rem64));
  const int64_t nvr = nvb - vb_u, nmr = nmb - mb_u;   // blocks from this unit on
  uint32_t lo[2];
  int cnth[2], vloc[2], mloc[2];
  bool vok[2], mok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    lo[j] = (uint32_t)(j * kHalf + 4 * lane);
    vloc[j] = (int)(lo[j] >> lbv);
    mloc[j] = (int)(lo[j] >> lbm);
    cnth[j] = FULL ? 4 : (lo[j] >= nrem ? 0 : ((nrem - lo[j]) >= 4u ? 4 : (int)(nrem - lo[j])));
    vok[j] = FULL || vloc[j] < nvr;
    mok[j] = kHasM && (FULL || mloc[j] < nmr);
  }
  const T* Gu = reinterpret_cast<const T*>(D.grad) + ub;
  T* Pu = reinterpret_cast<T*>(D.param) + ub;
  uint8_t* V8u = reinterpret_cast<uint8_t*>(D.v_q) + ub;
  uint16_t* V16u = reinterpret_cast<uint16_t*>(D.v_q) + ub;
  uint8_t* Mu8 = kHasM ? D.m_q + ub : nullptr;
  uint8_t* Mu4 = kHasM ? D.m_q + (ub >> 1) : nullptr;
  float* MSu = kHasM ? D.m_scale + mb_u : nullptr;
  float* VSu = D.v_scale + vb_u;
  float* VLu = D.v_min_log + vb_u;
  float* VBu = (kVbuf || MODE == 1) ? D.v_buf + ub : nullptr;
  const int mk = (MK == 1) ? 1 : h.mk;
  float* tabs = s_lds;
  float* xw = s_lds + ((VB == 8 && !kVbuf) ? nv_wg * 256 : 0);  // [0,16) partials, [16,32) fit

  // ---- stream loads, issued before the decode table and its barrier so that
  // their latency overlaps the table build
  float g[kEPT];
  pval_t<T> pin[kEPT];   // parameter values (double for fp64 parameters)
  uint32_t vq8[2] = {0u, 0u}, mq8[2] = {0u, 0u}, mq4[2] = {0u, 0u};
  u32x2 vq16[2] = {{0u, 0u}, {0u, 0u}};
  float ms[2] = {0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < kEPT; ++k) { g[k] = 0.0f; pin[k] = 0; }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (vok[j]) {
      if constexpr (!kVbuf) {
        if constexpr (VB == 8) vq8[j] = *gp(reinterpret_cast<const uint32_t*>(V8u + lo[j]));
        else vq16[j] = *gp(reinterpret_cast<const u32x2*>(V16u + lo[j]));
      }
      if (mok[j]) {
        ms[j] = gp(MSu)[mloc[j]];
        if (MK == 1 || !(mk == 2 || mk == 4)) mq8[j] = *gp(reinterpret_cast<const uint32_t*>(Mu8 + lo[j]));
        else mq4[j] = *gp(reinterpret_cast<const uint16_t*>(Mu4 + (lo[j] >> 1)));
      }
      if constexpr (FULL) {
        load4v<T>(Gu, lo[j], g + 4 * j);
        if constexpr (kWrite && !SR) load4v<T>(Pu, lo[j], pin + 4 * j);
      } else {
        load4n<T>(Gu, lo[j], nrem, g + 4 * j);
        if constexpr (kWrite && !SR) load4n<T>(Pu, lo[j], nrem, pin + 4 * j);
      }
    }
  }

  // ---- AL8 decode tables for this workgroup's V blocks
  if constexpr (VB == 8 && !kVbuf) {
    const int64_t vb0 = vb_u;
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
    float a = D.alpha ? *gp(D.alpha) : h.alpha_val;
    if (MODE == 2 && D.fira_scale) a = a * *gp(D.fira_scale);
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
  // per-half block statistics: max of non-negative floats as integer bit
  // patterns, and the non-zero minimum key
  uint32_t vmaxb[2] = {0u, 0u}, amaxb[2] = {0u, 0u};
  uint32_t vkey[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
  for (int k = 0; k < kEPT; ++k) { vn[k] = 0.0f; mn[k] = 0.0f; }

  if (vok[0]) {   // vok[1] implies vok[0]
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
      for (int k = 0; k < kEPT; ++k) vn[k] = (k & 3) < cnth[k >> 2] ? gp(VBu)[lo[k >> 2] + (k & 3)] : 0.0f;
    } else {
      float vo[kEPT];
      if constexpr (VB == 8) {
#pragma unroll
        for (int k = 0; k < kEPT; ++k)
          vo[k] = tabs[vloc[k >> 2] * 256 + ((vq8[k >> 2] >> (8 * (k & 3))) & 0xFFu)];
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float s_old = 0.0f, lm_old = 0.0f;
          if (vok[j]) { s_old = gp(VSu)[vloc[j]]; lm_old = gp(VLu)[vloc[j]]; }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t c = ((i < 2 ? vq16[j].x : vq16[j].y) >> (16 * (i & 1))) & 0xFFFFu;
            vo[4 * j + i] = c ? exp2_exact(((float)(c - 1) * s_old) / 65534.0f + lm_old) : 0.0f;
          }
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
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (mok[j]) {
        if (MK == 1) {
          const float s128 = ms[j] / 128.0f, b128 = -128.0f * s128;   // (q-128)*s128 == fma(q, s128, -128*s128)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            mo[4 * j + i] = __builtin_fmaf((float)((mq8[j] >> (8 * i)) & 0xFFu), s128, b128);
        } else if (mk == 2 || mk == 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t byte = (mq4[j] >> (8 * (i >> 1))) & 0xFFu;
            mo[4 * j + i] = m_decode(mk, (i & 1) ? (byte & 0x0Fu) : (byte >> 4), ms[j]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) mo[4 * j + i] = m_decode(mk, (mq8[j] >> (8 * i)) & 0xFFu, ms[j]);
        }
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
        for (int k = 0; k < kEPT; ++k) x[k] = g[k] * inv[k];
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
        for (int k = 0; k < kEPT; ++k) uu[k] = mn[k];
      } else {
#pragma unroll
        for (int k = 0; k < kEPT; ++k) uu[k] = mn[k] * inv[k];
      }
    } else {
#pragma unroll
      for (int k = 0; k < kEPT; ++k) uu[k] = g[k] * inv[k];
    }
    // elements beyond the tensor (the zero padding of its last blocks) hold zero state
#pragma unroll
    for (int k = 0; k < kEPT; ++k) {
      if ((k & 3) >= cnth[k >> 2]) { vn[k] = 0.0f; mn[k] = 0.0f; uu[k] = 0.0f; }
    }
    if constexpr (kSq) {
      // NORM / LAG: the update (momentum-only: U = g*inv before clipping); MNORM: M'
#pragma unroll
      for (int k = 0; k < kEPT; ++k) {
        const float t = (MODE == 4) ? mn[k] : ((mom && (k & 3) < cnth[k >> 2]) ? g[k] * inv[k] : uu[k]);
        sq = __builtin_fmaf(t, t, sq);
      }
    }
    if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < kEPT; ++k)
        if ((k & 3) < cnth[k >> 2]) gp(VBu)[lo[k >> 2] + (k & 3)] = vn[k];
    }
#pragma unroll
    for (int k = 0; k < kEPT; ++k) {
      const int j = k >> 2;
      vmaxb[j] = max(vmaxb[j], __float_as_uint(vn[k]));
      vkey[j] = min(vkey[j], nz_key(vn[k]));
      amaxb[j] = max(amaxb[j], __float_as_uint(mn[k]) & 0x7FFFFFFFu);
    }

    // ---- parameter write
    if constexpr (kWrite) {
      const bool has_dec = D.decay || h.has_decay;
      const float dec = D.decay ? *gp(D.decay) : (h.has_decay ? h.decay_val : 1.0f);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (!vok[j]) continue;
        if constexpr (SR) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (i < cnth[j]) {
              const uint32_t e = lo[j] + i;
              const float pv = ld1<T>(Pu, e);
              const T r = sr_round<T>(pv * dec - step * uu[4 * j + i], D.sr_seed, h.sr_step,
                                      (uint64_t)(ub + (int64_t)e));
              uint16_t bits;
              __builtin_memcpy(&bits, &r, 2);
              gp(reinterpret_cast<uint16_t*>(Pu))[e] = bits;
            }
          }
        } else {
          pval_t<T> p[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) p[i] = pin[4 * j + i];
          if (has_dec) {  // decoupled weight decay: p*decay rounded, then the update (optimizer.py:2039)
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = pdec(p[i], dec);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) p[i] = pupd(step, uu[4 * j + i], p[i]);
          store4n<T>(Pu, lo[j], nrem, p);
        }
      }
    }
  }

  // ---- V refit + codes
  if constexpr (!kVbuf) {
    const float lm2 = VB == 8 ? 254.0f : 65534.0f;
    ALFit f[2];
    if (vwhole) {
      // one block per workgroup: reduce over all lanes and both halves; wave 0
      // computes the fit (lane pair 0/1) and shares it through LDS, so the
      // other waves do not repeat the correctly rounded logarithms
      float bmax = grp_max(__uint_as_float(max(vmaxb[0], vmaxb[1])), 64);
      uint32_t bkey = grp_umin(min(vkey[0], vkey[1]), 64);
      if ((lane & 63) == 0) { xw[wave * 4 + 0] = bmax; xw[wave * 4 + 1] = __uint_as_float(bkey); }
      __syncthreads();
      if (wave == 0) {
        const float mx = fmaxf(fmaxf(xw[0], xw[4]), fmaxf(xw[8], xw[12]));
        const uint32_t ky = min(min(__float_as_uint(xw[1]), __float_as_uint(xw[5])),
                                min(__float_as_uint(xw[9]), __float_as_uint(xw[13])));
        const float mn_ = (ky == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(ky + 1u);
        const ALFit ft = al_refit_pair(mx, mn_, h.floor_, lm2, lane);
        if (lane == 0) {
          float* xf = xw + 16;
          xf[0] = ft.lmin; xf[1] = ft.s; xf[2] = ft.k; xf[3] = ft.c1; xf[4] = ft.kmar; xf[5] = ft.cmar;
        }
      }
      __syncthreads();
      const float* xf = xw + 16;
      f[0].lmin = xf[0]; f[0].s = xf[1]; f[0].k = xf[2]; f[0].c1 = xf[3]; f[0].kmar = xf[4]; f[0].cmar = xf[5];
      f[1] = f[0];
    } else {
      float bmax[2];
      uint32_t bkey[2];
      const int G = VLh < 64 ? VLh : 64;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bmax[j] = grp_max(__uint_as_float(vmaxb[j]), G);
        bkey[j] = grp_umin(vkey[j], G);
      }
      if (VLh > 64) {
        // a block spans VLh/64 waves of one half: exchange one partial per wave and half
        if ((lane & 63) == 0) {
#pragma unroll
          for (int j = 0; j < 2; ++j) { xw[wave * 4 + 2 * j] = bmax[j]; xw[wave * 4 + 2 * j + 1] = __uint_as_float(bkey[j]); }
        }
        __syncthreads();
        const int wpb = VLh >> 6;                 // waves per block
        const int w0 = (wave / wpb) * wpb;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float mx = xw[w0 * 4 + 2 * j];
          uint32_t ky = __float_as_uint(xw[w0 * 4 + 2 * j + 1]);
          for (int w = 1; w < wpb; ++w) {
            mx = fmaxf(mx, xw[(w0 + w) * 4 + 2 * j]);
            ky = min(ky, __float_as_uint(xw[(w0 + w) * 4 + 2 * j + 1]));
          }
          bmax[j] = mx;
          bkey[j] = ky;
        }
      }
      // the two fits of a lane's blocks: lanes 4q+0/1 take log2 of half 0's max/min,
      // 4q+2/3 of half 1's (a block spans >= 32 lanes, so the quad shares both)
      const float mn0 = (bkey[0] == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey[0] + 1u);
      const float mn1 = (bkey[1] == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey[1] + 1u);
      const int qs = lane & 3;
      const float x = qs == 0 ? bmax[0] : (qs == 1 ? mn0 : (qs == 2 ? bmax[1] : mn1));
      const float l = log2_exact(fmaxf(x, kLogClampIn));
      const int qb = lane & ~3;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float lmax = __shfl(l, qb + 2 * j, 64);
        float lmin = __shfl(l, qb + 2 * j + 1, 64);
        lmin = fmaxf(lmin, h.floor_);
        if (lmin >= lmax) lmin = lmax - 1.0f;
        f[j].lmin = lmin;
        f[j].s = fmaxf(lmax - lmin, 1e-12f);
        al_fit_consts(f[j], lm2);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (!vok[j]) continue;
      if constexpr (VB == 8) {
        float r[4];
        bool bad[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = al8_round_fast(vn[4 * j + i], f[j], bad[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (bad[i]) r[i] = al_round_exact<254>(vn[4 * j + i], f[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = al_clamp<254>(vn[4 * j + i], r[i]);
        *gp(reinterpret_cast<uint32_t*>(V8u + lo[j])) = pack4(r[0], r[1], r[2], r[3]);
      } else {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = al_finish<65534>(vn[4 * j + i], al_round_exact<65534>(vn[4 * j + i], f[j]));
        *gp(reinterpret_cast<u32x2*>(V16u + lo[j])) =
            u32x2{q[0] | (q[1] << 16), q[2] | (q[3] << 16)};
      }
      if ((lane & (VLh - 1)) == 0 && (vwhole ? j == 0 : true)) {
        gp(VSu)[vloc[j]] = f[j].s;
        gp(VLu)[vloc[j]] = f[j].lmin;
      }
    }
  }

  // ---- M refit + codes
  if constexpr (kWrite && kHasM) {
    float bam[2];
    if (mwhole) {
      float a = grp_max(__uint_as_float(max(amaxb[0], amaxb[1])), 64);
      __syncthreads();
      if ((lane & 63) == 0) xw[wave * 4 + 2] = a;
      __syncthreads();
      a = fmaxf(fmaxf(xw[2], xw[6]), fmaxf(xw[10], xw[14]));
      bam[0] = bam[1] = a;
    } else {
      const int G = MLh < 64 ? MLh : 64;
#pragma unroll
      for (int j = 0; j < 2; ++j) bam[j] = grp_max(__uint_as_float(amaxb[j]), G);
      if (MLh > 64) {
        __syncthreads();
        if ((lane & 63) == 0) { xw[wave * 4 + 2] = bam[0]; xw[wave * 4 + 3] = bam[1]; }
        __syncthreads();
        const int wpb = MLh >> 6;
        const int w0 = (wave / wpb) * wpb;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float a = xw[w0 * 4 + 2 + j];
          for (int w = 1; w < wpb; ++w) a = fmaxf(a, xw[(w0 + w) * 4 + 2 + j]);
          bam[j] = a;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (!mok[j]) continue;
      const float am = fmaxf(bam[j], 1e-12f);
      const float ram = fast_rcp(am);
      if (MK == 1) {
        const float kam = 128.0f * ram;
        float r[4];
        bool bad[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = uf_round_fast<128>(mn[4 * j + i], kam, bad[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (bad[i]) r[i] = uf_round_exact<128>(mn[4 * j + i], am);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = uf_clamp<128>(r[i]);
        *gp(reinterpret_cast<uint32_t*>(Mu8 + lo[j])) = pack4(r[0], r[1], r[2], r[3]);
      } else if (mk == 2 || mk == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const uint32_t hi = m_encode(mk, mn[4 * j + 2 * q], am, ram);
          const uint32_t lo = m_encode(mk, mn[4 * j + 2 * q + 1], am, ram);
          w |= ((hi << 4) | lo) << (8 * q);
        }
        *gp(reinterpret_cast<uint16_t*>(Mu4 + (lo[j] >> 1))) = (uint16_t)w;
      } else {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) w |= m_encode(mk, mn[4 * j + i], am, ram) << (8 * i);
        *gp(reinterpret_cast<uint32_t*>(Mu8 + lo[j])) = w;
      }
      if ((lane & (MLh - 1)) == 0 && (mwhole ? j == 0 : true)) gp(MSu)[mloc[j]] = am;
    }
  }

  // ---- sum of squares for NORM / LAG / MNORM: this workgroup's partial
  if constexpr (kSq) {
    __shared__ float s_nw[4];
    const double t = wg_partial<4>(sq, s_nw);
    if (lane == 0) gp(D.norm_part)[wl] = t;
  }
}

// Occupancy 7 waves per SIMD (at most 72 VGPRs): measured best on MI355X for
// this streaming step (more resident waves hide the HBM latency of the loads).
template <typename T, int VB, int MODE, bool SR, int MK>
__global__ __launch_bounds__(kLanes) __attribute__((amdgpu_waves_per_eu(7)))
void k_update1d(Desc1D one, const Desc1D* __restrict__ table, int ntab, Hyper1D h) {
  extern __shared__ float s_lds[];  // [nv_wg * 256] AL8 tables | cross-wave partials and fits
  if (h.dsc) {
    const a8_step_scalars sc = load_step_scalars(h.dsc);
    h.bv = (float)sc.beta_val;
    h.eps_d = sc.eps_d;
    h.alpha_val = sc.alpha;
    h.decay_val = sc.decay;
    h.sr_step = sc.step;
  }
  Desc1D D;
  if (table != nullptr) D = load_desc(table, ntab, (int)blockIdx.x);
  else D = one;
  const int64_t wl = (int64_t)blockIdx.x - D.wg_begin;
  if (D.numel - wl * kWGElems >= kWGElems) unit_step<T, VB, MODE, SR, MK, true>(D, h, wl, s_lds);
  else unit_step<T, VB, MODE, SR, MK, false>(D, h, wl, s_lds);
}

// ------------------------------------------------------------ any block size
// The reference accepts any B_V that is a multiple of 128 and any B_M that is a
// multiple of 4, at least 32 and a divisor of B_V (optimizer.py:1395-1416).  The
// unit layout above needs powers of two; every other size takes this kernel: one
// workgroup per V block, lanes over its quads (four consecutive elements: a quad
// never straddles an M block, since B_M % 4 == 0), block statistics through LDS
// (the V max and non-zero minimum, one M absmax per M block of the V block, all
// exact max/min).  Pass 1 forms v', m', u, writes p (and v_buf in NORM) and the
// statistics; pass 2, after the block fit, forms v' and m' again from the same
// inputs (the same bits) and writes the codes.  The element arithmetic is
// unit_step's, element for element.
constexpr int kGenMaxBV = 65536;
constexpr int kGenMaxMB = kGenMaxBV / 32;

template <typename T, int VB, int MODE, bool SR, int MK>
__global__ __launch_bounds__(kLanes) void k_update1d_gen(Desc1D one, const Desc1D* __restrict__ table, int ntab,
                                                         Hyper1D h) {
  constexpr bool kHasM = MK != 0;
  constexpr bool kVbuf = MODE == 2 || MODE == 4;
  constexpr bool kSq = MODE == 1 || MODE == 3 || MODE == 4;
  constexpr bool kWrite = MODE == 0 || MODE == 2 || MODE == 3;
  constexpr float LM2 = VB == 8 ? 254.0f : 65534.0f;
  __shared__ float s_tab[256];
  __shared__ uint32_t s_st[2];           // V max bits, V non-zero minimum key
  __shared__ float s_fit[2];             // new l_min, scale
  __shared__ uint32_t s_mab[kGenMaxMB];  // |m'| max bits per M block of this V block
  if (h.dsc) {
    const a8_step_scalars sc = load_step_scalars(h.dsc);
    h.bv = (float)sc.beta_val;
    h.eps_d = sc.eps_d;
    h.alpha_val = sc.alpha;
    h.decay_val = sc.decay;
    h.sr_step = sc.step;
  }
  const Desc1D D = table != nullptr ? load_desc(table, ntab, (int)blockIdx.x) : one;
  const int lane = threadIdx.x;
  const int BV = h.block_size, BM = h.m_block_size;
  const int64_t blk = (int64_t)blockIdx.x - D.wg_begin;
  const int64_t n = D.numel, base = blk * BV;
  const int nq = BV >> 2;
  const int mpb = kHasM ? BV / BM : 0;                        // M blocks per V block
  const int64_t nmb = kHasM ? (n + BM - 1) / BM : 0;          // M blocks of the tensor
  const int mk = (MK == 1) ? 1 : h.mk;
  const T* G = reinterpret_cast<const T*>(D.grad);
  T* P = reinterpret_cast<T*>(D.param);
  const float s_old = kVbuf ? 0.0f : gp(D.v_scale)[blk], lm_old = kVbuf ? 0.0f : gp(D.v_min_log)[blk];
  if (lane == 0) { s_st[0] = 0u; s_st[1] = 0xFFFFFFFFu; }
  for (int i = lane; i < mpb; i += kLanes) s_mab[i] = 0u;
  if (VB == 8 && !kVbuf) s_tab[lane] = lane ? exp2_exact(((float)(lane - 1) * s_old) / 254.0f + lm_old) : 0.0f;
  __syncthreads();

  // step scale (unit_step's)
  float step = 0.0f, ut_clip = 1.0f;
  if constexpr (MODE != 1) {
    float a = D.alpha ? *gp(D.alpha) : h.alpha_val;
    if (MODE == 2 && D.fira_scale) a = a * *gp(D.fira_scale);
    if constexpr (MODE == 0) {
      step = a;
    } else {
      float denom = 1.0f;
      if (h.d > 0.0f) {
        const float nrm = (MODE == 2) ? sqrtf(*gp(D.norm_buf))
                          : (MODE == 4 ? sqrtf(*gp(D.prev_norm)) : *gp(D.prev_norm));
        if (h.momentum_only && kHasM)
          denom = fmaxf(1.0f, (nrm / (float)sqrt((double)n)) / h.d);
        else
          denom = fmaxf(1.0f, nrm / (float)(sqrt((double)n) * (double)h.d));
      }
      if (h.momentum_only && kHasM) { step = a; ut_clip = denom; }
      else { step = a / denom; }
    }
  }
  const bool mom = kHasM && h.momentum_only;

  // v' and m' of quad q (elements beyond the tensor: zero), and the quad's M block
  auto quad_state = [&](int q, float* g, float* vn, float* mn, float* inv, int& cnt, int& mb, bool& m_ok) {
    const int64_t i0 = base + 4 * q;
    cnt = i0 >= n ? 0 : (n - i0 >= 4 ? 4 : (int)(n - i0));
    load4n<T>(G, i0, n, g);
#pragma unroll
    for (int k = 0; k < 4; ++k) g[k] = scrub(g[k]);
    if constexpr (kVbuf) {
#pragma unroll
      for (int k = 0; k < 4; ++k) vn[k] = k < cnt ? gp(D.v_buf)[i0 + k] : 0.0f;
    } else {
      float vo[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t c;
        if constexpr (VB == 8) c = gp(reinterpret_cast<const uint8_t*>(D.v_q))[i0 + k];
        else c = gp(reinterpret_cast<const uint16_t*>(D.v_q))[i0 + k];
        vo[k] = (VB == 8) ? s_tab[c] : (c ? exp2_exact(((float)(c - 1) * s_old) / LM2 + lm_old) : 0.0f);
        float gsq = g[k] * g[k];
        if (h.eps_g != 0.0f) gsq = gsq + h.eps_g;
        vn[k] = fabsf(h.bv) < 0.5f ? __builtin_fmaf(h.bv, gsq - vo[k], vo[k])
                                   : __builtin_fmaf(h.bv - 1.0f, gsq - vo[k], gsq);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (mom) inv[k] = 1.0f / sqrtf(fmaxf(vn[k], h.eps_sq));
      else if (h.adam_denom) inv[k] = fast_rcp(fast_sqrt(vn[k]) + h.eps_d);
      else inv[k] = __builtin_amdgcn_rsqf(fmaxf(vn[k], h.eps_sq));
    }
    mb = kHasM ? (4 * q) / BM : 0;
    m_ok = kHasM && blk * mpb + mb < nmb;
    if constexpr (kHasM) {
      float mo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (m_ok) {
        const float ms = gp(D.m_scale)[blk * mpb + mb];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t e = i0 + k;
          uint32_t c;
          if (mk == 2 || mk == 4) {
            const uint32_t byte = gp(D.m_q)[e >> 1];
            c = (e & 1) ? (byte & 0x0Fu) : (byte >> 4);
          } else {
            c = gp(D.m_q)[e];
          }
          mo[k] = m_decode(mk, c, ms);
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float x = g[k];
        if (mom) {
          x = g[k] * inv[k];
          if (ut_clip != 1.0f) x = x / ut_clip;
        }
        mn[k] = fabsf(h.w_m) < 0.5f ? __builtin_fmaf(h.w_m, x - mo[k], mo[k])
                                    : __builtin_fmaf(h.w_m - 1.0f, x - mo[k], x);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k >= cnt) { vn[k] = 0.0f; mn[k] = 0.0f; }
  };

  // ---- pass 1: update, parameter, statistics
  float sq = 0.0f;
  uint32_t vmax = 0u, vkey = 0xFFFFFFFFu;
  for (int q = lane; q < nq; q += kLanes) {
    float g[4], vn[4], mn[4] = {0.0f, 0.0f, 0.0f, 0.0f}, inv[4], uu[4];
    int cnt, mb;
    bool m_ok;
    quad_state(q, g, vn, mn, inv, cnt, mb, m_ok);
    const int64_t i0 = base + 4 * q;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uu[k] = kHasM ? (mom ? mn[k] : mn[k] * inv[k]) : g[k] * inv[k];
      if (k >= cnt) uu[k] = 0.0f;
      if constexpr (kSq) {
        const float t = (MODE == 4) ? mn[k] : ((mom && k < cnt) ? g[k] * inv[k] : uu[k]);
        sq = __builtin_fmaf(t, t, sq);
      }
      vmax = max(vmax, __float_as_uint(vn[k]));
      vkey = min(vkey, __float_as_uint(vn[k]) - 1u);
    }
    if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < cnt) gp(D.v_buf)[i0 + k] = vn[k];
    }
    if constexpr (kWrite && kHasM) {
      uint32_t ab = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) ab = max(ab, __float_as_uint(mn[k]) & 0x7FFFFFFFu);
      if (m_ok) atomicMax(&s_mab[mb], ab);
    }
    if constexpr (kWrite) {
      const bool has_dec = D.decay || h.has_decay;
      const float dec = D.decay ? *gp(D.decay) : (h.has_decay ? h.decay_val : 1.0f);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (k >= cnt) continue;
        if constexpr (SR) {
          const float pv = ld1<T>(P, i0 + k);
          const T r = sr_round<T>(pv * dec - step * uu[k], D.sr_seed, h.sr_step, (uint64_t)(i0 + k));
          uint16_t bits;
          __builtin_memcpy(&bits, &r, 2);
          gp(reinterpret_cast<uint16_t*>(P))[i0 + k] = bits;
        } else {
          pval_t<T> pv = ld1<T, pval_t<T>>(P, i0 + k);
          if (has_dec) pv = pdec(pv, dec);
          st1<T>(P, i0 + k, pupd(step, uu[k], pv));
        }
      }
    }
  }
  if constexpr (!kVbuf) {
    vmax = grp_red_u(vmax, 64, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
    vkey = grp_umin(vkey, 64);
    if ((lane & 63) == 0) {
      atomicMax(&s_st[0], vmax);
      atomicMin(&s_st[1], vkey);
    }
  }
  if constexpr (kSq) {   // this workgroup's partial sum of squares
    __shared__ float s_nw[4];
    const double t = wg_partial<4>(sq, s_nw);
    if (lane == 0) gp(D.norm_part)[blk] = t;
  }
  __syncthreads();
  if constexpr (kVbuf && !(kWrite && kHasM)) return;   // MNORM: no state written

  // ---- block fit (one lane pair) and pass 2: codes
  ALFit f{};
  if constexpr (!kVbuf) {
    if (lane < 64) {
      const uint32_t key = s_st[1];
      const float mnz = key == 0xFFFFFFFFu ? __builtin_inff() : __uint_as_float(key + 1u);
      const ALFit ft = al_refit_pair(__uint_as_float(s_st[0]), mnz, h.floor_, LM2, lane);
      if (lane == 0) { s_fit[0] = ft.lmin; s_fit[1] = ft.s; }
    }
    __syncthreads();
    f.lmin = s_fit[0];
    f.s = s_fit[1];
    al_fit_consts(f, LM2);
  }
  for (int q = lane; q < nq; q += kLanes) {
    float g[4], vn[4], mn[4] = {0.0f, 0.0f, 0.0f, 0.0f}, inv[4];
    int cnt, mb;
    bool m_ok;
    quad_state(q, g, vn, mn, inv, cnt, mb, m_ok);
    const int64_t i0 = base + 4 * q;
    if constexpr (!kVbuf) {
      uint32_t code[4];
      al_codes<(int)LM2, 4>(vn, f, code);
      if constexpr (VB == 8) {
        *gp(reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(D.v_q) + i0)) =
            code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
      } else {
        *gp(reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(D.v_q) + i0)) =
            u32x2{code[0] | (code[1] << 16), code[2] | (code[3] << 16)};
      }
    }
    if constexpr (kWrite && kHasM) {
      if (m_ok) {
        const float am = fmaxf(__uint_as_float(s_mab[mb]), 1e-12f);
        const float ram = fast_rcp(am);
        if (mk == 2 || mk == 4) {
          const uint32_t w = ((m_encode(mk, mn[0], am, ram) << 4) | m_encode(mk, mn[1], am, ram)) |
                             (((m_encode(mk, mn[2], am, ram) << 4) | m_encode(mk, mn[3], am, ram)) << 8);
          *gp(reinterpret_cast<uint16_t*>(D.m_q + (i0 >> 1))) = (uint16_t)w;
        } else {
          uint32_t w = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) w |= m_encode(mk, mn[k], am, ram) << (8 * k);
          *gp(reinterpret_cast<uint32_t*>(D.m_q + i0)) = w;
        }
      }
    }
  }
  __syncthreads();   // every lane has read the old block metadata
  if (!kVbuf && lane == 0) { gp(D.v_scale)[blk] = f.s; gp(D.v_min_log)[blk] = f.lmin; }
  if constexpr (kWrite && kHasM) {
    for (int i = lane; i < mpb; i += kLanes)
      if (blk * mpb + i < nmb) gp(D.m_scale)[blk * mpb + i] = fmaxf(__uint_as_float(s_mab[i]), 1e-12f);
  }
}

// ------------------------------------------------------------ norm finish
// Second launch of a NORM / LAG / MNORM pass: one workgroup per tensor adds the
// tensor's workgroup partials in index order (sum_parts) and adds the sum to its
// norm_buf, which the caller zeroed.  The sum is the same bits whatever order
// the pass's workgroups ran in, and the same in a batched launch as alone.
__global__ __launch_bounds__(kLanes) void k_update1d_fin(Desc1D one, const Desc1D* __restrict__ table, int ntab,
                                                        int64_t nwg) {
  __shared__ double s_w[4];
  const int i = (int)blockIdx.x;
  const Desc1D D = table ? table[i] : one;
  const int64_t end = table ? (i + 1 < ntab ? table[i + 1].wg_begin : nwg) : nwg;
  const double s = sum_parts(D.norm_part, end - D.wg_begin, s_w);
  if (threadIdx.x == 0) *gp(D.norm_buf) += (float)s;
}

static int finish_norm_1d(int mode, const Desc1D& one, const Desc1D* table, int ntab, int64_t nwg,
                          hipStream_t st) {
  if (mode != 1 && mode != 3 && mode != 4) return 0;
  hipLaunchKernelGGL(k_update1d_fin, dim3(table ? (unsigned)ntab : 1u), dim3(kLanes), 0, st, one, table, ntab,
                     nwg);
  return check_launch("k_update1d_fin");
}

// ------------------------------------------------------------ launch glue
static bool fast_shape_ok(int bv, int bm) {
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  return pow2(bv) && bv >= 128 && bv <= 2048 && pow2(bm) && bm >= 32 && bm <= bv;
}
// The reference's rules (optimizer.py:1395-1416), up to kGenMaxBV.
static bool gen_shape_ok(int bv, int bm) {
  return bv >= 128 && bv % 128 == 0 && bv <= kGenMaxBV && bm >= 32 && bm % 4 == 0 && bv % bm == 0;
}
// Elements per workgroup of the chosen kernel.
static int64_t unit_of(int bv, int bm) { return fast_shape_ok(bv, bm) ? kWGElems : bv; }

template <typename T, int VB, int MODE, bool SR, int MK>
static int launch_t(const Desc1D& one, const Desc1D* table, int ntab, int64_t nwg, const Hyper1D& h,
                    hipStream_t st) {
  const int nv_wg = h.gen ? 1 : kWGElems / h.block_size;
  size_t lds = ((VB == 8 && MODE != 2 && MODE != 4) ? (size_t)nv_wg * 256 : 0) * sizeof(float) +
               48 * sizeof(float);
  if (nwg <= 0) return 0;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "too many workgroups");
  if (h.gen) {
    hipLaunchKernelGGL((k_update1d_gen<T, VB, MODE, SR, MK>), dim3((unsigned)nwg), dim3(kLanes), 0, st, one,
                       table, ntab, h);
    return check_launch("k_update1d_gen");
  }
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
    case A8_F64: return launch_dispatch<double, false>(vbits, mode, one, table, ntab, nwg, h, st);
    default: return set_error(A8_ERR_DTYPE, "unsupported param dtype");
  }
}

static int check_common(int dtype, int64_t numel, int bv, int bm, int mbits, int mmode, int vbits,
                        bool has_m) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (vbits != 8 && vbits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  if (!has_m) bm = bv;
  if (!fast_shape_ok(bv, bm) && !gen_shape_ok(bv, bm))
    return set_error(A8_ERR_BLOCK, "block_size must be a multiple of 128 (at most 65536) and m_block_size a "
                                   "multiple of 4, at least 32, that divides block_size");
  if (has_m && !((mbits == 8 || mbits == 4) && (mmode == 0 || mmode == 1)))
    return set_error(A8_ERR_ARG, "m_bits must be 4/8 and m_mode 0/1");
  if (dtype != A8_F32 && dtype != A8_BF16 && dtype != A8_F16 && dtype != A8_F64)
    return set_error(A8_ERR_DTYPE, "dtype");
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
                          float* norm_buf, double* norm_parts, const float* alpha, const float* prev_norm,
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
  if ((mode == 1 || mode == 3 || mode == 4) && !norm_parts)
    return set_error(A8_ERR_ARG, "NORM/LAG/MNORM need norm_parts (a8_norm_parts_1d doubles)");
  if (!aligned16(param) || !aligned16(grad) || !aligned16(v_q) || (has_m && !aligned16(m_q)))
    return set_error(A8_ERR_ALIGN, "param/grad/code buffers must be 16-byte aligned");
  Desc1D D{};
  D.param = param; D.grad = grad; D.m_q = m_q; D.m_scale = m_scale;
  D.v_q = v_q; D.v_scale = v_scale; D.v_min_log = v_min_log; D.v_buf = v_buf;
  D.norm_buf = norm_buf; D.alpha = alpha; D.prev_norm = prev_norm; D.decay = decay;
  D.numel = numel; D.wg_begin = 0; D.sr_seed = sr_seed; D.norm_part = norm_parts;
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
  h.gen = fast_shape_ok(h.block_size, h.m_block_size) ? 0 : 1;
  const int64_t unit = unit_of(h.block_size, h.m_block_size);
  const int64_t nwg = (numel + unit - 1) / unit;
  rc = launch_any(dtype, sr, v_bits, mode, D, nullptr, 0, nwg, h, (hipStream_t)stream);
  if (rc) return rc;
  return finish_norm_1d(mode, D, nullptr, 0, nwg, (hipStream_t)stream);
}

// Validate a multi-tensor launch and, if `image` is non-null, write its device table
// image there (a8_table_bytes_1d(ntensors) bytes: the descriptors, then one int32
// first workgroup per tensor).  The workgroup count goes to *nwg_out.
static int table_image_1d(int mode, int dtype, const a8_tensor1d* tensors, int ntensors, int block_size,
                          int m_block_size, int m_bits, int m_mode, int v_bits, int momentum_only, char* image,
                          int64_t* nwg_out) {
  if (!tensors) return set_error(A8_ERR_ARG, "null tensor list");
  const bool has_m = tensors[0].m_q != nullptr;
  int rc = check_common(dtype, 0, block_size, m_block_size, m_bits, m_mode, v_bits, has_m);
  if (rc) return rc;
  if (mode < 0 || mode > 4) return set_error(A8_ERR_ARG, "mode must be 0..4");
  if (mode == 4 && !momentum_only) return set_error(A8_ERR_ARG, "MNORM needs momentum_only");
  Desc1D* tab = reinterpret_cast<Desc1D*>(image);
  int32_t* first = image ? reinterpret_cast<int32_t*>(image + sizeof(Desc1D) * (size_t)ntensors) : nullptr;
  const int64_t unit = unit_of(block_size, has_m ? m_block_size : block_size);
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
    if ((mode == 1 || mode == 3 || mode == 4) && !t.norm_parts)
      return set_error(A8_ERR_ARG, "NORM/LAG/MNORM need norm_parts (a8_norm_parts_1d doubles per tensor)");
    if (mode == 4 && !has_m) return set_error(A8_ERR_ARG, "MNORM needs momentum codes");
    if (!aligned16(t.param) || !aligned16(t.grad) || !aligned16(t.v_q) || (has_m && !aligned16(t.m_q)))
      return set_error(A8_ERR_ALIGN, "param/grad/code buffers must be 16-byte aligned");
    if (t.numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
    if (image) {
      Desc1D D{};
      D.param = t.param; D.grad = t.grad; D.m_q = t.m_q; D.m_scale = t.m_scale;
      D.v_q = t.v_q; D.v_scale = t.v_scale; D.v_min_log = t.v_min_log; D.v_buf = t.v_buf;
      D.norm_buf = t.norm_buf; D.alpha = t.alpha; D.prev_norm = t.prev_norm; D.decay = t.decay;
      D.numel = t.numel; D.wg_begin = wg; D.sr_seed = t.sr_seed; D.fira_scale = t.fira_scale;
      D.norm_part = t.norm_parts;
      std::memcpy(&tab[i], &D, sizeof(Desc1D));
      const int32_t f = (int32_t)(wg < 0x7FFFFFFF ? wg : 0x7FFFFFFF);
      std::memcpy(&first[i], &f, sizeof(int32_t));
    }
    wg += (t.numel + unit - 1) / unit;
  }
  if (wg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "too many workgroups");
  *nwg_out = wg;
  return 0;
}

static int launch_multi_1d(int mode, int stochastic, int dtype, bool has_m, int ntensors, const void* table_dev,
                           int64_t nwg, double beta1, double beta_val, float eps_for_denom, int use_adam_denom,
                           float log_floor, float eps_for_grad_sq, float eps_sq, int block_size, int m_block_size,
                           int m_bits, int m_mode, float d, int v_bits, int momentum_only, uint64_t sr_step,
                           float alpha_val, float decay_val, int has_decay, const void* dsc, hipStream_t st) {
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
  h.dsc = reinterpret_cast<const a8_step_scalars*>(dsc);
  h.gen = fast_shape_ok(h.block_size, h.m_block_size) ? 0 : 1;
  Desc1D none{};
  const Desc1D* tab = reinterpret_cast<const Desc1D*>(table_dev);
  const int rc = launch_any(dtype, stochastic, v_bits, mode, none, tab, ntensors, nwg, h, st);
  if (rc) return rc;
  return finish_norm_1d(mode, none, tab, ntensors, nwg, st);
}

// ------------------------------------------------------------ no-allocation table
// a8_fused_update_1d_multi_noalloc keeps its tensor table in this file-scope
// device array instead of a caller buffer.  In host code `scratch` names a host
// stand-in, not device memory: its device address is taken once per device with
// hipGetSymbolAddress (that device current) and only that address is used.  Every
// GPU holds its own copy until the process ends.
constexpr int kScratchBytes = 64 * 1024;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) char scratch[kScratchBytes];
static void* g_scratch_ptr[kScratchDevices];
static std::mutex g_scratch_mu;
alignas(16) static char g_stage[kScratchBytes];   // host image of the table (a8_fused_update_1d_multi_noalloc)
static std::mutex g_stage_mu;
// Per device: a fingerprint of the tensors whose table the scratch array holds, so
// that a call with upload == 0 is refused unless it names those same tensors.
struct ScratchPrint {
  uint64_t hash;
  int ntensors;
  int valid;
};
static ScratchPrint g_scratch_print[kScratchDevices];

// FNV-1a over the tensor records and the block sizes (the inputs of the table
// image; a8_tensor1d has no padding bytes).
static uint64_t table_print(const a8_tensor1d* t, int n, int block_size, int m_block_size) {
  uint64_t h = 1469598103934665603ull;
  auto mix = [&h](const void* p, size_t bytes) {
    const unsigned char* c = static_cast<const unsigned char*>(p);
    for (size_t i = 0; i < bytes; ++i) { h ^= c[i]; h *= 1099511628211ull; }
  };
  mix(&n, sizeof n);
  mix(&block_size, sizeof block_size);
  mix(&m_block_size, sizeof m_block_size);
  mix(t, sizeof(a8_tensor1d) * (size_t)n);
  return h;
}

static int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
    return set_error(A8_ERR_HIP, "no usable current device for the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      char msg[160];
      snprintf(msg, sizeof msg, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return set_error(A8_ERR_HIP, msg);
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

extern "C" {

int a8_fused_update_1d(int mode, int stochastic, int dtype, void* param, const void* grad,
                       uint8_t* m_q, float* m_scale, void* v_q, float* v_scale, float* v_min_log,
                       float* v_buf, float* norm_buf, double* norm_parts, const float* alpha,
                       const float* prev_norm, const float* decay, uint64_t sr_seed, uint64_t sr_step,
                       double beta1, double beta_val, float eps_for_denom, int use_adam_denom,
                       float log_floor, float eps_for_grad_sq, float eps_sq, int64_t numel,
                       int block_size, int m_block_size, int m_bits, int m_mode, float d, int v_bits,
                       int momentum_only, float alpha_val, float decay_val, int has_decay,
                       void* stream) {
  return update1d_entry(mode, stochastic, dtype, param, grad, m_q, m_scale, v_q, v_scale, v_min_log,
                        v_buf, norm_buf, norm_parts, alpha, prev_norm, decay, sr_seed, sr_step, beta1, beta_val,
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
                             float decay_val, int has_decay, int upload, const void* step_scalars,
                             void* stream) {
  if (ntensors <= 0) return 0;
  if (a8_table_bytes_1d(ntensors) > table_bytes)
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_table_bytes_1d(ntensors)");
  std::vector<char> image;
  if (upload) image.resize((size_t)a8_table_bytes_1d(ntensors));
  int64_t nwg = 0;
  int rc = table_image_1d(mode, dtype, tensors, ntensors, block_size, m_block_size, m_bits, m_mode, v_bits,
                          momentum_only, upload ? image.data() : nullptr, &nwg);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (upload && upload_table(table_dev, image.data(), image.size(), st) != hipSuccess)
    return set_error(A8_ERR_HIP, "table upload failed");
  return launch_multi_1d(mode, stochastic, dtype, tensors[0].m_q != nullptr, ntensors, table_dev, nwg, beta1,
                         beta_val, eps_for_denom, use_adam_denom, log_floor, eps_for_grad_sq, eps_sq, block_size,
                         m_block_size, m_bits, m_mode, d, v_bits, momentum_only, sr_step, alpha_val, decay_val,
                         has_decay, step_scalars, st);
}

int a8_fused_update_1d_multi_noalloc(int mode, int stochastic, int dtype, const a8_tensor1d* tensors,
                                     int ntensors, double beta1, double beta_val, float eps_for_denom,
                                     int use_adam_denom, float log_floor, float eps_for_grad_sq, float eps_sq,
                                     int block_size, int m_block_size, int m_bits, int m_mode, float d,
                                     int v_bits, int momentum_only, uint64_t sr_step, float alpha_val,
                                     float decay_val, int has_decay, int upload, const void* step_scalars,
                                     void* stream) {
  if (ntensors <= 0) return 0;
  if (a8_table_bytes_1d(ntensors) > (int64_t)kScratchBytes) {
    char msg[160];
    snprintf(msg, sizeof msg, "a8_fused_update_1d_multi_noalloc: %d tensors need %lld table bytes, above the %d-byte "
             "scratch (at most %d tensors)", ntensors, (long long)a8_table_bytes_1d(ntensors), kScratchBytes,
             a8_noalloc_max_tensors_1d());
    return set_error(A8_ERR_SIZE, msg);
  }
  void* table_dev = nullptr;
  int rc = scratch_of_current_device(&table_dev);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(A8_ERR_HIP, "hipGetDevice failed");
  const uint64_t print = table_print(tensors, ntensors, block_size, m_block_size);
  int64_t nwg = 0;
  if (upload) {
    // A captured graph would replay the copy from the library's host buffer as it is at
    // replay time, which a later call may have rewritten: the table must be uploaded
    // eagerly, and a captured call reuses it (upload == 0).
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess)
      return set_error(A8_ERR_HIP, "hipStreamIsCapturing failed");
    if (cs != hipStreamCaptureStatusNone)
      return set_error(A8_ERR_ARG, "a8_fused_update_1d_multi_noalloc: upload != 0 on a capturing stream; upload "
                                   "the table in an eager call first and capture with upload == 0");
    // The image is built in a host buffer of the library's own (no allocation) and
    // copied from there; the copy from pageable memory has consumed the buffer when
    // hipMemcpyAsync returns, so the next call may reuse it.
    std::lock_guard<std::mutex> lock(g_stage_mu);
    rc = table_image_1d(mode, dtype, tensors, ntensors, block_size, m_block_size, m_bits, m_mode, v_bits,
                        momentum_only, g_stage, &nwg);
    if (rc) return rc;
    if (hipMemcpyAsync(table_dev, g_stage, (size_t)a8_table_bytes_1d(ntensors), hipMemcpyHostToDevice, st) !=
        hipSuccess)
      return set_error(A8_ERR_HIP, "scratch table upload failed");
    std::lock_guard<std::mutex> plock(g_scratch_mu);
    g_scratch_print[dev] = ScratchPrint{print, ntensors, 1};
  } else {
    {
      std::lock_guard<std::mutex> plock(g_scratch_mu);
      const ScratchPrint& sp = g_scratch_print[dev];
      if (!sp.valid || sp.ntensors != ntensors || sp.hash != print)
        return set_error(A8_ERR_ARG, "a8_fused_update_1d_multi_noalloc: upload == 0, but the tensors (or block "
                                     "sizes) differ from those of the table last uploaded on this device");
    }
    rc = table_image_1d(mode, dtype, tensors, ntensors, block_size, m_block_size, m_bits, m_mode, v_bits,
                        momentum_only, nullptr, &nwg);
    if (rc) return rc;
  }
  return launch_multi_1d(mode, stochastic, dtype, tensors[0].m_q != nullptr, ntensors, table_dev, nwg, beta1,
                         beta_val, eps_for_denom, use_adam_denom, log_floor, eps_for_grad_sq, eps_sq, block_size,
                         m_block_size, m_bits, m_mode, d, v_bits, momentum_only, sr_step, alpha_val, decay_val,
                         has_decay, step_scalars, st);
}

int64_t a8_norm_parts_1d(int64_t numel, int block_size, int m_block_size) {
  if (block_size <= 0 || m_block_size <= 0) return -1;
  if (numel <= 0) return 0;
  const int64_t unit = unit_of(block_size, m_block_size);
  return (numel + unit - 1) / unit;
}

int a8_noalloc_max_tensors_1d(void) { return (int)(kScratchBytes / (sizeof(Desc1D) + sizeof(int32_t))); }

int64_t a8_table_bytes_1d(int ntensors) {
  return ((int64_t)sizeof(Desc1D) + (int64_t)sizeof(int32_t)) * (int64_t)ntensors;
}

int a8_set_qmap(const float* qmap8_host, const float* qmap4_host) {
  if (!qmap8_host || !qmap4_host) return set_error(A8_ERR_ARG, "null codebook");
  if (upload_qmap_tu(qmap8_host, qmap4_host) != hipSuccess ||
      a8::factored_upload_qmap(qmap8_host, qmap4_host) != hipSuccess ||
      a8::apollo_upload_qmap(qmap8_host, qmap4_host) != hipSuccess ||
      a8::decode_upload_qmap(qmap8_host, qmap4_host) != hipSuccess ||
      a8::sgd_upload_qmap(qmap8_host, qmap4_host) != hipSuccess ||
      a8::prims_upload_qmap(qmap8_host, qmap4_host) != hipSuccess)
    return set_error(A8_ERR_HIP, "codebook upload failed");
  return 0;
}

}  // extern "C"
