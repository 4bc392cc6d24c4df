// Kernels of the fused 1-D step and their launch templates, shared by the two
// translation units that instantiate them: a8_update1d.hip (KR = 0, the CPU
// quantiser's AL rule) and a8_update1d_k.hip (KR = 1, the reference kernels' AL
// rule, A8_AL_KERNEL_RULE).  KR is a template parameter so that each rule's kernel
// carries only its own refit code.
#pragma once
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
  int krule;        // host routing: the launch takes the KR = 1 instantiations (the reference kernels' AL rule)
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

// Block minimum keys: the bits of a non-negative float minus koff.  For v >= 0
// the unsigned order of the bits is the float order; with koff = 1 (the CPU
// rule) v == 0 maps to 0xFFFFFFFF, so an unsigned min over keys is the minimum
// over the non-zero entries; with koff = 0 (the kernels' rule) zeros count.

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
template <typename T, int VB, int MODE, bool SR, int MK, bool FULL, int KR>
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
        val = exp2_exact(al_dec_log<254>((float)(c - 1), sc, lm, KR));
      }
      tabs[c] = val;
    } else {
      for (int k = lane; k < nv_wg * 256; k += kLanes) {
        const int64_t b = vb0 + (k >> 8);
        const int c = k & 255;
        float val = 0.0f;
        if (b < nvb && c != 0) {
          const float sc = gp(D.v_scale)[b], lm = gp(D.v_min_log)[b];
          val = exp2_exact(al_dec_log<254>((float)(c - 1), sc, lm, KR));
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
        if (MODE == 3)   // LAG has no CPU branch: the CUDA kernels' pn / (sqrtf(numel) * d) in fp32 (kernels.cu:651-655)
          denom = fmaxf(1.0f, nrm / (sqrtf((float)n) * h.d));
        else if (h.momentum_only && kHasM)
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
  const uint32_t koff = KR ? 0u : 1u;
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
            vo[4 * j + i] = c ? exp2_exact(al_dec_log<65534>((float)(c - 1), s_old, lm_old, KR)) : 0.0f;
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
      // the block minimum: over non-zero v (CPU rule), or over every element of the
      // tensor including zeros (kernels' rule); keys past the tensor's end never count
      vkey[j] = min(vkey[j], (k & 3) < cnth[j] ? __float_as_uint(vn[k]) - koff : 0xFFFFFFFFu);
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
        const float mn_ = (ky == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(ky + koff);
        const ALFit ft = al_refit_pair(mx, mn_, h.floor_, lm2, lane, KR);
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
      const float mn0 = (bkey[0] == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey[0] + koff);
      const float mn1 = (bkey[1] == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey[1] + koff);
      const int qs = lane & 3;
      const float x = qs == 0 ? bmax[0] : (qs == 1 ? mn0 : (qs == 2 ? bmax[1] : mn1));
      const float l = KR ? al_klog(x, (qs & 1) ? -__builtin_inff() : -1e30f) : log2_exact(fmaxf(x, kLogClampIn));
      const int qb = lane & ~3;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float lmax = __shfl(l, qb + 2 * j, 64);
        float lmin = __shfl(l, qb + 2 * j + 1, 64);
        if (KR) {
          al_kfit(lmax, lmin, h.floor_, lm2, f[j]);
          continue;
        }
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
          if (bad[i]) r[i] = al_round_exact<254>(vn[4 * j + i], f[j], KR);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = al_clamp<254>(vn[4 * j + i], r[i]);
        *gp(reinterpret_cast<uint32_t*>(V8u + lo[j])) = pack4(r[0], r[1], r[2], r[3]);
      } else {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          q[i] = al_finish<65534>(vn[4 * j + i], al_round_exact<65534>(vn[4 * j + i], f[j], KR));
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
template <typename T, int VB, int MODE, bool SR, int MK, int KR>
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
  if (D.numel - wl * kWGElems >= kWGElems) unit_step<T, VB, MODE, SR, MK, true, KR>(D, h, wl, s_lds);
  else unit_step<T, VB, MODE, SR, MK, false, KR>(D, h, wl, s_lds);
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
// unit_step's, element for element.  A V block holding more than kGenMaxMB M
// blocks (B_V / B_M > 2048, so B_V > 65536) is taken in segments of kGenMaxMB M
// blocks: pass 1 and then the M codes and scales segment by segment (a segment's
// old scales are read only by its own quads), and after the last segment a pass
// that writes the V codes.
constexpr int kGenMaxMB = 2048;           // M blocks whose absmax LDS holds at once
constexpr int kGenMaxBV = 1 << 30;        // block_size is a 32-bit int

template <typename T, int VB, int MODE, bool SR, int MK, int KR>
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
  constexpr bool kSegM = kWrite && kHasM;                      // M codes written, absmaxes in LDS
  const int nseg = kSegM ? (mpb + kGenMaxMB - 1) / kGenMaxMB : 1;
  const int segq = nseg > 1 ? kGenMaxMB * (BM >> 2) : nq;      // quads per segment (< 2^28 when nseg > 1)
  const int64_t nmb = kHasM ? (n + BM - 1) / BM : 0;          // M blocks of the tensor
  const int mk = (MK == 1) ? 1 : h.mk;
  const T* G = reinterpret_cast<const T*>(D.grad);
  T* P = reinterpret_cast<T*>(D.param);
  const float s_old = kVbuf ? 0.0f : gp(D.v_scale)[blk], lm_old = kVbuf ? 0.0f : gp(D.v_min_log)[blk];
  if (lane == 0) { s_st[0] = 0u; s_st[1] = 0xFFFFFFFFu; }
  for (int i = lane; i < (mpb < kGenMaxMB ? mpb : kGenMaxMB); i += kLanes) s_mab[i] = 0u;
  if (VB == 8 && !kVbuf) s_tab[lane] = lane ? exp2_exact(al_dec_log<254>((float)(lane - 1), s_old, lm_old, KR)) : 0.0f;
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
        if (MODE == 3)   // LAG has no CPU branch: the CUDA kernels' pn / (sqrtf(numel) * d) in fp32 (kernels.cu:651-655)
          denom = fmaxf(1.0f, nrm / (sqrtf((float)n) * h.d));
        else if (h.momentum_only && kHasM)
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
  // need_m = false: v' only (the V-code pass after segmented M codes, whose M
  // state is already the new one)
  auto quad_state = [&](int q, float* g, float* vn, float* mn, float* inv, int& cnt, int& mb, bool& m_ok,
                        bool need_m = true) {
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
        vo[k] = (VB == 8) ? s_tab[c] : (c ? exp2_exact(al_dec_log<(int)LM2>((float)(c - 1), s_old, lm_old, KR)) : 0.0f);
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
    m_ok = kHasM && need_m && blk * mpb + mb < nmb;
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

  // the M codes of a quad from its M block's absmax bits
  auto write_m = [&](int64_t i0, const float* mn, float ab) {
    const float am = fmaxf(ab, 1e-12f);
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
  };

  // ---- pass 1: update, parameter, statistics (by segments, see above)
  float sq = 0.0f;
  uint32_t vmax = 0u, vkey = 0xFFFFFFFFu;
  const uint32_t koff = KR ? 0u : 1u;   // block minimum keys, as unit_step
  for (int seg = 0; seg < nseg; ++seg) {
    const int qb = seg * segq, qe = (nq - qb < segq) ? nq : qb + segq, mb0 = seg * kGenMaxMB;
    for (int q = qb + lane; q < qe; q += kLanes) {
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
        vkey = min(vkey, k < cnt ? __float_as_uint(vn[k]) - koff : 0xFFFFFFFFu);
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
        if (m_ok) atomicMax(&s_mab[mb - mb0], ab);
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
    if (nseg > 1) {
      if constexpr (kSegM) {
        __syncthreads();   // the segment's absmaxes are complete
        for (int q = qb + lane; q < qe; q += kLanes) {
          float g[4], vn[4], mn[4] = {0.0f, 0.0f, 0.0f, 0.0f}, inv[4];
          int cnt, mb;
          bool m_ok;
          quad_state(q, g, vn, mn, inv, cnt, mb, m_ok);
          if (m_ok) write_m(base + 4 * q, mn, __uint_as_float(s_mab[mb - mb0]));
        }
        __syncthreads();   // every lane has read the segment's old scales
        const int nm = (mpb - mb0 < kGenMaxMB) ? mpb - mb0 : kGenMaxMB;
        for (int i = lane; i < nm; i += kLanes) {
          if (blk * mpb + mb0 + i < nmb)
            gp(D.m_scale)[blk * mpb + mb0 + i] = fmaxf(__uint_as_float(s_mab[i]), 1e-12f);
          s_mab[i] = 0u;
        }
        __syncthreads();
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
  if (kVbuf && nseg > 1) return;   // APPLY in segments: M codes and scales are written, V has none

  // ---- block fit (one lane pair) and pass 2: codes
  ALFit f{};
  if constexpr (!kVbuf) {
    if (lane < 64) {
      const uint32_t key = s_st[1];
      const float mnz = key == 0xFFFFFFFFu ? __builtin_inff() : __uint_as_float(key + koff);
      const ALFit ft = al_refit_pair(__uint_as_float(s_st[0]), mnz, h.floor_, LM2, lane, KR);
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
    quad_state(q, g, vn, mn, inv, cnt, mb, m_ok, nseg == 1);
    const int64_t i0 = base + 4 * q;
    if constexpr (!kVbuf) {
      uint32_t code[4];
      al_codes<(int)LM2, 4>(vn, f, code, KR);
      if constexpr (VB == 8) {
        *gp(reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(D.v_q) + i0)) =
            code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
      } else {
        *gp(reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(D.v_q) + i0)) =
            u32x2{code[0] | (code[1] << 16), code[2] | (code[3] << 16)};
      }
    }
    if constexpr (kSegM) {
      if (m_ok) write_m(i0, mn, __uint_as_float(s_mab[mb]));   // one segment: mb0 = 0
    }
  }
  __syncthreads();   // every lane has read the old block metadata
  if (!kVbuf && lane == 0) { gp(D.v_scale)[blk] = f.s; gp(D.v_min_log)[blk] = f.lmin; }
  if constexpr (kSegM) {
    if (nseg == 1) {
      for (int i = lane; i < mpb; i += kLanes)
        if (blk * mpb + i < nmb) gp(D.m_scale)[blk * mpb + i] = fmaxf(__uint_as_float(s_mab[i]), 1e-12f);
    }
  }
}

// ------------------------------------------------------------ launch glue
static bool fast_shape_ok(int bv, int bm) {
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  return pow2(bv) && bv >= 128 && bv <= 2048 && pow2(bm) && bm >= 32 && bm <= bv;
}
// The reference's rules (optimizer.py:1395-1416).
static bool gen_shape_ok(int bv, int bm) {
  return bv >= 128 && bv % 128 == 0 && bv <= kGenMaxBV && bm >= 32 && bm % 4 == 0 && bv % bm == 0;
}
// Elements per workgroup of the chosen kernel.
static int64_t unit_of(int bv, int bm) { return fast_shape_ok(bv, bm) ? kWGElems : bv; }

template <typename T, int VB, int MODE, bool SR, int MK, int KR>
static int launch_t(const Desc1D& one, const Desc1D* table, int ntab, int64_t nwg, const Hyper1D& h,
                    hipStream_t st) {
  const int nv_wg = h.gen ? 1 : kWGElems / h.block_size;
  size_t lds = ((VB == 8 && MODE != 2 && MODE != 4) ? (size_t)nv_wg * 256 : 0) * sizeof(float) +
               48 * sizeof(float);
  if (nwg <= 0) return 0;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "too many workgroups");
  if (h.gen) {
    hipLaunchKernelGGL((k_update1d_gen<T, VB, MODE, SR, MK, KR>), dim3((unsigned)nwg), dim3(kLanes), 0, st, one,
                       table, ntab, h);
    return check_launch("k_update1d_gen");
  }
  hipLaunchKernelGGL((k_update1d<T, VB, MODE, SR, MK, KR>), dim3((unsigned)nwg), dim3(kLanes), lds, st, one,
                     table, ntab, h);
  return check_launch("k_update1d");
}

template <typename T, bool SR, int MK, int KR>
static int launch_mode(int vbits, int mode, const Desc1D& one, const Desc1D* table, int ntab,
                       int64_t nwg, const Hyper1D& h, hipStream_t st) {
#define A8_L(VB, MO) return launch_t<T, VB, MO, SR, MK, KR>(one, table, ntab, nwg, h, st)
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

template <typename T, bool SR, int KR>
static int launch_dispatch(int vbits, int mode, const Desc1D& one, const Desc1D* table, int ntab,
                           int64_t nwg, const Hyper1D& h, hipStream_t st) {
  switch (h.mk) {
    case 0: return launch_mode<T, SR, 0, KR>(vbits, mode, one, table, ntab, nwg, h, st);
    case 1: return launch_mode<T, SR, 1, KR>(vbits, mode, one, table, ntab, nwg, h, st);
    default: return launch_mode<T, SR, 2, KR>(vbits, mode, one, table, ntab, nwg, h, st);
  }
}

// Every instantiation of one AL rule (KR = 0: the CPU quantiser's, 1: the reference
// kernels'); each rule's instantiations live in their own translation unit.
template <int KR>
static int launch_rule(int dtype, int sr, int vbits, int mode, const Desc1D& one, const Desc1D* table,
                       int ntab, int64_t nwg, const Hyper1D& h, hipStream_t st) {
  if ((mode == 1 || mode == 4) && sr) sr = 0;
  switch (dtype) {
    case A8_F32: return launch_dispatch<float, false, KR>(vbits, mode, one, table, ntab, nwg, h, st);
    case A8_BF16:
      return sr ? launch_dispatch<__hip_bfloat16, true, KR>(vbits, mode, one, table, ntab, nwg, h, st)
                : launch_dispatch<__hip_bfloat16, false, KR>(vbits, mode, one, table, ntab, nwg, h, st);
    case A8_F16:
      return sr ? launch_dispatch<__half, true, KR>(vbits, mode, one, table, ntab, nwg, h, st)
                : launch_dispatch<__half, false, KR>(vbits, mode, one, table, ntab, nwg, h, st);
    case A8_F64: return launch_dispatch<double, false, KR>(vbits, mode, one, table, ntab, nwg, h, st);
    default: return set_error(A8_ERR_DTYPE, "unsupported param dtype");
  }
}


// KR = 1 instantiations (a8_update1d_k.hip).
int launch_any_kernel_rule(int dtype, int sr, int vbits, int mode, const Desc1D& one, const Desc1D* table,
                           int ntab, int64_t nwg, const Hyper1D& h, hipStream_t st);

}  // namespace a8
