// Momentum codecs (UF8/UF4/D8/D4), the dynamic codebook and the stochastic
// rounding writeback, shared by the fused step kernels.  Each translation unit
// holds its own copy of the codebook in constant memory; a8_set_qmap uploads
// every copy.
#pragma once
#include <type_traits>
#include "a8_common.cuh"

namespace a8 {

static __constant__ float c_qmap8[256];
static __constant__ float c_qmap4[16];

// Upload this translation unit's codebook copy (host side).
static inline hipError_t upload_qmap_tu(const float* q8, const float* q4) {
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(c_qmap8), q8, 256 * sizeof(float));
  if (e != hipSuccess) return e;
  return hipMemcpyToSymbol(HIP_SYMBOL(c_qmap4), q4, 16 * sizeof(float));
}

// ------------------------------------------------------------ SR writeback
// SplitMix64 counter stream keyed by (seed, step, element) and the bf16/fp16
// stochastic rounding rules of the reference (kernels.cu:48-161).
//
// sm_hi(z): the high 32 bits of the mix of counter z before its last xorshift,
// in 32-bit halves: z ^ (z >> k) takes one funnel shift (v_alignbit) for the low
// word, a 64 x 64 product keeps only what its low 64 bits need (the second one
// only its high word).  The stream's 32 random bits are hi ^ (hi >> 31) (the high
// word of z ^ (z >> 31)); every consumer here reads bits >> 8 or less, to which
// that xor is invisible, so the decisions take hi itself.  sm_hi_yh takes
// yhc = (zh ^ (zh >> 30)) * 0x1CE4E5B9, the high word's share of the first
// product, which counters that differ only in their low word share.
// sm_hi_ys: the same given the low word of z >> 30 (sh30), which counters that
// agree in their bits from 30 up share.
__device__ __forceinline__ uint32_t sm_hi_ys(uint32_t zl, uint32_t sh30, uint32_t yhc) {
  const uint32_t yl = zl ^ sh30;
  const uint64_t p = (uint64_t)yl * 0x1CE4E5B9u;   // * 0xBF58476D1CE4E5B9
  const uint32_t z1l = (uint32_t)p;
  const uint32_t z1h = (uint32_t)(p >> 32) + yl * 0xBF58476Du + yhc;
  const uint32_t y2l = z1l ^ __builtin_amdgcn_alignbit(z1h, z1l, 27), y2h = z1h ^ (z1h >> 27);
  return __umulhi(y2l, 0x133111EBu) + y2l * 0x94D049BBu + y2h * 0x133111EBu;   // * 0x94D049BB133111EB
}
__device__ __forceinline__ uint32_t sm_hi_yh(uint32_t zl, uint32_t zh, uint32_t yhc) {
  const uint32_t yl = zl ^ __builtin_amdgcn_alignbit(zh, zl, 30);
  const uint64_t p = (uint64_t)yl * 0x1CE4E5B9u;   // * 0xBF58476D1CE4E5B9
  const uint32_t z1l = (uint32_t)p;
  const uint32_t z1h = (uint32_t)(p >> 32) + yl * 0xBF58476Du + yhc;
  const uint32_t y2l = z1l ^ __builtin_amdgcn_alignbit(z1h, z1l, 27), y2h = z1h ^ (z1h >> 27);
  return __umulhi(y2l, 0x133111EBu) + y2l * 0x94D049BBu + y2h * 0x133111EBu;   // * 0x94D049BB133111EB
}
__device__ __forceinline__ uint32_t sm_yhc(uint32_t zh) { return (zh ^ (zh >> 30)) * 0x1CE4E5B9u; }

__device__ __forceinline__ uint32_t sm_hi(uint64_t z) {
  return sm_hi_yh((uint32_t)z, (uint32_t)(z >> 32), sm_yhc((uint32_t)(z >> 32)));
}

__device__ __forceinline__ uint64_t sr_base(uint64_t seed, uint64_t step) {
  return seed * 0x9E3779B97F4A7C15ULL + step * 0xD1B54A32D192ED03ULL;
}

// sm_hi of the element's counter (seed * gamma + step * K + idx + gamma).
__device__ __forceinline__ uint32_t sr_hi_at(uint64_t base, uint64_t idx) {
  return sm_hi(base + idx + 0x9E3779B97F4A7C15ULL);
}

// bf16 stochastic rounding (kernels.cu:67-87) decided in integers: the reference
// takes x's upper bf16 neighbour when u < rem / 2^16 (rem: x's low 16 bits), with
// u = (bits >> 8) / 2^24; that is (bits >> 8) < rem * 2^8 exactly (both sides are
// exact in fp32), that is (bits >> 16) < rem, that is hi < rem * 2^16 = x's bits
// << 16 (bits and hi differ in bit 0 only).  Its three guards fold into one
// magnitude compare: rem == 0 never rounds up (the compare is false), and
// |x| >= 0x7F7F0000 (inf, NaN, or a truncation whose upper neighbour is inf) never
// rounds up either; NaN becomes the quiet NaN.
__device__ __forceinline__ uint16_t sr_bf16_hi(float x, uint32_t hi) {
  const uint32_t b = __float_as_uint(x);
  const uint32_t a = b & 0x7FFFFFFFu;
  const uint32_t up = (uint32_t)(hi < (b << 16)) & (uint32_t)(a < 0x7F7F0000u);
  const uint32_t rn = (b >> 16) + up;
  const uint32_t rq = ((b >> 16) & 0x8000u) | 0x7FC0u;
  return (uint16_t)(a > 0x7F800000u ? rq : rn);
}

__device__ __forceinline__ float sr_uniform(uint64_t seed, uint64_t step, uint64_t idx) {
  return (float)(sr_hi_at(sr_base(seed, step), idx) >> 8) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ uint16_t h_next_up(uint16_t h) {
  if (h == 0x7C00u) return h;
  if (h == 0x8000u) return 0x0001u;
  return (h & 0x8000u) ? (uint16_t)(h - 1u) : (uint16_t)(h + 1u);
}
__device__ __forceinline__ uint16_t h_next_down(uint16_t h) {
  if (h == 0xFC00u) return h;
  if (h == 0x0000u) return 0x8001u;
  return (h & 0x8000u) ? (uint16_t)(h + 1u) : (uint16_t)(h - 1u);
}

__device__ __forceinline__ uint16_t sr_fp16(float x, float u) {
  uint32_t b = __float_as_uint(x);
  uint16_t sign = (b & 0x80000000u) ? 0x8000u : 0u;
  if ((b & 0x7F800000u) == 0x7F800000u) return (b & 0x007FFFFFu) ? (sign | 0x7E00u) : (sign | 0x7C00u);
  if (fabsf(x) > 65504.0f) return sign | 0x7BFFu;
  __half nh = __float2half_rn(f32_value(x));
  uint16_t qb = __half_as_ushort(nh);
  float q = __half2float(nh);
  if (q == x) return qb;
  uint16_t lo, hi;
  if (q < x) { lo = qb; hi = h_next_up(qb); } else { hi = qb; lo = h_next_down(qb); }
  float flo = __half2float(__ushort_as_half(lo));
  float fhi = __half2float(__ushort_as_half(hi));
  float prob = (x - flo) / (fhi - flo);
  return (u < prob) ? hi : lo;
}

template <typename T>
__device__ __forceinline__ T sr_round(float x, uint64_t seed, uint64_t step, uint64_t idx) {
  if constexpr (std::is_same<T, __hip_bfloat16>::value) {
    return __ushort_as_bfloat16(sr_bf16_hi(x, sr_hi_at(sr_base(seed, step), idx)));
  } else if constexpr (sizeof(T) == 2) {
    return __ushort_as_half(sr_fp16(x, sr_uniform(seed, step, idx)));
  } else {
    return x;
  }
}

// ------------------------------------------------------------ M codecs
__device__ __forceinline__ float m_decode(int mk, uint32_t q, float s) {
  switch (mk) {
    case 1: return ((float)q - 128.0f) * (s / 128.0f);
    case 2: return ((float)q - 8.0f) * (s / 8.0f);
    case 3: return c_qmap8[q] * s;
    default: return c_qmap4[q] * s;
  }
}

// Nearest codebook entry with searchsorted semantics and sign fix
// (optimizer.py:454-476), on x = m / absmax computed with IEEE division.
template <int N>
__device__ __forceinline__ uint32_t d_code(float m, float amax) {
  const float* qm = (N == 256) ? c_qmap8 : c_qmap4;
  float x = m / amax;
  int lo = 0, hi = N;  // first index with qm[i] >= x
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (qm[mid] < x) lo = mid + 1; else hi = mid;
  }
  int idx = lo > N - 1 ? N - 1 : lo;
  int prev = idx - 1 < 0 ? 0 : idx - 1;
  if (fabsf(x - qm[prev]) < fabsf(x - qm[idx])) idx = prev;
  float sx = (x > 0.0f) ? 1.0f : ((x < 0.0f) ? -1.0f : 0.0f);
  float v = qm[idx];
  float sq = (v > 0.0f) ? 1.0f : ((v < 0.0f) ? -1.0f : 0.0f);
  if (sx != sq && sx != 0.0f) {
    if (sx > 0.0f && idx < N - 1) idx += 1;
    else if (sx < 0.0f && idx > 0) idx -= 1;
  }
  return (uint32_t)idx;
}

__device__ __forceinline__ uint32_t m_encode(int mk, float m, float amax, float ramax) {
  switch (mk) {
    case 1: return uf_code<128>(m, amax, ramax);
    case 2: return uf_code<8>(m, amax, ramax);
    case 3: return d_code<256>(m, amax);
    default: return d_code<16>(m, amax);
  }
}

// ------------------------------------------------------------ lane codecs
// Momentum of elements e0..e0+7 (one lane; e0 a multiple of 8) from codes
// padded to whole blocks of 2^lbm elements.  mb = e0 >> lbm; m_ok says the
// lane's block exists (mb < number of blocks).
__device__ __forceinline__ void mq_decode8(int mk, const uint8_t* m_q, const float* m_scale, int64_t e0,
                                           int64_t mb, bool m_ok, float* mo) {
#pragma unroll
  for (int k = 0; k < 8; ++k) mo[k] = 0.0f;
  if (!m_ok) return;
  const float ms = gp(m_scale)[mb];
  if (mk == 2 || mk == 4) {
    const uint32_t qw = *gp(reinterpret_cast<const uint32_t*>(m_q + (e0 >> 1)));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t byte = (qw >> (8 * (k >> 1))) & 0xFFu;
      mo[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
    }
  } else {
    const u32x2 qv = *gp(reinterpret_cast<const u32x2*>(m_q + e0));
#pragma unroll
    for (int k = 0; k < 8; ++k) mo[k] = m_decode(mk, ((k < 4 ? qv.x : qv.y) >> (8 * (k & 3))) & 0xFFu, ms);
  }
}

// Requantise the lane's 8 values m[] (zero beyond the tensor): absmax over the
// ML = B_M / 8 lanes of a block (across waves through xw[4] when ML > 64),
// codes and the block scale.  Every lane of the 256-lane workgroup calls it.
__device__ __forceinline__ void mq_encode8(int mk, uint8_t* m_q, float* m_scale, int64_t e0, int64_t mb, bool m_ok,
                                           const float* m, int ML, float* xw) {
  const int lane = threadIdx.x, wave = lane >> 6;
  uint32_t ab = 0u;
#pragma unroll
  for (int k = 0; k < 8; ++k) ab = max(ab, __float_as_uint(m[k]) & 0x7FFFFFFFu);
  float bam = grp_max(__uint_as_float(ab), ML < 64 ? ML : 64);
  if (ML > 64) {
    if ((lane & 63) == 0) xw[wave] = bam;
    __syncthreads();
    const int wpb = ML >> 6, w0 = (wave / wpb) * wpb;
    bam = xw[w0];
    for (int ww = 1; ww < wpb; ++ww) bam = fmaxf(bam, xw[w0 + ww]);
  }
  if (!m_ok) return;
  const float am = fmaxf(bam, 1e-12f);
  const float ram = __builtin_amdgcn_rcpf(am);
  if (mk == 2 || mk == 4) {
    uint32_t wq = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t hi4 = m_encode(mk, m[2 * j], am, ram);
      const uint32_t lo4 = m_encode(mk, m[2 * j + 1], am, ram);
      wq |= ((hi4 << 4) | lo4) << (8 * j);
    }
    *gp(reinterpret_cast<uint32_t*>(m_q + (e0 >> 1))) = wq;
  } else {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) w0 |= m_encode(mk, m[k], am, ram) << (8 * k);
#pragma unroll
    for (int k = 0; k < 4; ++k) w1 |= m_encode(mk, m[k + 4], am, ram) << (8 * k);
    *gp(reinterpret_cast<u32x2*>(m_q + e0)) = u32x2{w0, w1};
  }
  if ((lane & (ML - 1)) == 0) gp(m_scale)[mb] = am;
}

}  // namespace a8
