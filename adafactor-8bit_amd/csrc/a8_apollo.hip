// APOLLO optimizer step for MI355X (gfx950), all matrices of a group per launch.
//
// Follows _update_param_apollo (optimizer.py:2587-3084) on its non-factorised
// path without CAME (apollo_factorize=False, beta3=None):
//   G (R x C) is projected to rank r: right side (R >= C) g_low = G P^T (R x r),
//   left side g_low = P^T G (r x C), P the seeded Gaussian / sqrt(r);
//   NaN / Inf gradient entries count as zero (optimizer.py:2606);
//   low-rank V: first step v = g_low^2 * beta_v (AL floor -126), later
//   v = lerp(v, g_low^2, beta_v) (floor log2(eps^2)); low-rank M: lerp(m, g_low, 1-beta1);
//   u = m / (sqrt(v) + eps) (or g_low / (...) without beta1);
//   channel scale s = ||u_ch|| / (||g_low_ch|| + 1e-8) over rows (right) or
//   columns (left), or one tensor scale; Fira on sqrt(sum ||G_ch||^2 s^2) (or
//   ||G|| s); p <- p * decay + (step * G) * final_scale, step = -alpha / denom
//   with bias correction.
//
// One step of a group of matrices is five launches over a device table of
// per-matrix descriptors (each kernel finds its matrix by a binary search of a
// compact first-workgroup array):
//   k_ap_proj    bf16 G: MFMA projection (v_mfma_f32_32x32x16_bf16) of 64-row
//                (right) or 64-column (left) tiles of G against P^T split into
//                three bf16 terms (3 x 8 significand bits carry fp32's 24; all
//                products land in one fp32 accumulator), reading G once: the
//                same pass scrubs non-finite entries and accumulates the channel
//                norms of G.  fp32 G: the same tiles with G split into three
//                bf16 terms as well (six products per pair of terms).
//   k_ap_low     low-rank V/M EMA and re-encode, u
//   k_ap_scale   channel (or tensor) norms of u and g_low, per-workgroup partials
//   k_ap_scalars one workgroup per matrix: alpha, Fira, step, decay
//   k_ap_apply   full-rank writeback (deterministic or stochastic rounding)
#include <vector>
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kApTile = 64;     // G columns per left-side projection tile (and fp32 G's right-side tile)
constexpr int kApRB = 3;        // 32-row blocks per right-side bf16 projection tile
constexpr int kApTileR = 32 * kApRB;   // G rows per right-side bf16 projection tile
constexpr int kApPass = 256;    // low-rank outputs per projection pass (4 waves x 64)
constexpr int kApUnit = 2048;   // low-rank elements per k_ap_low workgroup (8 per lane)
constexpr int kApScR = 16;      // right side: g_low rows per k_ap_scale workgroup
constexpr int kApScL = 64;      // left side: g_low columns per k_ap_scale workgroup
constexpr int kApRuns = 2;      // runs of eight elements per k_ap_apply lane (4 measured slower)
constexpr int kApApp = 2048 * kApRuns;   // matrix elements per k_ap_apply workgroup

constexpr int kApWide = 256;     // channels per wide projection tile (bf16 G, rank % 256 == 0)
static_assert(kApWide == kApPass, "a wide tile covers one output pass");

// G channels per projection tile of a matrix: wide tiles for bf16 G at ranks
// that are a multiple of 256, else kApTileR rows (bf16, right side) or kApTile.
__host__ __device__ inline int64_t ap_tile(bool g16, int64_t R, int64_t C, int64_t r) {
  if (g16 && r % kApWide == 0) return kApWide;
  return (g16 && R >= C) ? kApTileR : kApTile;
}

// Workspace of one matrix (offsets in floats; partial arrays hold doubles).
struct ApL {
  int64_t n_low, nchg, K, Kp, rp, ntr, npass, ntile, nunit, nsc, napp;
  int64_t glow, u, ngsq, fin, scal, gpart, ppart, spart, psplit, total;
};

// trows: G channels (rows on the right side, columns on the left) per projection
// tile, as ap_tile picks it.
__host__ __device__ inline ApL ap_layout(int64_t R, int64_t C, int64_t r, int64_t trows) {
  ApL w;
  const bool right = R >= C;
  w.n_low = (right ? R : C) * r;
  w.nchg = right ? R : C;                  // channels of G: rows (right) / columns (left)
  w.K = right ? C : R;                     // reduction length of the projection
  w.Kp = (w.K + 63) / 64 * 64;
  w.rp = (r + 31) / 32 * 32;
  const int64_t tile = trows;
  w.ntr = (w.nchg + tile - 1) / tile;
  w.npass = (w.rp + kApPass - 1) / kApPass;
  w.ntile = w.ntr * w.npass;
  w.nunit = (w.n_low + kApUnit - 1) / kApUnit;
  w.nsc = right ? (R + kApScR - 1) / kApScR : (C + kApScL - 1) / kApScL;
  w.napp = (R * C + kApApp - 1) / kApApp;
  w.glow = 0;
  w.u = w.glow + w.n_low;
  w.ngsq = w.u + w.n_low;                  // ||G_ch||^2
  w.fin = w.ngsq + w.nchg;                 // channel scale s
  w.scal = w.fin + w.nchg;                 // 16 per-matrix scalars
  w.gpart = (w.scal + 16 + 1) / 2 * 2;     // double[ntr]  ||G||^2 per tile
  w.ppart = w.gpart + 2 * w.ntr;           // double[ntr]  ||p||^2 per tile
  w.spart = w.ppart + 2 * w.ntr;           // double[3 nsc] sum ngsq s^2, sum u^2, sum g_low^2
  w.psplit = (w.spart + 6 * w.nsc + 63) / 64 * 64;   // bf16[3][rp][Kp]  P rows, three terms
  w.total = w.psplit + (3 * w.rp * w.Kp + 1) / 2;
  return w;
}

// Scalars in ApL::scal: [0] step (-alpha/denom, bias-corrected), [1] decay,
// [3] tensor final scale, [4] alpha, [5] norm_unscaled, [6] fira scale.

// One matrix.  Read through the scalar cache: 8-byte words only.
struct ApDesc {
  const void* grad;
  void* param;
  float* ws;
  const float* proj_t;
  void* v_q;
  float* v_scale;
  float* v_min_log;
  float* v_fp32;
  uint8_t* m_q;
  float* m_scale;
  float* m_fp32;
  float* fira_prev;
  const float* lr;
  int64_t R, C, r;
  uint64_t sr_seed, step;
  float bias_factor;
  int32_t first, has_prev, valign;
  int32_t rtile_begin, ltile_begin, unit_begin, sc_begin, app_begin, gap;
  int64_t* pstate;   // device projection schedule {last_proj_step, seed, current seed, fresh}, or null
  int32_t trows;     // G channels per projection tile (see ap_tile)
  int32_t wtile_begin;
};
static_assert(sizeof(ApDesc) % 8 == 0, "descriptor is loaded as 64-bit words");

struct ApHyp {
  float bv, w_m, aeps, log_floor, lr_val, eps2, wd, d, margin, sv;
  int lbv, lbm, mk, channel, front, fira, scale_param, bias_mode, wd_mode;
  int rowsum;   // k_ap_low leaves row sums for k_ap_scale where ap_rowsum holds (the plain step)
  const a8_step_scalars* dsc;   // if set: the V lerp weight, rho, bias factor and SR step of this step
};

// A right-side matrix whose low-rank rows (r elements, a power of two in [8, 512])
// lie whole inside k_ap_low's units and within one wave: k_ap_low sums each row's
// u^2 and g_low^2 (double) and stores the two sums where u would go, and
// k_ap_scale reads them instead of u and g_low.  u itself is read by nothing else
// on this path, so it is not written.
__device__ __forceinline__ bool ap_rowsum(const ApDesc& D, const ApHyp& h) {
  return h.rowsum && D.R >= D.C && D.r >= 8 && D.r <= 512 && (D.r & (D.r - 1)) == 0;
}

// Table: ntab descriptors, then five int32 first-workgroup arrays (right-side
// projection tiles, left-side projection tiles, low units, scale workgroups,
// apply workgroups); a matrix without work of a kind repeats the next first
// index, and the search takes the last match.  Without a table the single
// descriptor comes as a kernel argument.
__device__ __forceinline__ ApDesc ap_pick(const ApDesc& one, const ApDesc* tab, int ntab, int which, int wg,
                                          int& local) {
  if (tab == nullptr) {
    local = wg;
    return one;
  }
  const A8_C ApDesc* ct = cp(tab);
  const A8_C int32_t* fb = (const A8_C int32_t*)(ct + ntab) + (int64_t)which * ntab;
  int lo = 0, hi = ntab - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (fb[mid] <= wg) lo = mid; else hi = mid - 1;
  }
  const A8_C uint64_t* w = (const A8_C uint64_t*)(ct + lo);
  uint64_t buf[sizeof(ApDesc) / 8];
#pragma unroll
  for (int i = 0; i < (int)(sizeof(ApDesc) / 8); ++i) buf[i] = w[i];
  ApDesc d;
  __builtin_memcpy(&d, buf, sizeof(ApDesc));
  local = wg - fb[lo];
  return d;
}

__device__ __forceinline__ double ws_d(const float* ws, int64_t off, int64_t i) {
  return gp(reinterpret_cast<const double*>(ws + off))[i];
}
__device__ __forceinline__ void ws_d_set(float* ws, int64_t off, int64_t i, double v) {
  gp(reinterpret_cast<double*>(ws + off))[i] = v;
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

// ------------------------------------------------------------ bf16 helpers
// Eight bf16 of a row: one 16-byte load when all eight are in range and the row
// is 16-byte aligned, element loads otherwise (cnt in 0..8, the rest zero).
__device__ __forceinline__ u32x4 ldg8(const uint16_t* base, int64_t off, int cnt, int vec) {
  if (vec && cnt == 8) return *gp(reinterpret_cast<const u32x4*>(base + off));
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (j < cnt) w[j >> 1] |= (uint32_t)gp(base)[off + j] << (16 * (j & 1));
  return u32x4{w[0], w[1], w[2], w[3]};
}
// NaN / Inf (exponent all ones) -> +0 in both halves of a word.  A half's
// exponent field plus 0x0080 reaches bit 15 only when it is all ones (0x7F80 ->
// 0x8000; the low half cannot carry into the high one), and a 16-bit arithmetic
// shift by 15 turns that bit into the half's mask: four instructions a word.
typedef short i16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t scrub2(uint32_t w) {
  const uint32_t u = (w & 0x7F807F80u) + 0x00800080u;
  const i16x2 m = __builtin_bit_cast(i16x2, u) >> (i16x2){15, 15};
  return w & ~__builtin_bit_cast(uint32_t, m);
}
__device__ __forceinline__ u32x4 scrub8(u32x4 q) {
  return u32x4{scrub2(q.x), scrub2(q.y), scrub2(q.z), scrub2(q.w)};
}
// Sum of squares of eight (scrubbed) bf16 values: the products are exact in fp32.
__device__ __forceinline__ double sq8(u32x4 q) {
  double s = 0.0;
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xFFFF0000u);
    s += (double)(a * a);
    s += (double)(b * b);
  }
  return s;
}
__device__ __forceinline__ bf16x8 as_bf8(u32x4 q) { return __builtin_bit_cast(bf16x8, q); }
// 16 bytes at a workgroup-uniform base plus a 32-bit per-lane byte offset (the
// address form that keeps the base in SGPRs).
__device__ __forceinline__ u32x4 ldu(const void* base, uint32_t off) {
  return *gp(reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + off));
}
__device__ __forceinline__ bf16x8 ldp8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *gp(reinterpret_cast<const u32x4*>(p)));
}
__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// ||G_ch||^2 as torch.linalg.vector_norm(...).square(): the norm rounded to fp32, squared.
__device__ __forceinline__ float norm_sq(double s) {
  const float nrm = sqrtf((float)s);
  return nrm * nrm;
}

// ------------------------------------------------------------ P^T split
// The projection's P operand (rows of P: output index n, reduction index k) in
// three bf16 terms hi + mid + lo = the fp32 value exactly, stored in MFMA
// fragment order so that one wave's fragment load is 1 KB of contiguous memory:
// 16-byte unit u = (((kc * 3 + t) * nblk + blk) * 2 + j) * 64 + l holds
// P[32 blk + l % 32][32 kc + 16 (l / 32) + 8 j .. +8] of term t (zero padded to
// rp x Kp).  With lane half hi = l / 32 holding k = 16 hi + 8 j, sub-step j of
// a 32-k chunk takes the same k permutation on both operands, which leaves the
// sum unchanged.  A 32-k chunk's units are contiguous per term, so a wide tile
// copies a chunk's eight output blocks as three 16 KB runs.
__device__ __forceinline__ int64_t psw_unit(int64_t t, int64_t blk, int64_t kc, int j, int l, int64_t nblk,
                                            int64_t nkc) {
  (void)nkc;
  return (((kc * 3 + t) * nblk + blk) * 2 + j) * 64 + l;
}

// One 16-byte unit u of the split (three terms), from P^T values pv(row, k).
template <typename PV>
__device__ __forceinline__ void split_unit(int64_t u, int64_t nblk, int64_t nkc, int64_t r, int64_t K,
                                           PV pv, u32x4* __restrict__ out) {
  const int l = (int)(u & 63), j = (int)((u >> 6) & 1);
  const int64_t c = u >> 7, kc = c % nkc, blk = c / nkc;
  const int64_t row = 32 * blk + (l & 31), k0 = 32 * kc + 16 * (l >> 5) + 8 * j;
  uint32_t w[3][4] = {};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t k = k0 + e;
    const float x = (row < r && k < K) ? pv(row, k) : 0.0f;
    const __hip_bfloat16 h = __float2bfloat16(x);
    const float r1 = x - __bfloat162float(h);
    const __hip_bfloat16 m = __float2bfloat16(r1);
    const __hip_bfloat16 lo = __float2bfloat16(r1 - __bfloat162float(m));
    uint16_t bh, bm, bl;
    __builtin_memcpy(&bh, &h, 2);
    __builtin_memcpy(&bm, &m, 2);
    __builtin_memcpy(&bl, &lo, 2);
    w[0][e >> 1] |= (uint32_t)bh << (16 * (e & 1));
    w[1][e >> 1] |= (uint32_t)bm << (16 * (e & 1));
    w[2][e >> 1] |= (uint32_t)bl << (16 * (e & 1));
  }
#pragma unroll
  for (int t = 0; t < 3; ++t)
    gp(out)[psw_unit(t, blk, kc, j, l, nblk, nkc)] = u32x4{w[t][0], w[t][1], w[t][2], w[t][3]};
}

__global__ __launch_bounds__(256) void k_ap_split(const float* __restrict__ pt, int64_t r, int64_t K, int right,
                                                 int64_t rp, int64_t Kp, u32x4* __restrict__ out) {
  const int64_t nblk = rp / 32, nkc = Kp / 32;
  const int64_t nu = nblk * nkc * 128;   // units per term
  auto pv = [&](int64_t row, int64_t k) { return right ? gp(pt)[k * r + row] : gp(pt)[row * K + k]; };
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < nu; u += (int64_t)gridDim.x * 256)
    split_unit(u, nblk, nkc, r, K, pv, out);
}

// ------------------------------------------------------------ device projection schedule
// Capturable steps decide the projection refresh on the device (the host's
// _get_apollo_proj_matrix, optimizer.py:2557-2584), so the seed chain and the
// generator run there too.
//
// next_seed (optimizer.py:152-155) is the last of 15 torch.randint(0, 2^63 - 1)
// draws from a CPU generator seeded with the seed.  That generator is MT19937
// (Matsumoto and Nishimura, 1998) initialised from the seed's low 32 bits; a 64-bit
// draw joins two consecutive 32-bit outputs, the first as the high word, and is
// reduced modulo 2^63 - 1.  The 15th draw is outputs 28 and 29.  Output i (< 227)
// is the tempered word mt'[i] = mt[i + 397] ^ twist(mt[i], mt[i + 1]) of the first
// regeneration, which reads initial words only: the initialisation runs to word 426.
__device__ __forceinline__ uint32_t mt_twist_word(uint32_t a, uint32_t b, uint32_t c) {
  const uint32_t y = (a & 0x80000000u) | (b & 0x7FFFFFFFu);
  return c ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
}
__device__ __forceinline__ uint32_t mt_temper(uint32_t y) {
  y ^= y >> 11;
  y ^= (y << 7) & 0x9D2C5680u;
  y ^= (y << 15) & 0xEFC60000u;
  y ^= y >> 18;
  return y;
}
__device__ uint64_t mt_next_seed(uint64_t seed) {
  uint32_t x = (uint32_t)seed;
  uint32_t w28 = 0, w29 = 0, w30 = 0, w425 = 0, w426 = 0;
  for (uint32_t j = 1; j <= 426; ++j) {
    x = 1812433253u * (x ^ (x >> 30)) + j;
    if (j == 28) w28 = x;
    else if (j == 29) w29 = x;
    else if (j == 30) w30 = x;
    else if (j == 425) w425 = x;
    else if (j == 426) w426 = x;
  }
  const uint32_t hi = mt_temper(mt_twist_word(w28, w29, w425));
  const uint32_t lo = mt_temper(mt_twist_word(w29, w30, w426));
  return (((uint64_t)hi << 32) | lo) % 0x7FFFFFFFFFFFFFFFull;
}

// The generator: P's element k (row-major) is z / sqrt(r) with z the Box-Muller
// transform (Box and Muller, 1958) of two uniforms from SplitMix64 (Steele, Lea
// and Flood, 2014) seeded with the projection seed, outputs 2k + 1 and 2k + 2.
__device__ __forceinline__ uint64_t sm64_out(uint64_t seed, uint64_t i) {
  uint64_t z = seed + i * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float proj_value(uint64_t seed, uint64_t k, float rsq) {
  const uint64_t a = sm64_out(seed, 2 * k + 1), b = sm64_out(seed, 2 * k + 2);
  const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
  const double u2 = (double)(b >> 11) * 0x1.0p-53;
  const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
  return (float)z / rsq;
}

// One lane per matrix: t - last_proj_step >= gap starts a new projection.
__global__ __launch_bounds__(64) void k_ap_decide(ApDesc one, const ApDesc* tab, int ntab,
                                                  const a8_step_scalars* dsc) {
  const int i = (int)(blockIdx.x * 64 + threadIdx.x);
  if (i >= (tab ? ntab : 1)) return;
  const ApDesc D = tab ? tab[i] : one;
  if (!D.pstate) return;
  int64_t* ps = D.pstate;
  const int64_t t = (int64_t)load_step_scalars(dsc).step;
  if (t - gp(ps)[0] >= (int64_t)D.gap) {
    const uint64_t cur = (uint64_t)gp(ps)[1];
    gp(ps)[2] = (int64_t)cur;
    gp(ps)[1] = (int64_t)mt_next_seed(cur);
    gp(ps)[0] = t;
    gp(ps)[3] = 1;
  }
}

// kPGen workgroups per matrix: with fresh == 1 they generate P^T from the current
// seed (written to proj_t) and its split; with 2, the split of proj_t as given;
// with 0 (no refresh this step) they exit.  k_ap_scalars clears fresh.
constexpr int kPGen = 32;
__global__ __launch_bounds__(256) void k_ap_pgen(ApDesc one, const ApDesc* tab, int ntab) {
  const int i = (int)blockIdx.x / kPGen, slot = (int)blockIdx.x % kPGen;
  const ApDesc D = tab ? tab[i] : one;
  if (!D.pstate) return;
  const int64_t fresh = gp(D.pstate)[3];
  if (fresh == 0) return;
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const bool right = D.R >= D.C;
  const int64_t r = D.r, K = L.K, nblk = L.rp / 32, nkc = L.Kp / 32, nu = nblk * nkc * 128;
  u32x4* out = reinterpret_cast<u32x4*>(D.ws + L.psplit);
  float* pt = const_cast<float*>(D.proj_t);
  const uint64_t seed = (uint64_t)gp(D.pstate)[2];
  const float rsq = (float)sqrt((double)r);
  for (int64_t u = (int64_t)slot * 256 + threadIdx.x; u < nu; u += (int64_t)kPGen * 256) {
    if (fresh == 1) {
      auto pv = [&](int64_t row, int64_t k) {
        // right: P is r x C, element (row, k); left: P is R x r, element (k, row)
        const float v = proj_value(seed, right ? (uint64_t)(row * K + k) : (uint64_t)(k * r + row), rsq);
        gp(pt)[right ? k * r + row : row * K + k] = v;
        return v;
      };
      split_unit(u, nblk, nkc, r, K, pv, out);
    } else {
      auto pv = [&](int64_t row, int64_t k) { return right ? gp(pt)[k * r + row] : gp(pt)[row * K + k]; };
      split_unit(u, nblk, nkc, r, K, pv, out);
    }
  }
}

// a8_apollo_proj_gen: P^T of one matrix with the generator above.
__global__ __launch_bounds__(256) void k_proj_gen(float* __restrict__ pt, int64_t R, int64_t C, int64_t r,
                                                 uint64_t seed) {
  const bool right = R >= C;
  const int64_t K = right ? C : R, n = r * K;
  const float rsq = (float)sqrt((double)r);
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    // e runs over P^T row-major: right [K x r] (k, row), left [r x K] (row, k)
    const int64_t a = e / (right ? r : K), b = e - a * (right ? r : K);
    const int64_t row = right ? b : a, k = right ? a : b;
    gp(pt)[e] = proj_value(seed, right ? (uint64_t)(row * K + k) : (uint64_t)(k * r + row), rsq);
  }
}

__global__ __launch_bounds__(64) void k_next_seed(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                  int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (i < n) gp(out)[i] = mt_next_seed(gp(in)[i]);
}

// ------------------------------------------------------------ MFMA projection (bf16)
// 32x32x16 lane layout (gfx950): A: lane l holds row l%32, k = 8(l/32)..+8;
// B: column l%32, same k; D: column l%32, acc v at row 8(v/4) + 4(l/32) + v%4.
__device__ __forceinline__ void store_acc(const f32x16& acc, float* out, int64_t ld, int64_t row0, int64_t col,
                                          int64_t nrow, int64_t ncol, int hi) {
  if (col >= ncol) return;
  if (row0 + 32 <= nrow) {   // the whole 32-row block exists
#pragma unroll
    for (int v = 0; v < 16; ++v) gp(out)[(row0 + 8 * (v >> 2) + 4 * hi + (v & 3)) * ld + col] = acc[v];
    return;
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t row = row0 + 8 * (v >> 2) + 4 * hi + (v & 3);
    if (row < nrow) gp(out)[row * ld + col] = acc[v];
  }
}

// Eight squares of a scrubbed bf16 fragment: exact products, an 8-term fp32 sum.
__device__ __forceinline__ float sq8f(u32x4 q) {
  float s = 0.0f;
  const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = __uint_as_float(wv[i] << 16), b = __uint_as_float(wv[i] & 0xFFFF0000u);
    s = __builtin_fmaf(a, a, s);
    s = __builtin_fmaf(b, b, s);
  }
  return s;
}

constexpr int kApGS = 72;   // LDS row stride (halves) of the right side's 64-row x 64-k G slab
constexpr int kApTS = 40;   // LDS row stride (halves) of the left side's transposed 32-row slab

// Right side: tile = kApTileR rows of G (kApRB blocks of 32) x 256 outputs (one
// pass); wave w owns outputs [64w, 64w + 64) of the pass as two 32-column blocks
// (NB of them active), for every row block of the tile.  Each 64-k slab of the
// tile's G rows is loaded once per workgroup with row loads (eight lanes per
// 128-byte row segment, kApRB rows per lane), scrubbed, squared into the row
// norms and stored to LDS (double buffered); the MFMA A fragments come from LDS,
// the B fragments (P) from the fragment-ordered split.  A wave's B fragments
// serve all kApRB row blocks, so the split P streamed through L1 per MFMA falls
// as the tile grows.  FULL: all rows exist, K % 64 == 0 and rows are 16-byte
// aligned.
template <bool FULL, int NB>
__device__ __forceinline__ void proj_right(const ApDesc& D, const ApL& L, int tile, uint16_t* lds, double* sred) {
  constexpr int RB = kApRB;
  const int lane = threadIdx.x, l = lane & 63, l32 = l & 31, hi = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(lane >> 6);
  const int pass = (int)(tile / L.ntr);
  const int64_t rt = tile - (int64_t)pass * L.ntr;
  const int64_t R = D.R, C = D.C, r = D.r, K = C;
  const int64_t row0 = rt * kApTileR;
  const int64_t cb0 = (int64_t)pass * kApPass + w * 64;
  constexpr bool act1 = NB >= 2;
  const int64_t nblk = L.rp / 32, nkc = L.Kp / 32;
  const int64_t blk0 = cb0 / 32;
  const uint16_t* G = reinterpret_cast<const uint16_t*>(D.grad);
  const u32x4* Ps = reinterpret_cast<const u32x4*>(D.ws + L.psplit);
  const int lr = lane >> 3, lc = (lane & 7) * 8;   // loader: rows lr + 32 q, k chunk lc
  const bool pass0 = pass == 0;
  f32x16 acc0[RB], acc1[RB];
#pragma unroll
  for (int q = 0; q < RB; ++q) { acc0[q] = f32x16{}; acc1[q] = f32x16{}; }
  double nr[RB];
#pragma unroll
  for (int q = 0; q < RB; ++q) nr[q] = 0.0;
  auto ldG = [&](int64_t k0, u32x4* x) {
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int64_t ga = row0 + lr + 32 * q;
      if constexpr (FULL) {
        x[q] = ldu(G + k0, (uint32_t)((ga * C + lc) * 2));
      } else {
        const int64_t k = k0 + lc;
        const int cnt = K - k >= 8 ? 8 : (K - k > 0 ? (int)(K - k) : 0);
        x[q] = ldg8(G, ga * C + k, ga < R ? cnt : 0, D.valign);
      }
    }
  };
  auto ldB = [&](int64_t kc, int t, u32x4* x0, u32x4* x1) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      x0[j] = gp(Ps)[psw_unit(t, blk0, kc, j, l, nblk, nkc)];
      if constexpr (act1) x1[j] = gp(Ps)[psw_unit(t, blk0 + 1, kc, j, l, nblk, nkc)];
    }
  };
  u32x4 f[RB];   // the next slab's G, prefetched
  ldG(0, f);
  u32x4 b0[2], b1[2], c0[2], c1[2];
  if constexpr (NB > 0) ldB(0, 0, b0, b1);
  int buf = 0;
  for (int64_t k0 = 0; k0 < K; k0 += 64) {
    u32x4 x[RB];
#pragma unroll
    for (int q = 0; q < RB; ++q) x[q] = scrub8(f[q]);
    if (k0 + 64 < K) ldG(k0 + 64, f);
    if (pass0) {
#pragma unroll
      for (int q = 0; q < RB; ++q) nr[q] += (double)sq8f(x[q]);
    }
    uint16_t* sl = lds + buf * (kApTileR * kApGS);
#pragma unroll
    for (int q = 0; q < RB; ++q) *reinterpret_cast<u32x4*>(&sl[(lr + 32 * q) * kApGS + lc]) = x[q];
    __syncthreads();   // the slab is in LDS; the other buffer's readers finished a barrier ago
    if constexpr (NB > 0) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int64_t kcg = k0 / 32 + kc;
        u32x4 ar[RB][2];
#pragma unroll
        for (int q = 0; q < RB; ++q) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
            ar[q][j] = *reinterpret_cast<const u32x4*>(&sl[(32 * q + l32) * kApGS + 32 * kc + 16 * hi + 8 * j]);
        }
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          // the next term's (or the next chunk's first term's) P fragments
          const bool last = kc == 1 && t == 2;
          if (t < 2) ldB(kcg, t + 1, c0, c1);
          else if (!last || k0 + 64 < K) ldB(kcg + 1, 0, c0, c1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q = 0; q < RB; ++q) {
              acc0[q] = mfma(as_bf8(ar[q][j]), as_bf8(b0[j]), acc0[q]);
              if constexpr (act1) acc1[q] = mfma(as_bf8(ar[q][j]), as_bf8(b1[j]), acc1[q]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            b0[j] = c0[j];
            if constexpr (act1) b1[j] = c1[j];
          }
        }
      }
    }
    buf ^= 1;
  }
  float* glow = D.ws + L.glow;
#pragma unroll
  for (int q = 0; q < RB; ++q) {
    if constexpr (NB > 0) store_acc(acc0[q], glow, r, row0 + 32 * q, cb0 + l32, R, r, hi);
    if constexpr (act1) store_acc(acc1[q], glow, r, row0 + 32 * q, cb0 + 32 + l32, R, r, hi);
  }
  if (!pass0) return;
  // row norms: the eight lanes of a row (consecutive lanes) combine
  double t = 0.0;
#pragma unroll
  for (int q = 0; q < RB; ++q) {
    double nq = nr[q];
    nq += __shfl_xor(nq, 1, 64);
    nq += __shfl_xor(nq, 2, 64);
    nq += __shfl_xor(nq, 4, 64);
    const int64_t ga = row0 + lr + 32 * q;
    if ((lane & 7) == 0 && ga < R) { gp(D.ws + L.ngsq)[ga] = norm_sq(nq); t += nq; }
  }
  t = ap_wg_sum(t, sred);
  if (lane == 0) ws_d_set(D.ws, L.gpart, rt, t);
}

// Left side: tile = 64 columns of G x 256 outputs (one pass).  The A operand is
// P (rows of the low-rank output, from the fragment-ordered split); the B
// operand needs consecutive rows of G per lane, so each 32-row slab of the tile
// is loaded with row loads (eight lanes per 128-byte row segment) and stored
// transposed to LDS (double buffered).  The loading lanes also sum squares per
// column.  FULL: all 64 columns exist, K % 32 == 0 and rows are 16-byte aligned.
template <bool FULL, int NB>
__device__ __forceinline__ void proj_left(const ApDesc& D, const ApL& L, int tile, uint16_t* ldsT, double* sred) {
  const int lane = threadIdx.x, l = lane & 63, l32 = l & 31, hi = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(lane >> 6);
  const int pass = (int)(tile / L.ntr);
  const int64_t ct = tile - (int64_t)pass * L.ntr;
  const int64_t C = D.C, r = D.r, K = D.R;
  const int64_t n0 = ct * kApTile;
  const int64_t mb0 = (int64_t)pass * kApPass + w * 64;
  constexpr bool act1 = NB >= 2;
  const int64_t nblk = L.rp / 32, nkc = L.Kp / 32;
  const int64_t blk0 = mb0 / 32;
  const uint16_t* G = reinterpret_cast<const uint16_t*>(D.grad);
  const u32x4* Ps = reinterpret_cast<const u32x4*>(D.ws + L.psplit);
  const int lr = lane >> 3, lc = (lane & 7) * 8;   // loader: row lr of the slab, 8 columns
  const int64_t gc = n0 + lc;
  const int cc = C - gc >= 8 ? 8 : (C - gc > 0 ? (int)(C - gc) : 0);
  const bool pass0 = pass == 0;
  f32x16 a00 = {}, a01 = {}, a10 = {}, a11 = {};
  double cs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) cs[j] = 0.0;
  auto ldG = [&](int64_t row) {
    if constexpr (FULL) return ldu(G, (uint32_t)((row * C + gc) * 2));
    else return ldg8(G, row * C + gc, row < K ? cc : 0, D.valign);
  };
  auto ldA = [&](int64_t kc, int t, u32x4* x0, u32x4* x1) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      x0[j] = gp(Ps)[psw_unit(t, blk0, kc, j, l, nblk, nkc)];
      if constexpr (act1) x1[j] = gp(Ps)[psw_unit(t, blk0 + 1, kc, j, l, nblk, nkc)];
    }
  };
  u32x4 f = ldG(lr);   // the next slab's row, prefetched
  u32x4 p0[2], p1[2], q0[2], q1[2];
  if constexpr (NB > 0) ldA(0, 0, p0, p1);
  int buf = 0;
  for (int64_t k0 = 0; k0 < K; k0 += 32) {
    const u32x4 q = scrub8(f);
    if (k0 + 32 < K) f = ldG(k0 + 32 + lr);
    const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
    if (pass0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = __uint_as_float((j & 1) ? (wv[j >> 1] & 0xFFFF0000u) : (wv[j >> 1] << 16));
        cs[j] += (double)(x * x);
      }
    }
    uint16_t* sl = ldsT + buf * (kApTile * kApTS);
#pragma unroll
    for (int j = 0; j < 8; ++j) sl[(lc + j) * kApTS + lr] = (uint16_t)((wv[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
    __syncthreads();   // the slab is in LDS; the other buffer's readers finished a barrier ago
    if constexpr (NB > 0) {
      const int64_t kcg = k0 / 32;
      u32x4 bc0[2], bc1[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bc0[j] = *reinterpret_cast<const u32x4*>(&sl[l32 * kApTS + 16 * hi + 8 * j]);
        bc1[j] = *reinterpret_cast<const u32x4*>(&sl[(32 + l32) * kApTS + 16 * hi + 8 * j]);
      }
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        if (t < 2) ldA(kcg, t + 1, q0, q1);
        else if (k0 + 32 < K) ldA(kcg + 1, 0, q0, q1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          a00 = mfma(as_bf8(p0[j]), as_bf8(bc0[j]), a00);
          a01 = mfma(as_bf8(p0[j]), as_bf8(bc1[j]), a01);
          if constexpr (act1) {
            a10 = mfma(as_bf8(p1[j]), as_bf8(bc0[j]), a10);
            a11 = mfma(as_bf8(p1[j]), as_bf8(bc1[j]), a11);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          p0[j] = q0[j];
          if constexpr (act1) p1[j] = q1[j];
        }
      }
    }
    buf ^= 1;
  }
  float* glow = D.ws + L.glow;
  if constexpr (NB > 0) {
    store_acc(a00, glow, C, mb0, n0 + l32, r, C, hi);
    store_acc(a01, glow, C, mb0, n0 + 32 + l32, r, C, hi);
  }
  if constexpr (act1) {
    store_acc(a10, glow, C, mb0 + 32, n0 + l32, r, C, hi);
    store_acc(a11, glow, C, mb0 + 32, n0 + 32 + l32, r, C, hi);
  }
  if (!pass0) return;
  // column sums: lanes with equal (lane & 7) share columns; xor over 8, 16, 32
  // within the wave, then the four waves through LDS
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    double x = cs[j];
    x += __shfl_xor(x, 8, 64);
    x += __shfl_xor(x, 16, 64);
    x += __shfl_xor(x, 32, 64);
    cs[j] = x;
  }
  if (l < 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) sred[w * 64 + l * 8 + j] = cs[j];
  }
  __syncthreads();
  double t = 0.0;
  if (w == 0) {
    const double s = ((sred[l] + sred[64 + l]) + sred[128 + l]) + sred[192 + l];
    if (n0 + l < C) {
      gp(D.ws + L.ngsq)[n0 + l] = norm_sq(s);
      t = s;
    }
    t = grp_sum_d(t, 64);
  }
  if (lane == 0) ws_d_set(D.ws, L.gpart, ct, t);
}

// ------------------------------------------------------------ MFMA projection, wide tiles
// bf16 G at ranks that are a multiple of 256 (C4's rank 256): a workgroup
// computes a 256-channel x 256-output tile of g_low (channels: G rows on the
// right side, G columns on the left).  Per 32-k slab the workgroup stages both
// operands in LDS, double buffered: G, scrubbed, as [channel][k] rows, and the
// chunk's split P for the tile's eight output blocks (fragment order, a plain
// copy).  Each P unit is then fetched from L2 once per 256 channels: 6 bytes of
// split P per G element (the narrower tiles above fetch it per wave, 16 bytes
// per element at 96 rows).  The global loads of slab s + 1 are in flight while
// slab s is multiplied; one barrier per slab publishes the next.  The squares
// of each channel are summed from the staged slab for the channel norms.
// FULL: all 256 channels exist, K % 32 == 0 and rows are 16-byte aligned.
constexpr int kApW = kApWide;             // channels and outputs of a wide tile
constexpr int kApWS = 40;                 // LDS row stride (halves) of the G slab: 32 k + 8 pad
constexpr int kApWGh = kApW * kApWS;      // halves per G slab buffer (20 KB)
constexpr int kApWPu = 3 * 8 * 2 * 64;    // 16-byte P units per slab: 3 terms x 8 blocks x 2 j x 64 lanes (48 KB)

// Eight waves per wide tile, two per SIMD: waves (channel half gh, output quarter
// oq) each own a 128 x 64 block (4 x 2 MFMA tiles, 128 accumulators), so one
// wave's MFMAs issue while the other of its SIMD waits on LDS or staging.  The
// staging of the next slab is split over 512 lanes (8 loads and 8 LDS stores
// each), and a channel's squares over two lanes (k 0-15 and 16-31 of every slab),
// added once at the end.  A lane's 16 squares of a slab are exact products summed
// in fp32 by v_dot2_f32_bf16 (its rounding is the hardware's, within an ulp of
// the fp32 sum); the slabs' sums accumulate in double.
template <bool RIGHT, bool FULL>
__device__ __forceinline__ void proj_wide8(const ApDesc& D, const ApL& L, int tile, uint16_t* gsl, u32x4* psl,
                                           double* sred) {
  const int tid = threadIdx.x, l = tid & 63, l32 = l & 31, hi = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gh = w >> 2, oq = w & 3;   // the wave's channel half and output quarter
  const int pass = (int)(tile / L.ntr);
  const int64_t gt = tile - (int64_t)pass * L.ntr;
  const int64_t R = D.R, C = D.C, r = D.r;
  const int64_t K = RIGHT ? C : R, nch = RIGHT ? R : C;
  const int64_t ch0 = gt * kApW;
  const int64_t nblk = L.rp / 32;
  const int64_t nslab = (K + 31) / 32;
  const uint16_t* G = reinterpret_cast<const uint16_t*>(D.grad);
  const u32x4* Ps = reinterpret_cast<const u32x4*>(D.ws + L.psplit);
  const bool pass0 = pass == 0;
  // G loader.  Right: rows (tid >> 2) + 128 i, eight k at 8 (tid & 3).  Left: k
  // rows 2 (tid & 15) + i, eight columns at 8 (tid >> 4), stored transposed as
  // pairs of k in one 32-bit word.
  auto ldG1 = [&](int64_t k0, int i) -> u32x4 {
    if constexpr (RIGHT) {
      const int64_t row = ch0 + (tid >> 2) + 128 * i, k = k0 + 8 * (tid & 3);
      if constexpr (FULL) return ldu(G, (uint32_t)((row * C + k) * 2));
      const int cnt = K - k >= 8 ? 8 : (K - k > 0 ? (int)(K - k) : 0);
      return ldg8(G, row * C + k, row < R ? cnt : 0, D.valign);
    } else {
      const int64_t row = k0 + 2 * (tid & 15) + i, col = ch0 + 8 * (tid >> 4);
      if constexpr (FULL) return ldu(G, (uint32_t)((row * C + col) * 2));
      const int cnt = C - col >= 8 ? 8 : (C - col > 0 ? (int)(C - col) : 0);
      return ldg8(G, row * C + col, row < K ? cnt : 0, D.valign);
    }
  };
  // G store, piece i of 2: right, row piece i; left, columns 4 i .. 4 i + 3 of the
  // lane's eight (both k rows)
  auto stG1 = [&](const u32x4* f, uint16_t* sl, int i) {
    if constexpr (RIGHT) {
      *reinterpret_cast<u32x4*>(&sl[((tid >> 2) + 128 * i) * kApWS + 8 * (tid & 3)]) = scrub8(f[i]);
    } else {
      const int kp = 2 * (tid & 15), c0 = 8 * (tid >> 4);
      const u32x4 a = scrub8(f[0]), b = scrub8(f[1]);   // k rows kp, kp + 1
      const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 4 * i; e < 4 * i + 4; ++e) {
        const uint32_t lo = (e & 1) ? (wa[e >> 1] >> 16) : (wa[e >> 1] & 0xFFFFu);
        const uint32_t hv = (e & 1) ? (wb[e >> 1] & 0xFFFF0000u) : (wb[e >> 1] << 16);
        *reinterpret_cast<uint32_t*>(&sl[(c0 + e) * kApWS + kp]) = lo | hv;
      }
    }
  };
  // P: units tid + 512 i of the slab's 3072 (term i / 2)
  auto ldP1 = [&](int64_t kc, int i) -> u32x4 {
    return gp(Ps)[((kc * 3 + (i >> 1)) * nblk + 8 * pass) * 128 + tid + 512 * (i & 1)];
  };
  f32x16 acc[4][2];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[q][c] = f32x16{};
  double nsq = 0.0;   // squares of channel ch0 + (tid & 255), k half tid >> 8
  u32x4 fg[2], fp[6];   // the next slab, between its loads and its LDS stores
  // One slab from LDS buffer b, 48 MFMAs, the other instructions placed between
  // them in a fixed order (scheduling fences):
  //   before MFMA 0: sub-step 0's G fragments, its first P term, the two
  //     channel-row reads;
  //   sub-step 0 (MFMAs 0-23): after MFMA m the squares of channel elements
  //     2m, 2m + 1 (m < 8, one v_dot2); P terms 1-2 (m 0-3), the next slab's 8 global loads (m 4-11),
  //     sub-step 1's G fragments (m 12-15), its P terms 0-1 (m 16-19, into the
  //     registers of sub-step 0's dead terms);
  //   sub-step 1 (MFMAs 24-47): its P term 2 (m 0-1), then after every third
  //     MFMA one of the next slab's 8 LDS stores (6 P units, 2 G pieces).
  auto slab = [&](const int b, const int64_t kn, auto next) {
    constexpr bool NEXT = decltype(next)::value;
    const uint16_t* gs = gsl + b * kApWGh;
    const u32x4* ps = psl + b * kApWPu;
    uint16_t* gn = gsl + (b ^ 1) * kApWGh;
    u32x4* pn = psl + (b ^ 1) * kApWPu;
    u32x4 ga[4], gb[4], pa[3][2], pb[3][2], cr[2];
    float sq16 = 0.0f;
    auto rdG = [&](int j, int q) {
      return *reinterpret_cast<const u32x4*>(&gs[(gh * 128 + 32 * q + l32) * kApWS + 16 * hi + 8 * j]);
    };
    auto rdP = [&](int j, int t, int c) { return ps[((t * 8 + oq * 2 + c) * 2 + j) * 64 + l]; };
    auto rdC = [&](int g) {
      return *reinterpret_cast<const u32x4*>(&gs[(tid & 255) * kApWS + 16 * (tid >> 8) + 8 * g]);
    };
#pragma unroll
    for (int q = 0; q < 4; ++q) ga[q] = rdG(0, q);
#pragma unroll
    for (int c = 0; c < 2; ++c) pa[0][c] = rdP(0, 0, c);
    cr[0] = rdC(0);
    cr[1] = rdC(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < 24; ++m) {
      const int t = m / 8, c = (m / 4) % 2, q = m % 4;
      if constexpr (RIGHT) acc[q][c] = mfma(as_bf8(ga[q]), as_bf8(pa[t][c]), acc[q][c]);
      else acc[q][c] = mfma(as_bf8(pa[t][c]), as_bf8(ga[q]), acc[q][c]);
      if (m < 8) {   // two squares per MFMA (v_dot2), the slab's 16 in fp32, then into double
        const uint32_t wv = cr[m / 4][m % 4];
        sq16 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wv), __builtin_bit_cast(bf16x2, wv), sq16,
                                               false);
        if (m == 7) nsq += (double)sq16;
      }
      if (m < 4) {
        pa[1 + m / 2][m % 2] = rdP(0, 1 + m / 2, m % 2);
      } else if (m < 12) {
        if constexpr (NEXT) {
          if (m < 10) fp[m - 4] = ldP1(kn, m - 4);
          else fg[m - 10] = ldG1(32 * kn, m - 10);
        }
      } else if (m < 16) {
        gb[m - 12] = rdG(1, m - 12);
      } else if (m < 20) {
        pb[(m - 16) / 2][m % 2] = rdP(1, (m - 16) / 2, m % 2);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int m = 0; m < 24; ++m) {
      const int t = m / 8, c = (m / 4) % 2, q = m % 4;
      if constexpr (RIGHT) acc[q][c] = mfma(as_bf8(gb[q]), as_bf8(pb[t][c]), acc[q][c]);
      else acc[q][c] = mfma(as_bf8(pb[t][c]), as_bf8(gb[q]), acc[q][c]);
      if (m < 2) pb[2][m] = rdP(1, 2, m);
      if constexpr (NEXT) {
        if (m % 3 == 2) {
          const int pc = m / 3;
          if (pc < 6) pn[tid + 512 * pc] = fp[pc];
          else stG1(fg, gn, pc - 6);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int i = 0; i < 2; ++i) fg[i] = ldG1(0, i);
#pragma unroll
  for (int i = 0; i < 6; ++i) psl[tid + 512 * i] = ldP1(0, i);
  stG1(fg, gsl, 0);
  stG1(fg, gsl, 1);
  __syncthreads();
  // slab s's LDS stores go to the other buffer, whose readers finished slab s - 1
  // before the last barrier
  for (int64_t s = 0; s + 1 < nslab; ++s) {
    slab((int)(s & 1), s + 1, std::true_type{});
    __syncthreads();
  }
  slab((int)((nslab - 1) & 1), nslab, std::false_type{});
  float* glow = D.ws + L.glow;
  const int64_t gx0 = ch0 + gh * 128, ox0 = (int64_t)pass * kApW + oq * 64;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if constexpr (RIGHT) store_acc(acc[q][c], glow, r, gx0 + 32 * q, ox0 + 32 * c + l32, R, r, hi);
      else store_acc(acc[q][c], glow, C, ox0 + 32 * c, gx0 + 32 * q + l32, r, C, hi);
    }
  if (!pass0) return;
  // a channel's two k halves, then the tile's channels in the order of four waves
  double* half1 = sred + 8;
  if (tid >= kApW) half1[tid - kApW] = nsq;
  __syncthreads();
  double tot = 0.0;
  if (tid < kApW) {
    const int64_t ch = ch0 + tid;
    if (ch < nch) {
      tot = nsq + half1[tid];
      gp(D.ws + L.ngsq)[ch] = norm_sq(tot);
    }
  }
  tot = grp_sum_d(tot, 64);
  if ((tid & 63) == 0) sred[tid >> 6] = tot;
  __syncthreads();
  if (tid == 0) ws_d_set(D.ws, L.gpart, gt, ((sred[0] + sred[1]) + sred[2]) + sred[3]);
}

// ------------------------------------------------------------ MFMA projection (fp32 G)
// fp32 G (fp32 parameters; fp16 / fp64 ones project grad.float()) takes the same
// tiles with G split as P is: hi + mid + lo bf16 terms that sum to the fp32 value
// exactly (24 significand bits in three 8-bit pieces).  The split happens once,
// when a slab is stored to LDS (three planes); the MFMAs take the six products
// whose weight is at least 2^-16 of the leading one -- G_hi P_hi, G_hi P_mid,
// G_mid P_hi, G_hi P_lo, G_mid P_mid, G_lo P_hi -- all exact in the fp32
// accumulator.  The three dropped ones weigh at most 2^-24 (about one fp32
// rounding of each product), so g_low keeps an fp32 GEMM's error bound.
// Non-finite G entries count as zero (optimizer.py:2606); the channel norms take
// fp32 squares summed in double.

// x (fp32, finite or not) -> three bf16 terms of scrub(x); returns scrub(x).
__device__ __forceinline__ float split3(float x, uint16_t& h, uint16_t& m, uint16_t& lo) {
  x = scrub(x);
  const __hip_bfloat16 bh = __float2bfloat16(x);
  const float r1 = x - __bfloat162float(bh);
  const __hip_bfloat16 bm = __float2bfloat16(r1);
  const __hip_bfloat16 bl = __float2bfloat16(r1 - __bfloat162float(bm));
  __builtin_memcpy(&h, &bh, 2);
  __builtin_memcpy(&m, &bm, 2);
  __builtin_memcpy(&lo, &bl, 2);
  return x;
}
// Eight fp32 values -> three planes of eight bf16 (u32x4 each); adds their squares.
__device__ __forceinline__ void split8(const float* x, u32x4* pl, double& sq) {
  uint32_t w[3][4] = {};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint16_t h, m, lo;
    const float v = split3(x[e], h, m, lo);
    sq += (double)(v * v);
    w[0][e >> 1] |= (uint32_t)h << (16 * (e & 1));
    w[1][e >> 1] |= (uint32_t)m << (16 * (e & 1));
    w[2][e >> 1] |= (uint32_t)lo << (16 * (e & 1));
  }
#pragma unroll
  for (int t = 0; t < 3; ++t) pl[t] = u32x4{w[t][0], w[t][1], w[t][2], w[t][3]};
}
// Eight fp32 of a row at element offset off: two 16-byte loads when all eight exist
// and the row is aligned, element loads otherwise (missing ones zero).
__device__ __forceinline__ void ldf8(const float* base, int64_t off, int cnt, int vec, float* x) {
  if (vec && cnt == 8) {
    const f32x4 a = *gp(reinterpret_cast<const f32x4*>(base + off));
    const f32x4 b = *gp(reinterpret_cast<const f32x4*>(base + off + 4));
    x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
    x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = e < cnt ? gp(base)[off + e] : 0.0f;
}

constexpr int kApPlaneR = 2 * kApTile * kApGS;   // halves per G plane (two buffers), right side
constexpr int kApPlaneL = 2 * kApTile * kApTS;   // left side

template <bool FULL, int NB>
__device__ __forceinline__ void proj_right32(const ApDesc& D, const ApL& L, int tile, uint16_t* lds, double* sred) {
  const int lane = threadIdx.x, l = lane & 63, l32 = l & 31, hi = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(lane >> 6);
  const int pass = (int)(tile / L.ntr);
  const int64_t rt = tile - (int64_t)pass * L.ntr;
  const int64_t R = D.R, C = D.C, r = D.r, K = C;
  const int64_t row0 = rt * kApTile;
  const int64_t cb0 = (int64_t)pass * kApPass + w * 64;
  constexpr bool act1 = NB >= 2;
  const int64_t nblk = L.rp / 32, nkc = L.Kp / 32;
  const int64_t blk0 = cb0 / 32;
  const float* G = reinterpret_cast<const float*>(D.grad);
  const u32x4* Ps = reinterpret_cast<const u32x4*>(D.ws + L.psplit);
  const int lr = lane >> 3, lc = (lane & 7) * 8;   // loader: rows lr and lr + 32, k chunk lc
  const int64_t ga = row0 + lr, gb = row0 + lr + 32;
  const bool pass0 = pass == 0;
  f32x16 a00 = {}, a01 = {}, a10 = {}, a11 = {};
  double na = 0.0, nb = 0.0;
  auto ldG = [&](int64_t k0, float* x, float* y) {
    const int64_t k = k0 + lc;
    const int cnt = FULL ? 8 : (K - k >= 8 ? 8 : (K - k > 0 ? (int)(K - k) : 0));
    ldf8(G, ga * C + k, (FULL || ga < R) ? cnt : 0, FULL ? 1 : D.valign, x);
    ldf8(G, gb * C + k, (FULL || gb < R) ? cnt : 0, FULL ? 1 : D.valign, y);
  };
  auto ldB = [&](int64_t kc, int t, u32x4* x0, u32x4* x1) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      x0[j] = gp(Ps)[psw_unit(t, blk0, kc, j, l, nblk, nkc)];
      if constexpr (act1) x1[j] = gp(Ps)[psw_unit(t, blk0 + 1, kc, j, l, nblk, nkc)];
    }
  };
  float fx[8], fy[8];   // the next slab's G, prefetched
  ldG(0, fx, fy);
  u32x4 b0[2], b1[2], c0[2], c1[2];
  if constexpr (NB > 0) ldB(0, 0, b0, b1);
  int buf = 0;
  for (int64_t k0 = 0; k0 < K; k0 += 64) {
    u32x4 px[3], py[3];
    double sa = 0.0, sb = 0.0;
    split8(fx, px, sa);
    split8(fy, py, sb);
    if (pass0) { na += sa; nb += sb; }
    if (k0 + 64 < K) ldG(k0 + 64, fx, fy);
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      uint16_t* sl = lds + t * kApPlaneR + buf * (kApTile * kApGS);
      *reinterpret_cast<u32x4*>(&sl[lr * kApGS + lc]) = px[t];
      *reinterpret_cast<u32x4*>(&sl[(lr + 32) * kApGS + lc]) = py[t];
    }
    __syncthreads();   // the slab is in LDS; the other buffer's readers finished a barrier ago
    if constexpr (NB > 0) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int64_t kcg = k0 / 32 + kc;
        u32x4 ar0[3][2], ar1[3][2];
#pragma unroll
        for (int t = 0; t < 3; ++t) {
          const uint16_t* sl = lds + t * kApPlaneR + buf * (kApTile * kApGS);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            ar0[t][j] = *reinterpret_cast<const u32x4*>(&sl[l32 * kApGS + 32 * kc + 16 * hi + 8 * j]);
            ar1[t][j] = *reinterpret_cast<const u32x4*>(&sl[(32 + l32) * kApGS + 32 * kc + 16 * hi + 8 * j]);
          }
        }
#pragma unroll
        for (int tb = 0; tb < 3; ++tb) {   // P term tb meets G planes 0 .. 2 - tb
          const bool last = kc == 1 && tb == 2;
          if (tb < 2) ldB(kcg, tb + 1, c0, c1);
          else if (!last || k0 + 64 < K) ldB(kcg + 1, 0, c0, c1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int ta = 0; ta < 3 - tb; ++ta) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              a00 = mfma(as_bf8(ar0[ta][j]), as_bf8(b0[j]), a00);
              a10 = mfma(as_bf8(ar1[ta][j]), as_bf8(b0[j]), a10);
              if constexpr (act1) {
                a01 = mfma(as_bf8(ar0[ta][j]), as_bf8(b1[j]), a01);
                a11 = mfma(as_bf8(ar1[ta][j]), as_bf8(b1[j]), a11);
              }
            }
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            b0[j] = c0[j];
            if constexpr (act1) b1[j] = c1[j];
          }
        }
      }
    }
    buf ^= 1;
  }
  float* glow = D.ws + L.glow;
  if constexpr (NB > 0) {
    store_acc(a00, glow, r, row0, cb0 + l32, R, r, hi);
    store_acc(a10, glow, r, row0 + 32, cb0 + l32, R, r, hi);
  }
  if constexpr (act1) {
    store_acc(a01, glow, r, row0, cb0 + 32 + l32, R, r, hi);
    store_acc(a11, glow, r, row0 + 32, cb0 + 32 + l32, R, r, hi);
  }
  if (!pass0) return;
  na += __shfl_xor(na, 1, 64);
  na += __shfl_xor(na, 2, 64);
  na += __shfl_xor(na, 4, 64);
  nb += __shfl_xor(nb, 1, 64);
  nb += __shfl_xor(nb, 2, 64);
  nb += __shfl_xor(nb, 4, 64);
  double t = 0.0;
  if ((lane & 7) == 0) {
    if (ga < R) { gp(D.ws + L.ngsq)[ga] = norm_sq(na); t += na; }
    if (gb < R) { gp(D.ws + L.ngsq)[gb] = norm_sq(nb); t += nb; }
  }
  t = ap_wg_sum(t, sred);
  if (lane == 0) ws_d_set(D.ws, L.gpart, rt, t);
}

template <bool FULL, int NB>
__device__ __forceinline__ void proj_left32(const ApDesc& D, const ApL& L, int tile, uint16_t* ldsT, double* sred) {
  const int lane = threadIdx.x, l = lane & 63, l32 = l & 31, hi = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(lane >> 6);
  const int pass = (int)(tile / L.ntr);
  const int64_t ct = tile - (int64_t)pass * L.ntr;
  const int64_t C = D.C, r = D.r, K = D.R;
  const int64_t n0 = ct * kApTile;
  const int64_t mb0 = (int64_t)pass * kApPass + w * 64;
  constexpr bool act1 = NB >= 2;
  const int64_t nblk = L.rp / 32, nkc = L.Kp / 32;
  const int64_t blk0 = mb0 / 32;
  const float* G = reinterpret_cast<const float*>(D.grad);
  const u32x4* Ps = reinterpret_cast<const u32x4*>(D.ws + L.psplit);
  const int lr = lane >> 3, lc = (lane & 7) * 8;   // loader: row lr of the slab, 8 columns
  const int64_t gc = n0 + lc;
  const int cc = C - gc >= 8 ? 8 : (C - gc > 0 ? (int)(C - gc) : 0);
  const bool pass0 = pass == 0;
  f32x16 a00 = {}, a01 = {}, a10 = {}, a11 = {};
  double cs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) cs[j] = 0.0;
  auto ldG = [&](int64_t row, float* x) {
    ldf8(G, row * C + gc, (FULL || row < K) ? (FULL ? 8 : cc) : 0, FULL ? 1 : D.valign, x);
  };
  auto ldA = [&](int64_t kc, int t, u32x4* x0, u32x4* x1) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      x0[j] = gp(Ps)[psw_unit(t, blk0, kc, j, l, nblk, nkc)];
      if constexpr (act1) x1[j] = gp(Ps)[psw_unit(t, blk0 + 1, kc, j, l, nblk, nkc)];
    }
  };
  float f[8];   // the next slab's row, prefetched
  ldG(lr, f);
  u32x4 p0[2], p1[2], q0[2], q1[2];
  if constexpr (NB > 0) ldA(0, 0, p0, p1);
  int buf = 0;
  for (int64_t k0 = 0; k0 < K; k0 += 32) {
    uint16_t h[3][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = split3(f[j], h[0][j], h[1][j], h[2][j]);
      if (pass0) cs[j] += (double)(v * v);
    }
    if (k0 + 32 < K) ldG(k0 + 32 + lr, f);
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      uint16_t* sl = ldsT + t * kApPlaneL + buf * (kApTile * kApTS);
#pragma unroll
      for (int j = 0; j < 8; ++j) sl[(lc + j) * kApTS + lr] = h[t][j];
    }
    __syncthreads();   // the slab is in LDS; the other buffer's readers finished a barrier ago
    if constexpr (NB > 0) {
      const int64_t kcg = k0 / 32;
      u32x4 bc0[3][2], bc1[3][2];
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        const uint16_t* sl = ldsT + t * kApPlaneL + buf * (kApTile * kApTS);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bc0[t][j] = *reinterpret_cast<const u32x4*>(&sl[l32 * kApTS + 16 * hi + 8 * j]);
          bc1[t][j] = *reinterpret_cast<const u32x4*>(&sl[(32 + l32) * kApTS + 16 * hi + 8 * j]);
        }
      }
#pragma unroll
      for (int ta = 0; ta < 3; ++ta) {   // P term ta meets G planes 0 .. 2 - ta
        if (ta < 2) ldA(kcg, ta + 1, q0, q1);
        else if (k0 + 32 < K) ldA(kcg + 1, 0, q0, q1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tb = 0; tb < 3 - ta; ++tb) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            a00 = mfma(as_bf8(p0[j]), as_bf8(bc0[tb][j]), a00);
            a01 = mfma(as_bf8(p0[j]), as_bf8(bc1[tb][j]), a01);
            if constexpr (act1) {
              a10 = mfma(as_bf8(p1[j]), as_bf8(bc0[tb][j]), a10);
              a11 = mfma(as_bf8(p1[j]), as_bf8(bc1[tb][j]), a11);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          p0[j] = q0[j];
          if constexpr (act1) p1[j] = q1[j];
        }
      }
    }
    buf ^= 1;
  }
  float* glow = D.ws + L.glow;
  if constexpr (NB > 0) {
    store_acc(a00, glow, C, mb0, n0 + l32, r, C, hi);
    store_acc(a01, glow, C, mb0, n0 + 32 + l32, r, C, hi);
  }
  if constexpr (act1) {
    store_acc(a10, glow, C, mb0 + 32, n0 + l32, r, C, hi);
    store_acc(a11, glow, C, mb0 + 32, n0 + 32 + l32, r, C, hi);
  }
  if (!pass0) return;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    double x = cs[j];
    x += __shfl_xor(x, 8, 64);
    x += __shfl_xor(x, 16, 64);
    x += __shfl_xor(x, 32, 64);
    cs[j] = x;
  }
  if (l < 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) sred[w * 64 + l * 8 + j] = cs[j];
  }
  __syncthreads();
  double t = 0.0;
  if (w == 0) {
    const double s = ((sred[l] + sred[64 + l]) + sred[128 + l]) + sred[192 + l];
    if (n0 + l < C) {
      gp(D.ws + L.ngsq)[n0 + l] = norm_sq(s);
      t = s;
    }
    t = grp_sum_d(t, 64);
  }
  if (lane == 0) ws_d_set(D.ws, L.gpart, ct, t);
}

// Workgroups are dealt to the 8 XCDs round-robin by index, each XCD with its own
// L2.  Consecutive projection tiles of a matrix share its P split (3 x 2 r K
// bytes, ~3 MB at r = 256, K = 2048), so tile order is remapped to give each XCD
// one contiguous range of tiles: its resident workgroups then work on one or two
// matrices at a time and re-read P from their L2.
__device__ __forceinline__ int xcd_order(int b, int nwg) {
  constexpr int kXcd = 8;
  const int x = b % kXcd, slot = b / kXcd;
  const int q = nwg / kXcd, rem = nwg % kXcd;
  return x < rem ? x * (q + 1) + slot : rem * (q + 1) + (x - rem) * q + slot;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_ap_proj_r(ApDesc one, const ApDesc* tab, int ntab) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kApTileR * kApGS];
  __shared__ double sred[8];
  int local;
  const ApDesc D = ap_pick(one, tab, ntab, 0, xcd_order((int)blockIdx.x, (int)gridDim.x), local);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t row0 = (local % L.ntr) * kApTileR;
  const bool full = D.valign && row0 + kApTileR <= D.R && D.C % 64 == 0;
  const int64_t cb0 = (int64_t)(local / L.ntr) * kApPass + (threadIdx.x >> 6) * 64;
  const int nb = cb0 + 32 < L.rp ? 2 : (cb0 < L.rp ? 1 : 0);   // uniform per wave
  // every wave runs the slab loop (it holds the workgroup barriers)
  if (full) {
    if (nb == 2) proj_right<true, 2>(D, L, local, lds, sred);
    else if (nb == 1) proj_right<true, 1>(D, L, local, lds, sred);
    else proj_right<true, 0>(D, L, local, lds, sred);
  } else {
    if (nb == 2) proj_right<false, 2>(D, L, local, lds, sred);
    else if (nb == 1) proj_right<false, 1>(D, L, local, lds, sred);
    else proj_right<false, 0>(D, L, local, lds, sred);
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_ap_proj_l(ApDesc one, const ApDesc* tab, int ntab) {
  __shared__ __attribute__((aligned(16))) uint16_t ldsT[2 * kApTile * kApTS];
  __shared__ double sred[4 * 64 + 4];
  int local;
  const ApDesc D = ap_pick(one, tab, ntab, 1, xcd_order((int)blockIdx.x, (int)gridDim.x), local);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t n0 = (local % L.ntr) * kApTile;
  const bool full = D.valign && n0 + kApTile <= D.C && D.R % 32 == 0;
  const int64_t mb0 = (int64_t)(local / L.ntr) * kApPass + (threadIdx.x >> 6) * 64;
  const int nb = mb0 + 32 < L.rp ? 2 : (mb0 < L.rp ? 1 : 0);   // uniform per wave
  if (full) {
    if (nb == 2) proj_left<true, 2>(D, L, local, ldsT, sred);
    else if (nb == 1) proj_left<true, 1>(D, L, local, ldsT, sred);
    else proj_left<true, 0>(D, L, local, ldsT, sred);
  } else {
    if (nb == 2) proj_left<false, 2>(D, L, local, ldsT, sred);
    else if (nb == 1) proj_left<false, 1>(D, L, local, ldsT, sred);
    else proj_left<false, 0>(D, L, local, ldsT, sred);
  }
}

// Wide tiles of both sides, eight waves (one workgroup per CU: 138 KB of LDS).
// Workgroups are dealt to the 8 XCDs round-robin by index; XCD x takes the
// contiguous tile range [start[x], start[x + 1]) in order (its L2 then holds
// the P split of one or two matrices at a time).  The host cuts the ranges at
// equal cost (slabs of K) rather than equal tile counts: K differs between
// matrices (k / v against the rest), and count-equal ranges left one XCD with
// 12% more work than the average.  Slots past an XCD's range exit at once.
struct ApXcd {
  int32_t start[9];
};
__global__ __launch_bounds__(512) void k_ap_proj_w8(ApDesc one, const ApDesc* tab, int ntab, ApXcd xs) {
  __shared__ __attribute__((aligned(16))) uint16_t gsl[2 * kApWGh];
  __shared__ u32x4 psl[2 * kApWPu];
  __shared__ double sred[8 + kApW];
  const int x = (int)blockIdx.x % 8;
  const int wg = xs.start[x] + (int)blockIdx.x / 8;
  if (wg >= xs.start[x + 1]) return;
  int local;
  const ApDesc D = ap_pick(one, tab, ntab, 5, wg, local);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t ch0 = (local % L.ntr) * kApW;
  if (D.R >= D.C) {
    if (D.valign && ch0 + kApW <= D.R && D.C % 32 == 0) proj_wide8<true, true>(D, L, local, gsl, psl, sred);
    else proj_wide8<true, false>(D, L, local, gsl, psl, sred);
  } else {
    if (D.valign && ch0 + kApW <= D.C && D.R % 32 == 0) proj_wide8<false, true>(D, L, local, gsl, psl, sred);
    else proj_wide8<false, false>(D, L, local, gsl, psl, sred);
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_ap_proj_r32(ApDesc one, const ApDesc* tab, int ntab) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[3 * kApPlaneR];
  __shared__ double sred[8];
  int local;
  const ApDesc D = ap_pick(one, tab, ntab, 0, xcd_order((int)blockIdx.x, (int)gridDim.x), local);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t row0 = (local % L.ntr) * kApTile;
  const bool full = D.valign && row0 + kApTile <= D.R && D.C % 64 == 0;
  const int64_t cb0 = (int64_t)(local / L.ntr) * kApPass + (threadIdx.x >> 6) * 64;
  const int nb = cb0 + 32 < L.rp ? 2 : (cb0 < L.rp ? 1 : 0);   // uniform per wave
  if (full) {
    if (nb == 2) proj_right32<true, 2>(D, L, local, lds, sred);
    else if (nb == 1) proj_right32<true, 1>(D, L, local, lds, sred);
    else proj_right32<true, 0>(D, L, local, lds, sred);
  } else {
    if (nb == 2) proj_right32<false, 2>(D, L, local, lds, sred);
    else if (nb == 1) proj_right32<false, 1>(D, L, local, lds, sred);
    else proj_right32<false, 0>(D, L, local, lds, sred);
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_ap_proj_l32(ApDesc one, const ApDesc* tab, int ntab) {
  __shared__ __attribute__((aligned(16))) uint16_t ldsT[3 * kApPlaneL];
  __shared__ double sred[4 * 64 + 4];
  int local;
  const ApDesc D = ap_pick(one, tab, ntab, 1, xcd_order((int)blockIdx.x, (int)gridDim.x), local);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t n0 = (local % L.ntr) * kApTile;
  const bool full = D.valign && n0 + kApTile <= D.C && D.R % 32 == 0;
  const int64_t mb0 = (int64_t)(local / L.ntr) * kApPass + (threadIdx.x >> 6) * 64;
  const int nb = mb0 + 32 < L.rp ? 2 : (mb0 < L.rp ? 1 : 0);   // uniform per wave
  if (full) {
    if (nb == 2) proj_left32<true, 2>(D, L, local, ldsT, sred);
    else if (nb == 1) proj_left32<true, 1>(D, L, local, ldsT, sred);
    else proj_left32<true, 0>(D, L, local, ldsT, sred);
  } else {
    if (nb == 2) proj_left32<false, 2>(D, L, local, ldsT, sred);
    else if (nb == 1) proj_left32<false, 1>(D, L, local, ldsT, sred);
    else proj_left32<false, 0>(D, L, local, ldsT, sred);
  }
}

// ------------------------------------------------------------ ||p||^2 (scale_parameter)
// ntr workgroups per matrix, each summing a contiguous share of p^2 in double;
// only the total (k_ap_scalars) is used.
template <typename T>
__global__ __launch_bounds__(256) void k_ap_psq(ApDesc D) {
  __shared__ double sd[4];
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t n = D.R * D.C;
  const int64_t chunk = (n + L.ntr - 1) / L.ntr;
  const int64_t b = (int64_t)blockIdx.x * chunk, e = b + chunk < n ? b + chunk : n;
  const T* P = reinterpret_cast<const T*>(D.param);
  double s = 0.0;
  for (int64_t i = b + threadIdx.x; i < e; i += 256) {
    const float p = ld1<T>(P, i);
    s += (double)(p * p);
  }
  s = ap_wg_sum(s, sd);
  if (threadIdx.x == 0) ws_d_set(D.ws, L.ppart, blockIdx.x, s);
}

// ------------------------------------------------------------ low-rank V / M and u
// Flat 2048-element units of g_low (8 contiguous per lane).  V block B_V and M
// block B_M are powers of two (B_V in [128, 2048], B_M in [32, B_V]), so a
// block is B/8 consecutive lanes.  Arithmetic as optimizer.py:2765-2790, 2911-2951
// (quantised states through _quant_v / _m_ema_pytorch, fp32 states through
// lerp_): v = first ? g^2 * bv : lerp(v, g^2, bv); m = lerp(m, g, 1 - beta1);
// u = m / (sqrt(v) + eps).  u enters the step only through the norms ||u_ch||
// (the channel or tensor scale, optimizer.py:2997-3001), so it takes the hardware
// square root and reciprocal (<= 2 ulp), as the 1-D step's Adam denominator does.  FULL: the unit lies
// inside g_low and u is 16-byte aligned, so every access is a vector access.
// AL8 blocks of >= 512 elements decode through an LDS table of the block's
// 255 code values (one correctly rounded exp2 per lane per block).
template <int VB, int MK, bool FULL>
__device__ __forceinline__ void ap_low_unit(const ApDesc& D, const ApL& L, int unit, const ApHyp& h, float* xw,
                                            float* dtab) {
  const int64_t n = L.n_low;
  float* ws = D.ws;
  const int lane = threadIdx.x, wave = lane >> 6;
  const int64_t e0 = (int64_t)unit * kApUnit + (int64_t)lane * 8;
  const int lbv = h.lbv, lbm = h.lbm;
  const int VL = (1 << lbv) >> 3, ML = (1 << lbm) >> 3;
  const int64_t nvb = VB ? (n + (1 << lbv) - 1) >> lbv : 0;
  const int64_t nmb = (n + (1 << lbm) - 1) >> lbm;
  const int64_t vb = e0 >> lbv, mb = e0 >> lbm;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);
  const bool v_ok = VB ? vb < nvb : cnt > 0;
  const bool m_ok = (MK == 1 || MK == 2) && mb < nmb;   // codes padded to whole M blocks
  const int mk = MK == 1 ? 1 : h.mk;
  const bool first = D.first != 0;
  const float floor_ = first ? -126.0f : h.log_floor;
  float g[8], v[8], m[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) { g[k] = 0.0f; v[k] = 0.0f; m[k] = 0.0f; }
  if constexpr (FULL) {
    const f32x4 a = *gp(reinterpret_cast<const f32x4*>(ws + L.glow + e0));
    const f32x4 b = *gp(reinterpret_cast<const f32x4*>(ws + L.glow + e0 + 4));
    g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w; g[4] = b.x; g[5] = b.y; g[6] = b.z; g[7] = b.w;
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) g[k] = gp(ws)[L.glow + e0 + k];
  }
  // The code streams are loaded here, before the AL8 decode table and its
  // barrier, so that their latency overlaps the table build.
  uint32_t cw[2] = {0u, 0u};   // AL8 codes (table path)
  if constexpr (VB == 8) {
    if (!first && VL >= 64) {
      if constexpr (FULL) {
        const u32x2 q = *gp(reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(D.v_q) + e0));
        cw[0] = q.x; cw[1] = q.y;
      } else if (v_ok) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          cw[k >> 2] |= (uint32_t)gp(reinterpret_cast<const uint8_t*>(D.v_q))[e0 + k] << (8 * (k & 3));
      }
    }
  }
  float ms_old = 0.0f;   // M block scale and codes
  u32x2 mqv = {0u, 0u};
  if constexpr (MK == 1 || MK == 2) {
    if (m_ok) {
      ms_old = gp(D.m_scale)[mb];
      if (mk == 2 || mk == 4) mqv.x = *gp(reinterpret_cast<const uint32_t*>(D.m_q + (e0 >> 1)));
      else mqv = *gp(reinterpret_cast<const u32x2*>(D.m_q + e0));
    }
  }
  // ---- V
  float vo[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) vo[k] = 0.0f;
  if (!first) {
    if constexpr (VB == 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k < cnt) vo[k] = gp(D.v_fp32)[e0 + k];
    } else if (VB == 8 && VL >= 64) {
      // one block per VL lanes (VL / 64 waves); its 255 decoded values into LDS
      const int bw = lane / VL;   // block of this unit
      const int64_t vbb = (int64_t)unit * (kApUnit >> lbv) + bw;
      const bool bok = vbb < nvb;   // a tail unit may end before its last block slot
      const float s_old = bok ? gp(D.v_scale)[vbb] : 0.0f, lm_old = bok ? gp(D.v_min_log)[vbb] : 0.0f;
      for (int c = lane % VL; c < 256; c += VL)
        dtab[bw * 256 + c] = c ? exp2_exact(((float)(c - 1) * s_old) / 254.0f + lm_old) : 0.0f;
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 8; ++k) vo[k] = dtab[bw * 256 + ((cw[k >> 2] >> (8 * (k & 3))) & 0xFFu)];
    } else if (v_ok) {
      const float s_old = gp(D.v_scale)[vb], lm_old = gp(D.v_min_log)[vb];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        uint32_t c;
        if constexpr (VB == 8) c = gp(reinterpret_cast<const uint8_t*>(D.v_q))[e0 + k];
        else c = gp(reinterpret_cast<const uint16_t*>(D.v_q))[e0 + k];
        const float lm2 = VB == 8 ? 254.0f : 65534.0f;
        vo[k] = c ? exp2_exact(((float)(c - 1) * s_old) / lm2 + lm_old) : 0.0f;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float g2 = g[k] * g[k];
    v[k] = first ? g2 * h.bv : lerp_ref(vo[k], g2, h.bv);
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
        if (k < cnt) mo[k] = gp(D.m_fp32)[e0 + k];
    } else if (m_ok) {
      const float ms = ms_old;
      if (mk == 2 || mk == 4) {
        const uint32_t qw = mqv.x;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t byte = (qw >> (8 * (k >> 1))) & 0xFFu;
          mo[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
        }
      } else {
        const u32x2 qv = mqv;
#pragma unroll
        for (int k = 0; k < 8; ++k) mo[k] = m_decode(mk, ((k < 4 ? qv.x : qv.y) >> (8 * (k & 3))) & 0xFFu, ms);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) m[k] = (k < cnt) ? lerp_ref(mo[k], g[k], h.w_m) : 0.0f;
  }
  // ---- u, or the row sums of u^2 and g_low^2 (ap_rowsum)
  if (ap_rowsum(D, h)) {
    double su = 0.0, sg = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k < cnt) {
        const float uk = (MK != 0 ? m[k] : g[k]) * fast_rcp(fast_sqrt(v[k]) + h.aeps);
        su += (double)(uk * uk);
        sg += (double)(g[k] * g[k]);
      }
    }
    const int G = (int)(D.r >> 3);   // lanes of a row, <= 64
    su = grp_sum_d(su, G);
    sg = grp_sum_d(sg, G);
    const int64_t row = e0 / D.r;
    if ((lane & (G - 1)) == 0 && row < D.R) {
      ws_d_set(ws, L.u, 2 * row, su);
      ws_d_set(ws, L.u, 2 * row + 1, sg);
    }
  } else if constexpr (FULL) {
    float uu[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) uu[k] = (MK != 0 ? m[k] : g[k]) * fast_rcp(fast_sqrt(v[k]) + h.aeps);
    *gp(reinterpret_cast<f32x4*>(ws + L.u + e0)) = f32x4{uu[0], uu[1], uu[2], uu[3]};
    *gp(reinterpret_cast<f32x4*>(ws + L.u + e0 + 4)) = f32x4{uu[4], uu[5], uu[6], uu[7]};
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k < cnt) {
        const float x = MK != 0 ? m[k] : g[k];
        gp(ws)[L.u + e0 + k] = x * fast_rcp(fast_sqrt(v[k]) + h.aeps);
      }
    }
  }
  // ---- V state
  if constexpr (VB == 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) gp(D.v_fp32)[e0 + k] = v[k];
  } else {
    uint32_t vmaxb = 0u, vkey = 0xFFFFFFFFu;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      vmaxb = max(vmaxb, __float_as_uint(v[k]));
      vkey = min(vkey, __float_as_uint(v[k]) - 1u);
    }
    float bmax = grp_max(__uint_as_float(vmaxb), VL < 64 ? VL : 64);
    uint32_t bkey = vkey;
    bkey = grp_umin(bkey, VL < 64 ? VL : 64);
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
    const float mnz = (bkey == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(bkey + 1u);
    constexpr int LM2 = VB == 8 ? 254 : 65534;
    // the two correctly rounded logarithms of a block: one lane pair per wave
    // (al_refit_pair); a block spanning several waves is fitted by its first wave
    // only and shared through LDS, so the others skip the double-precision work
    ALFit f;
    if (VL > 64) {   // uniform
      const int wpb = VL >> 6, bw = wave / wpb;
      if (wave % wpb == 0) {
        f = al_refit_pair(bmax, mnz, floor_, (float)LM2, lane);
        if ((lane & 63) == 0) { xw[12 + 2 * bw] = f.lmin; xw[13 + 2 * bw] = f.s; }
      }
      __syncthreads();
      f.lmin = xw[12 + 2 * bw];
      f.s = xw[13 + 2 * bw];
      al_fit_consts(f, (float)LM2);
    } else {
      f = al_refit_pair(bmax, mnz, floor_, (float)LM2, lane);
    }
    if (v_ok) {
      uint32_t code[8];
      al_codes<LM2, 8>(v, f, code);
      if constexpr (FULL && VB == 8) {
        uint32_t cw[2] = {0u, 0u};
#pragma unroll
        for (int k = 0; k < 8; ++k) cw[k >> 2] |= code[k] << (8 * (k & 3));
        *gp(reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(D.v_q) + e0)) = u32x2{cw[0], cw[1]};
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if constexpr (VB == 8) gp(reinterpret_cast<uint8_t*>(D.v_q))[e0 + k] = (uint8_t)code[k];
          else gp(reinterpret_cast<uint16_t*>(D.v_q))[e0 + k] = (uint16_t)code[k];
        }
      }
      if ((lane & (VL - 1)) == 0) { gp(D.v_scale)[vb] = f.s; gp(D.v_min_log)[vb] = f.lmin; }
    }
  }
  // ---- M state
  if constexpr (MK == 3) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k < cnt) gp(D.m_fp32)[e0 + k] = m[k];
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
      for (int ww = 1; ww < wpb; ++ww) bam = fmaxf(bam, xw[8 + w0 + ww]);
    }
    if (m_ok) {
      const float am = fmaxf(bam, 1e-12f);
      const float ram = fast_rcp(am);
      if (mk == 2 || mk == 4) {
        uint32_t wq = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t hi4 = m_encode(mk, m[2 * j], am, ram);
          const uint32_t lo4 = m_encode(mk, m[2 * j + 1], am, ram);
          wq |= ((hi4 << 4) | lo4) << (8 * j);
        }
        *gp(reinterpret_cast<uint32_t*>(D.m_q + (e0 >> 1))) = wq;
      } else {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w0 |= m_encode(mk, m[k], am, ram) << (8 * k);
#pragma unroll
        for (int k = 0; k < 4; ++k) w1 |= m_encode(mk, m[k + 4], am, ram) << (8 * k);
        *gp(reinterpret_cast<u32x2*>(D.m_q + e0)) = u32x2{w0, w1};
      }
      if ((lane & (ML - 1)) == 0) gp(D.m_scale)[mb] = am;
    }
  }
}

template <int VB, int MK>
__global__ __launch_bounds__(256) void k_ap_low(ApDesc one, const ApDesc* tab, int ntab, ApHyp h) {
  __shared__ float xw[16];
  __shared__ float dtab[4 * 256];
  int unit;
  const ApDesc D = ap_pick(one, tab, ntab, 2, (int)blockIdx.x, unit);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  ApHyp hh = h;
  if (hh.dsc) hh.bv = (float)load_step_scalars(hh.dsc).beta_val;
  if ((int64_t)(unit + 1) * kApUnit <= L.n_low && (L.u & 3) == 0) ap_low_unit<VB, MK, true>(D, L, unit, hh, xw, dtab);
  else ap_low_unit<VB, MK, false>(D, L, unit, hh, xw, dtab);
}

// ------------------------------------------------------------ scale
// s_ch = ||u_ch|| / (||g_low_ch|| + 1e-8) (optimizer.py:2997-3001), norms as
// sqrt of fp32 squares summed in double.  Right side: one wave per g_low row
// (16 rows per workgroup); left side: one lane per g_low column walking a
// quarter of the r rows, the four waves combined in LDS (64 columns per
// workgroup).  Partials per workgroup: sum ngsq * s^2 (channel) or sum u^2 and
// sum g_low^2 (tensor).
__global__ __launch_bounds__(256) void k_ap_scale(ApDesc one, const ApDesc* tab, int ntab, ApHyp h) {
  __shared__ double sd[2 * 256 + 4];
  int wg;
  const ApDesc D = ap_pick(one, tab, ntab, 3, (int)blockIdx.x, wg);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const int64_t R = D.R, C = D.C, r = D.r;
  const float* U = D.ws + L.u;
  const float* GL = D.ws + L.glow;
  const int lane = threadIdx.x, w = lane >> 6, l = lane & 63;
  const bool rs = ap_rowsum(D, h);
  double a0 = 0.0, a1 = 0.0, a2 = 0.0;
  if (R >= C) {
#pragma unroll 1
    for (int i = 0; i < kApScR / 4; ++i) {
      const int64_t row = (int64_t)wg * kApScR + w * (kApScR / 4) + i;
      if (row >= R) break;
      double su = 0.0, sg = 0.0;
      if (rs) {   // k_ap_low's row sums
        if (l == 0) {
          su = ws_d(D.ws, L.u, 2 * row);
          sg = ws_d(D.ws, L.u, 2 * row + 1);
        }
      } else {
        for (int64_t k = l; k < r; k += 64) {
          const float u = gp(U)[row * r + k], g = gp(GL)[row * r + k];
          su += (double)(u * u);
          sg += (double)(g * g);
        }
        su = grp_sum_d(su, 64);
        sg = grp_sum_d(sg, 64);
      }
      if (l == 0) {
        if (h.channel) {
          float s = sqrtf((float)su) / (sqrtf((float)sg) + 1e-8f);
          if (h.front) s = s * h.sv;
          gp(D.ws + L.fin)[row] = s;
          a0 += (double)(gp(D.ws + L.ngsq)[row] * (s * s));
        } else {
          a1 += su;
          a2 += sg;
        }
      }
    }
  } else {
    const int64_t c = (int64_t)wg * kApScL + l;
    double su = 0.0, sg = 0.0;
    if (c < C) {
#pragma unroll 4
      for (int64_t k = w; k < r; k += 4) {
        const float u = gp(U)[k * C + c], g = gp(GL)[k * C + c];
        su += (double)(u * u);
        sg += (double)(g * g);
      }
    }
    sd[w * 64 + l] = su;
    sd[256 + w * 64 + l] = sg;
    __syncthreads();
    if (w == 0 && c < C) {
      su = ((sd[l] + sd[64 + l]) + sd[128 + l]) + sd[192 + l];
      sg = ((sd[256 + l] + sd[320 + l]) + sd[384 + l]) + sd[448 + l];
      if (h.channel) {
        float s = sqrtf((float)su) / (sqrtf((float)sg) + 1e-8f);
        if (h.front) s = s * h.sv;
        gp(D.ws + L.fin)[c] = s;
        a0 = (double)(gp(D.ws + L.ngsq)[c] * (s * s));
      } else {
        a1 = su;
        a2 = sg;
      }
    }
  }
  const double t0 = ap_wg_sum(a0, sd + 512);
  const double t1 = ap_wg_sum(a1, sd + 512);
  const double t2 = ap_wg_sum(a2, sd + 512);
  if (lane == 0) {
    ws_d_set(D.ws, L.spart, 3 * (int64_t)wg, t0);
    ws_d_set(D.ws, L.spart, 3 * (int64_t)wg + 1, t1);
    ws_d_set(D.ws, L.spart, 3 * (int64_t)wg + 2, t2);
  }
}

// ------------------------------------------------------------ per-matrix scalars
// One workgroup per matrix: alpha (optimizer.py:832-856), norm_unscaled and Fira
// on it (optimizer.py:3003-3024, 760-782 with the key scaled_grad_norm_prev),
// the RMS denominator, the step -alpha/denom with bias correction, the decay.
__global__ __launch_bounds__(256) void k_ap_scalars(ApDesc one, const ApDesc* tab, int ntab, ApHyp h) {
  __shared__ double sd[4];
  ApDesc D;
  if (tab == nullptr) {
    D = one;
  } else {
    const A8_C uint64_t* wsrc = (const A8_C uint64_t*)(cp(tab) + blockIdx.x);
    uint64_t buf[sizeof(ApDesc) / 8];
#pragma unroll
    for (int i = 0; i < (int)(sizeof(ApDesc) / 8); ++i) buf[i] = wsrc[i];
    __builtin_memcpy(&D, buf, sizeof(ApDesc));
  }
  (void)ntab;
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  float* ws = D.ws;
  const int lane = threadIdx.x;
  double pg = 0.0, pp = 0.0, s0 = 0.0, s1 = 0.0, s2 = 0.0;
  for (int64_t k = lane; k < L.ntr; k += 256) { pg += ws_d(ws, L.gpart, k); pp += ws_d(ws, L.ppart, k); }
  for (int64_t k = lane; k < L.nsc; k += 256) {
    s0 += ws_d(ws, L.spart, 3 * k);
    s1 += ws_d(ws, L.spart, 3 * k + 1);
    s2 += ws_d(ws, L.spart, 3 * k + 2);
  }
  pg = ap_wg_sum(pg, sd);
  pp = ap_wg_sum(pp, sd);
  s0 = ap_wg_sum(s0, sd);
  s1 = ap_wg_sum(s1, sd);
  s2 = ap_wg_sum(s2, sd);
  if (lane != 0) return;
  if (D.pstate) gp(D.pstate)[3] = 0;   // this step's projection refresh (if any) is done
  float lr_val = h.lr_val, bias_factor = D.bias_factor;
  if (h.dsc) {
    const a8_step_scalars sc = load_step_scalars(h.dsc);
    lr_val = sc.rho;
    bias_factor = sc.apollo_bias;
  }
  const int64_t numel = D.R * D.C;
  const float rho = D.lr ? *gp(D.lr) : lr_val;
  float alpha = rho;
  if (h.scale_param) {
    const float rms = sqrtf((float)pp) / (float)sqrt((double)numel);
    alpha = fmaxf(rms, h.eps2) * rho;
  }
  float s_t = 1.0f;   // tensor scale
  float nun;          // norm_unscaled
  if (h.channel) {
    nun = sqrtf((float)s0);
  } else {
    s_t = sqrtf((float)s1) / (sqrtf((float)s2) + 1e-8f);
    if (h.front) s_t = s_t * h.sv;
    nun = sqrtf((float)pg) * s_t;
  }
  float fs = 1.0f;
  if (h.fira) {
    const float curr = __builtin_isfinite(nun) ? nun : 0.0f;
    float next = curr;
    if (D.has_prev) {
      const float p = *gp(D.fira_prev);
      const float ratio = curr / (p + 1e-8f);
      const float lim = (ratio != ratio ? ratio : fmaxf(ratio, h.margin)) / h.margin;
      const bool reset = p < 1e-6f;
      fs = reset ? 1.0f : 1.0f / lim;
      next = reset ? curr : curr * fs;
    }
    *gp(D.fira_prev) = next;
  }
  float denom = 1.0f;
  if (h.d > 0.0f) denom = fmaxf(nun / (float)(sqrt((double)numel) * (double)h.d), 1.0f);
  float step = -alpha / denom;
  if (h.bias_mode == 1) step = step * bias_factor;
  else if (h.bias_mode == 2) step = step / bias_factor;
  float dec = 1.0f;
  if (h.wd_mode == 1) dec = 1.0f - alpha * h.wd;
  else if (h.wd_mode == 2) dec = 1.0f - rho * h.wd;
  float fin_t = s_t;
  if (h.fira) fin_t = fin_t * fs;
  if (!h.front) fin_t = fin_t * h.sv;
  float* sl = ws + L.scal;
  gp(sl)[0] = step;
  gp(sl)[1] = dec;
  gp(sl)[3] = fin_t;
  gp(sl)[4] = alpha;
  gp(sl)[5] = nun;
  gp(sl)[6] = fs;
}

// ------------------------------------------------------------ full-rank writeback
// Deterministic (optimizer.py:3071-3077): p := p * decay (rounded to T), then
// channel p + (step * G) * f_ch (addcmul) or tensor fma(step * f, G, p) (add_),
// rounded to T; f_ch = (s_ch * fira) * sqrt(apollo_scale) at the back.  SR
// (optimizer.py:3058-3063 with the stream of kernels.cu:48-87):
// x = (p * decay) + (G * f) * step in fp32, stochastically rounded.  Eight
// consecutive elements per lane (16-byte loads and stores for 16-bit types);
// with C % 8 == 0 they share one row, so one channel scale (right side) or
// eight consecutive ones (left side).
template <typename T>
__device__ __forceinline__ float ap_fch(const float* fin, int64_t ch, float fs, const ApHyp& h) {
  float f = gp(fin)[ch];
  if (h.fira) f = f * fs;
  if (!h.front) f = f * h.sv;
  return f;
}

// GT: the gradient's element type (the parameter's, or fp32 for fp16 params,
// whose projection runs on an fp32 copy of G).
template <typename T, bool SR, typename GT = T>
__global__ __launch_bounds__(256) void k_ap_apply(ApDesc one, const ApDesc* tab, int ntab, ApHyp h) {
  int unit;
  const ApDesc D = ap_pick(one, tab, ntab, 4, (int)blockIdx.x, unit);
  const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
  const uint32_t R = (uint32_t)D.R, C = (uint32_t)D.C, n = R * C;   // n < 2^31
  const bool right = R >= C;
  const float* ws = D.ws;
  const float* fin = ws + L.fin;
  const float* sl = ws + L.scal;
  const float step = gp(sl)[0], dec = gp(sl)[1], fin_t = gp(sl)[3], fs = gp(sl)[6];
  const bool has_dec = h.wd_mode != 0;
  T* P = reinterpret_cast<T*>(D.param);
  const GT* G = reinterpret_cast<const GT*>(D.grad);
  // kApRuns runs of eight per lane, 2048 elements apart; every run's loads are
  // issued before the first is computed (a wave keeps several kilobytes in flight)
  const uint32_t ea = (uint32_t)unit * kApApp + threadIdx.x * 8u;
  if (ea >= n) return;
  const uint64_t sr_step = SR && h.dsc ? load_step_scalars(h.dsc).step : D.step;
  float gr[kApRuns][8];
  pval_t<T> pr[kApRuns][8];   // double for fp64 parameters
#pragma unroll
  for (int q = 0; q < kApRuns; ++q) {
    const uint32_t e = ea + 2048u * q;
    if (q == 0 || e < n) {
      load8<GT>(G, e, n, gr[q]);
      load8<T>(P, e, n, pr[q]);
    }
  }
  auto run8 = [&](const uint32_t e0, float* g, pval_t<T>* p) {
    float f[8];
    const uint32_t row = e0 / C, col = e0 - row * C;
    if (!h.channel) {
#pragma unroll
      for (int k = 0; k < 8; ++k) f[k] = fin_t;
    } else if (D.valign && e0 + 8 <= n) {   // all eight in one row
      if (right) {
        const float fr = ap_fch<T>(fin, row, fs, h);
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] = fr;
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) f[k] = ap_fch<T>(fin, col + k, fs, h);
      }
    } else {
      uint32_t rr = row, cc = col;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        f[k] = (e0 + k < n) ? ap_fch<T>(fin, right ? rr : cc, fs, h) : 0.0f;
        if (++cc == C) { cc = 0; ++rr; }
      }
    }
    const float ts = step * fin_t;   // tensor: alpha = step * final_scale
    if constexpr (SR) {
      // The lane's first counter; element k's is zb + k.  The random words come
      // first: unless the eight counters cross a multiple of 2^30 (a lane in 1.5e8),
      // they share their bits from 30 up, hence the high word's share of the first
      // product and the low word of z >> 30.
      const uint64_t zb = sr_base(D.sr_seed, sr_step) + 0x9E3779B97F4A7C15ULL + (uint64_t)e0;
      const uint32_t zl = (uint32_t)zb, zh = (uint32_t)(zb >> 32);
      uint32_t hv[8];
      if ((zl & 0x3FFFFFFFu) <= 0x3FFFFFF8u) {   // the eight agree from bit 30 up
        const uint32_t yhc = sm_yhc(zh), sh30 = __builtin_amdgcn_alignbit(zh, zl, 30);
#pragma unroll
        for (int k = 0; k < 8; ++k) hv[k] = sm_hi_ys(zl + (uint32_t)k, sh30, yhc);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) hv[k] = sm_hi(zb + (uint64_t)k);
      }
      float xv[8];   // (p * decay) + (g * f) * step; the decay branch is uniform
      if (has_dec) {
#pragma unroll
        for (int k = 0; k < 8; ++k) xv[k] = (p[k] * dec) + (scrub(g[k]) * f[k]) * step;
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) xv[k] = p[k] + (scrub(g[k]) * f[k]) * step;
      }
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if constexpr (std::is_same<T, __half>::value) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          w[k >> 1] |= (uint32_t)sr_fp16(xv[k], (float)(hv[k] >> 8) * (1.0f / 16777216.0f)) << (16 * (k & 1));
      } else {
        uint32_t amax = 0u;
#pragma unroll
        for (int k = 0; k < 8; ++k) amax = max(amax, __float_as_uint(xv[k]) & 0x7FFFFFFFu);
        if (amax < 0x7F7F0000u) {
          // all eight finite and below the largest value that can round up:
          // sr_bf16_hi without its guards.  It rounds up when (hv >> 16) < (b &
          // 0xFFFF), which is when b + (0xFFFF - (hv >> 16)) carries into the high
          // half; the two high halves of a pair then make one word (v_perm).
          uint32_t sv[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) sv[k] = __float_as_uint(xv[k]) + (~hv[k] >> 16);
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = __builtin_amdgcn_perm(sv[2 * j + 1], sv[2 * j], 0x07060302u);
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) w[k >> 1] |= (uint32_t)sr_bf16_hi(xv[k], hv[k]) << (16 * (k & 1));
        }
      }
      if (e0 + 8 <= n) {
        *gp(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(P) + e0)) = u32x4{w[0], w[1], w[2], w[3]};
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (e0 + k < n) gp(reinterpret_cast<uint16_t*>(P))[e0 + k] = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
      }
    } else if constexpr (sizeof(T) == 8) {
      // fp64 parameter (G read as fp32): p.mul_(decay), then addcmul_ / add_ in
      // double, as torch computes them on a float64 tensor with fp32 operands
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double gk = (double)scrub(g[k]);
        double x = p[k];
        if (has_dec) x = pdec(x, dec);
        if (h.channel) x = x + ((double)step * gk) * (double)f[k];
        else x = __builtin_fma((double)ts, gk, x);
        p[k] = x;
      }
      store8<T>(P, e0, n, p);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float gk = scrub(g[k]);
        float x = p[k];
        if (has_dec) x = to_f<T>(from_f<T>(x * dec));
        if (h.channel) x = x + (step * gk) * f[k];
        else x = __builtin_fmaf(ts, gk, x);
        p[k] = x;
      }
      store8<T>(P, e0, n, p);
    }
  };
#pragma unroll
  for (int q = 0; q < kApRuns; ++q)
    if (q == 0 || ea + 2048u * q < n) run8(ea + 2048u * q, gr[q], pr[q]);
}

hipError_t apollo_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

// ------------------------------------------------------------ rocBLAS (fp32 G)

template <int VB>
static void launch_low(int mkt, unsigned nb, const ApDesc& one, const ApDesc* tab, int ntab, const ApHyp& h,
                       hipStream_t st) {
  switch (mkt) {
    case 0: hipLaunchKernelGGL((k_ap_low<VB, 0>), dim3(nb), dim3(256), 0, st, one, tab, ntab, h); break;
    case 1: hipLaunchKernelGGL((k_ap_low<VB, 1>), dim3(nb), dim3(256), 0, st, one, tab, ntab, h); break;
    case 3: hipLaunchKernelGGL((k_ap_low<VB, 3>), dim3(nb), dim3(256), 0, st, one, tab, ntab, h); break;
    default: hipLaunchKernelGGL((k_ap_low<VB, 2>), dim3(nb), dim3(256), 0, st, one, tab, ntab, h); break;
  }
}

static int64_t table_bytes(int n) { return (int64_t)n * (int64_t)(sizeof(ApDesc) + 6 * sizeof(int32_t)); }

// phase 0: the whole step; 1: projection (and the norms of G) only, leaving
// g_low in workspace[0, n_low); 2: scale, scalars and writeback from the update
// the caller wrote to workspace[n_low, 2 n_low) (the factorised / CAME low-rank
// stage of a8_apollo_lowrank_x runs between the two); 3: as 2, reading the row
// sums that stage left in place of u for the matrices where ap_rowsum holds.
static int apollo_run(int phase, int dtype, int stochastic, const a8_apollo_tensor* ts, int n, void* table_dev,
                      int64_t tbytes, double beta_val, double beta1, int has_m, float apollo_eps, float log_floor,
                      int v_bits, int block_size, int m_bits, int m_mode, int m_fp32, int m_block_size, int channel,
                      float apollo_scale, int scale_front, int fira, float fira_margin, float d, float lr_val,
                      float eps2, int scale_parameter, int bias_mode, float weight_decay, int wd_mode,
                      int upload, const a8_step_scalars* dsc, void* stream) {
  if (n <= 0) return 0;
  if (!ts) return set_error(A8_ERR_ARG, "null tensor list");
  if (dtype != A8_F32 && dtype != A8_BF16 && dtype != A8_F16 && dtype != A8_F64)
    return set_error(A8_ERR_DTYPE, "APOLLO supports fp32, bf16, fp16 and fp64 params");
  if (v_bits != 0 && v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 0, 8 or 16");
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  if (v_bits && !(pow2(block_size) && block_size >= 128 && block_size <= 2048))
    return set_error(A8_ERR_BLOCK, "APOLLO V block_size must be a power of two in [128, 2048]");
  if (has_m && !m_fp32 && !(pow2(m_block_size) && m_block_size >= 32 && m_block_size <= 2048))
    return set_error(A8_ERR_BLOCK, "APOLLO m_block_size must be a power of two in [32, 2048]");
  if (n > 1 && (!table_dev || tbytes < table_bytes(n)))
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_apollo_table_bytes(n)");
  if (dtype == A8_F64 && scale_parameter)   // the reference takes an fp32 norm of the fp64 tensor, which torch refuses
    return set_error(A8_ERR_ARG, "scale_parameter is not available for fp64 APOLLO parameters");
  if (stochastic && (dtype == A8_F32 || dtype == A8_F64)) stochastic = 0;
  std::vector<ApDesc> tab((size_t)n);
  std::vector<int32_t> first((size_t)6 * n);
  int64_t nrt = 0, nlt = 0, nwt = 0, nunit = 0, nsc = 0, napp = 0;
  for (int i = 0; i < n; ++i) {
    const a8_apollo_tensor& t = ts[i];
    if (!t.param || !t.grad || !t.proj_t || !t.workspace) return set_error(A8_ERR_ARG, "null pointer");
    if (t.rows <= 0 || t.cols <= 0 || t.rank <= 0) return set_error(A8_ERR_SIZE, "empty APOLLO tensor");
    if (t.rows * t.cols >= ((int64_t)1 << 31)) return set_error(A8_ERR_SIZE, "APOLLO tensor too large");
    if (phase == 0 && (v_bits ? !(t.v_q && t.v_scale && t.v_min_log) : !t.v_fp32))
      return set_error(A8_ERR_ARG, "APOLLO V state missing");
    if (phase == 0 && has_m && (m_fp32 ? !t.m_fp32 : !(t.m_q && t.m_scale)))
      return set_error(A8_ERR_ARG, "APOLLO M state missing");
    if (fira && !t.fira_prev) return set_error(A8_ERR_ARG, "APOLLO Fira needs scaled_grad_norm_prev");
    if (dsc && (!t.proj_state || t.proj_gap <= 0))
      return set_error(A8_ERR_ARG, "APOLLO with step_scalars needs each record's proj_state and proj_gap > 0");
    if (!aligned16(t.param) || !aligned16(t.grad) || !aligned16(t.workspace))
      return set_error(A8_ERR_ALIGN, "APOLLO param, grad and workspace must be 16-byte aligned");
    const int64_t trows = ap_tile(dtype == A8_BF16, t.rows, t.cols, t.rank);
    const ApL L = ap_layout(t.rows, t.cols, t.rank, trows);
    ApDesc& D = tab[(size_t)i];
    D.grad = t.grad; D.param = t.param; D.ws = t.workspace; D.proj_t = t.proj_t;
    D.trows = (int32_t)trows;
    D.v_q = t.v_q; D.v_scale = t.v_scale; D.v_min_log = t.v_min_log; D.v_fp32 = t.v_fp32;
    D.m_q = t.m_q; D.m_scale = t.m_scale; D.m_fp32 = t.m_fp32;
    D.fira_prev = t.fira_prev; D.lr = t.lr;
    D.R = t.rows; D.C = t.cols; D.r = t.rank;
    D.sr_seed = t.sr_seed; D.step = dsc ? 0 : t.step; D.bias_factor = dsc ? 0.0f : t.bias_factor;
    D.first = t.first_step ? 1 : 0; D.has_prev = t.has_fira_prev ? 1 : 0;
    D.pstate = dsc ? t.proj_state : nullptr; D.gap = dsc ? t.proj_gap : 0;
    D.valign = (t.cols % 8) == 0 ? 1 : 0;   // a k_ap_apply unit (8 elements) stays in one row
    D.rtile_begin = (int32_t)nrt; D.ltile_begin = (int32_t)nlt; D.unit_begin = (int32_t)nunit;
    D.sc_begin = (int32_t)nsc; D.app_begin = (int32_t)napp;
    first[(size_t)i] = D.rtile_begin;
    first[(size_t)n + i] = D.ltile_begin;
    first[(size_t)2 * n + i] = D.unit_begin;
    first[(size_t)3 * n + i] = D.sc_begin;
    first[(size_t)4 * n + i] = D.app_begin;
    D.wtile_begin = (int32_t)nwt;
    first[(size_t)5 * n + i] = D.wtile_begin;
    if (trows == kApWide) nwt += L.ntile;
    else if (t.rows >= t.cols) nrt += L.ntile;
    else nlt += L.ntile;
    nunit += L.nunit; nsc += L.nsc; napp += L.napp;
    if (nrt > 0x7FFFFFFF || nlt > 0x7FFFFFFF || nwt > 0x7FFFFFFF || nunit > 0x7FFFFFFF || nsc > 0x7FFFFFFF || napp > 0x7FFFFFFF)
      return set_error(A8_ERR_SIZE, "too many workgroups");
  }
  hipStream_t st = (hipStream_t)stream;
  const ApDesc* dtab = nullptr;
  if (n > 1) {
    if (upload) {
      std::vector<char> blob((size_t)table_bytes(n));
      std::memcpy(blob.data(), tab.data(), sizeof(ApDesc) * (size_t)n);
      std::memcpy(blob.data() + sizeof(ApDesc) * (size_t)n, first.data(), sizeof(int32_t) * 6 * (size_t)n);
      if (upload_table(table_dev, blob.data(), blob.size(), st) != hipSuccess)
        return set_error(A8_ERR_HIP, "table upload failed");
    }
    dtab = reinterpret_cast<const ApDesc*>(table_dev);
  }
  const ApDesc& one = tab[0];
  ApHyp h{};
  h.bv = (float)beta_val; h.w_m = (float)(1.0 - beta1); h.aeps = apollo_eps; h.log_floor = log_floor;
  h.lr_val = lr_val; h.eps2 = eps2; h.wd = weight_decay; h.d = d;
  h.margin = (float)(1.0 + (double)fira_margin); h.sv = (float)sqrt((double)apollo_scale);
  int lbv = 0, lbm = 0;
  while ((1 << lbv) < (v_bits ? block_size : 2048)) ++lbv;
  while ((1 << lbm) < ((has_m && !m_fp32) ? m_block_size : 32)) ++lbm;
  h.lbv = lbv; h.lbm = lbm;
  h.mk = has_m && !m_fp32 ? (m_mode == 0 ? (m_bits == 8 ? 1 : 2) : (m_bits == 8 ? 3 : 4)) : 0;
  h.channel = channel ? 1 : 0; h.front = scale_front ? 1 : 0; h.fira = fira ? 1 : 0;
  h.scale_param = scale_parameter ? 1 : 0; h.bias_mode = bias_mode; h.wd_mode = wd_mode;
  // phase 2 finishes a low-rank stage that wrote u itself, phase 3 one that left
  // the row sums (a8_apollo_x_args.u_rowsums) where ap_rowsum holds
  h.rowsum = (phase == 0 || phase == 3) ? 1 : 0;
  h.dsc = dsc;
  int rc;
  // projection (+ channel norms of G)
  if (phase >= 2) {
    // the projection ran in phase 1
  } else {
    // P^T's split: on the device schedule (capturable steps), or when a record says it changed
    if (dsc) {
      hipLaunchKernelGGL(k_ap_decide, dim3((unsigned)((n + 63) / 64)), dim3(64), 0, st, one, dtab, n, dsc);
      if ((rc = check_launch("k_ap_decide"))) return rc;
      hipLaunchKernelGGL(k_ap_pgen, dim3((unsigned)(n * kPGen)), dim3(256), 0, st, one, dtab, n);
      if ((rc = check_launch("k_ap_pgen"))) return rc;
    }
    for (int i = 0; i < n && !dsc; ++i) {
      if (!ts[i].proj_fresh) continue;
      const ApDesc& D = tab[(size_t)i];
      const ApL L = ap_layout(D.R, D.C, D.r, D.trows);
      const int64_t nb = (L.rp * L.Kp / 8 + 255) / 256;
      hipLaunchKernelGGL(k_ap_split, dim3((unsigned)(nb < 4096 ? nb : 4096)), dim3(256), 0, st, D.proj_t, D.r, L.K,
                         (int)(D.R >= D.C), L.rp, L.Kp, reinterpret_cast<u32x4*>(D.ws + L.psplit));
      if ((rc = check_launch("k_ap_split"))) return rc;
    }
    // g_low = G P^T / P^T G with the channel norms of G: bf16 G as it is, fp32 G in three terms
    const bool g16 = dtype == A8_BF16;
    if (nrt > 0) {
      if (g16) hipLaunchKernelGGL(k_ap_proj_r, dim3((unsigned)nrt), dim3(256), 0, st, one, dtab, n);
      else hipLaunchKernelGGL(k_ap_proj_r32, dim3((unsigned)nrt), dim3(256), 0, st, one, dtab, n);
      if ((rc = check_launch("k_ap_proj_r"))) return rc;
    }
    if (nlt > 0) {
      if (g16) hipLaunchKernelGGL(k_ap_proj_l, dim3((unsigned)nlt), dim3(256), 0, st, one, dtab, n);
      else hipLaunchKernelGGL(k_ap_proj_l32, dim3((unsigned)nlt), dim3(256), 0, st, one, dtab, n);
      if ((rc = check_launch("k_ap_proj_l"))) return rc;
    }
    if (nwt > 0) {
      // cost-balanced XCD ranges over the wide tiles in table order (cost of a
      // tile: its slabs of K plus a few for the prologue and epilogue)
      ApXcd xs{};
      int64_t total = 0;
      for (int i = 0; i < n; ++i)
        if (tab[(size_t)i].trows == kApWide) {
          const ApL L = ap_layout(tab[(size_t)i].R, tab[(size_t)i].C, tab[(size_t)i].r, kApWide);
          total += L.ntile * ((L.K + 31) / 32 + 4);
        }
      int xi = 1;
      int64_t cum = 0, wg = 0;
      for (int i = 0; i < n; ++i) {
        if (tab[(size_t)i].trows != kApWide) continue;
        const ApL L = ap_layout(tab[(size_t)i].R, tab[(size_t)i].C, tab[(size_t)i].r, kApWide);
        const int64_t c = (L.K + 31) / 32 + 4;
        for (int64_t j = 0; j < L.ntile; ++j, ++wg, cum += c)
          while (xi < 8 && cum * 8 >= total * xi) xs.start[xi++] = (int32_t)wg;
      }
      while (xi <= 8) xs.start[xi++] = (int32_t)wg;
      int32_t most = 0;
      for (int k = 0; k < 8; ++k) most = std::max(most, xs.start[k + 1] - xs.start[k]);
      hipLaunchKernelGGL(k_ap_proj_w8, dim3((unsigned)(8 * most)), dim3(512), 0, st, one, dtab, n, xs);
      if ((rc = check_launch("k_ap_proj_w8"))) return rc;
    }
    if (h.scale_param) {   // ||p||^2 of the parameter (fp64 parameters refuse scale_parameter above)
      for (int i = 0; i < n; ++i) {
        const ApDesc& D = tab[(size_t)i];
        const dim3 grid((unsigned)ap_layout(D.R, D.C, D.r, D.trows).ntr);
        if (dtype == A8_BF16) hipLaunchKernelGGL(k_ap_psq<__hip_bfloat16>, grid, dim3(256), 0, st, D);
        else if (dtype == A8_F16) hipLaunchKernelGGL(k_ap_psq<__half>, grid, dim3(256), 0, st, D);
        else hipLaunchKernelGGL(k_ap_psq<float>, grid, dim3(256), 0, st, D);
        if ((rc = check_launch("k_ap_psq"))) return rc;
      }
    }
  }
  if (phase == 1) return 0;
  if (phase == 0) {
    const int mkt = !has_m ? 0 : (m_fp32 ? 3 : (h.mk == 1 ? 1 : 2));
    if (v_bits == 8) launch_low<8>(mkt, (unsigned)nunit, one, dtab, n, h, st);
    else if (v_bits == 16) launch_low<16>(mkt, (unsigned)nunit, one, dtab, n, h, st);
    else launch_low<0>(mkt, (unsigned)nunit, one, dtab, n, h, st);
    if ((rc = check_launch("k_ap_low"))) return rc;
  }
  hipLaunchKernelGGL(k_ap_scale, dim3((unsigned)nsc), dim3(256), 0, st, one, dtab, n, h);
  if ((rc = check_launch("k_ap_scale"))) return rc;
  hipLaunchKernelGGL(k_ap_scalars, dim3((unsigned)n), dim3(256), 0, st, one, dtab, n, h);
  if ((rc = check_launch("k_ap_scalars"))) return rc;
  if (dtype == A8_F32)
    hipLaunchKernelGGL((k_ap_apply<float, false>), dim3((unsigned)napp), dim3(256), 0, st, one, dtab, n, h);
  else if (dtype == A8_F64)
    hipLaunchKernelGGL((k_ap_apply<double, false, float>), dim3((unsigned)napp), dim3(256), 0, st, one, dtab, n, h);
  else if (dtype == A8_F16 && stochastic)
    hipLaunchKernelGGL((k_ap_apply<__half, true, float>), dim3((unsigned)napp), dim3(256), 0, st, one, dtab, n, h);
  else if (dtype == A8_F16)
    hipLaunchKernelGGL((k_ap_apply<__half, false, float>), dim3((unsigned)napp), dim3(256), 0, st, one, dtab, n, h);
  else if (stochastic)
    hipLaunchKernelGGL((k_ap_apply<__hip_bfloat16, true>), dim3((unsigned)napp), dim3(256), 0, st, one, dtab, n, h);
  else
    hipLaunchKernelGGL((k_ap_apply<__hip_bfloat16, false>), dim3((unsigned)napp), dim3(256), 0, st, one, dtab, n, h);
  return check_launch("k_ap_apply");
}

}  // namespace a8

using namespace a8;

extern "C" {

int64_t a8_apollo_workspace_floats(int64_t rows, int64_t cols, int64_t rank, int channel) {
  (void)channel;
  if (rows <= 0 || cols <= 0 || rank <= 0) return 0;
  // either tile height (the dtype is not known here): the larger workspace
  int64_t m = 0;
  for (int g16 = 0; g16 < 2; ++g16) {
    const int64_t a = ap_layout(rows, cols, rank, ap_tile(g16 != 0, rows, cols, rank)).total;
    m = a > m ? a : m;
  }
  return m;
}

int64_t a8_apollo_table_bytes(int ntensors) { return ntensors > 0 ? table_bytes(ntensors) : 0; }

int a8_apollo_step(int dtype, int stochastic, const a8_apollo_tensor* t, int first_step, int proj_fresh,
                   double beta_val, double beta1, int has_m, float apollo_eps, float log_floor, int v_bits,
                   int block_size, int m_bits, int m_mode, int m_fp32, int m_block_size, int channel,
                   float apollo_scale, int scale_front, int fira, float fira_margin, float d, float lr_val,
                   float eps2, int scale_parameter, int bias_mode, float bias_factor, float weight_decay,
                   int wd_mode, uint64_t sr_step, void* stream) {
  if (!t) return set_error(A8_ERR_ARG, "null pointer");
  a8_apollo_tensor one = *t;
  one.first_step = first_step;
  one.proj_fresh = proj_fresh;
  one.step = sr_step;
  one.bias_factor = bias_factor;
  one.proj_state = nullptr;
  return apollo_run(0, dtype, stochastic, &one, 1, nullptr, 0, beta_val, beta1, has_m, apollo_eps, log_floor, v_bits,
                    block_size, m_bits, m_mode, m_fp32, m_block_size, channel, apollo_scale, scale_front, fira,
                    fira_margin, d, lr_val, eps2, scale_parameter, bias_mode, weight_decay, wd_mode, 1, nullptr,
                    stream);
}

int a8_apollo_step_multi(int dtype, int stochastic, const a8_apollo_tensor* ts, int ntensors, void* table_dev,
                         int64_t table_bytes_, double beta_val, double beta1, int has_m, float apollo_eps,
                         float log_floor, int v_bits, int block_size, int m_bits, int m_mode, int m_fp32,
                         int m_block_size, int channel, float apollo_scale, int scale_front, int fira,
                         float fira_margin, float d, float lr_val, float eps2, int scale_parameter, int bias_mode,
                         float weight_decay, int wd_mode, int upload, const void* step_scalars, void* stream) {
  return apollo_run(0, dtype, stochastic, ts, ntensors, table_dev, table_bytes_, beta_val, beta1, has_m, apollo_eps,
                    log_floor, v_bits, block_size, m_bits, m_mode, m_fp32, m_block_size, channel, apollo_scale,
                    scale_front, fira, fira_margin, d, lr_val, eps2, scale_parameter, bias_mode, weight_decay,
                    wd_mode, upload, reinterpret_cast<const a8_step_scalars*>(step_scalars), stream);
}

int a8_apollo_proj_gen(float* proj_t, int64_t rows, int64_t cols, int64_t rank, uint64_t seed, void* stream) {
  if (!proj_t) return set_error(A8_ERR_ARG, "null proj_t");
  if (rows <= 0 || cols <= 0 || rank <= 0) return set_error(A8_ERR_SIZE, "empty projection");
  const int64_t n = rank * (rows >= cols ? cols : rows);
  const int64_t nb = (n + 255) / 256;
  hipLaunchKernelGGL(k_proj_gen, dim3((unsigned)(nb < 8192 ? nb : 8192)), dim3(256), 0, (hipStream_t)stream,
                     proj_t, rows, cols, rank, seed);
  return check_launch("k_proj_gen");
}

int a8_apollo_next_seed(const uint64_t* seeds, uint64_t* out, int64_t n, void* stream) {
  if (n < 0) return set_error(A8_ERR_SIZE, "n < 0");
  if (n == 0) return 0;
  if (!seeds || !out) return set_error(A8_ERR_ARG, "null pointer");
  hipLaunchKernelGGL(k_next_seed, dim3((unsigned)((n + 63) / 64)), dim3(64), 0, (hipStream_t)stream, seeds, out, n);
  return check_launch("k_next_seed");
}

int a8_apollo_step_multi_phase(int phase, int dtype, int stochastic, const a8_apollo_tensor* ts, int ntensors,
                               void* table_dev, int64_t table_bytes_, double beta_val, double beta1, int has_m,
                               float apollo_eps, float log_floor, int v_bits, int block_size, int m_bits, int m_mode,
                               int m_fp32, int m_block_size, int channel, float apollo_scale, int scale_front,
                               int fira, float fira_margin, float d, float lr_val, float eps2, int scale_parameter,
                               int bias_mode, float weight_decay, int wd_mode, int upload, const void* step_scalars,
                               void* stream) {
  if (phase < 1 || phase > 3)
    return set_error(A8_ERR_ARG, "phase must be 1 (projection), 2 or 3 (finish)");
  return apollo_run(phase, dtype, stochastic, ts, ntensors, table_dev, table_bytes_, beta_val, beta1, has_m,
                    apollo_eps, log_floor, v_bits, block_size, m_bits, m_mode, m_fp32, m_block_size, channel,
                    apollo_scale, scale_front, fira, fira_margin, d, lr_val, eps2, scale_parameter, bias_mode,
                    weight_decay, wd_mode, upload, reinterpret_cast<const a8_step_scalars*>(step_scalars), stream);
}

}  // extern "C"
