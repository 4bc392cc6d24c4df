// Factored (Adafactor row/column) optimizer step for MI355X (gfx950).
//
// One group step is a few launches over every tensor of the group:
//   k_fstats   2-D tiles of up to kTRS rows x 1024 columns: row sums and column
//              sums of g^2 (and sum p^2 for the relative step size), written as
//              per-tile partials -- no atomics, so the result is deterministic;
//   k_fcolsum  (tensors of more than kSplit row strips) the column partials
//              summed over groups of kSplit strips, in parallel;
//   k_fblock   one workgroup per AL block of each row/column vector: reduce the
//              partials in a fixed order, EMA the second moment, refit and
//              re-encode the block (columns: inv_col in place);
//   k_frows    one workgroup per tensor: the row mean, inv_row, the step size
//              and the weight-decay factor;
//   k_fupdt    on tiles of 32 rows x 1024 columns (k_fupdate, flat 2048-element units, for
//              the few tensors whose column count rules tiles out): the update
//              u = (x * inv_row) * inv_col with x = g or the momentum EMA, the
//              parameter write and the momentum re-encode.  With RMS clipping
//              or Fira it runs twice: first for sum(u^2) per tile, then (after
//              k_fnorm) to apply;
//   k_fnorm    one workgroup per tensor: ||u||, the Fira limiter and the step.
// CAME (beta3) adds, between k_frows and the update:
//   k_fclip    the RMS clip factor of U = (g * inv_row) * inv_col (after a
//              norm pass over U, only when d > 0);
//   k_came1    the same 2-D tiles as k_fstats: U / clip, the momentum EMA M',
//              and row/column sums of the residual (U - M')^2 + eps_came;
//   k_fcolsum, k_fblock, k_frows again, on the residual sums: the confidence
//              EMA, its AL re-encode and inv_conf_row / inv_conf_col;
// and the update becomes (M' * inv_conf_row) * inv_conf_col (optimizer.py:929-956).
// Numbers follow the reference's PyTorch path (optimizer.py:2198-2252 and
// _fallback_2d_update 920-970): means are sum/count of the fp32 squares,
// inv_row = 1/sqrt(row/r) and inv_col = 1/sqrt(col) with IEEE division and
// square root, and u is formed as (x * inv_row) * inv_col.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

constexpr int kTR = 32;      // minimum rows per statistics tile
constexpr int kTC = 1024;    // columns per statistics tile (256 lanes x 4)
constexpr int kUnit = 2048;  // elements per update workgroup
constexpr int kScal = 8;     // per-tensor scalars in the workspace
constexpr int kMkFp32 = 5;   // HyperF::mk of fp32 momentum (codecs are 1-4)

// Per-tensor workspace layout (offsets in floats).  The partial sums are doubles:
// every statistic (row / column means, sum p^2, ||u||^2) is accumulated in double
// from its first term and rounded to float once, so it is the correctly rounded
// sum in all but vanishingly rare cases, whatever the tiling.  The double regions
// come first and have even sizes, so each starts 8-byte aligned (the workspace
// itself is 256-byte aligned).
struct FWs {
  int64_t rowpart;   // double [nchunk][B*R]       row partial sums
  int64_t colpart;   // double [B][nstrip][C]      column partial sums
  int64_t colsum;    // double [B][nsplit][C]      column sums over groups of kSplit strips
  int64_t p2;        // double [ntile]             partial sum p^2
  int64_t npart;     // double [max(nunit, nutile)] partial sums u^2 (per unit or per update tile)
  int64_t invr;      // [B*R]              new row V, then inv_row
  int64_t invc;      // [B*C]              new column V, then inv_col
  int64_t icr;       // [B*R]              CAME: new row confidence, then its inverse root
  int64_t icc;       // [B*C]              CAME: new column confidence, then its inverse root
  int64_t scal;      // [8]: alpha, step, fira scale, decay, CAME clip factor
  int64_t total;
  int64_t nchunk, nstrip, ntile, nunit;
  int64_t nsplit;    // strip groups of the column reduction (1: k_fblock reads colpart)
  int64_t tr;        // rows per statistics tile
  int64_t nustrip, nutile;   // update tiles: kTR rows x 1024 columns
};

// Tile geometry.  The update passes (k_fupdt) run on tiles of kTR = 32 rows x
// 1024 columns, which stream best for them.  The statistics passes (k_fstats,
// k_came1) take up to kTRS rows per tile: each tile ends with a write of its row
// and column partials, and such writes spread through the read stream cost far
// more bandwidth than their bytes, so fewer, taller tiles write less often.  The
// column partials of tall matrices are reduced in parallel by k_fcolsum, kSplit
// strips per workgroup, before k_fblock.
#ifndef A8_TRS
#define A8_TRS 256
#endif
constexpr int kTRS = A8_TRS;
constexpr int kSplit = 32;

__host__ __device__ inline int64_t fws_tile_rows(int64_t R) {
  const int64_t r = (R + kTR - 1) / kTR * kTR;
  return r < kTRS ? r : kTRS;
}

__host__ __device__ inline FWs fws_layout(int64_t B, int64_t R, int64_t C) {
  FWs w;
  w.nchunk = (C + kTC - 1) / kTC;
  w.tr = fws_tile_rows(R);
  w.nstrip = (R + w.tr - 1) / w.tr;
  w.ntile = B * w.nstrip * w.nchunk;
  w.nustrip = (R + kTR - 1) / kTR;
  w.nutile = B * w.nustrip * w.nchunk;
  w.nunit = (B * R * C + kUnit - 1) / kUnit;
  w.nsplit = (w.nstrip > kSplit) ? (w.nstrip + kSplit - 1) / kSplit : 1;
  w.rowpart = 0;
  w.colpart = w.rowpart + 2 * w.nchunk * B * R;
  w.colsum = w.colpart + 2 * B * w.nstrip * C;
  w.p2 = w.colsum + (w.nsplit > 1 ? 2 * B * w.nsplit * C : 0);
  w.npart = w.p2 + 2 * w.ntile;
  w.invr = w.npart + 2 * (w.nunit > w.nutile ? w.nunit : w.nutile);
  w.invc = w.invr + B * R;
  w.icr = w.invc + B * C;
  w.icc = w.icr + B * R;
  w.scal = w.icc + B * C;
  w.total = w.scal + kScal;
  return w;
}

__device__ __forceinline__ double* ws_dp(float* ws, int64_t off) { return reinterpret_cast<double*>(ws + off); }
__device__ __forceinline__ const double* ws_dp(const float* ws, int64_t off) {
  return reinterpret_cast<const double*>(ws + off);
}

struct DescF {
  void* param;
  const void* grad;
  uint8_t* m_q;
  float* m_scale;
  void* row_q;
  float* row_scale;
  float* row_min_log;
  float* row_var;
  void* col_q;
  float* col_scale;
  float* col_min_log;
  float* col_var;
  void* crow_q;        // CAME confidence state (codes or fp32), as row/col V
  float* crow_scale;
  float* crow_min_log;
  float* crow_var;
  void* ccol_q;
  float* ccol_scale;
  float* ccol_min_log;
  float* ccol_var;
  float* ws;
  const float* lr;
  float* fira_prev;
  float* m;            // fp32 momentum (MK 3), or null
  int64_t B, R, C, numel;
  int64_t tile_begin;  // first statistics tile of this tensor
  int64_t utile_begin; // first update tile
  int64_t unit_begin;
  int64_t fblk_begin;  // first k_fblock workgroup of this tensor
  int64_t cs_begin;    // first k_fcolsum workgroup of this tensor
  int64_t nbr;         // AL blocks of the row vector (the column vector follows)
  uint64_t sr_seed;
  int has_fira_prev;
  int vec4;            // every row starts 16-byte aligned
  int tiled;           // update runs on the statistics tiles (k_fupdt), else flat units
};

struct HyperF {
  float bv;            // V lerp weight
  float eps1;
  float eps2;
  float lr_val;
  float bias_factor;
  float wd;
  float d;
  float margin;        // 1 + fira_margin
  float floor_;
  float w_m;           // momentum lerp weight (1 - beta1)
  float w_c;           // CAME confidence lerp weight (1 - beta3)
  float eps_came;
  int came;
  int bias_mode;
  int scale_param;
  int wd_mode;
  int fira;
  int block_size;      // V block size
  int mk;              // momentum codec (0 none, 1 UF8, 2 UF4, 3 D8, 4 D4)
  int lbm;             // log2(m_block_size); -1: B_M not a power of two in [32, 2048]
  int bm;              // B_M when lbm < 0 (k_fupdate_gen), else 0
  int unit;            // elements per k_fupdate_gen workgroup (a whole number of M blocks)
  uint64_t sr_step;
  const a8_step_scalars* dsc;   // if set: this step's V lerp weight, lr, bias factor and SR step
};

// The per-step fields from the device block of a8_step_advance, when given.
__device__ __forceinline__ void hf_step(HyperF& h) {
  if (!h.dsc) return;
  const a8_step_scalars sc = load_step_scalars(h.dsc);
  h.bv = (float)sc.beta_val;
  h.lr_val = sc.rho;
  h.bias_factor = sc.bias_factor;
  h.sr_step = sc.step;
}

__device__ __forceinline__ const DescF* find_tile(const DescF* tab, int n, int64_t wg) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (tab[mid].tile_begin <= wg) lo = mid; else hi = mid - 1;
  }
  return tab + lo;
}

__device__ __forceinline__ const DescF* find_utile(const DescF* tab, int n, int64_t wg) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (tab[mid].utile_begin <= wg) lo = mid; else hi = mid - 1;
  }
  return tab + lo;
}

__device__ __forceinline__ const DescF* find_unit(const DescF* tab, int n, int64_t wg) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (tab[mid].unit_begin <= wg) lo = mid; else hi = mid - 1;
  }
  return tab + lo;
}

// Workgroup-wide reductions (256 lanes, 4 waves) through 4 LDS slots; every
// lane gets the result.  The cross-wave order is fixed.
__device__ __forceinline__ double wg_sum_d(double x, double* s4) {
  x = grp_sum_d(x, 64);
  const int lane = threadIdx.x;
  __syncthreads();
  if ((lane & 63) == 0) s4[lane >> 6] = x;
  __syncthreads();
  return ((s4[0] + s4[1]) + s4[2]) + s4[3];
}

__device__ __forceinline__ uint32_t nz_key_f(float v) { return __float_as_uint(v) - 1u; }

__device__ __forceinline__ void wg_maxkey(float& mx, uint32_t& key, float* s8) {
  mx = grp_max(mx, 64);
  key = grp_umin(key, 64);
  const int lane = threadIdx.x;
  __syncthreads();
  if ((lane & 63) == 0) {
    s8[lane >> 6] = mx;
    s8[4 + (lane >> 6)] = __uint_as_float(key);
  }
  __syncthreads();
  mx = fmaxf(fmaxf(s8[0], s8[1]), fmaxf(s8[2], s8[3]));
  key = min(min(__float_as_uint(s8[4]), __float_as_uint(s8[5])),
            min(__float_as_uint(s8[6]), __float_as_uint(s8[7])));
}

// Four consecutive row elements starting at column c0 (zero beyond C).
template <typename T, typename V>
__device__ __forceinline__ void load4(const T* base, int64_t rowbase, int64_t c0, int64_t C, bool vec,
                                      V* out) {
  if (vec && c0 + 4 <= C) {
    if constexpr (sizeof(T) == 8) {
      ld4d<V>(reinterpret_cast<const double*>(base) + rowbase + c0, out);
    } else if constexpr (sizeof(T) == 4) {
      const f32x4 a = *gp(reinterpret_cast<const f32x4*>(base + rowbase + c0));
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    } else {
      const u32x2 a = *gp(reinterpret_cast<const u32x2*>(base + rowbase + c0));
      const T* h = reinterpret_cast<const T*>(&a);
#pragma unroll
      for (int k = 0; k < 4; ++k) out[k] = to_f<T>(h[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = (c0 + k < C) ? ld1<T, V>(base, rowbase + c0 + k) : (V)0;
  }
}

// ------------------------------------------------------------ statistics
// Tile layout of the two statistics kernels (k_fstats, k_came1): wave w of the
// workgroup owns columns c_base + 256 w .. + 255 of every row of the tile, a lane
// one 4-column window.  A lane's column sums therefore cover the whole tile in
// four registers (double), written straight to the column partials; the row sums
// are kept per lane for kRB rows at a time and then reduce-scattered across the
// wave (one 6-step butterfly for all kRB rows), the four waves' row partials
// meeting in LDS at the end of the tile.  Every load of a batch of rows is issued
// before its arithmetic: rows beyond the tile and windows beyond C read a valid
// address (the tile's first row, column 0) and count zero.
constexpr int kRB = 4;   // rows per row-sum batch

// Sum of v[0..3] over the 64 lanes of the wave for each k, scattered: on return
// every lane holds the total of v[k] for k = row_of_lane(lane).
__device__ __forceinline__ double reduce_scatter4(const double* v, int wl) {
  const bool b5 = (wl & 32) != 0, b4 = (wl & 16) != 0;
  double a[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const double mine = b5 ? v[k + 2] : v[k];
    const double other = b5 ? v[k] : v[k + 2];
    a[k] = mine + __shfl_xor(other, 32, 64);
  }
  double x = (b4 ? a[1] : a[0]) + __shfl_xor(b4 ? a[0] : a[1], 16, 64);
  x += __shfl_xor(x, 8, 64);
  x += __shfl_xor(x, 4, 64);
  x += __shfl_xor(x, 2, 64);
  x += __shfl_xor(x, 1, 64);
  return x;
}

__device__ __forceinline__ int row_of_lane(int wl) { return ((wl >> 5) & 1) * 2 + ((wl >> 4) & 1); }

// Four consecutive elements at a per-lane 32-bit element offset from a
// workgroup-uniform row pointer.  The offset is scaled to bytes in 32 bits (rows
// of a tensor are far below 4 GiB apart... the offset is below C * sizeof(T)), so
// the address is a scalar base plus a zero-extended vector offset: the saddr form
// of the global load, with no 64-bit address per lane.
// (The row pointer passes through readfirstlane: it is uniform anyway, and the
// opaque step keeps loop strength reduction from turning base + offset back into
// one 64-bit induction pointer per load.)
template <typename T>
__device__ __forceinline__ const char* at_off(const T* row, uint32_t off) {
  const uint64_t v = reinterpret_cast<uint64_t>(row);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo) + (off * (uint32_t)sizeof(T));
}

template <typename T, typename V>
__device__ __forceinline__ void load4o(const T* row, uint32_t off, V* out) {
  if constexpr (sizeof(T) == 8) {
    ld4d<V>(reinterpret_cast<const double*>(at_off(row, off)), out);
  } else if constexpr (sizeof(T) == 4) {
    const f32x4 a = __builtin_nontemporal_load(gp(reinterpret_cast<const f32x4*>(at_off(row, off))));
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  } else {
    const u32x2 a = __builtin_nontemporal_load(gp(reinterpret_cast<const u32x2*>(at_off(row, off))));
    const T* h = reinterpret_cast<const T*>(&a);
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = to_f<T>(h[k]);
  }
}

// Where a statistics workgroup sits: tensor-local tile t, chunk, strip, batch.
struct TilePos {
  int64_t t, ch, s, b, r_lo, r_hi, c_base;
};

// (UPD: an update tile of kTR rows, else a statistics tile of W.tr rows.)
template <bool UPD>
__device__ __forceinline__ TilePos tile_pos(const DescF& D, const FWs& W) {
  TilePos q;
  q.t = (int64_t)blockIdx.x - (UPD ? D.utile_begin : D.tile_begin);
  const int64_t tr = UPD ? kTR : W.tr;
  const uint32_t t32 = (uint32_t)q.t, nch = (uint32_t)W.nchunk, nst = (uint32_t)(UPD ? W.nustrip : W.nstrip);
  const uint32_t bs = t32 / nch;
  q.ch = (int64_t)(t32 - bs * nch);
  q.b = (int64_t)(bs / nst);
  q.s = (int64_t)(bs - (uint32_t)q.b * nst);
  q.r_lo = q.s * tr;
  q.r_hi = (q.r_lo + tr < D.R) ? q.r_lo + tr : D.R;
  q.c_base = q.ch * kTC;
  return q;
}

// The four waves' row partials of the tile (LDS, [4][kTRS]) summed in a fixed
// order into the chunk's row partials.
__device__ __forceinline__ void tile_rows_out(const double* s_row, double* rowpart, int64_t r_lo, int64_t r_hi) {
  __syncthreads();
  for (int i = threadIdx.x; i < r_hi - r_lo; i += 256) {
    const double v = ((s_row[i] + s_row[kTRS + i]) + s_row[2 * kTRS + i]) + s_row[3 * kTRS + i];
    gp(rowpart)[r_lo + i] = v;
  }
}

template <typename T, bool PSQ, bool RAGGED>
__device__ __forceinline__ void fstats_tile(const DescF& D, const TilePos& q, int64_t c0, bool act, double* acc,
                                            double& psq, double* s_row) {
  const T* G = reinterpret_cast<const T*>(D.grad);
  const T* P = reinterpret_cast<const T*>(D.param);
  const int64_t R = D.R, C = D.C;
  const int wl = threadIdx.x & 63;
  const uint32_t cl = act ? (uint32_t)c0 : 0u;
  const bool vec = D.vec4 != 0;
  float g[kRB][4], pv[kRB][PSQ ? 4 : 1];
  bool rv[kRB];
  auto issue = [&](int64_t r0) {
#pragma unroll
    for (int k = 0; k < kRB; ++k) {
      const int64_t r = r0 + k;
      rv[k] = r < q.r_hi;
      const int64_t rowbase = (q.b * R + (rv[k] ? r : q.r_lo)) * C;
      if constexpr (RAGGED) {
        load4<T>(G, rowbase, c0, C, vec, g[k]);
        if constexpr (PSQ) load4<T>(P, rowbase, c0, C, vec, pv[k]);
      } else {
        load4o<T>(G + rowbase, cl, g[k]);
        if constexpr (PSQ) load4o<T>(P + rowbase, cl, pv[k]);
      }
    }
  };
  double rp[kRB];
  auto consume = [&]() {
#pragma unroll
    for (int k = 0; k < kRB; ++k) {
      const bool ok = rv[k] && act;
      double rk = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // the float square g*g is the reference's term (g32.square(), optimizer.py:2213)
        const float gg = ok ? scrub(g[k][e]) : 0.0f;
        const double sq = (double)(gg * gg);
        acc[e] += sq;
        rk += sq;
        if constexpr (PSQ) {
          const double pd = ok ? (double)pv[k][e] : 0.0;
          psq = __builtin_fma(pd, pd, psq);
        }
      }
      rp[k] = rk;
    }
  };
  auto reduce = [&](int64_t r0) {
    const double tot = reduce_scatter4(rp, wl);
    if ((wl & 15) == 0) s_row[(r0 - q.r_lo) + row_of_lane(wl)] = tot;
  };
  // Each batch's row-sum reduction runs while the next batch's loads are in
  // flight (issued just before it).
  issue(q.r_lo);
  __builtin_amdgcn_sched_barrier(0);
  consume();
  int64_t r0 = q.r_lo + kRB;
  for (; r0 < q.r_hi; r0 += kRB) {
    __builtin_amdgcn_sched_barrier(0);
    issue(r0);
    __builtin_amdgcn_sched_barrier(0);
    reduce(r0 - kRB);
    __builtin_amdgcn_sched_barrier(0);
    consume();
  }
  reduce(r0 - kRB);
}

// Row sums and column sums of g^2 (and sum p^2) as per-tile partials, accumulated
// in double (optimizer.py:2211-2219).
template <typename T, bool PSQ>
__global__ __launch_bounds__(256) void k_fstats(const DescF* __restrict__ table, int ntab) {
  __shared__ double s_row[4 * kTRS];
  __shared__ double s4[4];
  const DescF D = *find_tile(table, ntab, (int64_t)blockIdx.x);
  const FWs W = fws_layout(D.B, D.R, D.C);
  const TilePos q = tile_pos<false>(D, W);
  const int lane = threadIdx.x, wl = lane & 63;
  const int wave = __builtin_amdgcn_readfirstlane(lane >> 6);
  const int64_t C = D.C;
  const int64_t c0 = q.c_base + 256 * wave + 4 * wl;
  const bool act = c0 < C;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  double psq = 0.0;
  double* srow = s_row + kTRS * wave;
  if (q.c_base + 256 * wave >= C) {   // the wave's columns lie beyond C
    for (int i = wl; i < kTRS; i += 64) srow[i] = 0.0;
  }
  else if ((C & 3) == 0) fstats_tile<T, PSQ, false>(D, q, c0, act, acc, psq, srow);
  else fstats_tile<T, PSQ, true>(D, q, c0, act, acc, psq, srow);
  float* ws = D.ws;
  double* colp = ws_dp(ws, W.colpart) + (q.b * W.nstrip + q.s) * C;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c0 + e < C) gp(colp)[c0 + e] = acc[e];
  tile_rows_out(s_row, ws_dp(ws, W.rowpart) + q.ch * (D.B * D.R) + q.b * D.R, q.r_lo, q.r_hi);
  if constexpr (PSQ) {
    const double tot = wg_sum_d(psq, s4);
    if (lane == 0) gp(ws_dp(ws, W.p2))[q.t] = tot;
  }
}

// ------------------------------------------------------------ CAME residual statistics
// Old momentum of the element at flat index e (codec mk: 1 UF8, 2 UF4, 3 D8,
// 4 D4; UF4/D4 keep the even element in the high nibble).
// M block of flat index e: a shift for the power-of-two sizes (lbm >= 0), else a
// division by B_M.
__device__ __forceinline__ int64_t m_blk(int64_t e, int lbm, int bm) { return lbm >= 0 ? e >> lbm : e / bm; }

__device__ __forceinline__ float m_old_at(int mk, const uint8_t* mq, const float* msc, int64_t e, int lbm, int bm) {
  const float ms = gp(msc)[m_blk(e, lbm, bm)];
  uint32_t q;
  if (mk == 2 || mk == 4) {
    const uint32_t byte = gp(mq)[e >> 1];
    q = (e & 1) ? (byte & 0x0Fu) : (byte >> 4);
  } else {
    q = gp(mq)[e];
  }
  return m_decode(mk, q, ms);
}

// Old momentum of four consecutive elements e .. e+3 of one row (zero beyond
// `avail`).  The vector form needs e % 4 == 0 (the four share an M block).
template <int MK>
__device__ __forceinline__ void m_old4(int mkr, const uint8_t* mq, const float* msc, int64_t e, int64_t avail,
                                       bool vec, int lbm, int bm, float* out) {
  const int mk = MK == 1 ? 1 : mkr;
  if (vec && avail >= 4) {
    const float ms = gp(msc)[m_blk(e, lbm, bm)];
    if (mk == 2 || mk == 4) {
      const uint32_t w = *gp(reinterpret_cast<const uint16_t*>(mq + (e >> 1)));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t byte = (w >> (8 * (k >> 1))) & 0xFFu;
        out[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
      }
    } else {
      const uint32_t w = *gp(reinterpret_cast<const uint32_t*>(mq + e));
#pragma unroll
      for (int k = 0; k < 4; ++k) out[k] = m_decode(mk, (w >> (8 * k)) & 0xFFu, ms);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = (k < avail) ? m_old_at(mk, mq, msc, e + k, lbm, bm) : 0.0f;
  }
}

// CAME pass 1 over the statistics tiles of one workgroup (layout of fstats_tile):
// U = ((g * inv_row) * inv_col) / clip, M' = lerp(M, U, 1 - beta1),
// res = (U - M')^2 + eps_came, row and column sums of res (optimizer.py:929-937).
template <typename T, int MK, bool RAGGED>
__device__ __forceinline__ void came1_tile(const DescF& D, const FWs& W, const TilePos& q, const HyperF& h,
                                           int64_t c0, bool act, const float* icol, float clip, double* acc,
                                           double* s_row) {
  const T* G = reinterpret_cast<const T*>(D.grad);
  const int64_t R = D.R, C = D.C;
  const int wl = threadIdx.x & 63;
  const uint32_t cl = act ? (uint32_t)c0 : 0u;
  const bool vec = D.vec4 != 0;
  const float* ws = D.ws;
  const int mk = MK == 1 ? 1 : h.mk;
  const bool nib = (mk == 2 || mk == 4);
  const LerpW lw = lerp_weight(h.w_m);
  const float rclip = 1.0f / clip;
  float g[kRB][4], mo[kRB][4], ir[kRB];
  uint32_t qv[kRB];
  float ms[kRB];
  bool rv[kRB];
  auto issue = [&](int64_t r0) {
#pragma unroll
    for (int k = 0; k < kRB; ++k) {
      const int64_t r = r0 + k;
      rv[k] = r < q.r_hi;
      const int64_t rr = rv[k] ? r : q.r_lo;
      const int64_t rowbase = (q.b * R + rr) * C;
      ir[k] = cp(ws)[W.invr + q.b * R + rr];
      if constexpr (RAGGED) {
        load4<T>(G, rowbase, c0, C, vec, g[k]);
        if constexpr (MK == 3) load4<float>(D.m, rowbase, c0, C, vec, mo[k]);
        else m_old4<MK>(h.mk, D.m_q, D.m_scale, rowbase + c0, C - c0, vec, h.lbm, h.bm, mo[k]);
      } else {
        load4o<T>(G + rowbase, cl, g[k]);
        if constexpr (MK == 3) {
          load4o<float>(D.m + rowbase, cl, mo[k]);
        } else {
          const int64_t e = rowbase + cl;
          ms[k] = gp(D.m_scale)[m_blk(e, h.lbm, h.bm)];
          if (MK == 1 || !nib) qv[k] = __builtin_nontemporal_load(gp(reinterpret_cast<const uint32_t*>(D.m_q + e)));
          else qv[k] = __builtin_nontemporal_load(gp(reinterpret_cast<const uint16_t*>(D.m_q + (e >> 1))));
        }
      }
    }
  };
  double rp[kRB];
  auto consume = [&]() {
    float mk4[kRB][4];
#pragma unroll
    for (int k = 0; k < kRB; ++k) {
      if constexpr (!RAGGED && MK != 3) {
        if (MK == 1 || !nib) {
#pragma unroll
          for (int e = 0; e < 4; ++e) mk4[k][e] = m_decode(mk, (qv[k] >> (8 * e)) & 0xFFu, ms[k]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t byte = (qv[k] >> (8 * (e >> 1))) & 0xFFu;
            mk4[k][e] = m_decode(mk, (e & 1) ? (byte & 0x0Fu) : (byte >> 4), ms[k]);
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) mk4[k][e] = mo[k][e];
      }
    }
#pragma unroll
    for (int k = 0; k < kRB; ++k) {
      float xs[4], ug[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) xs[e] = (scrub(g[k][e]) * ir[k]) * icol[e];
      div_by<4>(ug, xs, clip, rclip);
      double rk = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = rv[k] && (RAGGED ? c0 + e < C : act);
        const float mn = lerp_u(mk4[k][e], ug[e], lw);
        const float dd = ug[e] - mn;
        const double res = ok ? (double)(dd * dd + h.eps_came) : 0.0;
        acc[e] += res;
        rk += res;
      }
      rp[k] = rk;
    }
  };
  auto reduce = [&](int64_t r0) {
    const double tot = reduce_scatter4(rp, wl);
    if ((wl & 15) == 0) s_row[(r0 - q.r_lo) + row_of_lane(wl)] = tot;
  };
  // next batch's loads in flight during the row-sum reduction, as in fstats_tile
  issue(q.r_lo);
  __builtin_amdgcn_sched_barrier(0);
  consume();
  int64_t r0 = q.r_lo + kRB;
  for (; r0 < q.r_hi; r0 += kRB) {
    __builtin_amdgcn_sched_barrier(0);
    issue(r0);
    __builtin_amdgcn_sched_barrier(0);
    reduce(r0 - kRB);
    __builtin_amdgcn_sched_barrier(0);
    consume();
  }
  reduce(r0 - kRB);
}

// CAME pass 1: the residual's row and column sums as per-tile partials in the
// g^2 partial arrays (consumed by then).
template <typename T, int MK>
__global__ __launch_bounds__(256) void k_came1(const DescF* __restrict__ table, int ntab, HyperF h) {
  __shared__ double s_row[4 * kTRS];
  const DescF D = *find_tile(table, ntab, (int64_t)blockIdx.x);
  const FWs W = fws_layout(D.B, D.R, D.C);
  const TilePos q = tile_pos<false>(D, W);
  const int lane = threadIdx.x, wl = lane & 63;
  const int wave = __builtin_amdgcn_readfirstlane(lane >> 6);
  const int64_t C = D.C;
  const int64_t c0 = q.c_base + 256 * wave + 4 * wl;
  const bool act = c0 < C;
  float* ws = D.ws;
  const float clip = cp(ws)[W.scal + 4];
  float icol[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) icol[e] = (c0 + e < C) ? gp(ws)[W.invc + q.b * C + c0 + e] : 0.0f;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  double* srow = s_row + kTRS * wave;
  if (q.c_base + 256 * wave >= C) {   // the wave's columns lie beyond C
    for (int i = wl; i < kTRS; i += 64) srow[i] = 0.0;
  }
  else if ((C & 3) == 0) came1_tile<T, MK, false>(D, W, q, h, c0, act, icol, clip, acc, srow);
  else came1_tile<T, MK, true>(D, W, q, h, c0, act, icol, clip, acc, srow);
  double* colp = ws_dp(ws, W.colpart) + (q.b * W.nstrip + q.s) * C;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c0 + e < C) gp(colp)[c0 + e] = acc[e];
  tile_rows_out(s_row, ws_dp(ws, W.rowpart) + q.ch * (D.B * D.R) + q.b * D.R, q.r_lo, q.r_hi);
}

// ------------------------------------------------------------ row/column V EMA
template <int VB>
__device__ __forceinline__ float fv_decode(const void* q, const float* sc, const float* ml, int64_t i,
                                           int64_t bsz) {
  if constexpr (VB == 8) {
    const uint32_t c = gp(reinterpret_cast<const uint8_t*>(q))[i];
    if (!c) return 0.0f;
    const int64_t bi = i / bsz;
    return exp2_exact(((float)(c - 1) * gp(sc)[bi]) / 254.0f + gp(ml)[bi]);
  } else {
    const uint32_t c = gp(reinterpret_cast<const uint16_t*>(q))[i];
    if (!c) return 0.0f;
    const int64_t bi = i / bsz;
    return exp2_exact(((float)(c - 1) * gp(sc)[bi]) / 65534.0f + gp(ml)[bi]);
  }
}

__device__ __forceinline__ const DescF* find_cs(const DescF* tab, int n, int64_t wg) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (tab[mid].cs_begin <= wg) lo = mid; else hi = mid - 1;
  }
  return tab + lo;
}

// First level of the column reduction for tensors of more than kSplit strips:
// one workgroup per (batch, 256 columns, group of kSplit strips) sums its strips'
// partials in strip order (double) into colsum.  k_fblock then adds the nsplit
// group sums in order.
__global__ __launch_bounds__(256) void k_fcolsum(const DescF* __restrict__ table, int ntab) {
  const DescF D = *find_cs(table, ntab, (int64_t)blockIdx.x);
  const FWs W = fws_layout(D.B, D.R, D.C);
  if (W.nsplit <= 1) return;
  const int64_t C = D.C;
  const int64_t ncg = (C + 255) / 256;
  const int64_t w = (int64_t)blockIdx.x - D.cs_begin;
  const int64_t sg = w % W.nsplit;
  const int64_t cg = (w / W.nsplit) % ncg;
  const int64_t b = w / (W.nsplit * ncg);
  const int64_t c = cg * 256 + threadIdx.x;
  if (c >= C) return;
  const int64_t k0 = sg * kSplit;
  const int64_t k1 = (k0 + kSplit < W.nstrip) ? k0 + kSplit : W.nstrip;
  const double* src = ws_dp(D.ws, W.colpart) + b * W.nstrip * C + c;
  double sum = 0.0;
  int64_t k = k0;
  for (; k + 8 <= k1; k += 8) {   // eight loads in flight, summed in order
    double t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = gp(src)[(k + u) * C];
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += t[u];
  }
  for (; k < k1; ++k) sum += gp(src)[k * C];
  gp(ws_dp(D.ws, W.colsum))[(b * W.nsplit + sg) * C + c] = sum;
}

__device__ __forceinline__ const DescF* find_fblk(const DescF* tab, int n, int64_t wg) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (tab[mid].fblk_begin <= wg) lo = mid; else hi = mid - 1;
  }
  return tab + lo;
}

// Row/column second moment (CONF = false) or CAME confidence (CONF = true), one
// workgroup per AL block of the flattened row or column vector of a tensor:
// reduce the statistics tiles' partials in a fixed order (double), mean (g^2:
// sum/count + eps1; residual: sum/count), EMA with the decoded state (lerp
// weight 1 - beta2 / step^decay, or 1 - beta3), refit and re-encode the block
// (optimizer.py:2204-2238, 941-948).  The new values go to the workspace vector;
// on the column side they are replaced by inv_col = 1/sqrt(v) (optimizer.py:818-821,
// 951-953).  VB is the state's codec (8 / 16 bits, 0 = fp32 state, blocks of the
// same size only partition the work).
template <int VB, bool CONF>
__global__ __launch_bounds__(256) void k_fblock(const DescF* __restrict__ table, int ntab, HyperF h) {
  hf_step(h);
  __shared__ float sf[8];
  const DescF D = *find_fblk(table, ntab, (int64_t)blockIdx.x);
  const FWs W = fws_layout(D.B, D.R, D.C);
  const int64_t lb = (int64_t)blockIdx.x - D.fblk_begin;
  const bool is_row = lb < D.nbr;
  const int64_t bi = is_row ? lb : lb - D.nbr;
  const int lane = threadIdx.x;
  const int64_t B = D.B, R = D.R, C = D.C;
  const int64_t n = is_row ? B * R : B * C;
  float* ws = D.ws;
  float* vec;
  void* q;
  float *sc, *ml, *fst;
  if constexpr (CONF) {
    vec = ws + (is_row ? W.icr : W.icc);
    q = is_row ? D.crow_q : D.ccol_q;
    sc = is_row ? D.crow_scale : D.ccol_scale;
    ml = is_row ? D.crow_min_log : D.ccol_min_log;
    fst = is_row ? D.crow_var : D.ccol_var;
  } else {
    vec = ws + (is_row ? W.invr : W.invc);
    q = is_row ? D.row_q : D.col_q;
    sc = is_row ? D.row_scale : D.col_scale;
    ml = is_row ? D.row_min_log : D.col_min_log;
    fst = is_row ? D.row_var : D.col_var;
  }
  const float cnt = is_row ? (float)C : (float)R;
  const int64_t bsz = h.block_size;
  const float w = CONF ? h.w_c : h.bv;
  const int64_t i0 = bi * bsz;
  const int64_t i1 = (i0 + bsz < n) ? i0 + bsz : n;

  // 1. means and EMA (each lane keeps its own entries for step 2)
  float mx = 0.0f;
  uint32_t key = 0xFFFFFFFFu;
  for (int64_t i = i0 + lane; i < i1; i += 256) {
    double sum = 0.0;
    if (is_row) {
      for (int64_t k = 0; k < W.nchunk; ++k) sum += gp(ws_dp(ws, W.rowpart))[k * n + i];
    } else {
      // the column's strip partials, or k_fcolsum's sums of kSplit strips each
      const int64_t b = i / C, c = i - b * C;
      const int64_t np = W.nsplit > 1 ? W.nsplit : W.nstrip;
      const double* cp0 = ws_dp(ws, W.nsplit > 1 ? W.colsum : W.colpart) + b * np * C + c;
      int64_t k = 0;
      for (; k + 8 <= np; k += 8) {   // eight loads in flight, summed in order
        double t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = gp(cp0)[(k + u) * C];
#pragma unroll
        for (int u = 0; u < 8; ++u) sum += t[u];
      }
      for (; k < np; ++k) sum += gp(cp0)[k * C];
    }
    float mean = (float)sum / cnt;
    if constexpr (!CONF) mean = mean + h.eps1;
    float old;
    if constexpr (VB == 0) old = gp(fst)[i];
    else old = fv_decode<VB>(q, sc, ml, i, bsz);
    const float nv = lerp_ref(old, mean, w);
    gp(vec)[i] = nv;
    if constexpr (VB == 0) {
      gp(fst)[i] = nv;
      if (!is_row) gp(vec)[i] = 1.0f / sqrtf(nv);
    }
    mx = fmaxf(mx, nv);
    key = min(key, nz_key_f(nv));
  }

  // 2. refit and re-encode the block (zero padding beyond n -> code 0)
  if constexpr (VB != 0) {
    constexpr int LM2 = VB == 8 ? 254 : 65534;
    wg_maxkey(mx, key, sf);
    const float mnz = (key == 0xFFFFFFFFu) ? __builtin_inff() : __uint_as_float(key + 1u);
    const ALFit f = al_refit(mx, mnz, h.floor_, (float)LM2);
    for (int64_t k = lane; k < bsz; k += 256) {
      const int64_t i = i0 + k;
      const float v = i < n ? gp(vec)[i] : 0.0f;
      const uint32_t code = al_finish<LM2>(v, al_round_exact<LM2>(v, f));
      if constexpr (VB == 8) gp(reinterpret_cast<uint8_t*>(q))[i] = (uint8_t)code;
      else gp(reinterpret_cast<uint16_t*>(q))[i] = (uint16_t)code;
      if (!is_row && i < n) gp(vec)[i] = 1.0f / sqrtf(v);
    }
    if (lane == 0) { gp(sc)[bi] = f.s; gp(ml)[bi] = f.lmin; }
  }
}

// One workgroup per tensor: r = max(mean_r(row), eps1) per batch and
// inv_row = 1/sqrt(row / r) (optimizer.py:2221, 818-821; the confidence's r_c,
// 951-952), then (CONF = false) the step size and weight-decay factor
// (optimizer.py:832-856, 2020-2039).
template <bool CONF>
__global__ __launch_bounds__(256) void k_frows(const DescF* __restrict__ table, HyperF h) {
  hf_step(h);
  __shared__ double sd[4];
  const DescF D = table[blockIdx.x];
  const FWs W = fws_layout(D.B, D.R, D.C);
  const int lane = threadIdx.x;
  const int64_t B = D.B, R = D.R;
  float* ws = D.ws;
  float* vec = ws + (CONF ? W.icr : W.invr);
  for (int64_t b = 0; b < B; ++b) {
    float* v = vec + b * R;
    double s = 0.0;
    int64_t r = lane;
    for (; r + 7 * 256 < R; r += 8 * 256) {   // eight loads in flight, summed in order
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = gp(v)[r + 256 * u];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += (double)t[u];
    }
    for (; r < R; r += 256) s += (double)gp(v)[r];
    s = wg_sum_d(s, sd);
    const float rmv = fmaxf((float)s / (float)R, h.eps1);
    r = lane;
    for (; r + 3 * 256 < R; r += 4 * 256) {
      float t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = gp(v)[r + 256 * u];
#pragma unroll
      for (int u = 0; u < 4; ++u) gp(v)[r + 256 * u] = 1.0f / sqrtf(t[u] / rmv);
    }
    for (; r < R; r += 256) gp(v)[r] = 1.0f / sqrtf(gp(v)[r] / rmv);
  }
  if constexpr (!CONF) {
    const float rho = D.lr ? *gp(D.lr) : h.lr_val;
    float alpha = rho;
    if (h.scale_param) {
      double s = 0.0;
      for (int64_t k = lane; k < W.ntile; k += 256) s += gp(ws_dp(ws, W.p2))[k];
      s = wg_sum_d(s, sd);
      const float nrm = sqrtf((float)s);
      const float rms = nrm / (float)sqrt((double)D.numel);
      alpha = fmaxf(rms, h.eps2) * rho;
    }
    if (h.bias_mode == 1) alpha = alpha * h.bias_factor;
    else if (h.bias_mode == 2) alpha = alpha / h.bias_factor;
    if (lane == 0) {
      float* sl = ws + W.scal;
      gp(sl)[0] = alpha;
      gp(sl)[1] = alpha;
      gp(sl)[2] = 1.0f;
      float dec = 1.0f;
      if (h.wd_mode == 1) dec = 1.0f - alpha * h.wd;
      else if (h.wd_mode == 2) dec = 1.0f - rho * h.wd;
      gp(sl)[3] = dec;
      gp(sl)[4] = 1.0f;   // CAME clip factor unless k_fclip sets it
    }
  }
}

// ------------------------------------------------------------ update
// MODE 0: write with step = alpha; 1: sum(u^2) per unit; 2: write with the
// step and Fira scale of k_fnorm.  MK: 0 no momentum, 1 UF8, 2 other codecs, 3 fp32 momentum.
// CM (CAME): the momentum EMA runs on U = ((g * inv_row) * inv_col) / clip and
// the update is (M' * inv_conf_row) * inv_conf_col (optimizer.py:929-956).
template <typename T, int MODE, bool SR, int MK, bool CM>
__global__ __launch_bounds__(256) void k_fupdate(const DescF* __restrict__ table, int ntab, HyperF h) {
  if constexpr (SR) hf_step(h);
  static_assert(!CM || MK != 0, "CAME needs momentum");
  __shared__ float s4[8];
  __shared__ double s4d[4];
  constexpr bool kHasM = MK != 0;
  const DescF D = *find_unit(table, ntab, (int64_t)blockIdx.x);
  if (D.tiled) return;   // updated by k_fupdt
  const FWs W = fws_layout(D.B, D.R, D.C);
  const int64_t wl = (int64_t)blockIdx.x - D.unit_begin;
  const int lane = threadIdx.x;
  const int64_t n = D.numel;
  const int64_t e0 = wl * kUnit + (int64_t)lane * 8;
  const int64_t rem = n - e0;
  const int cnt = rem <= 0 ? 0 : (rem >= 8 ? 8 : (int)rem);
  const int64_t R = D.R, C = D.C;
  const float* ws = D.ws;
  const float* invr = ws + W.invr;
  const float* invc = ws + W.invc;
  const float* icr = ws + W.icr;
  const float* icc = ws + W.icc;
  const float* sl = ws + W.scal;
  const int lbm = h.lbm;
  const int BM = 1 << lbm;
  const int ML = BM >> 3;
  const int64_t mb = e0 >> lbm;
  const int mk = (MK == 1) ? 1 : h.mk;

  float g[8], mn[8], u[8], mo[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) { g[k] = 0.0f; mn[k] = 0.0f; u[k] = 0.0f; mo[k] = 0.0f; }
  double sq = 0.0;   // sum u^2 (MODE 1), accumulated in double
  uint32_t amaxb = 0u;
  if (cnt > 0) {
    load8<T>(reinterpret_cast<const T*>(D.grad), e0, n, g);
#pragma unroll
    for (int k = 0; k < 8; ++k) g[k] = scrub(g[k]);
    if constexpr (MK == 3) {
      load8<float>(D.m, e0, n, mo);
    } else if constexpr (kHasM) {
      const float ms = gp(D.m_scale)[mb];
      if (MK == 1) {
        const u32x2 qv = *gp(reinterpret_cast<const u32x2*>(D.m_q + e0));
        const float s128 = ms / 128.0f, b128 = -128.0f * s128;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          mo[k] = __builtin_fmaf((float)(((k < 4 ? qv.x : qv.y) >> (8 * (k & 3))) & 0xFFu), s128, b128);
      } else if (mk == 2 || mk == 4) {
        const uint32_t qw = *gp(reinterpret_cast<const uint32_t*>(D.m_q + (e0 >> 1)));
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t byte = (qw >> (8 * (k >> 1))) & 0xFFu;
          mo[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
        }
      } else {
        const u32x2 qv = *gp(reinterpret_cast<const u32x2*>(D.m_q + e0));
#pragma unroll
        for (int k = 0; k < 8; ++k) mo[k] = m_decode(mk, ((k < 4 ? qv.x : qv.y) >> (8 * (k & 3))) & 0xFFu, ms);
      }
    }
    if constexpr (kHasM && !CM) {
#pragma unroll
      for (int k = 0; k < 8; ++k) mn[k] = (k < cnt) ? lerp_ref(mo[k], g[k], h.w_m) : 0.0f;
    }
    const float clip = CM ? gp(sl)[4] : 1.0f;
    // element (row, column): row = e / C, column index b*C + c with b = row / R
    int64_t row = e0 / C;
    int64_t c = e0 - row * C;
    int64_t b = row / R;
    int64_t rr = row - b * R;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k < cnt) {
        if constexpr (CM) {
          const float ug = ((g[k] * gp(invr)[row]) * gp(invc)[b * C + c]) / clip;
          mn[k] = lerp_ref(mo[k], ug, h.w_m);
          u[k] = (mn[k] * gp(icr)[row]) * gp(icc)[b * C + c];
        } else {
          const float x = kHasM ? mn[k] : g[k];
          u[k] = (x * gp(invr)[row]) * gp(invc)[b * C + c];
        }
        if (MODE == 1) sq = __builtin_fma((double)u[k], (double)u[k], sq);
      }
      if (++c == C) {
        c = 0;
        ++row;
        if (++rr == R) { rr = 0; ++b; }
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) amaxb = max(amaxb, __float_as_uint(mn[k]) & 0x7FFFFFFFu);

    if constexpr (MODE != 1) {
      const float step = (MODE == 0) ? gp(sl)[0] : gp(sl)[1];
      const float fs = (MODE == 2) ? gp(sl)[2] : 1.0f;
      const float dec = gp(sl)[3];
      const bool has_dec = h.wd_mode != 0;
      if (MODE == 2) {
#pragma unroll
        for (int k = 0; k < 8; ++k) u[k] = u[k] * fs;
      }
      T* P = reinterpret_cast<T*>(D.param);
      if constexpr (SR) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (k < cnt) {
            const float pv = ld1<T>(P, e0 + k);
            const T r = sr_round<T>((has_dec ? pv * dec : pv) - step * u[k], D.sr_seed, h.sr_step,
                                    (uint64_t)(e0 + k));
            uint16_t bits;
            __builtin_memcpy(&bits, &r, 2);
            gp(reinterpret_cast<uint16_t*>(P))[e0 + k] = bits;
          }
        }
      } else {
        pval_t<T> p[8];
        load8<T>(P, e0, n, p);
        if (has_dec) {
#pragma unroll
          for (int k = 0; k < 8; ++k) p[k] = pdec(p[k], dec);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = pupd(step, u[k], p[k]);
        store8<T>(P, e0, n, p);
      }
    }
  }

  if constexpr (MODE == 1) {
    const double tot = wg_sum_d(sq, s4d);
    if (lane == 0) gp(ws_dp(const_cast<float*>(ws), W.npart))[wl] = tot;
  }

  if constexpr (MODE != 1 && MK == 3) {
    if (cnt > 0) store8<float>(D.m, e0, n, mn);
  }
  // momentum re-encode: absmax over B_M elements = ML lanes
  if constexpr (MODE != 1 && kHasM && MK != 3) {
    const int wave = lane >> 6;
    float bam = grp_max(__uint_as_float(amaxb), ML < 64 ? ML : 64);
    if (ML > 64) {
      __syncthreads();
      if ((lane & 63) == 0) s4[wave] = bam;
      __syncthreads();
      const int w0 = (lane >> (lbm - 3)) * (ML >> 6);
      bam = s4[w0];
      for (int w = 1; w < (ML >> 6); ++w) bam = fmaxf(bam, s4[w0 + w]);
    }
    if (cnt > 0) {
      const float am = fmaxf(bam, 1e-12f);
      const float ram = fast_rcp(am);
      if (MK == 1) {
        const float kam = 128.0f * ram;
        float r[8];
        bool bad[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = uf_round_fast<128>(mn[k], kam, bad[k]);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (bad[k]) r[k] = uf_round_exact<128>(mn[k], am);
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = uf_clamp<128>(r[k]);
        *gp(reinterpret_cast<u32x2*>(D.m_q + e0)) = u32x2{pack4(r[0], r[1], r[2], r[3]), pack4(r[4], r[5], r[6], r[7])};
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
}

// k_fupdate for coded momentum whose block size the unit layout cannot take
// (B_M a multiple of 4 in [32, 2^30], not a power of two up to 2048).  One
// workgroup covers h.unit = B_M * ceil(2048 / B_M) elements, a whole number of M
// blocks and at least kUnit, so a tensor takes no more workgroups than its
// W.nunit norm-partial slots; its last workgroup zeroes the slots it does not
// use.  Lanes take quads (a quad never straddles an M block, B_M % 4 == 0); each
// block's absmax meets in LDS (an exact max).  Pass 1 forms M' and u and writes
// the parameter (MODE 1: the partial sum of u^2); pass 2, after the absmaxes,
// forms M' again from the same inputs and writes the codes; the scales follow
// once every lane has read the old ones.  Element for element the arithmetic is
// k_fupdate's.  MK: 0 no momentum (the CAME clip pass), 2 any codec (h.mk).
constexpr int kFGenMaxMB = 64;

template <typename T, int MODE, bool SR, int MK, bool CM>
__global__ __launch_bounds__(256) void k_fupdate_gen(const DescF* __restrict__ table, int ntab, HyperF h) {
  if constexpr (SR) hf_step(h);
  static_assert(MK == 0 || MK == 2, "codes through m_decode / m_encode");
  static_assert(!CM || MK != 0, "CAME needs momentum");
  __shared__ uint32_t s_mab[kFGenMaxMB];
  __shared__ double s4d[4];
  const DescF D = *find_unit(table, ntab, (int64_t)blockIdx.x);
  if (D.tiled) return;
  const FWs W = fws_layout(D.B, D.R, D.C);
  const int lane = threadIdx.x;
  const int BM = h.bm, U = h.unit, mpu = U / BM;
  const int64_t wl = (int64_t)blockIdx.x - D.unit_begin;
  const int64_t n = D.numel;
  const int64_t base = wl * U;
  const int64_t mb0 = base / BM, nmb = (n + BM - 1) / BM;
  const int64_t R = D.R, C = D.C;
  float* ws = D.ws;
  const float* invr = ws + W.invr;
  const float* invc = ws + W.invc;
  const float* icr = ws + W.icr;
  const float* icc = ws + W.icc;
  const float* sl = ws + W.scal;
  const T* G = reinterpret_cast<const T*>(D.grad);
  T* P = reinterpret_cast<T*>(D.param);
  const int mk = h.mk;
  const bool nib = mk == 2 || mk == 4;
  const float clip = CM ? gp(sl)[4] : 1.0f;
  if constexpr (MK != 0 && MODE != 1) {
    for (int i = lane; i < mpu; i += 256) s_mab[i] = 0u;
    __syncthreads();
  }

  // M' and u of the quad at unit offset 4q (zero past the tensor)
  auto quad = [&](int q, float* g, float* mn, float* u, int& cnt, int& mb, bool& m_ok) {
    const int64_t i0 = base + 4 * q;
    cnt = i0 >= n ? 0 : (n - i0 >= 4 ? 4 : (int)(n - i0));
    load4n<T>(G, i0, n, g);
#pragma unroll
    for (int k = 0; k < 4; ++k) g[k] = scrub(g[k]);
    mb = (4 * q) / BM;
    m_ok = MK != 0 && mb0 + mb < nmb;   // codes are padded to whole blocks
    float mo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (m_ok) {
      const float ms = gp(D.m_scale)[mb0 + mb];
      if (nib) {
        const uint32_t w = *gp(reinterpret_cast<const uint16_t*>(D.m_q + (i0 >> 1)));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t byte = (w >> (8 * (k >> 1))) & 0xFFu;
          mo[k] = m_decode(mk, (k & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
        }
      } else {
        const uint32_t w = *gp(reinterpret_cast<const uint32_t*>(D.m_q + i0));
#pragma unroll
        for (int k = 0; k < 4; ++k) mo[k] = m_decode(mk, (w >> (8 * k)) & 0xFFu, ms);
      }
    }
    int64_t row = i0 / C;
    int64_t c = i0 - row * C;
    int64_t b = row / R;
    int64_t rr = row - b * R;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      mn[k] = 0.0f;
      u[k] = 0.0f;
      if (k < cnt) {
        if constexpr (CM) {
          const float ug = ((g[k] * gp(invr)[row]) * gp(invc)[b * C + c]) / clip;
          mn[k] = lerp_ref(mo[k], ug, h.w_m);
          u[k] = (mn[k] * gp(icr)[row]) * gp(icc)[b * C + c];
        } else {
          if constexpr (MK != 0) mn[k] = lerp_ref(mo[k], g[k], h.w_m);
          const float x = MK != 0 ? mn[k] : g[k];
          u[k] = (x * gp(invr)[row]) * gp(invc)[b * C + c];
        }
      }
      if (++c == C) {
        c = 0;
        ++row;
        if (++rr == R) { rr = 0; ++b; }
      }
    }
  };

  float step = 0.0f, fs = 1.0f, dec = 1.0f;
  if constexpr (MODE != 1) {
    step = (MODE == 0) ? gp(sl)[0] : gp(sl)[1];
    fs = (MODE == 2) ? gp(sl)[2] : 1.0f;
    dec = gp(sl)[3];
  }
  const bool has_dec = h.wd_mode != 0;

  // ---- pass 1
  double sq = 0.0;
  for (int q = lane; q < (U >> 2); q += 256) {
    float g[4], mn[4], u[4];
    int cnt, mb;
    bool m_ok;
    quad(q, g, mn, u, cnt, mb, m_ok);
    const int64_t i0 = base + 4 * q;
    if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < cnt) sq = __builtin_fma((double)u[k], (double)u[k], sq);
    } else {
      if (MODE == 2) {
#pragma unroll
        for (int k = 0; k < 4; ++k) u[k] = u[k] * fs;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (k >= cnt) continue;
        if constexpr (SR) {
          const float pv = ld1<T>(P, i0 + k);
          const T r = sr_round<T>((has_dec ? pv * dec : pv) - step * u[k], D.sr_seed, h.sr_step,
                                  (uint64_t)(i0 + k));
          uint16_t bits;
          __builtin_memcpy(&bits, &r, 2);
          gp(reinterpret_cast<uint16_t*>(P))[i0 + k] = bits;
        } else {
          const pval_t<T> pv = ld1<T, pval_t<T>>(P, i0 + k);
          st1<T>(P, i0 + k, pupd(step, u[k], has_dec ? pdec(pv, dec) : pv));
        }
      }
      if constexpr (MK != 0) {
        uint32_t ab = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) ab = max(ab, __float_as_uint(mn[k]) & 0x7FFFFFFFu);
        if (m_ok) atomicMax(&s_mab[mb], ab);
      }
    }
  }
  if constexpr (MODE == 1) {
    const double tot = wg_sum_d(sq, s4d);
    const int64_t nu = (n + U - 1) / U;
    if (lane == 0) gp(ws_dp(ws, W.npart))[wl] = tot;
    if (wl == nu - 1)
      for (int64_t k = nu + lane; k < W.nunit; k += 256) gp(ws_dp(ws, W.npart))[k] = 0.0;
    return;
  }
  if constexpr (MK != 0) {
    __syncthreads();
    // ---- pass 2: codes
    for (int q = lane; q < (U >> 2); q += 256) {
      float g[4], mn[4], u[4];
      int cnt, mb;
      bool m_ok;
      quad(q, g, mn, u, cnt, mb, m_ok);
      if (!m_ok) continue;
      const int64_t i0 = base + 4 * q;
      const float am = fmaxf(__uint_as_float(s_mab[mb]), 1e-12f);
      const float ram = fast_rcp(am);
      if (nib) {
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
    __syncthreads();   // every lane has read the old scales
    for (int i = lane; i < mpu; i += 256)
      if (mb0 + i < nmb) gp(D.m_scale)[mb0 + i] = fmaxf(__uint_as_float(s_mab[i]), 1e-12f);
  }
}

// Tiled form of k_fupdate for tensors whose columns allow it (C % 4 == 0 and,
// with momentum, B_M <= 256 dividing C): the statistics tiles (tr rows x 1024
// columns), each wave walking rows, lanes holding 4 consecutive columns of each
// 256-column chunk (1 KB-contiguous accesses).  The tile's inv_col (and CAME
// inv_conf_col) are staged in LDS once, a row's inv_row arrives through a scalar
// load, and an M block is B_M/4 lanes of one chunk of one row.  Same arithmetic
// and operation order as k_fupdate; MODE 1 writes one partial per tile.
// Pins four values in VGPRs at this point, so the arithmetic that forms them (and
// the waits for its loads) stays ahead of a following lane-conditional store
// instead of being sunk into it; a load left unconsumed on the store-skipping path
// would make the next row's loads wait for every outstanding store.
template <typename V>
__device__ __forceinline__ void keep4(const V* v) {
  asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
}

template <typename T, int MODE, bool SR, int MK, bool CM>
__global__ __launch_bounds__(256) void k_fupdt(const DescF* __restrict__ table, int ntab, HyperF h) {
  if constexpr (SR) hf_step(h);
  static_assert(!CM || MK != 0, "CAME needs momentum");
  __shared__ float s_ic[2 * kTC];
  __shared__ double s4d[4];
  constexpr bool kHasM = MK != 0;
  const DescF D = *find_utile(table, ntab, (int64_t)blockIdx.x);
  if (!D.tiled) return;   // updated by k_fupdate
  const FWs W = fws_layout(D.B, D.R, D.C);
  const TilePos q = tile_pos<true>(D, W);
  const int64_t R = D.R, C = D.C, b = q.b, c_base = q.c_base;
  const int lane = threadIdx.x, wl = lane & 63;
  const int wave = __builtin_amdgcn_readfirstlane(lane >> 6);
  float* ws = D.ws;
  for (int k = lane; k < kTC; k += 256) {
    const int64_t c = c_base + k;
    s_ic[k] = c < C ? gp(ws)[W.invc + b * C + c] : 0.0f;
    if constexpr (CM) s_ic[kTC + k] = c < C ? gp(ws)[W.icc + b * C + c] : 0.0f;
  }
  __syncthreads();
  const float* sl = ws + W.scal;
  const int lbm = h.lbm;
  const int G = (1 << lbm) >> 2;          // lanes per M block
  const int mk = (MK == 1) ? 1 : h.mk;
  const float clip = CM ? cp(sl)[4] : 1.0f;
  const float rclip = 1.0f / clip;
  const LerpW lw = lerp_weight(h.w_m);
  float step = 0.0f, fs = 1.0f, dec = 1.0f;
  if constexpr (MODE != 1) {
    step = (MODE == 0) ? cp(sl)[0] : cp(sl)[1];
    fs = (MODE == 2) ? cp(sl)[2] : 1.0f;
    dec = cp(sl)[3];
  }
  const bool has_dec = h.wd_mode != 0;
  const T* G0 = reinterpret_cast<const T*>(D.grad);
  T* P0 = reinterpret_cast<T*>(D.param);
  // A lane's four 4-column windows.  C % 4 == 0, so a window holds all four
  // columns or none; one beyond C is pointed at the tile's first window (a valid
  // address), computed on like the others and never stored.  Loads and their
  // arithmetic are unconditional, so nothing is left in flight across rows.
  uint32_t cl[4];
  bool act[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c0 = c_base + 256 * j + 4 * wl;
    act[j] = c0 < C;
    cl[j] = act[j] ? (uint32_t)c0 : (uint32_t)c_base;
  }
  // Rows r, r + 4, r + 8 and r + 12 in one pass for the plain update (the loads
  // of all four in flight together: 2.40 -> 2.33 ms at C2 against two rows); one
  // row per pass with momentum (two rows measured slower there: 172 registers)
  // and in the read-only norm pass, where registers are better spent on
  // occupancy.  A row beyond the tile reads the first one again and stores nothing.
  constexpr int NRW = (kHasM || MODE == 1) ? 1 : 4;
  double sq = 0.0;   // sum u^2 (MODE 1), accumulated in double
  for (int64_t r0 = q.r_lo + wave; r0 < q.r_hi; r0 += 4 * NRW) {
    int64_t rowb[NRW];
    bool rv[NRW];
    float irw[NRW], icrw[NRW];
    float gj[NRW][4][4], msj[NRW][4];
    pval_t<T> pj[NRW][4][4];   // double for fp64 parameters
    float mfj[NRW][MK == 3 ? 4 : 1][4];
    uint32_t qj[NRW][4];
#pragma unroll
    for (int rr = 0; rr < NRW; ++rr) {
      rv[rr] = r0 + 4 * rr < q.r_hi;
      const int64_t r = rv[rr] ? r0 + 4 * rr : r0;
      rowb[rr] = (b * R + r) * C;
      irw[rr] = cp(ws)[W.invr + b * R + r];
      icrw[rr] = CM ? cp(ws)[W.icr + b * R + r] : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t e = rowb[rr] + cl[j];
        load4o<T>(G0 + rowb[rr], cl[j], gj[rr][j]);
        if constexpr (MK == 3) {
          load4o<float>(D.m + rowb[rr], cl[j], mfj[rr][j]);
        } else if constexpr (kHasM) {
          msj[rr][j] = gp(D.m_scale)[e >> lbm];
          if (MK == 1 || !(mk == 2 || mk == 4)) qj[rr][j] = *gp(reinterpret_cast<const uint32_t*>(D.m_q + e));
          else qj[rr][j] = *gp(reinterpret_cast<const uint16_t*>(D.m_q + (e >> 1)));
        }
        if constexpr (MODE != 1 && !SR) load4o<T>(P0 + rowb[rr], cl[j], pj[rr][j]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load of the pass is issued before its arithmetic
#pragma unroll
    for (int rr = 0; rr < NRW; ++rr)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q0 = 256 * j + 4 * wl;
      const int64_t e = rowb[rr] + cl[j];
      const float ir = irw[rr], icrr = icrw[rr];
      const bool st = rv[rr] && act[j];   // this window of this row is stored
      float mo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      float mn[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4];
      pval_t<T>* pv = pj[rr][j];
      if constexpr (MK == 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) mo[i] = mfj[rr][j][i];
      } else if constexpr (kHasM) {
        const float ms = msj[rr][j];
        const uint32_t qv = qj[rr][j];
        if (MK == 1) {
          const float s128 = ms / 128.0f, b128 = -128.0f * s128;
#pragma unroll
          for (int i = 0; i < 4; ++i) mo[i] = __builtin_fmaf((float)((qv >> (8 * i)) & 0xFFu), s128, b128);
        } else if (mk == 2 || mk == 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t byte = (qv >> (8 * (i >> 1))) & 0xFFu;
            mo[i] = m_decode(mk, (i & 1) ? (byte & 0x0Fu) : (byte >> 4), ms);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) mo[i] = m_decode(mk, (qv >> (8 * i)) & 0xFFu, ms);
        }
      }
      float ugj[4];
      if constexpr (CM) {
        float xs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[i] = (scrub(gj[rr][j][i]) * ir) * s_ic[q0 + i];
        div_by<4>(ugj, xs, clip, rclip);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gi = scrub(gj[rr][j][i]);
        const float ic = s_ic[q0 + i];
        if constexpr (CM) {
          mn[i] = lerp_u(mo[i], ugj[i], lw);
          u[i] = (mn[i] * icrr) * s_ic[kTC + q0 + i];
        } else {
          float x = gi;
          if constexpr (kHasM) { mn[i] = lerp_u(mo[i], gi, lw); x = mn[i]; }
          u[i] = (x * ir) * ic;
        }
        if (MODE == 1) {
          const double ud = st ? (double)u[i] : 0.0;
          sq = __builtin_fma(ud, ud, sq);
        }
      }
      if constexpr (MODE != 1) {
        if (MODE == 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) u[i] = u[i] * fs;
        }
        if constexpr (SR) {
          keep4(u);
          if (st) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float p = ld1<T>(P0, e + i);
              const T rr = sr_round<T>((has_dec ? p * dec : p) - step * u[i], D.sr_seed, h.sr_step,
                                       (uint64_t)(e + i));
              uint16_t bits;
              __builtin_memcpy(&bits, &rr, 2);
              gp(reinterpret_cast<uint16_t*>(P0))[e + i] = bits;
            }
          }
        } else {
          if (has_dec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) pv[i] = pdec(pv[i], dec);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) pv[i] = pupd(step, u[i], pv[i]);
          keep4(pv);
          if (st) store4n<T>(P0, e, e + 4, pv);
        }
        if constexpr (MK == 3) {
          keep4(mn);
          if (st) store4n<float>(D.m, e, e + 4, mn);
        } else if constexpr (kHasM) {
          // momentum re-encode: absmax over the block's G lanes.  C is a multiple
          // of the M block, so a block is wholly inside or wholly beyond C.
          uint32_t ab = 0u;
#pragma unroll
          for (int i = 0; i < 4; ++i) ab = max(ab, st ? (__float_as_uint(mn[i]) & 0x7FFFFFFFu) : 0u);
          const float bam = grp_max_dpp(__uint_as_float(ab), G);
          if (st) {
            const float am = fmaxf(bam, 1e-12f);
            const float ram = fast_rcp(am);
            if (MK == 1) {
              const float kam = 128.0f * ram;
              float rr[4];
              bool bad[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) rr[i] = uf_round_fast<128>(mn[i], kam, bad[i]);
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (bad[i]) rr[i] = uf_round_exact<128>(mn[i], am);
#pragma unroll
              for (int i = 0; i < 4; ++i) rr[i] = uf_clamp<128>(rr[i]);
              *gp(reinterpret_cast<uint32_t*>(D.m_q + e)) = pack4(rr[0], rr[1], rr[2], rr[3]);
            } else if (mk == 2 || mk == 4) {
              uint32_t w = 0;
#pragma unroll
              for (int k = 0; k < 2; ++k) {
                const uint32_t hi = m_encode(mk, mn[2 * k], am, ram);
                const uint32_t lo = m_encode(mk, mn[2 * k + 1], am, ram);
                w |= ((hi << 4) | lo) << (8 * k);
              }
              *gp(reinterpret_cast<uint16_t*>(D.m_q + (e >> 1))) = (uint16_t)w;
            } else {
              uint32_t w = 0;
#pragma unroll
              for (int i = 0; i < 4; ++i) w |= m_encode(mk, mn[i], am, ram) << (8 * i);
              *gp(reinterpret_cast<uint32_t*>(D.m_q + e)) = w;
            }
            if ((wl & (G - 1)) == 0) gp(D.m_scale)[e >> lbm] = am;
          }
        }
      }
    }
  }
  if constexpr (MODE == 1) {
    const double tot = wg_sum_d(sq, s4d);
    if (lane == 0) gp(ws_dp(ws, W.npart))[q.t] = tot;
  }
}

// ------------------------------------------------------------ norm, Fira, step
// _apply_update_pytorch with Fira (optimizer.py:796-810, 859-875).
__global__ __launch_bounds__(256) void k_fnorm(const DescF* __restrict__ table, HyperF h) {
  __shared__ double sd[4];
  const DescF D = table[blockIdx.x];
  const FWs W = fws_layout(D.B, D.R, D.C);
  float* ws = D.ws;
  double s = 0.0;
  const int64_t np = D.tiled ? W.nutile : W.nunit;
  for (int64_t k = threadIdx.x; k < np; k += 256) s += gp(ws_dp(ws, W.npart))[k];
  s = wg_sum_d(s, sd);
  if (threadIdx.x == 0) {
    float* sl = ws + W.scal;
    float nrm = sqrtf((float)s);
    float fs = 1.0f;
    if (h.fira) {
      const bool fin = __builtin_isfinite(nrm);
      if (!fin) nrm = 0.0f;            // u.zero_(); norm.zero_()
      float next = nrm;
      if (D.has_fira_prev) {
        const float p = *gp(D.fira_prev);
        const float ratio = nrm / (p + 1e-8f);
        const float lim = (ratio != ratio ? ratio : fmaxf(ratio, h.margin)) / h.margin;
        const bool reset = p < 1e-6f;
        fs = reset ? 1.0f : 1.0f / lim;
        next = reset ? nrm : nrm * fs;
      }
      *gp(D.fira_prev) = next;
      if (!fin) fs = 0.0f;
    }
    float denom = 1.0f;   // CAME applies its update unclipped (optimizer.py:955)
    if (h.d > 0.0f && !h.came) denom = fmaxf(nrm / (float)(sqrt((double)D.numel) * (double)h.d), 1.0f);
    const float alpha = gp(sl)[0];
    gp(sl)[1] = alpha / denom;
    gp(sl)[2] = fs;
  }
}

// CAME clip factor of U = (g * inv_row) * inv_col (optimizer.py:824-829):
// clip = max((||U|| / sqrt(n)) / d, 1), from the norm pass's unit partials.
__global__ __launch_bounds__(256) void k_fclip(const DescF* __restrict__ table, HyperF h) {
  __shared__ double sd[4];
  const DescF D = table[blockIdx.x];
  const FWs W = fws_layout(D.B, D.R, D.C);
  float* ws = D.ws;
  double s = 0.0;
  const int64_t np = D.tiled ? W.nutile : W.nunit;
  for (int64_t k = threadIdx.x; k < np; k += 256) s += gp(ws_dp(ws, W.npart))[k];
  s = wg_sum_d(s, sd);
  if (threadIdx.x == 0) {
    const float rms = sqrtf((float)s) / (float)sqrt((double)D.numel);
    gp(ws)[W.scal + 4] = fmaxf(rms / h.d, 1.0f);
  }
}

hipError_t factored_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

// ------------------------------------------------------------ launch glue
template <typename T>
static int launch_stats(bool psq, const DescF* tab, int ntab, int64_t ntiles, hipStream_t st) {
  if (psq) hipLaunchKernelGGL((k_fstats<T, true>), dim3((unsigned)ntiles), dim3(256), 0, st, tab, ntab);
  else hipLaunchKernelGGL((k_fstats<T, false>), dim3((unsigned)ntiles), dim3(256), 0, st, tab, ntab);
  return check_launch("k_fstats");
}

// Work split of the update passes: tensors with the tiled layout (k_fupdt,
// over the statistics tiles) and the rest (k_fupdate, over flat units).
struct UpdGrid {
  int64_t ntiles, nunits;
  bool any_tiled, any_flat;
};

template <typename T, int MODE, bool SR, bool CM>
static int launch_update_m(int mk, const DescF* tab, int ntab, const UpdGrid& ug, const HyperF& h,
                           hipStream_t st) {
  const dim3 b(256);
  if (ug.any_tiled) {
    const dim3 g((unsigned)ug.ntiles);
    if constexpr (CM) {
      if (mk == 1) hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 1, true>), g, b, 0, st, tab, ntab, h);
      else if (mk == kMkFp32) hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 3, true>), g, b, 0, st, tab, ntab, h);
      else hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 2, true>), g, b, 0, st, tab, ntab, h);
    } else {
      switch (mk) {
        case 0: hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 0, false>), g, b, 0, st, tab, ntab, h); break;
        case 1: hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 1, false>), g, b, 0, st, tab, ntab, h); break;
        case kMkFp32: hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 3, false>), g, b, 0, st, tab, ntab, h); break;
        default: hipLaunchKernelGGL((k_fupdt<T, MODE, SR, 2, false>), g, b, 0, st, tab, ntab, h); break;
      }
    }
    int rc = check_launch("k_fupdt");
    if (rc) return rc;
  }
  if (ug.any_flat && h.lbm < 0) {   // general B_M: every tensor is flat, units of h.unit
    const dim3 g((unsigned)ug.nunits);
    if constexpr (CM) hipLaunchKernelGGL((k_fupdate_gen<T, MODE, SR, 2, true>), g, b, 0, st, tab, ntab, h);
    else if (mk == 0) hipLaunchKernelGGL((k_fupdate_gen<T, MODE, SR, 0, false>), g, b, 0, st, tab, ntab, h);
    else hipLaunchKernelGGL((k_fupdate_gen<T, MODE, SR, 2, false>), g, b, 0, st, tab, ntab, h);
    return check_launch("k_fupdate_gen");
  }
  if (ug.any_flat) {
    const dim3 g((unsigned)ug.nunits);
    if constexpr (CM) {
      if (mk == 1) hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 1, true>), g, b, 0, st, tab, ntab, h);
      else if (mk == kMkFp32) hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 3, true>), g, b, 0, st, tab, ntab, h);
      else hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 2, true>), g, b, 0, st, tab, ntab, h);
    } else {
      switch (mk) {
        case 0: hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 0, false>), g, b, 0, st, tab, ntab, h); break;
        case 1: hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 1, false>), g, b, 0, st, tab, ntab, h); break;
        case kMkFp32: hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 3, false>), g, b, 0, st, tab, ntab, h); break;
        default: hipLaunchKernelGGL((k_fupdate<T, MODE, SR, 2, false>), g, b, 0, st, tab, ntab, h); break;
      }
    }
    return check_launch("k_fupdate");
  }
  return 0;
}

template <typename T, bool SR, bool CM>
static int launch_update(int mode, int mk, const DescF* tab, int ntab, const UpdGrid& ug, const HyperF& h,
                         hipStream_t st) {
  switch (mode) {
    case 0: return launch_update_m<T, 0, SR, CM>(mk, tab, ntab, ug, h, st);
    case 1: return launch_update_m<T, 1, false, CM>(mk, tab, ntab, ug, h, st);
    default: return launch_update_m<T, 2, SR, CM>(mk, tab, ntab, ug, h, st);
  }
}

static int launch_colsum(const DescF* tab, int ntab, int64_t ncs, hipStream_t st) {
  if (ncs <= 0) return 0;
  hipLaunchKernelGGL(k_fcolsum, dim3((unsigned)ncs), dim3(256), 0, st, tab, ntab);
  return check_launch("k_fcolsum");
}

template <bool CONF>
static int launch_finish(int bits, const DescF* tab, int ntab, int64_t nfblk, const HyperF& h,
                         hipStream_t st) {
  const dim3 g((unsigned)nfblk), b(256);
  switch (bits) {
    case 8: hipLaunchKernelGGL((k_fblock<8, CONF>), g, b, 0, st, tab, ntab, h); break;
    case 16: hipLaunchKernelGGL((k_fblock<16, CONF>), g, b, 0, st, tab, ntab, h); break;
    default: hipLaunchKernelGGL((k_fblock<0, CONF>), g, b, 0, st, tab, ntab, h); break;
  }
  int rc = check_launch("k_fblock");
  if (rc) return rc;
  hipLaunchKernelGGL((k_frows<CONF>), dim3((unsigned)ntab), b, 0, st, tab, h);
  return check_launch("k_frows");
}

// Launch sequence of one group step.  Plain factored: stats, finish, then the
// update (with a norm pass + k_fnorm first when clipping or Fira is on).  CAME:
// stats, finish, [U norm + k_fclip when d > 0], k_came1, confidence finish,
// [update norm + k_fnorm with Fira], update.
template <typename T, bool SR>
static int run_group(const DescF* tab, int ntab, int64_t ntiles, const UpdGrid& ug, int64_t nfblk, int64_t ncs,
                     int vbits, int cbits, bool clip, const HyperF& h, hipStream_t st) {
  int rc = launch_stats<T>(h.scale_param != 0, tab, ntab, ntiles, st);
  if (rc) return rc;
  if ((rc = launch_colsum(tab, ntab, ncs, st))) return rc;
  if ((rc = launch_finish<false>(vbits, tab, ntab, nfblk, h, st))) return rc;
  if (h.came) {
    if (h.d > 0.0f) {
      if ((rc = launch_update<T, false, false>(1, 0, tab, ntab, ug, h, st))) return rc;
      hipLaunchKernelGGL(k_fclip, dim3((unsigned)ntab), dim3(256), 0, st, tab, h);
      if ((rc = check_launch("k_fclip"))) return rc;
    }
    if (h.mk == 1) hipLaunchKernelGGL((k_came1<T, 1>), dim3((unsigned)ntiles), dim3(256), 0, st, tab, ntab, h);
    else if (h.mk == kMkFp32) hipLaunchKernelGGL((k_came1<T, 3>), dim3((unsigned)ntiles), dim3(256), 0, st, tab, ntab, h);
    else hipLaunchKernelGGL((k_came1<T, 2>), dim3((unsigned)ntiles), dim3(256), 0, st, tab, ntab, h);
    if ((rc = check_launch("k_came1"))) return rc;
    if ((rc = launch_colsum(tab, ntab, ncs, st))) return rc;
    if ((rc = launch_finish<true>(cbits, tab, ntab, nfblk, h, st))) return rc;
    if (!h.fira) return launch_update<T, SR, true>(0, h.mk, tab, ntab, ug, h, st);
    if ((rc = launch_update<T, false, true>(1, h.mk, tab, ntab, ug, h, st))) return rc;
    hipLaunchKernelGGL(k_fnorm, dim3((unsigned)ntab), dim3(256), 0, st, tab, h);
    if ((rc = check_launch("k_fnorm"))) return rc;
    return launch_update<T, SR, true>(2, h.mk, tab, ntab, ug, h, st);
  }
  if (!clip) return launch_update<T, SR, false>(0, h.mk, tab, ntab, ug, h, st);
  if ((rc = launch_update<T, false, false>(1, h.mk, tab, ntab, ug, h, st))) return rc;
  hipLaunchKernelGGL(k_fnorm, dim3((unsigned)ntab), dim3(256), 0, st, tab, h);
  if ((rc = check_launch("k_fnorm"))) return rc;
  return launch_update<T, SR, false>(2, h.mk, tab, ntab, ug, h, st);
}

static int mk_code(int mbits, int mmode) {
  if (mmode == 0) return mbits == 8 ? 1 : 2;
  return mbits == 8 ? 3 : 4;
}

}  // namespace a8

using namespace a8;

extern "C" {

int64_t a8_factored_workspace_floats(int64_t batch, int64_t rows, int64_t cols) {
  if (batch <= 0 || rows <= 0 || cols <= 0) return 0;
  return fws_layout(batch, rows, cols).total;
}

int64_t a8_table_bytes_2d(int ntensors) { return (int64_t)sizeof(DescF) * (int64_t)ntensors; }

int a8_factored_step(int dtype, int stochastic, const a8_tensor2d* tensors, int ntensors,
                     void* table_dev, int64_t table_bytes, int upload, double beta_val, float eps1,
                     float eps2, float lr_val, int scale_parameter, int bias_mode, float bias_factor,
                     float weight_decay, int wd_mode, float d, int fira, float fira_margin,
                     float log_floor, int v_bits, int block_size, double beta1, int m_block_size,
                     int m_bits, int m_mode, uint64_t sr_step, int came, double beta3, float eps_came,
                     int c_bits, const void* step_scalars, void* stream) {
  if (ntensors <= 0) return 0;
  if (dtype != A8_F32 && dtype != A8_BF16 && dtype != A8_F16 && dtype != A8_F64)
    return set_error(A8_ERR_DTYPE, "dtype");
  if (v_bits != 0 && v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 0, 8 or 16");
  if (came && c_bits != 0 && c_bits != 8 && c_bits != 16) return set_error(A8_ERR_ARG, "c_bits must be 0, 8 or 16");
  if (block_size <= 0) return set_error(A8_ERR_BLOCK, "block_size must be positive");
  if ((int64_t)sizeof(DescF) * ntensors > table_bytes)
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_table_bytes_2d(ntensors)");
  const bool m32 = tensors[0].m != nullptr;
  const bool has_m = tensors[0].m_q != nullptr || m32;
  int lbm = 5, gbm = 0, gunit = 0;
  if (has_m && !m32) {
    if (!((m_bits == 8 || m_bits == 4) && (m_mode == 0 || m_mode == 1)))
      return set_error(A8_ERR_ARG, "m_bits must be 4/8 and m_mode 0/1");
    if (m_block_size < 32 || m_block_size > (1 << 30) || (m_block_size & 3))
      return set_error(A8_ERR_BLOCK, "m_block_size must be a multiple of 4 in [32, 2^30]");
    if (m_block_size <= kUnit && !(m_block_size & (m_block_size - 1))) {
      lbm = 0;
      while ((1 << lbm) < m_block_size) ++lbm;
    } else {   // k_fupdate_gen: whole M blocks per workgroup, at least kUnit elements
      lbm = -1;
      gbm = m_block_size;
      gunit = m_block_size * ((kUnit + m_block_size - 1) / m_block_size);
    }
  }
  if (came && !has_m) return set_error(A8_ERR_ARG, "CAME needs momentum (m_q or m)");
  if (stochastic && dtype == A8_F32) stochastic = 0;
  std::vector<DescF> tab((size_t)ntensors);
  int64_t tiles = 0, utiles = 0, units = 0, fblks = 0, csw = 0;
  bool any_tiled = false, any_flat = false;
  const size_t esz = dtype == A8_F32 ? 4 : (dtype == A8_F64 ? 8 : 2);
  for (int i = 0; i < ntensors; ++i) {
    const a8_tensor2d& t = tensors[i];
    if (t.batch <= 0 || t.rows <= 0 || t.cols <= 0) return set_error(A8_ERR_SIZE, "empty factored tensor");
    if (!t.param || !t.grad || !t.workspace) return set_error(A8_ERR_ARG, "null param/grad/workspace");
    if ((t.m_q != nullptr) != (has_m && !m32) || (t.m != nullptr) != m32)
      return set_error(A8_ERR_ARG, "mixed momentum kinds in one launch");
    if (v_bits ? !(t.row_q && t.col_q && t.row_scale && t.col_scale && t.row_min_log && t.col_min_log)
               : !(t.row_var && t.col_var))
      return set_error(A8_ERR_ARG, "row/column state missing");
    if (fira && !t.fira_prev_norm) return set_error(A8_ERR_ARG, "fira needs fira_prev_norm");
    if (came && (c_bits ? !(t.conf_row_q && t.conf_col_q && t.conf_row_scale && t.conf_col_scale &&
                            t.conf_row_min_log && t.conf_col_min_log)
                        : !(t.conf_row && t.conf_col)))
      return set_error(A8_ERR_ARG, "CAME confidence state missing");
    if (!aligned16(t.param) || !aligned16(t.grad) || (has_m && !aligned16(m32 ? (const void*)t.m : t.m_q)))
      return set_error(A8_ERR_ALIGN, "param/grad/momentum buffers must be 16-byte aligned");
    const int64_t numel = t.batch * t.rows * t.cols;
    if (numel >= ((int64_t)1 << 40)) return set_error(A8_ERR_SIZE, "tensor too large");
    DescF& D = tab[(size_t)i];
    D.param = t.param; D.grad = t.grad; D.m_q = t.m_q; D.m_scale = t.m_scale; D.m = t.m;
    D.row_q = t.row_q; D.row_scale = t.row_scale; D.row_min_log = t.row_min_log; D.row_var = t.row_var;
    D.col_q = t.col_q; D.col_scale = t.col_scale; D.col_min_log = t.col_min_log; D.col_var = t.col_var;
    D.crow_q = t.conf_row_q; D.crow_scale = t.conf_row_scale; D.crow_min_log = t.conf_row_min_log;
    D.crow_var = t.conf_row; D.ccol_q = t.conf_col_q; D.ccol_scale = t.conf_col_scale;
    D.ccol_min_log = t.conf_col_min_log; D.ccol_var = t.conf_col;
    D.ws = t.workspace; D.lr = t.lr; D.fira_prev = t.fira_prev_norm; D.has_fira_prev = t.has_fira_prev;
    D.B = t.batch; D.R = t.rows; D.C = t.cols; D.numel = numel;
    D.sr_seed = t.sr_seed;
    D.vec4 = ((t.cols * esz) % 16 == 0) ? 1 : 0;
    D.tiled = (t.cols % 4 == 0) &&
              (!has_m || m32 || (lbm >= 0 && m_block_size <= 256 && t.cols % m_block_size == 0)) ? 1 : 0;
    (D.tiled ? any_tiled : any_flat) = true;
    const FWs W = fws_layout(t.batch, t.rows, t.cols);
    D.tile_begin = tiles;
    D.utile_begin = utiles;
    D.unit_begin = units;
    D.fblk_begin = fblks;
    D.cs_begin = csw;
    D.nbr = (t.batch * t.rows + block_size - 1) / block_size;
    tiles += W.ntile;
    utiles += W.nutile;
    units += lbm >= 0 ? W.nunit : (numel + gunit - 1) / gunit;   // gunit >= kUnit: within W.nunit slots
    fblks += D.nbr + (t.batch * t.cols + block_size - 1) / block_size;
    if (W.nsplit > 1) csw += t.batch * ((t.cols + 255) / 256) * W.nsplit;
  }
  if (tiles > 0x7FFFFFFF || utiles > 0x7FFFFFFF || units > 0x7FFFFFFF || fblks > 0x7FFFFFFF || csw > 0x7FFFFFFF)
    return set_error(A8_ERR_SIZE, "too many workgroups");
  hipStream_t st = (hipStream_t)stream;
  if (upload && upload_table(table_dev, tab.data(), sizeof(DescF) * (size_t)ntensors, st) != hipSuccess)
    return set_error(A8_ERR_HIP, "table upload failed");
  HyperF h{};
  h.bv = (float)beta_val;
  h.eps1 = eps1; h.eps2 = eps2; h.lr_val = lr_val;
  h.bias_factor = bias_factor; h.bias_mode = bias_mode;
  h.scale_param = scale_parameter;
  h.wd = weight_decay; h.wd_mode = wd_mode;
  h.d = d; h.fira = fira; h.margin = (float)(1.0 + (double)fira_margin);
  h.floor_ = log_floor;
  h.w_m = (float)(1.0 - beta1);
  h.came = came ? 1 : 0;
  h.w_c = (float)(1.0 - beta3);
  h.eps_came = eps_came;
  h.block_size = block_size;
  h.mk = m32 ? kMkFp32 : (has_m ? mk_code(m_bits, m_mode) : 0);
  h.lbm = lbm;
  h.bm = gbm;
  h.unit = gunit;
  h.sr_step = sr_step;
  h.dsc = reinterpret_cast<const a8_step_scalars*>(step_scalars);
  const bool clip = d > 0.0f || fira;
  const DescF* dt = reinterpret_cast<const DescF*>(table_dev);
  const UpdGrid ug{utiles, units, any_tiled, any_flat};
  switch (dtype) {
    case A8_F32: return run_group<float, false>(dt, ntensors, tiles, ug, fblks, csw, v_bits, c_bits, clip, h, st);
    case A8_BF16:
      return stochastic ? run_group<__hip_bfloat16, true>(dt, ntensors, tiles, ug, fblks, csw, v_bits, c_bits, clip, h, st)
                        : run_group<__hip_bfloat16, false>(dt, ntensors, tiles, ug, fblks, csw, v_bits, c_bits, clip, h, st);
    case A8_F64: return run_group<double, false>(dt, ntensors, tiles, ug, fblks, csw, v_bits, c_bits, clip, h, st);
    default:
      return stochastic ? run_group<__half, true>(dt, ntensors, tiles, ug, fblks, csw, v_bits, c_bits, clip, h, st)
                        : run_group<__half, false>(dt, ntensors, tiles, ug, fblks, csw, v_bits, c_bits, clip, h, st);
  }
}

}  // extern "C"
