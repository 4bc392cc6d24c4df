// APOLLO low-rank stage of the factorised and CAME variants, and of the plain
// variant at block sizes the fused k_ap_low does not take.
//
// Follows _update_param_apollo (optimizer.py:2587-3084) on the branches its
// CPU fallback takes (no CUDA module) for what a8_apollo_step's fused k_ap_low
// does not cover:
//   factorised (apollo_factorize, optimizer.py:2689-2758): row / column means of
//     g_low^2 plus FLT_MIN into fp32 EMAs r, c (first step mean * bv, later
//     fma(bv, mean, x * (1 - bv)), the order of mul_(1-bv).add_(mean, alpha=bv));
//     v = (r_i c_j) / max(mean(r), eps); u = x / (sqrt(v) + eps), x = g_low or its
//     momentum lerp(m, g_low, 1 - beta1).  With beta3 (CAME): U = (g / sqrt(r_i /
//     max(mean r, FLT_MIN))) / sqrt(c_j), RMS clip, m EMA of U, res = (U - m)^2 +
//     eps_came, its row / column means into confidence EMAs (beta3; fp32, or AL
//     codes re-encoded from the lerped values, which are used), u = (m /
//     sqrt(cr_i / max(mean cr, FLT_MIN))) / sqrt(cc_j).
//   non-factorised CAME (beta3, optimizer.py:2759-2896): the low-rank V EMA of
//     the plain path (first step g^2 * bv at floor -126, later lerp at floor
//     log2(eps^2)); U = g / sqrt(max(v, eps^2)), RMS clip, m EMA of U, residual
//     EMA (beta3) of (U - m)^2 + eps_came in fp32 or AL codes (read back decoded
//     after the re-encode), u = m / sqrt(max(res, eps^2)).
//   plain (optimizer.py:2759-2799), for a coded low-rank V block that is not a
//     power of two in [128, 2048] or such a momentum block outside [32, 2048]:
//     the low-rank V EMA above, the momentum EMA of g_low (its lerped values),
//     u = x / (sqrt(v) + eps) with x = m or g_low and v the lerped V values.
//     The EMAs run in the general-block kernels of a8_prims / a8_sgd.
// RMS clip (optimizer.py:2715-2717, 2869-2871): U /= max((||U|| / sqrt(n)) / d, 1)
// for d > 0, ||U|| summed in double.  Row / column means are sums in double
// rounded to fp32 and divided by the count in fp32.  rsqrt is 1 / sqrt, both
// correctly rounded, as the CPU kernels compute it.
//
// The caller runs a8_apollo_step_multi_phase(1, ...) first (g_low in
// workspace[0, n_low) of the APOLLO workspace), then this with u pointing at
// workspace[n_low, 2 n_low), then phase 2 (channel scale, Fira, writeback).
#include "a8_common.cuh"
#include "a8_abi_impl.h"

namespace a8 {

constexpr int kXParts = 1024;     // max workgroups of an element pass (= partial sums of a reduction)
constexpr int kXRowChunk = 256;   // rows per column-sum partial
constexpr int kXColBlk = 256;     // columns per row-sum partial (four per lane)

// Extended workspace of one matrix (offsets in floats; part / cpart hold doubles).
struct XL {
  int64_t n, nch, ncb, xv, xu, xm, xr, rowm, colm, crow, ccol, scal, part, cpart, rpart, total;
};

__host__ __device__ inline XL x_layout(int64_t R, int64_t C) {
  XL w;
  w.n = R * C;
  w.nch = (R + kXRowChunk - 1) / kXRowChunk;
  w.ncb = (C + kXColBlk - 1) / kXColBlk;
  const int64_t n4 = (w.n + 3) / 4 * 4;   // regions start 16-byte aligned
  w.xv = 0;                    // V values of coded V (the lerped values)
  w.xu = w.xv + n4;            // U (CAME)
  w.xm = w.xu + n4;            // momentum values of coded M
  w.xr = w.xm + n4;            // residual, then its decoded EMA
  w.rowm = w.xr + n4;          // row means
  w.colm = w.rowm + (R + 3) / 4 * 4;   // column means
  w.crow = w.colm + (C + 3) / 4 * 4;   // confidence values of coded confidence
  w.ccol = w.crow + (R + 3) / 4 * 4;
  w.scal = w.ccol + (C + 3) / 4 * 4;   // [0] clip, [1] row-variance mean (clamped), [2] confidence row mean
  w.part = (w.scal + 16 + 1) / 2 * 2;
  w.cpart = w.part + 2 * kXParts;
  w.rpart = w.cpart + 2 * w.nch * C;
  w.total = w.rpart + 2 * w.ncb * R;
  return w;
}

// One matrix of a launch.
struct XK {
  const float* g;      // g_low, R x C row-major
  const float* src;    // input of the fp32 momentum EMA (g_low or U)
  float* dst;          // output of the U pass
  float* u;            // update_low (output)
  float* ws;           // extended workspace
  float* v;            // V values (fp32 state or ws + xv)
  float* m;            // momentum values (fp32 state or ws + xm)
  float* res;          // fp32 residual EMA state (null: coded, decoded into ws + xr)
  float* rv;           // factorised fp32 row / column EMAs
  float* cv;
  float* cr;           // confidence values (fp32 state or ws + crow / ccol)
  float* cc;
  int64_t R, C, n;
  float bv, omb, w1, w3, aeps, eps_sq, eps_came, d, sqn;
  int first, np;
  int v4;              // every stream of this matrix is 16-byte aligned and n % 4 == 0
};

// Launch kinds: each has its own grid over the batch, and a matrix owns the
// workgroups [wb[kind], wb[kind] + count) of it.
enum { XW_EL = 0, XW_ROWS, XW_CPART, XW_CFIN, XW_VEC, XW_ONE, XW_N };

struct XD {
  XK k;
  int64_t wb[XW_N];
};

// Where a launch finds its matrices: a device table, or one matrix by value;
// dsc: the device step block, whose V weight replaces the descriptors' bv.
struct XT {
  XD one;
  const XD* tab;
  int ntab;
  const a8_step_scalars* dsc;
};

// The V lerp weight bv and 1 - bv (derived in double, as the descriptor's are).
__device__ __forceinline__ void x_bv(const XT& t, const XK& k, float& bv, float& omb) {
  bv = k.bv;
  omb = k.omb;
  if (t.dsc) {
    const double b = load_step_scalars(t.dsc).beta_val;
    bv = (float)b;
    omb = (float)(1.0 - b);
  }
}

// The matrix that owns workgroup blockIdx.x of a launch of kind KIND, and the
// workgroup's index within that matrix.
template <int KIND>
__device__ __forceinline__ XK x_find(const XT& t, int64_t& local) {
  const int64_t wg = blockIdx.x;
  if (!t.tab) {
    local = wg;
    return t.one.k;
  }
  int lo = 0, hi = t.ntab - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.tab[mid].wb[KIND] <= wg) lo = mid; else hi = mid - 1;
  }
  local = wg - t.tab[lo].wb[KIND];
  return t.tab[lo].k;
}

enum {
  XE_SQB = 0,   // xv = (g^2) * bv
  XE_V32,       // fp32 V state: first ? g^2 * bv : lerp(v, g^2, bv)
  XE_U,         // dst = g / sqrt(max(v, eps^2)); partial sum of squares
  XE_FCU,       // dst = (g / sqrt(r_i / rmean)) / sqrt(c_j); partial sum of squares
  XE_DIV,       // dst /= clip
  XE_M32,       // fp32 m = lerp(m, src, 1 - beta1)
  XE_RES,       // xr = (U - m)^2 + eps_came; fp32 res state lerped toward it
  XE_UCAME,     // u = m / sqrt(max(res, eps^2))
  XE_FU,        // u = src / (sqrt((r_i c_j) / max(mean r, eps)) + eps)
  XE_FUC,       // u = (m / sqrt(cr_i / cmean)) / sqrt(cc_j)
  XE_AU         // u = x / (sqrt(v) + eps), x = m (momentum) or g
};

__device__ __forceinline__ float rsqrt_ref(float x) { return 1.0f / sqrtf(x); }

__device__ __forceinline__ double x_wg_sum(double v, double* sd) {
  v = grp_sum_d(v, 64);
  const int lane = threadIdx.x;
  __syncthreads();
  if ((lane & 63) == 0) sd[lane >> 6] = v;
  __syncthreads();
  return ((sd[0] + sd[1]) + sd[2]) + sd[3];
}

// Four consecutive elements of a stream: one 16-byte access when the matrix's
// streams are aligned (v4), else element by element inside n.
__device__ __forceinline__ void x_ld4(const float* p, int64_t i, int64_t n, int v4, float* o) {
  if (v4) {
    load4v<float>(p, i, o);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (i + e < n) ? gp(p)[i + e] : 0.0f;
  }
}
__device__ __forceinline__ void x_st4(float* p, int64_t i, int64_t n, int v4, const float* o) {
  if (v4) {
    store4n<float>(p, i, i + 4, o);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i + e < n) gp(p)[i + e] = o[e];
  }
}

// Element passes: lane t of local workgroup b handles elements 4(b*256 + t) ..
// +3, striding by the matrix's np workgroups.
template <int OP>
__global__ __launch_bounds__(256) void k_ax_el(XT t) {
  __shared__ double sd[4];
  int64_t lb;
  const XK k = x_find<XW_EL>(t, lb);
  float* ws = k.ws;
  const XL L = x_layout(k.R, k.C);
  const float clip = (OP == XE_DIV) ? gp(ws)[L.scal] : 1.0f;
  const float rmean = (OP == XE_FCU || OP == XE_FU) ? gp(ws)[L.scal + 1] : 1.0f;
  const float cmean = (OP == XE_FUC) ? gp(ws)[L.scal + 2] : 1.0f;
  float bv = 0.0f, omb = 0.0f;
  if constexpr (OP == XE_SQB || OP == XE_V32) x_bv(t, k, bv, omb);
  double acc = 0.0;
  const int64_t stride = (int64_t)k.np * 1024;
  for (int64_t i = (lb * 256 + threadIdx.x) * 4; i < k.n; i += stride) {
    float a[4], b[4], o[4];
    if constexpr (OP == XE_SQB) {
      x_ld4(k.g, i, k.n, k.v4, a);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (a[e] * a[e]) * bv;
      x_st4(ws + L.xv, i, k.n, k.v4, o);
    } else if constexpr (OP == XE_V32) {
      x_ld4(k.g, i, k.n, k.v4, a);
      if (!k.first) x_ld4(k.v, i, k.n, k.v4, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float g2 = a[e] * a[e];
        o[e] = k.first ? g2 * bv : lerp_ref(b[e], g2, bv);
      }
      x_st4(k.v, i, k.n, k.v4, o);
    } else if constexpr (OP == XE_U) {
      x_ld4(k.g, i, k.n, k.v4, a);
      x_ld4(k.v, i, k.n, k.v4, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = a[e] * rsqrt_ref(fmaxf(b[e], k.eps_sq));
        if (i + e < k.n) acc += (double)(o[e] * o[e]);
      }
      x_st4(k.dst, i, k.n, k.v4, o);
    } else if constexpr (OP == XE_DIV) {
      x_ld4(k.dst, i, k.n, k.v4, a);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = a[e] / clip;
      x_st4(k.dst, i, k.n, k.v4, o);
    } else if constexpr (OP == XE_M32) {
      x_ld4(k.m, i, k.n, k.v4, a);
      x_ld4(k.src, i, k.n, k.v4, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = lerp_ref(a[e], b[e], k.w1);
      x_st4(k.m, i, k.n, k.v4, o);
    } else if constexpr (OP == XE_RES) {
      x_ld4(ws + L.xu, i, k.n, k.v4, a);
      x_ld4(k.m, i, k.n, k.v4, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r = a[e] - b[e];
        r = r * r;
        o[e] = r + k.eps_came;
      }
      x_st4(ws + L.xr, i, k.n, k.v4, o);
      if (k.res) {
        x_ld4(k.res, i, k.n, k.v4, a);
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = lerp_ref(a[e], o[e], k.w3);
        x_st4(k.res, i, k.n, k.v4, a);
      }
    } else if constexpr (OP == XE_AU) {
      x_ld4(k.m ? k.m : k.g, i, k.n, k.v4, a);
      x_ld4(k.v, i, k.n, k.v4, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = a[e] / (sqrtf(b[e]) + k.aeps);
      x_st4(k.u, i, k.n, k.v4, o);
    } else if constexpr (OP == XE_UCAME) {
      x_ld4(k.m, i, k.n, k.v4, a);
      x_ld4(k.res ? k.res : ws + L.xr, i, k.n, k.v4, b);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = a[e] * rsqrt_ref(fmaxf(b[e], k.eps_sq));
      x_st4(k.u, i, k.n, k.v4, o);
    } else {   // XE_FCU, XE_FU, XE_FUC: row / column factors, (r, c) stepped from the first element
      x_ld4(OP == XE_FCU ? k.g : (OP == XE_FU ? k.src : k.m), i, k.n, k.v4, a);
      int64_t r = i / k.C, c = i - r * k.C;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (i + e < k.n) {
          if constexpr (OP == XE_FCU) {
            const float ir = rsqrt_ref(gp(k.rv)[r] / rmean);
            const float ic = rsqrt_ref(gp(k.cv)[c]);
            o[e] = (a[e] * ir) * ic;
            acc += (double)(o[e] * o[e]);
          } else if constexpr (OP == XE_FU) {
            const float ve = (gp(k.rv)[r] * gp(k.cv)[c]) / rmean;
            o[e] = a[e] / (sqrtf(ve) + k.aeps);
          } else {
            const float icr = rsqrt_ref(gp(k.cr)[r] / cmean);
            const float icc = rsqrt_ref(gp(k.cc)[c]);
            o[e] = (a[e] * icr) * icc;
          }
        } else {
          o[e] = 0.0f;
        }
        if (++c == k.C) { c = 0; ++r; }
      }
      x_st4(OP == XE_FCU ? k.dst : k.u, i, k.n, k.v4, o);
    }
  }
  if constexpr (OP == XE_U || OP == XE_FCU) {
    const double s = x_wg_sum(acc, sd);
    if (threadIdx.x == 0) reinterpret_cast<A8_G double*>(gp(ws) + L.part)[lb] = s;
  }
}

// Which vector a row / column pass reads: g_low^2, or the residual.
enum { XR_GSQ = 0, XR_RES };

template <int SRC>
__device__ __forceinline__ const float* x_src(const XK& k) {
  return SRC == XR_GSQ ? k.g : k.ws + x_layout(k.R, k.C).xr;
}

// Row and column sums of x (or x^2) in one read, over a tile of kXRowChunk rows
// and kXColBlk columns: each wave walks every fourth row of the tile, a lane
// holding four consecutive columns.  A row's sum over the tile's columns (lane
// sums, then the wave's fixed tree) is its mean when the matrix has one column
// block, else a partial in rpart; a lane's columns accumulate down its rows and
// the four waves combine in order into the chunk's column partial.
template <int SRC>
__global__ __launch_bounds__(256) void k_ax_rcpart(XT t, float add) {
  __shared__ double sd[4 * kXColBlk];
  int64_t lb;
  const XK k = x_find<XW_CPART>(t, lb);
  const float* x = x_src<SRC>(k);
  const XL L = x_layout(k.R, k.C);
  const int64_t by = lb / L.ncb, bx = lb - by * L.ncb;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t c0 = bx * kXColBlk + 4 * l;
  const int64_t r0 = by * kXRowChunk;
  const int64_t r1 = r0 + kXRowChunk < k.R ? r0 + kXRowChunk : k.R;
  const bool vec = k.v4 && (k.C & 3) == 0 && (SRC == XR_RES || (reinterpret_cast<uintptr_t>(x) & 15) == 0);
  double cs[4] = {0.0, 0.0, 0.0, 0.0};
  // four of the wave's rows per round, all loaded before any is summed
  for (int64_t rb = r0 + w; rb < r1; rb += 16) {   // uniform per wave
    float a[4][4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t r = rb + 4 * h;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[h][e] = 0.0f;
      if (r >= r1) continue;
      const float* xr = x + r * k.C;
      if (vec) {
        if (c0 < k.C) {
          const f32x4 q = *gp(reinterpret_cast<const f32x4*>(xr + c0));
          a[h][0] = q.x; a[h][1] = q.y; a[h][2] = q.z; a[h][3] = q.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c0 + e < k.C) a[h][e] = gp(xr)[c0 + e];
      }
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t r = rb + 4 * h;
      if (r >= r1) break;   // uniform per wave
      double rs = 0.0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double q = (double)(SRC == XR_GSQ ? a[h][e] * a[h][e] : a[h][e]);
        cs[e] += q;
        rs += q;
      }
      rs = grp_sum_d(rs, 64);
      if (l == 0) {
        if (L.ncb == 1) gp(k.ws)[L.rowm + r] = (float)rs / (float)k.C + add;
        else reinterpret_cast<A8_G double*>(gp(k.ws) + L.rpart)[bx * k.R + r] = rs;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) sd[w * kXColBlk + 4 * l + e] = cs[e];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * l + e;
      if (c0 + e < k.C)
        reinterpret_cast<A8_G double*>(gp(k.ws) + L.cpart)[by * k.C + c0 + e] =
            ((sd[j] + sd[kXColBlk + j]) + sd[2 * kXColBlk + j]) + sd[3 * kXColBlk + j];
    }
  }
}

// Row means from the column blocks' partials, in block order (matrices with
// more than one column block).
__global__ __launch_bounds__(256) void k_ax_rowfin(XT t, float add) {
  int64_t lb;
  const XK k = x_find<XW_ROWS>(t, lb);
  const XL L = x_layout(k.R, k.C);
  const int64_t r = lb * 256 + threadIdx.x;
  if (r >= k.R || L.ncb == 1) return;
  const A8_G double* part = reinterpret_cast<const A8_G double*>(gp(k.ws) + L.rpart);
  double s = 0.0;
  for (int64_t h = 0; h < L.ncb; ++h) s += part[h * k.R + r];
  gp(k.ws)[L.rowm + r] = (float)s / (float)k.C + add;
}

__global__ __launch_bounds__(256) void k_ax_colfin(XT t, float add) {
  int64_t lb;
  const XK k = x_find<XW_CFIN>(t, lb);
  const XL L = x_layout(k.R, k.C);
  const int64_t c = lb * 256 + threadIdx.x;
  if (c >= k.C) return;
  const A8_G double* part = reinterpret_cast<const A8_G double*>(gp(k.ws) + L.cpart);
  double s = 0.0;
  for (int64_t h = 0; h < L.nch; ++h) s += part[h * k.C + c];
  gp(k.ws)[L.colm + c] = (float)s / (float)k.R + add;
}

enum { XV_VAR = 0, XV_CONF };

// Row (index < R) and column (index >= R) vectors of the factorised EMAs.
template <int OP>
__global__ __launch_bounds__(256) void k_ax_vec(XT t) {
  int64_t lb;
  const XK k = x_find<XW_VEC>(t, lb);
  const XL L = x_layout(k.R, k.C);
  const int64_t j = lb * 256 + threadIdx.x;
  if (j >= k.R + k.C) return;
  const bool row = j < k.R;
  const int64_t i = row ? j : j - k.R;
  const float mean = gp(k.ws)[(row ? L.rowm : L.colm) + i];
  if constexpr (OP == XV_VAR) {
    float* s = row ? k.rv : k.cv;
    float bv, omb;
    x_bv(t, k, bv, omb);
    gp(s)[i] = k.first ? mean * bv : __builtin_fmaf(bv, mean, gp(s)[i] * omb);
  } else {
    float* s = row ? k.cr : k.cc;
    gp(s)[i] = lerp_ref(gp(s)[i], mean, k.w3);
  }
}

enum { XS_CLIP = 0, XS_RMEAN, XS_RMEAN_CAME, XS_CMEAN };

// One workgroup per matrix: the scalars between passes.
template <int OP>
__global__ __launch_bounds__(256) void k_ax_s(XT t) {
  __shared__ double sd[4];
  int64_t lb;
  const XK k = x_find<XW_ONE>(t, lb);
  float* ws = k.ws;
  const XL L = x_layout(k.R, k.C);
  double s = 0.0;
  if constexpr (OP == XS_CLIP) {
    const A8_G double* p = reinterpret_cast<const A8_G double*>(gp(ws) + L.part);
    for (int i = threadIdx.x; i < k.np; i += 256) s += p[i];
  } else {
    const float* x = OP == XS_CMEAN ? k.cr : k.rv;
    for (int64_t i = threadIdx.x; i < k.R; i += 256) s += (double)gp(x)[i];
  }
  s = x_wg_sum(s, sd);
  if (threadIdx.x != 0) return;
  if constexpr (OP == XS_CLIP) {
    const float rms = sqrtf((float)s) / k.sqn;
    gp(ws)[L.scal] = fmaxf(rms / k.d, 1.0f);
  } else {
    const float mean = (float)s / (float)k.R;
    if constexpr (OP == XS_RMEAN) gp(ws)[L.scal + 1] = fmaxf(mean, k.aeps);
    else if constexpr (OP == XS_RMEAN_CAME) gp(ws)[L.scal + 1] = fmaxf(mean, 1.17549435e-38f);
    else gp(ws)[L.scal + 2] = fmaxf(mean, 1.17549435e-38f);
  }
}

// Workgroups of an element pass over n elements (4 per lane): at most kXParts,
// which is also the number of partial sums a reduction leaves.
static int64_t x_grid(int64_t n) {
  const int64_t nb = (n + 1023) / 1024;
  return nb < kXParts ? (nb > 0 ? nb : 1) : kXParts;
}

// Workgroups of each launch kind for one matrix.
static void x_counts(const XK& k, int64_t* cnt) {
  const XL L = x_layout(k.R, k.C);
  cnt[XW_EL] = x_grid(k.n);
  cnt[XW_ROWS] = L.ncb > 1 ? (k.R + 255) / 256 : 0;
  cnt[XW_CPART] = L.ncb * L.nch;
  cnt[XW_CFIN] = (k.C + 255) / 256;
  cnt[XW_VEC] = (k.R + k.C + 255) / 256;
  cnt[XW_ONE] = 1;
}

// A batch of matrices that share every flag and hyper-parameter of the stage:
// their descriptors (wb filled in), the total grid of each launch kind, the
// device tables (null for a single matrix), and the arguments.
// The descriptors change within a stage (the momentum pass sets src and m): each
// version has a slot of its own in the table, so that a later call with the same
// arguments finds all of them in place and need not upload (upload == 0).
constexpr int kXSync = 3;
struct XB {
  std::vector<XD> d;
  std::vector<const a8_apollo_x_args*> a;
  int64_t total[XW_N];
  XD* tab_dev;          // kXSync slots of n descriptors
  void* mema_dev;       // m_ema_table_bytes(n)
  void* vema_dev;       // v_ema_table_bytes(2 n)
  void* tail_dev;       // the larger of came_tail_table_bytes(n) and fact_tail_table_bytes(n)
  hipStream_t st;
  int tail_rs;          // a fused tail wrote the row sums of u_rowsums matrices
  int upload;           // copy the tables (0: an earlier call with the same arguments left them)
  int slot;             // the next descriptor slot
  const XD* cur;        // the current descriptor version
  const a8_step_scalars* dsc;   // device step block (the V weight), or null
};

static XT x_tab(const XB& b) {
  XT t{};
  if (b.tab_dev) {
    t.tab = b.cur;
    t.ntab = (int)b.d.size();
  } else {
    t.one = b.d[0];
  }
  t.dsc = b.dsc;
  return t;
}

template <int OP>
static int x_el(const XB& b) {
  hipLaunchKernelGGL((k_ax_el<OP>), dim3((unsigned)b.total[XW_EL]), dim3(256), 0, b.st, x_tab(b));
  return check_launch("k_ax_el");
}

// Row means into ws.rowm and column means into ws.colm of g_low^2 or the residual, plus add.
template <int SRC>
static int x_rowcol(const XB& b, float add) {
  const XT t = x_tab(b);
  hipLaunchKernelGGL((k_ax_rcpart<SRC>), dim3((unsigned)b.total[XW_CPART]), dim3(256), 0, b.st, t, add);
  int rc = check_launch("k_ax_rcpart");
  if (rc) return rc;
  if (b.total[XW_ROWS] > 0) {
    hipLaunchKernelGGL(k_ax_rowfin, dim3((unsigned)b.total[XW_ROWS]), dim3(256), 0, b.st, t, add);
    if ((rc = check_launch("k_ax_rowfin"))) return rc;
  }
  hipLaunchKernelGGL(k_ax_colfin, dim3((unsigned)b.total[XW_CFIN]), dim3(256), 0, b.st, t, add);
  return check_launch("k_ax_colfin");
}

template <int OP>
static int x_vec(const XB& b) {
  hipLaunchKernelGGL((k_ax_vec<OP>), dim3((unsigned)b.total[XW_VEC]), dim3(256), 0, b.st, x_tab(b));
  return check_launch("k_ax_vec");
}

template <int OP>
static int x_s(const XB& b) {
  hipLaunchKernelGGL((k_ax_s<OP>), dim3((unsigned)b.total[XW_ONE]), dim3(256), 0, b.st, x_tab(b));
  return check_launch("k_ax_s");
}

// Clip of U in dst (partials of the preceding U pass) and the division.
static int x_clip(const XB& b) {
  if (!(b.a[0]->d > 0.0f)) return 0;
  int rc = x_s<XS_CLIP>(b);
  if (rc) return rc;
  return x_el<XE_DIV>(b);
}

// Publishes the descriptors (first, and after a change of the per-matrix
// pointers) in the next slot.
static int x_sync(XB& b) {
  if (!b.tab_dev) return 0;
  if (b.slot >= kXSync) return set_error(A8_ERR_ARG, "low-rank stage: descriptor slots exhausted");
  XD* dst = b.tab_dev + (size_t)b.slot * b.d.size();
  ++b.slot;
  b.cur = dst;
  if (b.upload && upload_table(dst, b.d.data(), sizeof(XD) * b.d.size(), b.st) != hipSuccess)
    return set_error(A8_ERR_HIP, "table upload failed");
  return 0;
}

// Momentum EMA of x (ws region XU or g_low): fp32 state in place, or codes
// re-encoded with the lerped values in ws.xm.  Sets each k.m.
static int x_momentum(XB& b, bool from_u) {
  const a8_apollo_x_args* a0 = b.a[0];
  const size_t n = b.d.size();
  for (size_t i = 0; i < n; ++i) {
    XK& k = b.d[i].k;
    k.src = from_u ? k.ws + x_layout(k.R, k.C).xu : k.g;
    k.m = a0->m_fp32 ? b.a[i]->m_fp32 : k.ws + x_layout(k.R, k.C).xm;
  }
  int rc = x_sync(b);
  if (rc) return rc;
  if (a0->m_fp32) return x_el<XE_M32>(b);
  std::vector<MEmaItem> it(n);
  for (size_t i = 0; i < n; ++i) it[i] = MEmaItem{b.a[i]->m_q, b.a[i]->m_scale, b.d[i].k.src, b.d[i].k.m, b.d[i].k.n};
  return m_ema_multi(it.data(), (int)n, b.mema_dev, a0->beta1, a0->m_block_size, a0->m_bits, a0->m_mode, b.st,
                     b.upload);
}

static int x_stage(XB& b) {
  const a8_apollo_x_args* a0 = b.a[0];
  const size_t n = b.d.size();
  int rc;
  if (a0->factorize) {
    if ((rc = x_rowcol<XR_GSQ>(b, 1.17549435e-38f))) return rc;
    if ((rc = x_vec<XV_VAR>(b))) return rc;
    if (!a0->came) {
      if ((rc = x_s<XS_RMEAN>(b))) return rc;
      if (a0->has_m) {
        // momentum EMA and update in one pass (power-of-two M blocks, aligned streams)
        bool tail = a0->m_fp32 || (a0->m_block_size >= 32 && a0->m_block_size <= 2048 &&
                                   (a0->m_block_size & (a0->m_block_size - 1)) == 0);
        for (size_t i = 0; tail && i < n; ++i) {
          const a8_apollo_x_args* a = b.a[i];
          tail = aligned16(b.d[i].k.g) && aligned16(b.d[i].k.u) && (a->m_fp32 ? aligned16(a->m_fp32) : aligned16(a->m_q));
        }
        if (tail) {
          std::vector<FactTailItem> it(n);
          for (size_t i = 0; i < n; ++i) {
            const a8_apollo_x_args* a = b.a[i];
            const XK& k = b.d[i].k;
            it[i] = FactTailItem{k.g, a->m_q, a->m_scale, a->m_fp32, k.rv, k.cv, k.ws + x_layout(k.R, k.C).scal + 1,
                                 k.u, k.n, k.C, a->u_rowsums ? 1 : 0};
          }
          b.tail_rs = 1;
          return fact_tail_multi(it.data(), (int)n, b.tail_dev, a0->beta1, a0->apollo_eps, a0->m_fp32 != nullptr,
                                 a0->m_bits, a0->m_mode, a0->m_block_size, b.st, b.upload);
        }
        if ((rc = x_momentum(b, false))) return rc;
        for (auto& e : b.d) e.k.src = e.k.m;
      } else {
        for (auto& e : b.d) e.k.src = e.k.g;
      }
      if ((rc = x_sync(b))) return rc;
      return x_el<XE_FU>(b);
    }
    if ((rc = x_s<XS_RMEAN_CAME>(b))) return rc;
    if ((rc = x_el<XE_FCU>(b))) return rc;
    if ((rc = x_clip(b))) return rc;
    if ((rc = x_momentum(b, true))) return rc;
    if ((rc = x_el<XE_RES>(b))) return rc;
    if ((rc = x_rowcol<XR_RES>(b, 0.0f))) return rc;
    if (a0->c_bits) {
      std::vector<VEmaItem> it(2 * n);
      for (size_t i = 0; i < n; ++i) {
        const a8_apollo_x_args* a = b.a[i];
        const XK& k = b.d[i].k;
        const XL L = x_layout(k.R, k.C);
        it[2 * i] = VEmaItem{a->crow_q, a->crow_scale, a->crow_min_log, k.ws + L.rowm, k.ws + L.crow, nullptr, k.R};
        it[2 * i + 1] = VEmaItem{a->ccol_q, a->ccol_scale, a->ccol_min_log, k.ws + L.colm, k.ws + L.ccol, nullptr,
                                 k.C};
      }
      if ((rc = v_ema_multi(it.data(), (int)(2 * n), b.vema_dev, 1.0 - a0->beta3, a0->block_size, 0, 0.0f,
                            -126.0f, a0->c_bits, b.st, b.upload)))
        return rc;
    } else if ((rc = x_vec<XV_CONF>(b))) {
      return rc;
    }
    if ((rc = x_s<XS_CMEAN>(b))) return rc;
    return x_el<XE_FUC>(b);
  }
  // non-factorised CAME: low-rank V
  if (a0->v_bits) {
    std::vector<VEmaItem> it(n);
    for (size_t i = 0; i < n; ++i) {
      const a8_apollo_x_args* a = b.a[i];
      const XK& k = b.d[i].k;
      it[i] = a0->first_step ? VEmaItem{a->v_q, a->v_scale, a->v_min_log, k.v, nullptr, nullptr, k.n}
                             : VEmaItem{a->v_q, a->v_scale, a->v_min_log, k.g, k.v, nullptr, k.n};
    }
    if (a0->first_step) {
      if ((rc = x_el<XE_SQB>(b))) return rc;
      if ((rc = v_ema_multi(it.data(), (int)n, b.vema_dev, 1.0, a0->block_size, 0, 0.0f, -126.0f, a0->v_bits,
                            b.st, b.upload)))
        return rc;
    } else if ((rc = v_ema_multi(it.data(), (int)n, b.vema_dev, a0->beta_v, a0->block_size, 1, 0.0f, a0->log_floor,
                                 a0->v_bits, b.st, b.upload, b.dsc))) {
      return rc;
    }
  } else if ((rc = x_el<XE_V32>(b))) {
    return rc;
  }
  if (!a0->came) {   // plain: u from the momentum values (x_momentum sets k.m) or g_low
    if (a0->has_m && (rc = x_momentum(b, false))) return rc;
    return x_el<XE_AU>(b);
  }
  if ((rc = x_el<XE_U>(b))) return rc;
  // the fused tail takes power-of-two blocks and 16-byte aligned streams (its lanes
  // read eight elements at a time); other batches run the passes one by one
  bool tail = a0->has_m && came_tail_ok(a0->m_fp32 != nullptr, a0->m_block_size, a0->c_bits, a0->block_size);
  for (size_t i = 0; tail && i < n; ++i) {
    const a8_apollo_x_args* a = b.a[i];
    const XK& k = b.d[i].k;
    tail = aligned16(k.dst) && aligned16(k.u) && (a->m_fp32 ? aligned16(a->m_fp32) : aligned16(a->m_q)) &&
           (a->c_bits || aligned16(a->res_fp32));
  }
  if (tail) {
    // the clip factor, then one kernel for division, momentum, residual, its EMA and u
    if (a0->d > 0.0f && (rc = x_s<XS_CLIP>(b))) return rc;
    std::vector<CameTailItem> it(n);
    for (size_t i = 0; i < n; ++i) {
      const a8_apollo_x_args* a = b.a[i];
      const XK& k = b.d[i].k;
      it[i] = CameTailItem{k.dst, a->d > 0.0f ? k.ws + x_layout(k.R, k.C).scal : nullptr, a->m_q, a->m_scale,
                           a->m_fp32, a->res_q, a->res_scale, a->res_min_log, a->res_fp32, k.u, k.n, k.g,
                           a->u_rowsums ? k.C : 0};
    }
    b.tail_rs = 1;
    return came_tail_multi(it.data(), (int)n, b.tail_dev, a0->beta1, a0->beta3, a0->eps_came, a0->eps_sq,
                           a0->m_fp32 != nullptr, a0->m_bits, a0->m_mode, a0->m_block_size, a0->c_bits,
                           a0->block_size, b.st, b.upload);
  }
  if ((rc = x_clip(b))) return rc;
  if (!a0->has_m) return 0;   // unreachable through the optimizer (beta3 needs beta1): u = clipped U
  if ((rc = x_momentum(b, true))) return rc;
  if ((rc = x_el<XE_RES>(b))) return rc;
  if (a0->c_bits) {
    // the residual EMA is read back decoded after its re-encode (optimizer.py:2857-2866)
    std::vector<VEmaItem> it(n);
    for (size_t i = 0; i < n; ++i) {
      const a8_apollo_x_args* a = b.a[i];
      const XK& k = b.d[i].k;
      float* xr = k.ws + x_layout(k.R, k.C).xr;
      it[i] = VEmaItem{a->res_q, a->res_scale, a->res_min_log, xr, nullptr, xr, k.n};
    }
    char* vt = b.vema_dev ? static_cast<char*>(b.vema_dev) + v_ema_table_bytes((int)n) : nullptr;
    if ((rc = v_ema_multi(it.data(), (int)n, vt, 1.0 - a0->beta3, a0->block_size, 0, 0.0f, -126.0f, a0->c_bits,
                          b.st, b.upload)))
      return rc;
  }
  return x_el<XE_UCAME>(b);
}

// The stage's descriptor of one matrix.
static XK x_desc(const a8_apollo_x_args* a) {
  const int64_t R = a->rows_low, C = a->cols_low;
  const XL L = x_layout(R, C);
  XK k{};
  k.g = a->g_low; k.u = a->u; k.ws = a->xws;
  k.R = R; k.C = C; k.n = L.n;
  k.bv = (float)a->beta_v; k.omb = (float)(1.0 - a->beta_v);
  k.w1 = (float)(1.0 - a->beta1); k.w3 = (float)(1.0 - a->beta3);
  k.aeps = a->apollo_eps; k.eps_sq = a->eps_sq; k.eps_came = a->eps_came; k.d = a->d;
  k.sqn = (float)sqrt((double)L.n);
  k.first = a->first_step ? 1 : 0;
  k.np = (int)x_grid(L.n);
  k.dst = a->xws + L.xu;
  if (a->factorize) {
    k.rv = a->row_var; k.cv = a->col_var;
    if (a->came) {
      k.cr = a->c_bits ? a->xws + L.crow : a->crow_fp32;
      k.cc = a->c_bits ? a->xws + L.ccol : a->ccol_fp32;
    }
  } else {
    k.v = a->v_bits ? a->xws + L.xv : a->v_fp32;
    k.res = a->c_bits ? nullptr : a->res_fp32;
    if (!a->has_m) k.dst = a->u;
  }
  const void* streams[] = {a->g_low, a->u, a->v_fp32, a->m_fp32, a->res_fp32};
  bool al = (L.n & 3) == 0;
  for (const void* p : streams) al = al && aligned16(p);   // aligned16(nullptr) holds
  k.v4 = al ? 1 : 0;
  return k;
}

static int x_check(const a8_apollo_x_args* a) {
  if (!a) return set_error(A8_ERR_ARG, "null pointer");
  if (a->rows_low <= 0 || a->cols_low <= 0) return set_error(A8_ERR_SIZE, "empty low-rank matrix");
  if (a->rows_low * a->cols_low >= ((int64_t)1 << 31)) return set_error(A8_ERR_SIZE, "low-rank matrix too large");
  if (!a->g_low || !a->u || !a->xws) return set_error(A8_ERR_ARG, "null g_low, u or workspace");
  if (!aligned16(a->xws)) return set_error(A8_ERR_ALIGN, "workspace must be 16-byte aligned");
  if (a->came && !a->has_m) return set_error(A8_ERR_ARG, "CAME (beta3) requires momentum (beta1)");
  if (a->u_rowsums && !rowsum_len_ok(a->cols_low))
    return set_error(A8_ERR_SIZE, "u_rowsums: cols_low must be a power of two in [8, 512]");
  const bool v_coded = !a->factorize && a->v_bits;
  const bool c_coded = a->came && a->c_bits;
  if ((v_coded || c_coded) && !(a->block_size >= 128 && a->block_size <= (1 << 30) && a->block_size % 128 == 0))
    return set_error(A8_ERR_BLOCK, "block_size must be a multiple of 128 in [128, 2^30]");
  if ((v_coded && a->v_bits != 8 && a->v_bits != 16) || (c_coded && a->c_bits != 8 && a->c_bits != 16))
    return set_error(A8_ERR_ARG, "v_bits / c_bits must be 0, 8 or 16");
  if (a->has_m) {
    if (a->m_fp32 == nullptr) {
      if (!a->m_q || !a->m_scale) return set_error(A8_ERR_ARG, "momentum state missing");
      if (!(a->m_block_size >= 32 && a->m_block_size <= (1 << 30) && a->m_block_size % 4 == 0))
        return set_error(A8_ERR_BLOCK, "m_block_size must be a multiple of 4 in [32, 2^30]");
    }
  }
  if (a->factorize) {
    if (!a->row_var || !a->col_var) return set_error(A8_ERR_ARG, "factorised row / column state missing");
    if (a->came && (a->c_bits ? !(a->crow_q && a->crow_scale && a->crow_min_log && a->ccol_q && a->ccol_scale &&
                                  a->ccol_min_log)
                              : !(a->crow_fp32 && a->ccol_fp32)))
      return set_error(A8_ERR_ARG, "confidence state missing");
  } else {
    if (a->v_bits ? !(a->v_q && a->v_scale && a->v_min_log) : !a->v_fp32)
      return set_error(A8_ERR_ARG, "low-rank V state missing");
    if (a->came && (a->c_bits ? !(a->res_q && a->res_scale && a->res_min_log) : !a->res_fp32))
      return set_error(A8_ERR_ARG, "residual state missing");
  }
  return 0;
}

// The stage, then the row sums of u^2 and g_low^2 of the u_rowsums matrices
// where no fused tail left them: summed from u into the workspace's V region
// (free once the stage is done) and copied over u.
static int x_run(XB& b) {
  b.tail_rs = 0;
  int rc = x_stage(b);
  if (rc || b.tail_rs) return rc;
  for (size_t i = 0; i < b.a.size(); ++i) {
    const a8_apollo_x_args* a = b.a[i];
    if (!a->u_rowsums) continue;
    const XK& k = b.d[i].k;
    double* tmp = reinterpret_cast<double*>(k.ws + x_layout(k.R, k.C).xv);
    if ((rc = rowsum_sq(a->u, a->g_low, k.n, k.C, tmp, b.st))) return rc;
    if (hipMemcpyAsync(a->u, tmp, sizeof(double) * 2 * (size_t)k.R, hipMemcpyDeviceToDevice, b.st) != hipSuccess)
      return set_error(A8_ERR_HIP, "row sums: copy failed");
  }
  return 0;
}

// Two matrices can share the stage's launches when every flag and
// hyper-parameter agrees.
static bool x_same(const a8_apollo_x_args* a, const a8_apollo_x_args* b) {
  return a->factorize == b->factorize && a->came == b->came && a->has_m == b->has_m &&
         a->first_step == b->first_step && (a->factorize || a->v_bits == b->v_bits) &&
         a->block_size == b->block_size && (a->m_fp32 == nullptr) == (b->m_fp32 == nullptr) &&
         a->m_bits == b->m_bits && a->m_mode == b->m_mode && a->m_block_size == b->m_block_size &&
         a->c_bits == b->c_bits && a->beta_v == b->beta_v && a->beta1 == b->beta1 && a->beta3 == b->beta3 &&
         a->apollo_eps == b->apollo_eps && a->eps_sq == b->eps_sq && a->log_floor == b->log_floor &&
         a->eps_came == b->eps_came && a->d == b->d;
}

// Table bytes of one batch of n matrices: descriptors, momentum and AL tables.
static int64_t x_round(int64_t b) { return (b + 255) / 256 * 256; }
static int64_t x_bytes(int n) {
  const int64_t tail = came_tail_table_bytes(n) > fact_tail_table_bytes(n) ? came_tail_table_bytes(n)
                                                                           : fact_tail_table_bytes(n);
  return kXSync * x_round((int64_t)sizeof(XD) * n) + x_round(m_ema_table_bytes(n)) +
         x_round(v_ema_table_bytes(2 * n)) + x_round(tail);
}

}  // namespace a8

using namespace a8;

extern "C" {

int64_t a8_apollo_x_workspace_floats(int64_t rows_low, int64_t cols_low) {
  if (rows_low <= 0 || cols_low <= 0) return 0;
  return x_layout(rows_low, cols_low).total;
}

int64_t a8_apollo_x_table_bytes(int nmat) { return nmat > 0 ? x_bytes(nmat) : 0; }

int a8_apollo_lowrank_x(const a8_apollo_x_args* a, void* stream) {
  int rc = x_check(a);
  if (rc) return rc;
  XB b{};
  b.d.resize(1);
  b.a.push_back(a);
  b.d[0].k = x_desc(a);
  x_counts(b.d[0].k, b.total);
  b.st = (hipStream_t)stream;
  b.upload = 1;
  return x_run(b);
}

int a8_apollo_lowrank_x_multi(const a8_apollo_x_args* args, int nmat, void* table_dev, int64_t table_bytes,
                              int upload, const void* step_scalars, void* stream) {
  if (nmat <= 0) return 0;
  if (!args) return set_error(A8_ERR_ARG, "null pointer");
  if (!table_dev || table_bytes < x_bytes(nmat))
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_apollo_x_table_bytes(nmat)");
  if (upload) {
    // a captured copy would replay from the library's host staging as it is at
    // replay time: the tables are uploaded by an eager call, and a captured one
    // passes upload == 0
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess)
      return set_error(A8_ERR_HIP, "hipStreamIsCapturing failed");
    if (cs != hipStreamCaptureStatusNone)
      return set_error(A8_ERR_ARG, "a8_apollo_lowrank_x_multi: upload != 0 on a capturing stream");
  }
  for (int i = 0; i < nmat; ++i) {
    const int rc = x_check(args + i);
    if (rc) return rc;
  }
  // batches of matrices that agree on every flag, in order of first appearance;
  // each takes its own slice of the table
  std::vector<int> batch_of((size_t)nmat, -1);
  char* base = static_cast<char*>(table_dev);
  for (int i = 0; i < nmat; ++i) {
    if (batch_of[(size_t)i] >= 0) continue;
    XB b{};
    b.st = (hipStream_t)stream;
    b.upload = upload ? 1 : 0;
    b.dsc = reinterpret_cast<const a8_step_scalars*>(step_scalars);
    for (int j = i; j < nmat; ++j) {
      if (batch_of[(size_t)j] >= 0 || !x_same(args + i, args + j)) continue;
      batch_of[(size_t)j] = i;
      b.a.push_back(args + j);
    }
    const int n = (int)b.a.size();
    b.d.resize((size_t)n);
    for (int e = 0; e < XW_N; ++e) b.total[e] = 0;
    for (int j = 0; j < n; ++j) {
      b.d[(size_t)j].k = x_desc(b.a[(size_t)j]);
      int64_t cnt[XW_N];
      x_counts(b.d[(size_t)j].k, cnt);
      for (int e = 0; e < XW_N; ++e) {
        b.d[(size_t)j].wb[e] = b.total[e];
        b.total[e] += cnt[e];
      }
    }
    for (int e = 0; e < XW_N; ++e)
      if (b.total[e] > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "low-rank batch too large");
    b.tab_dev = reinterpret_cast<XD*>(base);
    b.mema_dev = base + kXSync * x_round((int64_t)sizeof(XD) * n);
    b.vema_dev = static_cast<char*>(b.mema_dev) + x_round(m_ema_table_bytes(n));
    b.tail_dev = static_cast<char*>(b.vema_dev) + x_round(v_ema_table_bytes(2 * n));
    base += x_bytes(n);
    int rc = x_sync(b);
    if (rc) return rc;
    if ((rc = x_run(b))) return rc;
  }
  return 0;
}

}  // extern "C"
