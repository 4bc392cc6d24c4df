// APOLLO low-rank stage of the factorised and CAME variants, one matrix per call.
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

// Extended workspace of one matrix (offsets in floats; part / cpart hold doubles).
struct XL {
  int64_t n, nch, xv, xu, xm, xr, rowm, colm, crow, ccol, scal, part, cpart, total;
};

__host__ __device__ inline XL x_layout(int64_t R, int64_t C) {
  XL w;
  w.n = R * C;
  w.nch = (R + kXRowChunk - 1) / kXRowChunk;
  w.xv = 0;                    // V values of coded V (the lerped values)
  w.xu = w.xv + w.n;           // U (CAME)
  w.xm = w.xu + w.n;           // momentum values of coded M
  w.xr = w.xm + w.n;           // residual, then its decoded EMA
  w.rowm = w.xr + w.n;         // row means
  w.colm = w.rowm + R;         // column means
  w.crow = w.colm + C;         // confidence values of coded confidence
  w.ccol = w.crow + R;
  w.scal = w.ccol + C;         // [0] clip, [1] row-variance mean (clamped), [2] confidence row mean
  w.part = (w.scal + 16 + 1) / 2 * 2;
  w.cpart = w.part + 2 * kXParts;
  w.total = w.cpart + 2 * w.nch * C;
  return w;
}

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
};

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
  XE_FUC        // u = (m / sqrt(cr_i / cmean)) / sqrt(cc_j)
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

template <int OP>
__global__ __launch_bounds__(256) void k_ax_el(XK k) {
  __shared__ double sd[4];
  float* ws = k.ws;
  const XL L = x_layout(k.R, k.C);
  const float clip = (OP == XE_DIV) ? gp(ws)[L.scal] : 1.0f;
  double acc = 0.0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < k.n; i += stride) {
    if constexpr (OP == XE_SQB) {
      const float g = gp(k.g)[i];
      gp(ws)[L.xv + i] = (g * g) * k.bv;
    } else if constexpr (OP == XE_V32) {
      const float g = gp(k.g)[i];
      const float g2 = g * g;
      gp(k.v)[i] = k.first ? g2 * k.bv : lerp_ref(gp(k.v)[i], g2, k.bv);
    } else if constexpr (OP == XE_U) {
      const float x = gp(k.g)[i] * rsqrt_ref(fmaxf(gp(k.v)[i], k.eps_sq));
      gp(k.dst)[i] = x;
      acc += (double)(x * x);
    } else if constexpr (OP == XE_FCU) {
      const int64_t r = i / k.C, c = i - r * k.C;
      const float ir = rsqrt_ref(gp(k.rv)[r] / gp(ws)[L.scal + 1]);
      const float ic = rsqrt_ref(gp(k.cv)[c]);
      const float x = (gp(k.g)[i] * ir) * ic;
      gp(k.dst)[i] = x;
      acc += (double)(x * x);
    } else if constexpr (OP == XE_DIV) {
      gp(k.dst)[i] = gp(k.dst)[i] / clip;
    } else if constexpr (OP == XE_M32) {
      gp(k.m)[i] = lerp_ref(gp(k.m)[i], gp(k.src)[i], k.w1);
    } else if constexpr (OP == XE_RES) {
      float r = gp(ws)[L.xu + i] - gp(k.m)[i];
      r = r * r;
      r = r + k.eps_came;
      gp(ws)[L.xr + i] = r;
      if (k.res) gp(k.res)[i] = lerp_ref(gp(k.res)[i], r, k.w3);
    } else if constexpr (OP == XE_UCAME) {
      const float rd = k.res ? gp(k.res)[i] : gp(ws)[L.xr + i];
      gp(k.u)[i] = gp(k.m)[i] * rsqrt_ref(fmaxf(rd, k.eps_sq));
    } else if constexpr (OP == XE_FU) {
      const int64_t r = i / k.C, c = i - r * k.C;
      const float ve = (gp(k.rv)[r] * gp(k.cv)[c]) / gp(ws)[L.scal + 1];
      gp(k.u)[i] = gp(k.src)[i] / (sqrtf(ve) + k.aeps);
    } else {   // XE_FUC
      const int64_t r = i / k.C, c = i - r * k.C;
      const float icr = rsqrt_ref(gp(k.cr)[r] / gp(ws)[L.scal + 2]);
      const float icc = rsqrt_ref(gp(k.cc)[c]);
      gp(k.u)[i] = (gp(k.m)[i] * icr) * icc;
    }
  }
  if constexpr (OP == XE_U || OP == XE_FCU) {
    const double t = x_wg_sum(acc, sd);
    if (threadIdx.x == 0) reinterpret_cast<A8_G double*>(gp(ws) + L.part)[blockIdx.x] = t;
  }
}

// Row means of x (or x^2): one wave per row, 4 rows per workgroup.
__global__ __launch_bounds__(256) void k_ax_rows(const float* __restrict__ x, int sq, int64_t R, int64_t C,
                                                 float* __restrict__ out, float add) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  if (row >= R) return;
  double s = 0.0;
  for (int64_t j = l; j < C; j += 64) {
    const float v = gp(x)[row * C + j];
    s += (double)(sq ? v * v : v);
  }
  s = grp_sum_d(s, 64);
  if (l == 0) gp(out)[row] = (float)s / (float)C + add;
}

// Column sums of x (or x^2) over a chunk of kXRowChunk rows: 64 columns per
// workgroup, the four waves striding the chunk's rows, combined in order.
__global__ __launch_bounds__(256) void k_ax_colpart(const float* __restrict__ x, int sq, int64_t R, int64_t C,
                                                    double* __restrict__ part) {
  __shared__ double sd[256];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t c = (int64_t)blockIdx.x * 64 + l;
  const int64_t r0 = (int64_t)blockIdx.y * kXRowChunk;
  const int64_t r1 = r0 + kXRowChunk < R ? r0 + kXRowChunk : R;
  double s = 0.0;
  if (c < C) {
    for (int64_t r = r0 + w; r < r1; r += 4) {
      const float v = gp(x)[r * C + c];
      s += (double)(sq ? v * v : v);
    }
  }
  sd[threadIdx.x] = s;
  __syncthreads();
  if (w == 0 && c < C) gp(part)[(int64_t)blockIdx.y * C + c] = ((sd[l] + sd[64 + l]) + sd[128 + l]) + sd[192 + l];
}

__global__ __launch_bounds__(256) void k_ax_colfin(const double* __restrict__ part, int64_t nch, int64_t R,
                                                   int64_t C, float* __restrict__ out, float add) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  double s = 0.0;
  for (int64_t h = 0; h < nch; ++h) s += gp(part)[h * C + c];
  gp(out)[c] = (float)s / (float)R + add;
}

enum { XV_VAR = 0, XV_CONF };

// Row (index < R) and column (index >= R) vectors of the factorised EMAs.
template <int OP>
__global__ __launch_bounds__(256) void k_ax_vec(XK k) {
  const XL L = x_layout(k.R, k.C);
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= k.R + k.C) return;
  const bool row = j < k.R;
  const int64_t t = row ? j : j - k.R;
  const float mean = gp(k.ws)[(row ? L.rowm : L.colm) + t];
  if constexpr (OP == XV_VAR) {
    float* s = row ? k.rv : k.cv;
    gp(s)[t] = k.first ? mean * k.bv : __builtin_fmaf(k.bv, mean, gp(s)[t] * k.omb);
  } else {
    float* s = row ? k.cr : k.cc;
    gp(s)[t] = lerp_ref(gp(s)[t], mean, k.w3);
  }
}

enum { XS_CLIP = 0, XS_RMEAN, XS_RMEAN_CAME, XS_CMEAN };

// One workgroup: the scalars between passes.
template <int OP>
__global__ __launch_bounds__(256) void k_ax_s(XK k) {
  __shared__ double sd[4];
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

static unsigned x_grid(int64_t n) {
  const int64_t nb = (n + 255) / 256;
  return (unsigned)(nb < kXParts ? (nb > 0 ? nb : 1) : kXParts);
}

template <int OP>
static int x_el(const XK& k, hipStream_t st) {
  hipLaunchKernelGGL((k_ax_el<OP>), dim3(x_grid(k.n)), dim3(256), 0, st, k);
  return check_launch("k_ax_el");
}

// Row means into ws.rowm and column means into ws.colm of x (or x^2), plus add.
static int x_rowcol(const XK& k, const float* x, int sq, float add, hipStream_t st) {
  const XL L = x_layout(k.R, k.C);
  hipLaunchKernelGGL(k_ax_rows, dim3((unsigned)((k.R + 3) / 4)), dim3(256), 0, st, x, sq, k.R, k.C, k.ws + L.rowm,
                     add);
  int rc = check_launch("k_ax_rows");
  if (rc) return rc;
  double* cpart = reinterpret_cast<double*>(k.ws + L.cpart);
  hipLaunchKernelGGL(k_ax_colpart, dim3((unsigned)((k.C + 63) / 64), (unsigned)L.nch), dim3(256), 0, st, x, sq, k.R,
                     k.C, cpart);
  if ((rc = check_launch("k_ax_colpart"))) return rc;
  hipLaunchKernelGGL(k_ax_colfin, dim3((unsigned)((k.C + 255) / 256)), dim3(256), 0, st, cpart, L.nch, k.R, k.C,
                     k.ws + L.colm, add);
  return check_launch("k_ax_colfin");
}

template <int OP>
static int x_vec(const XK& k, hipStream_t st) {
  hipLaunchKernelGGL((k_ax_vec<OP>), dim3((unsigned)((k.R + k.C + 255) / 256)), dim3(256), 0, st, k);
  return check_launch("k_ax_vec");
}

template <int OP>
static int x_s(const XK& k, hipStream_t st) {
  hipLaunchKernelGGL((k_ax_s<OP>), dim3(1), dim3(256), 0, st, k);
  return check_launch("k_ax_s");
}

// Clip of U in dst (partials of the preceding U pass) and the division.
static int x_clip(XK& k, hipStream_t st) {
  if (!(k.d > 0.0f)) return 0;
  k.np = (int)x_grid(k.n);
  int rc = x_s<XS_CLIP>(k, st);
  if (rc) return rc;
  return x_el<XE_DIV>(k, st);
}

// Momentum EMA of x (n values): fp32 state in place, or codes re-encoded with the
// lerped values in ws.xm.  Sets k.m.
static int x_momentum(XK& k, const a8_apollo_x_args* a, const float* x, hipStream_t st) {
  const XL L = x_layout(k.R, k.C);
  if (a->m_fp32) {
    k.m = a->m_fp32;
    k.src = x;
    return x_el<XE_M32>(k, st);
  }
  k.m = k.ws + L.xm;
  return a8_m_quantize_lerp(a->m_q, a->m_scale, x, A8_F32, k.m, a->beta1, a->m_block_size, k.n, a->m_bits,
                            a->m_mode, st);
}

static int x_run(const a8_apollo_x_args* a, hipStream_t st) {
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
  int rc;
  if (a->factorize) {
    k.rv = a->row_var; k.cv = a->col_var;
    if ((rc = x_rowcol(k, a->g_low, 1, 1.17549435e-38f, st))) return rc;
    if ((rc = x_vec<XV_VAR>(k, st))) return rc;
    if (!a->came) {
      if ((rc = x_s<XS_RMEAN>(k, st))) return rc;
      k.src = a->g_low;
      if (a->has_m) {
        if ((rc = x_momentum(k, a, a->g_low, st))) return rc;
        k.src = k.m;
      }
      return x_el<XE_FU>(k, st);
    }
    if ((rc = x_s<XS_RMEAN_CAME>(k, st))) return rc;
    k.dst = k.ws + L.xu;
    if ((rc = x_el<XE_FCU>(k, st))) return rc;
    if ((rc = x_clip(k, st))) return rc;
    if ((rc = x_momentum(k, a, k.ws + L.xu, st))) return rc;
    k.res = nullptr;
    if ((rc = x_el<XE_RES>(k, st))) return rc;
    if ((rc = x_rowcol(k, k.ws + L.xr, 0, 0.0f, st))) return rc;
    if (a->c_bits) {
      if ((rc = a8_log_quantize_lerp(a->crow_q, a->crow_scale, a->crow_min_log, k.ws + L.rowm, A8_F32, k.ws + L.crow,
                                     1.0 - a->beta3, a->block_size, 0, 0.0f, R, -126.0f, a->c_bits, st)))
        return rc;
      if ((rc = a8_log_quantize_lerp(a->ccol_q, a->ccol_scale, a->ccol_min_log, k.ws + L.colm, A8_F32, k.ws + L.ccol,
                                     1.0 - a->beta3, a->block_size, 0, 0.0f, C, -126.0f, a->c_bits, st)))
        return rc;
      k.cr = k.ws + L.crow; k.cc = k.ws + L.ccol;
    } else {
      k.cr = a->crow_fp32; k.cc = a->ccol_fp32;
      if ((rc = x_vec<XV_CONF>(k, st))) return rc;
    }
    if ((rc = x_s<XS_CMEAN>(k, st))) return rc;
    return x_el<XE_FUC>(k, st);
  }
  // non-factorised CAME: low-rank V
  if (a->v_bits) {
    k.v = k.ws + L.xv;
    if (a->first_step) {
      if ((rc = x_el<XE_SQB>(k, st))) return rc;
      if ((rc = a8_log_quantize_lerp(a->v_q, a->v_scale, a->v_min_log, k.v, A8_F32, nullptr, 1.0, a->block_size, 0,
                                     0.0f, L.n, -126.0f, a->v_bits, st)))
        return rc;
    } else if ((rc = a8_log_quantize_lerp(a->v_q, a->v_scale, a->v_min_log, a->g_low, A8_F32, k.v, a->beta_v,
                                          a->block_size, 1, 0.0f, L.n, a->log_floor, a->v_bits, st))) {
      return rc;
    }
  } else {
    k.v = a->v_fp32;
    if ((rc = x_el<XE_V32>(k, st))) return rc;
  }
  if (!a->has_m) {   // unreachable through the optimizer (beta3 needs beta1); u = clipped U
    k.dst = a->u;
    if ((rc = x_el<XE_U>(k, st))) return rc;
    return x_clip(k, st);
  }
  k.dst = k.ws + L.xu;
  if ((rc = x_el<XE_U>(k, st))) return rc;
  if ((rc = x_clip(k, st))) return rc;
  if ((rc = x_momentum(k, a, k.ws + L.xu, st))) return rc;
  k.res = a->c_bits ? nullptr : a->res_fp32;
  if ((rc = x_el<XE_RES>(k, st))) return rc;
  if (a->c_bits) {
    if ((rc = a8_log_quantize_lerp(a->res_q, a->res_scale, a->res_min_log, k.ws + L.xr, A8_F32, nullptr,
                                   1.0 - a->beta3, a->block_size, 0, 0.0f, L.n, -126.0f, a->c_bits, st)))
      return rc;
    if ((rc = a8_dequantize_log_nonneg(k.ws + L.xr, a->res_q, a->res_scale, a->res_min_log, L.n, a->block_size,
                                       a->c_bits, st)))
      return rc;
  }
  return x_el<XE_UCAME>(k, st);
}

}  // namespace a8

using namespace a8;

extern "C" {

int64_t a8_apollo_x_workspace_floats(int64_t rows_low, int64_t cols_low) {
  if (rows_low <= 0 || cols_low <= 0) return 0;
  return x_layout(rows_low, cols_low).total;
}

int a8_apollo_lowrank_x(const a8_apollo_x_args* a, void* stream) {
  if (!a) return set_error(A8_ERR_ARG, "null pointer");
  if (a->rows_low <= 0 || a->cols_low <= 0) return set_error(A8_ERR_SIZE, "empty low-rank matrix");
  if (a->rows_low * a->cols_low >= ((int64_t)1 << 31)) return set_error(A8_ERR_SIZE, "low-rank matrix too large");
  if (!a->g_low || !a->u || !a->xws) return set_error(A8_ERR_ARG, "null g_low, u or workspace");
  if (!aligned16(a->xws)) return set_error(A8_ERR_ALIGN, "workspace must be 16-byte aligned");
  if (!a->factorize && !a->came)
    return set_error(A8_ERR_ARG, "plain APOLLO runs in a8_apollo_step; this entry is factorised or CAME");
  if (a->came && !a->has_m) return set_error(A8_ERR_ARG, "CAME (beta3) requires momentum (beta1)");
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  const bool v_coded = !a->factorize && a->v_bits;
  const bool c_coded = a->came && a->c_bits;
  if ((v_coded || c_coded) && !(pow2(a->block_size) && a->block_size >= 128 && a->block_size <= 2048))
    return set_error(A8_ERR_BLOCK, "block_size must be a power of two in [128, 2048]");
  if ((v_coded && a->v_bits != 8 && a->v_bits != 16) || (c_coded && a->c_bits != 8 && a->c_bits != 16))
    return set_error(A8_ERR_ARG, "v_bits / c_bits must be 0, 8 or 16");
  if (a->has_m) {
    if (a->m_fp32 == nullptr) {
      if (!a->m_q || !a->m_scale) return set_error(A8_ERR_ARG, "momentum state missing");
      if (!(pow2(a->m_block_size) && a->m_block_size >= 32 && a->m_block_size <= 2048))
        return set_error(A8_ERR_BLOCK, "m_block_size must be a power of two in [32, 2048]");
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
  return x_run(a, (hipStream_t)stream);
}

}  // extern "C"
