// Full-precision (fp32 V, optional fp32 M) 1-D step and the Fira scalar.
//
// Tensors below min_8bit_size keep fp32 state (optimizer.py:1640-1641); the
// reference steps them with fused_update_1d_full_kernel (kernels.cu:1261-1372)
// on the GPU and with mul_/addcmul_/lerp_ (optimizer.py:2186-2191, 886-917) on
// the CPU.  This kernel follows the CPU arithmetic:
//   v = fma(RN(bv*g), g, RN(v*(1-bv))) [+ bv*eps_g],  m = lerp(m, x, 1-beta1)
// Element-wise, 8 elements per lane, tensor-table capable like the
// quantised kernel.  Fira (kernels.cu:3030-3053, optimizer.py:760-782) is a
// one-lane-per-tensor scalar kernel.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

struct DescFull {
  void* param;
  const void* grad;
  float* v;
  float* m;
  float* norm_buf;
  const float* alpha;
  const float* prev_norm;
  const float* decay;
  int64_t numel;
  int64_t wg_begin;
  uint64_t sr_seed;
  float* psq;               // sum of p^2 (NORM pass with scale_param), read by the update passes
  const float* fira_scale;  // Fira limiter scale multiplied into the step, or null
  double* norm_part;        // NORM / LAG / MNORM: partial sums of u^2 (then of p^2), one per workgroup
};

struct HyperFull {
  float w_m;        // (float)(1 - beta1)
  float bv;         // (float)beta_val
  float v_keep;     // (float)(1 - beta_val)
  float eps_add;    // (float)(beta_val * eps_g), added when eps_g > 0
  float eps_d;
  float eps_sq;
  float d;
  int has_eps_add;
  int adam_denom;
  int momentum_only;
  float alpha_val;
  float decay_val;
  int has_decay;
  uint64_t sr_step;
  int scale_param;  // alpha = max(rms(p), eps2) * rho with rms from *psq (optimizer.py:851-855)
  float eps2;
  int wd_mode;      // 0: none here, 1: p *= 1 - alpha*wd, 2: p *= 1 - rho*wd (optimizer.py:2032-2039)
  float wd;
  int v_ready;      // V holds this step's second moment already (no EMA, not written)
  float eps_g;      // added to g^2 (times beta_val)
  const a8_step_scalars* dsc;   // if set: this step's beta_val, eps_d, alpha, decay and SR step
};

constexpr int kFLanes = 256;
constexpr int kFElems = kFLanes * 8;

// The tensor table is uniform per workgroup and read-only during the launch:
// it is read through the scalar cache (constant address space), the search
// probing each descriptor's wg_begin, the descriptor landing in SGPRs.
__device__ __forceinline__ DescFull load_full(const DescFull* tab, int n, int64_t wg) {
  const A8_C DescFull* ct = cp(tab);
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (ct[mid].wg_begin <= wg) lo = mid; else hi = mid - 1;
  }
  static_assert(sizeof(DescFull) % 8 == 0, "descriptor is loaded as 64-bit words");
  const A8_C uint64_t* w = (const A8_C uint64_t*)(ct + lo);
  uint64_t buf[sizeof(DescFull) / 8];
#pragma unroll
  for (int i = 0; i < (int)(sizeof(DescFull) / 8); ++i) buf[i] = w[i];
  DescFull d;
  __builtin_memcpy(&d, buf, sizeof(DescFull));
  return d;
}

// MODE: 0 single pass, 1 NORM (writes V, sums u^2 or U^2), 2 APPLY (reads V,
// writes M and p), 3 LAG, 4 MNORM (momentum-only: reads V, clips U by the NORM
// pass's sum of U^2 in prev_norm and sums M'^2 for Fira; writes nothing).
// SR: the parameter write is p * decay - step * u in fp32, stochastically
// rounded to T with the stream of kernels.cu:48-87 (write_param_update,
// kernels.cu:149-161), element index within the tensor.
template <typename T, int MODE, bool SR>
__global__ __launch_bounds__(kFLanes) void k_update1d_full(DescFull one, const DescFull* __restrict__ table,
                                                         int ntab, HyperFull h) {
  if (h.dsc) {   // the derived fields as make_hf forms them from beta_val
    const a8_step_scalars sc = load_step_scalars(h.dsc);
    h.bv = (float)sc.beta_val;
    h.v_keep = (float)(1.0 - sc.beta_val);
    h.eps_add = (float)(sc.beta_val * (double)h.eps_g);
    h.eps_d = sc.eps_d;
    h.alpha_val = sc.alpha;
    h.decay_val = sc.decay;
    h.sr_step = sc.step;
  }
  const DescFull D = table ? load_full(table, ntab, (int64_t)blockIdx.x) : one;
  const int64_t wl = (int64_t)blockIdx.x - D.wg_begin;
  const int lane = threadIdx.x;
  const int64_t n = D.numel;
  const int64_t e0 = wl * kFElems + (int64_t)lane * 8;
  float sq = 0.0f, psum = 0.0f;
  float step = 0.0f, ut_clip = 1.0f, wdec = 1.0f;
  if constexpr (MODE != 1) {
    float a = D.alpha ? *D.alpha : h.alpha_val;   // rho when scale_param
    const float rho = a;
    if (h.scale_param) a = fmaxf(sqrtf(*D.psq) / (float)sqrt((double)n), h.eps2) * a;
    if (h.wd_mode == 1) wdec = 1.0f - a * h.wd;
    else if (h.wd_mode == 2) wdec = 1.0f - rho * h.wd;
    if (D.fira_scale) a = a * *D.fira_scale;
    if constexpr (MODE == 0) {
      step = a;
    } else {
      float denom = 1.0f;
      if (h.d > 0.0f) {
        const float nrm = (MODE == 2) ? sqrtf(*D.norm_buf)
                          : (MODE == 4 ? sqrtf(*D.prev_norm) : *D.prev_norm);
        // U-clip of momentum_only divides by sqrt(n) then d (optimizer.py:894-895);
        // the update clip divides by sqrt(n)*d (optimizer.py:859-863)
        if (MODE == 3)   // LAG has no CPU branch: the CUDA kernels' pn / (sqrtf(numel) * d) in fp32 (kernels.cu:651-655)
          denom = fmaxf(1.0f, nrm / (sqrtf((float)n) * h.d));
        else if (h.momentum_only && D.m)
          denom = fmaxf(1.0f, (nrm / (float)sqrt((double)n)) / h.d);
        else
          denom = fmaxf(1.0f, nrm / (float)(sqrt((double)n) * (double)h.d));
      }
      if (h.momentum_only && D.m) { step = a; ut_clip = denom; }
      else { step = a / denom; }
    }
  }
  if (e0 < n) {
    const int cnt = (n - e0) < 8 ? (int)(n - e0) : 8;
    const T* G = reinterpret_cast<const T*>(D.grad);
    T* P = reinterpret_cast<T*>(D.param);
    // every input of the lane's elements is loaded before any store: the stores
    // could alias the loads as far as the compiler knows, so loads interleaved
    // with them would run one memory round trip per element
    constexpr bool kNeedP = MODE != 1 && MODE != 4;
    T graw[8], praw[8];
    float vin[8], min_[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k < cnt) {
        const int64_t i = e0 + k;
        graw[k] = G[i];
        if (kNeedP || (MODE == 1 && h.scale_param)) praw[k] = P[i];
        vin[k] = D.v[i];
        if (D.m) min_[k] = D.m[i];
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k >= cnt) break;
      const int64_t i = e0 + k;
      const float g = scrub(to_f<T>(graw[k]));
      if (MODE == 1 && h.scale_param) {
        const float pv = to_f<T>(praw[k]);
        psum += pv * pv;
      }
      float v;
      if (MODE == 2 || MODE == 4 || h.v_ready) {
        v = vin[k];
      } else {
        v = __builtin_fmaf(h.bv * g, g, vin[k] * h.v_keep);
        if (h.has_eps_add) v = v + h.eps_add;
        D.v[i] = v;
      }
      float inv = h.adam_denom ? 1.0f / (sqrtf(v) + h.eps_d) : 1.0f / sqrtf(fmaxf(v, h.eps_sq));
      float u;
      if (D.m) {
        float mo = min_[k];
        if (h.momentum_only) {
          const float ut = g * inv;
          if (MODE == 1 || MODE == 3) sq += ut * ut;
          if (MODE != 1) {
            const float m = lerp_ref(mo, ut_clip != 1.0f ? ut / ut_clip : ut, h.w_m);
            if (MODE == 4) sq += m * m;
            else D.m[i] = m;
            u = m;
          } else {
            u = ut;
          }
        } else {
          float m;
          if (MODE == 2) {
            m = mo;  // written by the NORM pass
          } else {
            m = lerp_ref(mo, g, h.w_m);
            D.m[i] = m;
          }
          u = m * inv;
          if (MODE == 1 || MODE == 3) sq += u * u;
        }
      } else {
        u = h.adam_denom ? g / (sqrtf(v) + h.eps_d) : g * inv;
        if (MODE == 1 || MODE == 3) sq += u * u;
      }
      if (MODE != 1 && MODE != 4) {
        pval_t<T> p = pv_of<T>(praw[k]);
        if constexpr (SR) {
          const float dec = D.decay ? *D.decay : (h.has_decay ? h.decay_val : (h.wd_mode ? wdec : 1.0f));
          P[i] = sr_round<T>(p * dec - step * u, D.sr_seed, h.sr_step, (uint64_t)i);
        } else {
          if (D.decay) p = pdec(p, *D.decay);
          else if (h.has_decay) p = pdec(p, h.decay_val);
          else if (h.wd_mode) p = pdec(p, wdec);
          P[i] = pv_to<T>(pupd(step, u, p));
        }
      }
    }
  }
  // Sums: this workgroup's partials (wg_partial: a fixed order), u^2 at
  // norm_part[wl] and p^2 at norm_part[np + wl] (np workgroups of the tensor);
  // k_full_fin adds them in index order.
  if constexpr (MODE == 1 || MODE == 3 || MODE == 4) {
    __shared__ float s4[4], s4p[4];
    const double t = wg_partial<4>(sq, s4);
    if (lane == 0) gp(D.norm_part)[wl] = t;
    if (MODE == 1 && h.scale_param) {
      const int64_t np = (n + kFElems - 1) / kFElems;
      const double tp = wg_partial<4>(psum, s4p);
      if (lane == 0) gp(D.norm_part)[np + wl] = tp;
    }
  }
}

// Second launch of a NORM / LAG / MNORM pass: one workgroup per tensor adds the
// tensor's partials in index order to norm_buf (and, with scale_param, the p^2
// partials to psq), both zeroed by the caller.
__global__ __launch_bounds__(kFLanes) void k_full_fin(DescFull one, const DescFull* __restrict__ table, int ntab,
                                                     int64_t nwg, int psq) {
  __shared__ double s_w[4];
  const int i = (int)blockIdx.x;
  const DescFull D = table ? table[i] : one;
  const int64_t np = (table ? (i + 1 < ntab ? table[i + 1].wg_begin : nwg) : nwg) - D.wg_begin;
  const double s = sum_parts(D.norm_part, np, s_w);
  if (threadIdx.x == 0) *gp(D.norm_buf) += (float)s;
  if (psq) {
    __syncthreads();   // lane 0 has read s_w
    const double t = sum_parts(D.norm_part + np, np, s_w);
    if (threadIdx.x == 0) *gp(D.psq) += (float)t;
  }
}

static int finish_full(int mode, const DescFull& one, const DescFull* tab, int ntab, int64_t nwg, int psq,
                       hipStream_t st) {
  if (mode != 1 && mode != 3 && mode != 4) return 0;
  hipLaunchKernelGGL(k_full_fin, dim3(tab ? (unsigned)ntab : 1u), dim3(kFLanes), 0, st, one, tab, ntab, nwg,
                     mode == 1 ? psq : 0);
  return check_launch("k_full_fin");
}

template <typename T, bool SR>
static int launch_full(int mode, const DescFull& one, const DescFull* tab, int ntab, int64_t nwg,
                       const HyperFull& h, hipStream_t st) {
  if (nwg <= 0) return 0;
  switch (mode) {
    case 0: hipLaunchKernelGGL((k_update1d_full<T, 0, SR>), dim3((unsigned)nwg), dim3(kFLanes), 0, st, one, tab, ntab, h); break;
    case 1: hipLaunchKernelGGL((k_update1d_full<T, 1, SR>), dim3((unsigned)nwg), dim3(kFLanes), 0, st, one, tab, ntab, h); break;
    case 2: hipLaunchKernelGGL((k_update1d_full<T, 2, SR>), dim3((unsigned)nwg), dim3(kFLanes), 0, st, one, tab, ntab, h); break;
    case 4: hipLaunchKernelGGL((k_update1d_full<T, 4, SR>), dim3((unsigned)nwg), dim3(kFLanes), 0, st, one, tab, ntab, h); break;
    default: hipLaunchKernelGGL((k_update1d_full<T, 3, SR>), dim3((unsigned)nwg), dim3(kFLanes), 0, st, one, tab, ntab, h); break;
  }
  return check_launch("k_update1d_full");
}

static int launch_full_any(int dtype, int stochastic, int mode, const DescFull& one, const DescFull* tab,
                           int ntab, int64_t nwg, const HyperFull& h, hipStream_t st) {
  switch (dtype) {
    case A8_F32: return launch_full<float, false>(mode, one, tab, ntab, nwg, h, st);
    case A8_BF16:
      return stochastic ? launch_full<__hip_bfloat16, true>(mode, one, tab, ntab, nwg, h, st)
                        : launch_full<__hip_bfloat16, false>(mode, one, tab, ntab, nwg, h, st);
    case A8_F16:
      return stochastic ? launch_full<__half, true>(mode, one, tab, ntab, nwg, h, st)
                        : launch_full<__half, false>(mode, one, tab, ntab, nwg, h, st);
    case A8_F64: return launch_full<double, false>(mode, one, tab, ntab, nwg, h, st);
    default: return set_error(A8_ERR_DTYPE, "unsupported param dtype");
  }
}

static HyperFull make_hf(double beta1, double beta_val, float eps_sq, float eps_d, int adam,
                         float eps_g, float d, int mom_only, uint64_t sr_step, float alpha_val,
                         float decay_val, int has_decay) {
  HyperFull h{};
  h.alpha_val = alpha_val; h.decay_val = decay_val; h.has_decay = has_decay;
  h.w_m = (float)(1.0 - beta1);
  h.bv = (float)beta_val;
  h.v_keep = (float)(1.0 - beta_val);
  h.eps_add = (float)(beta_val * (double)eps_g);
  h.has_eps_add = eps_g > 0.0f;
  h.eps_g = eps_g;
  h.eps_d = eps_d; h.eps_sq = eps_sq; h.d = d;
  h.adam_denom = adam; h.momentum_only = mom_only; h.sr_step = sr_step;
  return h;
}

// ------------------------------------------------------------ Fira scalar
// out[i] = scale (apply 0: x is the norm; 2: x is its square) or alpha*scale
// (apply 1: x is the square), out[n+i] = next prev-norm, out[2n+i] = finite(x) ? x : 0
__global__ void k_fira(const float* x, const float* prev, const float* alpha, float* out, int64_t n,
                       float margin, int apply, int has_prev) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float in = x[i];
  const float nrm = apply ? sqrtf(in) : in;
  const bool fin = __builtin_isfinite(nrm);
  const float curr = fin ? nrm : 0.0f;
  float scale = 1.0f, next = curr;
  if (has_prev) {
    const float p = prev[i];
    const float ratio = curr / (p + 1.0e-8f);
    const float lim = (ratio != ratio ? ratio : fmaxf(ratio, margin)) / margin;
    const bool reset = p < 1.0e-6f;
    scale = reset ? 1.0f : 1.0f / lim;
    next = reset ? curr : curr * scale;
  }
  out[i] = apply == 1 ? alpha[i] * scale : scale;
  out[n + i] = next;
  out[2 * n + i] = fin ? in : 0.0f;
}

}  // namespace a8

using namespace a8;

extern "C" {

int a8_fused_update_1d_full(int mode, int dtype, void* param, const void* grad, float* variance,
                            float* m, float* norm_buf, double* norm_parts, const float* alpha, const float* prev_norm,
                            const float* decay, double beta1, double beta_val, float eps_sq,
                            float eps_for_denom, int use_adam_denom, float eps_for_grad_sq,
                            int64_t numel, float d, int momentum_only, float alpha_val,
                            float decay_val, int has_decay, int stochastic, uint64_t sr_seed,
                            uint64_t sr_step, int v_ready, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (mode < 0 || mode > 4) return set_error(A8_ERR_ARG, "mode must be 0..4");
  if (!param && mode != 1 && mode != 4) return set_error(A8_ERR_ARG, "null param");
  if (!grad || !variance) return set_error(A8_ERR_ARG, "null grad/variance");
  if (mode != 0 && !norm_buf) return set_error(A8_ERR_ARG, "null norm_buf");
  if ((mode == 3 || mode == 4) && !prev_norm) return set_error(A8_ERR_ARG, "null prev_norm");
  if (mode == 4 && !(m && momentum_only)) return set_error(A8_ERR_ARG, "MNORM needs momentum and momentum_only");
  if ((mode == 1 || mode == 3 || mode == 4) && !norm_parts)
    return set_error(A8_ERR_ARG, "NORM/LAG/MNORM need norm_parts (a8_norm_parts_full doubles)");
  DescFull D{};
  D.param = param; D.grad = grad; D.v = variance; D.m = m; D.norm_buf = norm_buf; D.norm_part = norm_parts;
  D.alpha = alpha; D.prev_norm = prev_norm; D.decay = decay; D.numel = numel; D.sr_seed = sr_seed;
  HyperFull h = make_hf(beta1, beta_val, eps_sq, eps_for_denom, use_adam_denom, eps_for_grad_sq, d,
                        momentum_only, sr_step, alpha_val, decay_val, has_decay);
  h.v_ready = v_ready;
  const int64_t nwg = (numel + kFElems - 1) / kFElems;
  const int rc = launch_full_any(dtype, stochastic, mode, D, nullptr, 0, nwg, h, (hipStream_t)stream);
  if (rc) return rc;
  return finish_full(mode, D, nullptr, 0, nwg, 0, (hipStream_t)stream);
}

int a8_fused_update_1d_full_multi(int mode, int dtype, const a8_tensor_full* tensors, int ntensors,
                                  void* table_dev, int64_t table_bytes, double beta1, double beta_val,
                                  float eps_sq, float eps_for_denom, int use_adam_denom,
                                  float eps_for_grad_sq, float d, int momentum_only,
                                  float alpha_val, float decay_val, int has_decay, int stochastic,
                                  uint64_t sr_step, int scale_param, float eps2, int wd_mode, float wd,
                                  int v_ready, int upload, const void* step_scalars, void* stream) {
  if (ntensors <= 0) return 0;
  if (scale_param && mode != 1 && mode != 2 && mode != 4)
    return set_error(A8_ERR_ARG, "scale_param needs the NORM / MNORM / APPLY passes");
  if (wd_mode && has_decay) return set_error(A8_ERR_ARG, "give has_decay or wd_mode, not both");
  if ((int64_t)sizeof(DescFull) * ntensors > table_bytes)
    return set_error(A8_ERR_SIZE, "table_dev too small: need a8_table_bytes_full(ntensors)");
  if (mode < 0 || mode > 4) return set_error(A8_ERR_ARG, "mode must be 0..4");
  std::vector<DescFull> tab((size_t)ntensors);
  int64_t wg = 0;
  const bool has_m = tensors[0].m != nullptr;
  if (mode == 4 && !(has_m && momentum_only)) return set_error(A8_ERR_ARG, "MNORM needs momentum and momentum_only");
  for (int i = 0; i < ntensors; ++i) {
    const a8_tensor_full& t = tensors[i];
    if ((t.m != nullptr) != has_m) return set_error(A8_ERR_ARG, "mixed M / no-M tensors in one launch");
    if (t.numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
    if (!t.grad || !t.variance) return set_error(A8_ERR_ARG, "null grad/variance");
    if (!t.param && mode != 1 && mode != 4) return set_error(A8_ERR_ARG, "null param");
    if (mode != 0 && !t.norm_buf) return set_error(A8_ERR_ARG, "null norm_buf");
    if ((mode == 3 || mode == 4) && !t.prev_norm) return set_error(A8_ERR_ARG, "null prev_norm");
    if ((mode == 1 || mode == 3 || mode == 4) && !t.norm_parts)
      return set_error(A8_ERR_ARG, "NORM/LAG/MNORM need norm_parts (a8_norm_parts_full doubles per tensor)");
    DescFull& D = tab[(size_t)i];
    D.param = t.param; D.grad = t.grad; D.v = t.variance; D.m = t.m; D.norm_buf = t.norm_buf;
    D.alpha = t.alpha; D.prev_norm = t.prev_norm; D.decay = t.decay; D.numel = t.numel;
    D.sr_seed = t.sr_seed;
    D.psq = t.psq; D.fira_scale = t.fira_scale; D.norm_part = t.norm_parts;
    if (scale_param && (!t.psq || !t.param)) return set_error(A8_ERR_ARG, "scale_param needs psq and param");
    D.wg_begin = wg;
    wg += (t.numel + kFElems - 1) / kFElems;
  }
  hipStream_t st = (hipStream_t)stream;
  if (upload && upload_table(table_dev, tab.data(), sizeof(DescFull) * (size_t)ntensors, st) != hipSuccess)
    return set_error(A8_ERR_HIP, "table upload failed");
  HyperFull h = make_hf(beta1, beta_val, eps_sq, eps_for_denom, use_adam_denom, eps_for_grad_sq, d,
                        momentum_only, sr_step, alpha_val, decay_val, has_decay);
  h.scale_param = scale_param; h.eps2 = eps2; h.wd_mode = wd_mode; h.wd = wd; h.v_ready = v_ready;
  h.dsc = reinterpret_cast<const a8_step_scalars*>(step_scalars);
  DescFull none{};
  const DescFull* tabd = reinterpret_cast<const DescFull*>(table_dev);
  const int rc = launch_full_any(dtype, stochastic, mode, none, tabd, ntensors, wg, h, st);
  if (rc) return rc;
  return finish_full(mode, none, tabd, ntensors, wg, scale_param, st);
}

int64_t a8_table_bytes_full(int ntensors) { return (int64_t)sizeof(DescFull) * (int64_t)ntensors; }

int64_t a8_norm_parts_full(int64_t numel) {
  if (numel <= 0) return 0;
  return 2 * ((numel + kFElems - 1) / kFElems);
}

int a8_fira_scalar(const float* x, const float* prev, const float* alpha, float* out, int64_t n,
                   int has_prev, int apply, float margin, void* stream) {
  if (n < 0) return set_error(A8_ERR_SIZE, "n < 0");
  if (n == 0) return 0;
  if (apply < 0 || apply > 2) return set_error(A8_ERR_ARG, "apply must be 0, 1 or 2");
  if (!x || !out || (has_prev && !prev) || (apply == 1 && !alpha)) return set_error(A8_ERR_ARG, "null pointer");
  const int threads = 128;
  const int64_t blocks = (n + threads - 1) / threads;
  hipLaunchKernelGGL(k_fira, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream, x, prev, alpha,
                     out, n, margin, apply, has_prev);
  return check_launch("k_fira");
}

}  // extern "C"
