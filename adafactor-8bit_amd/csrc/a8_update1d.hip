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
#include "a8_update1d_kern.cuh"

#include <mutex>

namespace a8 {

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

static int launch_any(int dtype, int sr, int vbits, int mode, const Desc1D& one, const Desc1D* table,
                      int ntab, int64_t nwg, const Hyper1D& h, hipStream_t st) {
  if (h.krule) return launch_any_kernel_rule(dtype, sr, vbits, mode, one, table, ntab, nwg, h, st);
  return launch_rule<0>(dtype, sr, vbits, mode, one, table, ntab, nwg, h, st);
}

static int check_common(int dtype, int64_t numel, int bv, int bm, int mbits, int mmode, int vbits,
                        bool has_m) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (vbits != 8 && vbits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  if (!has_m) bm = bv;
  if (!fast_shape_ok(bv, bm) && !gen_shape_ok(bv, bm))
    return set_error(A8_ERR_BLOCK, "block_size must be a multiple of 128 (at most 2^30) and m_block_size a "
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
  const int krule = (v_bits & A8_AL_KERNEL_RULE) ? 1 : 0;
  v_bits &= ~A8_AL_KERNEL_RULE;
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
  h.krule = krule;
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
  int rc = check_common(dtype, 0, block_size, m_block_size, m_bits, m_mode, v_bits & ~A8_AL_KERNEL_RULE, has_m);
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
  h.krule = (v_bits & A8_AL_KERNEL_RULE) ? 1 : 0;
  v_bits &= ~A8_AL_KERNEL_RULE;
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
      a8::prims_upload_qmap(qmap8_host, qmap4_host) != hipSuccess ||
      a8::update1d_k_upload_qmap(qmap8_host, qmap4_host) != hipSuccess)
    return set_error(A8_ERR_HIP, "codebook upload failed");
  return 0;
}

}  // extern "C"
