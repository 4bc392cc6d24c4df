/* adafactor8bit_amd — C ABI of the MI355X (gfx950) fused optimizer-step library.
 *
 * Every entry point takes raw device pointers, element counts, float scalars
 * and a hipStream_t passed as void*, launches asynchronously on that stream and
 * returns 0 or a negative A8_ERR_* code (message: a8_last_error()).  No torch
 * types cross this boundary.  Buffers are caller-owned; kernels update state in
 * place exactly where the reference's kernels do.
 *
 * The reference binds its kernels as the pybind11 module "adafactor8bit_cuda"
 * (adafactor8bit/kernels.cu:3089-3150), loaded by _load_cuda_module
 * (adafactor8bit/optimizer.py:61-106).  Each function below names the
 * binding(s) it replaces.  The Python mirror of that module
 * (adafactor-8bit_amd/adafactor8bit/adafactor8bit_cuda.py) keeps the
 * reference's names and positional signatures and calls these functions.
 *
 * Numerics: quantised codes are decided as the reference's PyTorch path
 * decides them (optimizer.py:299-353, 504-532).
 */
#ifndef ADAFACTOR8BIT_AMD_H
#define ADAFACTOR8BIT_AMD_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define A8_OK 0
#define A8_ERR_ARG (-1)
#define A8_ERR_DTYPE (-2)
#define A8_ERR_BLOCK (-3)
#define A8_ERR_SIZE (-4)
#define A8_ERR_ALIGN (-5)
#define A8_ERR_HIP (-6)

/* parameter / gradient element types */
#define A8_F32 0
#define A8_BF16 1
#define A8_F16 2
/* fp64 parameters (the reference's kernels dispatch double too,
 * AT_DISPATCH_FLOATING_TYPES_AND2, kernels.cu:840): the gradient is read as fp32
 * and the parameter takes its update in double, as the reference's PyTorch path
 * does on a float64 tensor.  Accepted by the 1-D (quantised and fp32-state), SGD,
 * factored and APOLLO steps (APOLLO: grad is an fp32 copy, projected with the
 * fp32 GEMM; scale_parameter is refused, as torch refuses the reference's fp32
 * norm of a float64 tensor); no stochastic rounding. */
#define A8_F64 3

/* OR'd into v_bits of the 1-D quantised steps (a8_fused_update_1d, its _multi and
 * _multi_noalloc forms): refit and code V by the rule of the reference's fused 1-D
 * CUDA kernels (kernels.cu:686-687, 772-791, 318-326) instead of its CPU quantiser's
 * (optimizer.py:299-353, the default, which the reference's CPU path and this
 * library's parity tests follow).  The kernels' block minimum includes zeros and is
 * floored at log_floor (pass log2(max(eps1^2, FLT_MIN)), the kernels' log_eps_sq;
 * a block holding a zero V therefore takes the floor); l_max is capped at 126; a
 * block without a non-zero V gets scale 1e-12 and min_log -1e30; codes are
 * rint((log2 v - l_min) * ((L-2)/s)) + 1 and decode 2^(((q-1) * (1/(L-2))) * s +
 * l_min), each product and quotient rounded to fp32 in that order.  The logarithm
 * and power are correctly rounded, where the CUDA build uses log2f/exp2f, and the
 * element arithmetic (the V and M EMAs, M codes) stays the CPU path's. */
#define A8_AL_KERNEL_RULE 0x100

/* kernel modes (kernels.cu:19-24): single pass, norm pass, apply pass, lagged norm */
#define A8_MODE_NOCLIP 0
#define A8_MODE_NORM 1
#define A8_MODE_APPLY 2
#define A8_MODE_LAG 3
/* momentum-only norm of the new momentum M' for Fira (no counterpart in the
 * reference's kernels, whose CUDA path applies Fira to ||U||; its PyTorch path,
 * optimizer.py:890-896 with _apply_update_pytorch 866-875, applies it to ||M'||):
 * reads v_buf, clips U by sqrt(*prev_norm) (the NORM pass's sum of U^2) and
 * accumulates sum(M'^2) into norm_buf; writes no state. */
#define A8_MODE_MNORM 4

const char* a8_last_error(void);
const char* a8_version(void);

/* Replaces set_qmap (kernels.cu:32-37; called by _ensure_qmap, optimizer.py:109-133).
 * Uploads the 256- and 16-entry signed dynamic codebooks (host fp32 arrays)
 * to the current device. */
int a8_set_qmap(const float* qmap8_host, const float* qmap4_host);

/* Replaces fused_update_1d_{noclip,norm,apply,lag}[_sr] (kernels.cu:826-990)
 * and, with m_q == NULL, fused_update_1d_vonly_{noclip,norm,apply,lag}[_sr]
 * (kernels.cu:1100-1255); called from _dispatch_1d_cuda (optimizer.py:1080-1170).
 *   mode        A8_MODE_*; stochastic = SR writeback for bf16/fp16 params
 *   param/grad  numel elements of `dtype`, 16-byte aligned
 *   m_q/m_scale momentum codes (uf8/d8: 1 byte, uf4/d4: packed nibbles) padded to
 *               m_block_size, fp32 absmax per m block; NULL for no momentum
 *   v_q         AL8 uint8 / AL16 int16 codes padded to block_size; v_scale,
 *               v_min_log fp32 per block
 *   v_buf       fp32[numel] exact V written by NORM, read by APPLY
 *   norm_buf    fp32[1] sum of squares accumulated by NORM/LAG, read by APPLY
 *   norm_parts  NORM/LAG/MNORM: a8_norm_parts_1d(numel, block_size, m_block_size)
 *               doubles of workspace.  The pass writes one partial sum per workgroup
 *               there and a second launch adds them in index order to norm_buf, so
 *               the sum has the same bits run to run (the reference adds with float
 *               atomics, kernels.cu:297-316); NULL is allowed for modes 0 and 2
 *   alpha, prev_norm, decay: device fp32 scalars; alpha == NULL uses alpha_val,
 *               decay == NULL uses decay_val when has_decay (p := p*decay before
 *               the update, the decoupled weight decay of optimizer.py:2034-2039)
 *   beta1, beta_val  EMA coefficients as the host's doubles: the lerp weights are
 *               (float)(1 - beta1) and (float)beta_val, as torch.lerp_ receives them
 *   log_floor   lower bound of a block's l_min (-126 for the reference's CPU rule;
 *               log2(max(eps1^2, FLT_MIN)) with A8_AL_KERNEL_RULE)
 *   v_bits      8 (AL8) or 16 (AL16), optionally | A8_AL_KERNEL_RULE
 * block_size: a multiple of 128 up to 2^30; m_block_size: a multiple of 4, at least
 * 32, dividing block_size (the reference's rules, optimizer.py:1395-1416).  Powers of
 * two (block_size <= 2048) run the 2048-element unit layout, other sizes one
 * workgroup per V block. */
int a8_fused_update_1d(int mode, int stochastic, int dtype, void* param, const void* grad,
                       uint8_t* m_q, float* m_scale, void* v_q, float* v_scale, float* v_min_log,
                       float* v_buf, float* norm_buf, double* norm_parts, const float* alpha,
                       const float* prev_norm, const float* decay, uint64_t sr_seed, uint64_t sr_step,
                       double beta1, double beta_val, float eps_for_denom, int use_adam_denom,
                       float log_floor, float eps_for_grad_sq, float eps_sq, int64_t numel,
                       int block_size, int m_block_size, int m_bits, int m_mode, float d, int v_bits,
                       int momentum_only, float alpha_val, float decay_val, int has_decay,
                       void* stream);
/* Doubles of norm_parts workspace a NORM / LAG / MNORM pass of a8_fused_update_1d needs for
 * one tensor (the workgroups it runs; pass m_block_size = block_size without momentum). */
int64_t a8_norm_parts_1d(int64_t numel, int block_size, int m_block_size);

/* ---- Per-step scalars on the device (graph-capturable steps) ---------------
 * No counterpart in the reference, which forms these on the host per parameter
 * (optimizer.py:2012-2039, 832-856).  a8_step_advance adds one to a device step
 * counter and writes this step's scalars, derived from the counter as the host
 * derives them from its step: the V lerp weight 1 - beta2 or t^beta2_decay, the
 * step size rho (lr, or min(lr, 1/sqrt(t)) for the relative step) with its bias
 * correction, the Adam epsilon eps1 * sqrt(1 - beta2^t), the weight-decay factor
 * and the factored path's bias factor.  The multi-tensor entry points take
 * `step_scalars` (NULL: use their scalar arguments): with it, beta_val,
 * eps_for_denom, alpha_val, decay_val (when has_decay), the factored path's
 * lr_val and bias_factor, and sr_step are read from the device block instead, so
 * the launch sequence of a step can be captured once in a HIP graph and replayed. */
typedef struct a8_step_spec {
  double beta1, beta2, beta2_decay, eps1;
  double lr;
  float wd;
  int v_mode;          /* V lerp weight: 0 none (SGD), 1 1 - beta2, 2 t^beta2_decay */
  int relative_step;   /* rho = min(lr, 1/sqrt(t)) */
  int bias_mode;       /* 0 none; 1 alpha *= sqrt(bc2)/bc1 (and eps1 *= sqrt(bc2) when adam_denom);
                          2 alpha /= bc1 (beta2 = None) */
  int adam_denom;
  int wd_mode;         /* 0 none; 1 decay = 1 - alpha*wd; 2 decay = 1 - rho*wd */
  int fact_bias_mode;  /* factored path: 0 none; 1 sqrt(1 - beta2^t)/bc1; 2 bc1 */
  int apollo_bias_mode;   /* APOLLO (optimizer.py:3015-3023): 0 none; 1 sqrt(1 - beta2^t)/bc1; 2 bc1 */
  const float* lr_dev;    /* device fp32 learning rate read at each step (a scheduler may fill_ it
                             between graph replays), or NULL for lr */
} a8_step_spec;

typedef struct a8_step_scalars {
  double beta_val;     /* V lerp weight (double: the kernels derive 1 - beta_val from it as the host does) */
  float eps_d;         /* Adam denominator epsilon */
  float alpha;         /* step size, bias corrected (1-D paths) */
  float decay;         /* weight-decay factor (1 without decay) */
  float bias_factor;   /* factored path */
  float rho;           /* step size before the RMS scaling and bias correction */
  float apollo_bias;   /* APOLLO bias factor (apollo_bias_mode) */
  uint64_t step;       /* this step's number (the SR stream's step) */
} a8_step_scalars;

int a8_step_advance(const a8_step_spec* spec, int64_t* counter, a8_step_scalars* out, void* stream);

/* One tensor of a multi-tensor launch. */
typedef struct a8_tensor1d {
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
  uint64_t sr_seed;
  const float* fira_scale; /* APPLY: the step is multiplied by this Fira limiter scale (NULL: none) */
  double* norm_parts;      /* NORM/LAG/MNORM: a8_norm_parts_1d(numel, ...) doubles of workspace */
} a8_tensor1d;

/* Multi-tensor form of a8_fused_update_1d: one launch over `ntensors` tensors
 * that share hyper-parameters (the reference launches once per tensor from
 * its per-parameter loop, optimizer.py:1887).  `table_dev` is a device buffer
 * of at least a8_table_bytes_1d(ntensors) bytes that receives the tensor table
 * (stream-ordered upload) when `upload` is non-zero; with upload == 0 the table
 * already there from an earlier call with the same tensors is reused. */
int a8_fused_update_1d_multi(int mode, int stochastic, int dtype, const a8_tensor1d* tensors,
                             int ntensors, void* table_dev, int64_t table_bytes, double beta1,
                             double beta_val, float eps_for_denom, int use_adam_denom,
                             float log_floor, float eps_for_grad_sq, float eps_sq, int block_size,
                             int m_block_size, int m_bits, int m_mode, float d, int v_bits,
                             int momentum_only, uint64_t sr_step, float alpha_val,
                             float decay_val, int has_decay, int upload, const void* step_scalars,
                             void* stream);
int64_t a8_table_bytes_1d(int ntensors);

/* a8_fused_update_1d_multi without any allocation.  It has no counterpart in the
 * reference; it is for callers that cannot allocate device or pinned host memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid it).
 * Arguments are those of a8_fused_update_1d_multi minus table_dev / table_bytes:
 * the tensor table lives in a 64 KiB device array of the library, one per GPU,
 * held until the process ends, so at most a8_noalloc_max_tensors_1d() tensors
 * (468) fit; more returns A8_ERR_SIZE.  With `upload` non-zero the table is
 * written there (a stream-ordered copy from a host buffer of the library); this is
 * refused (A8_ERR_ARG) on a stream that is being captured, since a replay would
 * copy from that host buffer as it is at replay time.  With upload == 0 the table
 * of the last upload on this GPU is reused; the call is refused (A8_ERR_ARG) unless
 * it names the same tensors (every record field) and block sizes as that upload.
 * So under capture: one eager call with upload != 0, then capture calls with
 * upload == 0.  Every call on a GPU shares that GPU's array, which keeps the last
 * upload's table: calls that overlap on one GPU (two streams, or two host threads)
 * race.  NORM/LAG/MNORM need each record's norm_parts workspace, as in
 * a8_fused_update_1d_multi (the caller's memory, like v_buf and norm_buf). */
int a8_fused_update_1d_multi_noalloc(int mode, int stochastic, int dtype, const a8_tensor1d* tensors,
                                     int ntensors, double beta1, double beta_val, float eps_for_denom,
                                     int use_adam_denom, float log_floor, float eps_for_grad_sq, float eps_sq,
                                     int block_size, int m_block_size, int m_bits, int m_mode, float d,
                                     int v_bits, int momentum_only, uint64_t sr_step, float alpha_val,
                                     float decay_val, int has_decay, int upload, const void* step_scalars,
                                     void* stream);
int a8_noalloc_max_tensors_1d(void);

/* Replaces fused_update_1d_full_{noclip,norm,apply,lag}[_sr] (kernels.cu:1374-1515;
 * called at optimizer.py:2147-2183): fp32 V (and optional fp32 M, NULL for none)
 * for tensors below min_8bit_size or with quantize=False.  NORM writes V (and M
 * unless momentum_only) and accumulates sum(u^2) into norm_buf; APPLY reads them.
 * NORM/LAG/MNORM take norm_parts, a8_norm_parts_full(numel) doubles of workspace: one
 * partial per workgroup, added in index order by a second launch (same bits run to run).
 * stochastic (16-bit params): p * decay - step * u rounded with the (sr_seed,
 * sr_step, element index) stream of kernels.cu:48-87.  v_ready: variance already
 * holds this step's second moment (e.g. the fp32 output of a8_log_quantize_lerp for
 * quantised V with fp32 M, optimizer.py:2078-2087): no EMA, variance not written. */
int a8_fused_update_1d_full(int mode, int dtype, void* param, const void* grad, float* variance,
                            float* m, float* norm_buf, double* norm_parts, const float* alpha,
                            const float* prev_norm, const float* decay, double beta1, double beta_val, float eps_sq,
                            float eps_for_denom, int use_adam_denom, float eps_for_grad_sq,
                            int64_t numel, float d, int momentum_only, float alpha_val,
                            float decay_val, int has_decay, int stochastic, uint64_t sr_seed,
                            uint64_t sr_step, int v_ready, void* stream);

typedef struct a8_tensor_full {
  void* param;
  const void* grad;
  float* variance;
  float* m;
  float* norm_buf;
  const float* alpha;
  const float* prev_norm;
  const float* decay;
  int64_t numel;
  uint64_t sr_seed;        /* stochastic rounding seed (16-bit params) */
  float* psq;              /* sum of p^2 slot (zeroed by the caller) when scale_param, else null */
  const float* fira_scale; /* Fira scale multiplied into alpha by the update passes, or null */
  double* norm_parts;      /* NORM/LAG/MNORM: a8_norm_parts_full(numel) doubles of workspace */
} a8_tensor_full;

/* Multi-tensor form of a8_fused_update_1d_full (one launch per group).  Beyond the
 * single-tensor call: scale_param makes the NORM pass add sum(p^2) to each tensor's
 * psq slot and the APPLY pass take alpha = max(sqrt(psq)/sqrt(numel), eps2) * rho
 * (rho = alpha_val, or *alpha) (optimizer.py:851-855); wd_mode 1 / 2 multiplies p by
 * 1 - alpha*wd / 1 - rho*wd before the update (optimizer.py:2032-2039, instead of
 * has_decay); a tensor's fira_scale, when given, multiplies alpha after both
 * (_apply_fira_cuda, optimizer.py:785-793). */
int a8_fused_update_1d_full_multi(int mode, int dtype, const a8_tensor_full* tensors, int ntensors,
                                  void* table_dev, int64_t table_bytes, double beta1, double beta_val,
                                  float eps_sq, float eps_for_denom, int use_adam_denom,
                                  float eps_for_grad_sq, float d, int momentum_only,
                                  float alpha_val, float decay_val, int has_decay, int stochastic,
                                  uint64_t sr_step, int scale_param, float eps2, int wd_mode, float wd,
                                  int v_ready, int upload, const void* step_scalars, void* stream);
int64_t a8_table_bytes_full(int ntensors);
int64_t a8_norm_parts_full(int64_t numel);

/* Replaces fira_scalar (kernels.cu:3030-3084; used by _fira_scalar_cuda,
 * optimizer.py:735-757).  For i < n: norm = apply ? sqrt(x[i]) : x[i] (apply 0, 1, 2), zeroed when
 * non-finite; with a previous norm p: ratio = norm/(p+1e-8),
 * limiter = max(ratio, margin)/margin, scale = p < 1e-6 ? 1 : 1/limiter.
 * out[i] = apply == 1 ? alpha[i]*scale : scale (apply 2: x holds squared norms, the
 * scale alone is written); out[n+i] = next previous norm;
 * out[2n+i] = x[i] if finite else 0.  margin = 1 + fira_margin. */
int a8_fira_scalar(const float* x, const float* prev, const float* alpha, float* out, int64_t n,
                   int has_prev, int apply, float margin, void* stream);

/* ---- Factored second moment (Adafactor row/column statistics) ------------
 * One parameter of shape [batch, rows, cols] (leading dimensions flattened
 * into batch) with row/column V state.  V state is AL8/AL16 codes with
 * per-block scale/min_log over the flattened [batch*rows] (resp. [batch*cols])
 * vector, or fp32 vectors (row_var/col_var) when unquantised. */
typedef struct a8_tensor2d {
  void* param;
  const void* grad;
  uint8_t* m_q;            /* optional momentum codes (NULL: beta1 is None) */
  float* m_scale;
  void* row_q;             /* AL codes (NULL when row_var holds fp32 state) */
  float* row_scale;
  float* row_min_log;
  float* row_var;          /* fp32 row state, [batch*rows], or NULL */
  void* col_q;
  float* col_scale;
  float* col_min_log;
  float* col_var;
  void* conf_row_q;        /* CAME confidence state, as row/col V (codes or fp32 conf_row/conf_col) */
  float* conf_row_scale;
  float* conf_row_min_log;
  float* conf_row;
  void* conf_col_q;
  float* conf_col_scale;
  float* conf_col_min_log;
  float* conf_col;
  float* workspace;        /* a8_factored_workspace_floats(batch, rows, cols) floats */
  const float* lr;         /* device learning rate, or NULL for lr_val */
  float* fira_prev_norm;   /* 0-dim fp32 state when fira is on; written every step */
  int has_fira_prev;       /* 0 on the first Fira step (the state is created) */
  int64_t batch, rows, cols;
  uint64_t sr_seed;
  float* m;                /* fp32 momentum (m_quant_type 'fp32'), in place of m_q/m_scale, or NULL */
} a8_tensor2d;

/* Replaces the factored branch of one optimizer step for a group of tensors
 * (optimizer.py:2198-2252 statistics and V EMA, 2534-2552 with
 * _fallback_2d_update 920-970 for the update; kernels: compute_factored_sums
 * kernels.cu:1925-1944, fused_log_quantize_lerp 340-480, fused_update_2d
 * 1523-1647).  Per tensor:
 *   row_mean = mean_c(g^2) + eps1, col_mean = mean_r(g^2) + eps1 (deterministic);
 *   row/col V: decode, lerp(v, mean, beta_val), refit + re-encode (or fp32 state);
 *   r = mean_r(row V) clamped at eps1 per batch; inv_row = 1/sqrt(row/r), inv_col = 1/sqrt(col);
 *   alpha = lr (* max(rms(p), eps2) when scale_parameter) (* or / bias_factor);
 *   u = (x * inv_row) * inv_col with x = g, or the momentum EMA lerp(m, g, 1-beta1);
 *   d > 0 or fira: one extra pass for ||u||, Fira limiter, denom = max(1, ||u||/(sqrt(n) d));
 *   p <- p * (1 - wd*alpha | 1 - wd*lr) - (alpha/denom) * u   (SR for bf16/fp16 if stochastic).
 * bias_mode: 0 none, 1 alpha *= bias_factor, 2 alpha /= bias_factor.
 * wd_mode: 0 none, 1 decay uses alpha, 2 decay uses lr.
 * v_bits: 8 / 16 (codes) or 0 (fp32 row_var/col_var).  block_size: V block
 * (any positive size).  m_block_size: a multiple of 4 in [32, 2^30] (powers of
 * two up to 2048 take the tiled / unit layouts, other sizes whole M blocks per
 * workgroup).
 * table_dev: device buffer of a8_table_bytes_2d(ntensors) bytes (uploaded when upload != 0).
 *
 * came != 0 selects CAME (beta3; _fallback_2d_update optimizer.py:929-956, kernels
 * compute_ut_rms kernels.cu:1962-1984, fused_came_pass1 2003-2094, fused_came_pass2
 * 2097-2221, called at optimizer.py:2265-2340).  Momentum codes are required.  After the
 * row/column V step:
 *   U = ((g * inv_row) * inv_col) / clip, clip = max((||U0|| / sqrt(n)) / d, 1) (1 when d == 0);
 *   M' = lerp(M, U, 1 - beta1), res = (U - M')^2 + eps_came;
 *   conf_row/conf_col: lerp(conf, mean of res over columns/rows, 1 - beta3), re-encoded
 *   with c_bits (8 / 16 codes, 0 = fp32 state);
 *   u = (M' * inv_conf_row) * inv_conf_col with inv_conf_row = 1/sqrt(conf_row / r_c),
 *   r_c = mean_r(conf_row) clamped at eps1; Fira (when on) scales u; no RMS denominator;
 *   p <- p * decay - alpha * u, M' re-encoded. */
int a8_factored_step(int dtype, int stochastic, const a8_tensor2d* tensors, int ntensors,
                     void* table_dev, int64_t table_bytes, int upload, double beta_val, float eps1,
                     float eps2, float lr_val, int scale_parameter, int bias_mode, float bias_factor,
                     float weight_decay, int wd_mode, float d, int fira, float fira_margin,
                     float log_floor, int v_bits, int block_size, double beta1, int m_block_size,
                     int m_bits, int m_mode, uint64_t sr_step, int came, double beta3, float eps_came,
                     int c_bits, const void* step_scalars, void* stream);
int64_t a8_factored_workspace_floats(int64_t batch, int64_t rows, int64_t cols);
int64_t a8_table_bytes_2d(int ntensors);

/* ---- APOLLO (low-rank projected AdamW) ------------------------------------
 * One full-rank matrix (a 2-D view: rows x cols; higher-rank parameters are
 * viewed as [shape[0], -1]) per call. */
typedef struct a8_apollo_tensor {
  void* param;             /* fp32, bf16, fp16 or fp64, rows x cols */
  const void* grad;        /* same dtype as param; fp32 for fp16 and fp64 params (the
                              reference projects grad.float(), optimizer.py:2601).  The
                              projection runs on MFMA for bf16 and fp32 G alike */
  int64_t rows, cols;
  const float* proj_t;     /* projection P^T, fp32: right side (rows >= cols) [cols x rank],
                              left side [rank x rows] (P = stable_randn / sqrt(rank)) */
  int64_t rank;
  void* v_q;               /* low-rank V: AL8 uint8 / AL16 int16 codes ... */
  float* v_scale;
  float* v_min_log;
  float* v_fp32;           /* ... or fp32 v_low (NULL when coded) */
  uint8_t* m_q;            /* low-rank M: codes + scale, or fp32 m_low */
  float* m_scale;
  float* m_fp32;
  float* fira_prev;        /* scaled_grad_norm_prev (0-dim fp32 state) when Fira is on */
  int has_fira_prev;       /* 0 on the first Fira step */
  const float* lr;         /* device learning rate, or NULL for lr_val */
  float* workspace;        /* a8_apollo_workspace_floats(rows, cols, rank, channel) floats, kept
                              across steps (it caches the bf16 split of P^T) */
  uint64_t sr_seed;
  /* per-step fields, read by a8_apollo_step_multi (a8_apollo_step takes them as arguments) */
  int first_step;          /* V initialised as g_low^2 * beta_val (no low-rank state yet) */
  int proj_fresh;          /* P^T changed since the last call for this workspace */
  uint64_t step;           /* optimizer step (stochastic-rounding stream) */
  float bias_factor;       /* see bias_mode */
  /* device projection schedule (with step_scalars; NULL otherwise): int64[4] =
     {last_proj_step, apollo_seed, current_proj_seed, fresh}, see a8_apollo_step_multi */
  int64_t* proj_state;
  int proj_gap;            /* apollo_update_proj_gap */
} a8_apollo_tensor;

/* Replaces the APOLLO update of one parameter (_update_param_apollo,
 * optimizer.py:2587-3084, non-factorised, beta3 = None; kernels
 * fused_m_quantize_lerp kernels.cu:523-588, fused_log_quantize_lerp 340-517,
 * compute_apollo_norms 2410-2453, apollo_apply_* 2638-3000; the projection GEMM
 * torch.matmul at optimizer.py:2678-2681).  first_step: V initialised as
 * g_low^2 * beta_val (AL floor -126); later steps lerp with floor log_floor
 * (log2(max(apollo_eps^2, FLT_MIN))).  proj_fresh: P^T changed since the last
 * call for this workspace (its bf16 split is recomputed).  has_m: beta1 is set;
 * m_fp32 selects fp32 m_low.  channel: apollo_scale_type "channel" (else
 * "tensor").  bias_mode 0/1/2: none / step *= bias_factor / step /= bias_factor.
 * wd_mode 0/1/2: none / decay uses alpha / decay uses lr.  V block_size and
 * m_block_size are powers of two (V: 128..2048, M: 32..2048); other sizes run
 * the low-rank stage of a8_apollo_lowrank_x between the phases of
 * a8_apollo_step_multi_phase. */
int a8_apollo_step(int dtype, int stochastic, const a8_apollo_tensor* t, int first_step, int proj_fresh,
                   double beta_val, double beta1, int has_m, float apollo_eps, float log_floor, int v_bits,
                   int block_size, int m_bits, int m_mode, int m_fp32, int m_block_size, int channel,
                   float apollo_scale, int scale_front, int fira, float fira_margin, float d, float lr_val,
                   float eps2, int scale_parameter, int bias_mode, float bias_factor, float weight_decay,
                   int wd_mode, uint64_t sr_step, void* stream);
int64_t a8_apollo_workspace_floats(int64_t rows, int64_t cols, int64_t rank, int channel);

/* The APOLLO update of every matrix of a parameter group in five launches over a
 * device descriptor table (the reference loops _update_param_apollo per
 * parameter, optimizer.py:1886-1898; this batching has no counterpart there).
 * Same hyper-parameters as a8_apollo_step; per-matrix step, first_step,
 * proj_fresh and bias_factor come from the tensor records.  table_dev: device
 * memory of a8_apollo_table_bytes(ntensors) bytes, written by this call (stream
 * ordered) when `upload` is non-zero; with upload == 0 the table already there
 * (from a call with the same records) is used.  Calls that share a table_dev
 * must not overlap.
 *
 * step_scalars (NULL: host scalars as above): the device block of a8_step_advance.
 * The V lerp weight, lr (rho), the bias factor (apollo_bias) and the SR step then
 * come from it, and each record's proj_state schedules the projection on the
 * device, as _get_apollo_proj_matrix does on the host (optimizer.py:2557-2584):
 * with t the device step, when t - last_proj_step >= proj_gap the step takes
 * current_proj_seed = apollo_seed, apollo_seed = next_seed(that seed) (the
 * reference's seed chain, optimizer.py:152-155, restated on the device) and
 * last_proj_step = t, and regenerates P^T (proj_t, written in place) and its bf16
 * split with a8_apollo_proj_gen's generator; fresh = 2 set by the caller rebuilds
 * only the split from proj_t.  proj_fresh, step and bias_factor of the records are
 * then not read, so a step so launched can be captured in a HIP graph and
 * replayed. */
int a8_apollo_step_multi(int dtype, int stochastic, const a8_apollo_tensor* tensors, int ntensors,
                         void* table_dev, int64_t table_bytes, double beta_val, double beta1, int has_m,
                         float apollo_eps, float log_floor, int v_bits, int block_size, int m_bits, int m_mode,
                         int m_fp32, int m_block_size, int channel, float apollo_scale, int scale_front, int fira,
                         float fira_margin, float d, float lr_val, float eps2, int scale_parameter, int bias_mode,
                         float weight_decay, int wd_mode, int upload, const void* step_scalars, void* stream);

/* The device projection generator of capturable APOLLO steps (no counterpart in
 * the reference, whose stable_randn draws from a torch generator seeded on the
 * host, optimizer.py:139-149).  Writes P^T for a rows x cols matrix at rank r
 * (right side, rows >= cols: [cols x r]; left: [r x rows]) with P[i][j] = z / sqrt(r)
 * (fp32 IEEE division), z = (float)(sqrt(-2 ln u1) cos(2 pi u2)) (Box-Muller, in
 * double), u1 = ((a >> 11) + 1) 2^-53, u2 = (b >> 11) 2^-53, where a and b are
 * outputs 2k + 1 and 2k + 2 of SplitMix64 seeded with `seed` and k = i * (P's
 * columns) + j is P's row-major index. */
int a8_apollo_proj_gen(float* proj_t, int64_t rows, int64_t cols, int64_t rank, uint64_t seed, void* stream);
/* out[i] = next_seed(seeds[i]) (optimizer.py:152-155) on the device: the 15th
 * torch.randint(0, 2^63 - 1) draw of a CPU generator seeded with the seed (MT19937
 * from its low 32 bits; a draw is two outputs, first high, modulo 2^63 - 1).  Device
 * arrays of n uint64. */
int a8_apollo_next_seed(const uint64_t* seeds, uint64_t* out, int64_t n, void* stream);
int64_t a8_apollo_table_bytes(int ntensors);

/* a8_apollo_step_multi split around the low-rank stage, for the factorised and
 * CAME variants (optimizer.py:2689-2896), and the plain variant at block sizes
 * the fused stage does not take, whose stage is a8_apollo_lowrank_x.
 * phase 1: projection g_low = G P^T / P^T G into workspace[0, n_low) (n_low =
 * max(rows, cols) * rank; row-major rows x rank on the right side, rank x cols on
 * the left) plus the norms of G (and of p for scale_parameter); V / M fields of
 * the records and v_bits, m_* are not used.  phase 2: channel (or tensor) scale
 * of the update the caller wrote to workspace[n_low, 2 n_low) against g_low,
 * Fira, alpha, step and writeback, with the same arguments as phase 1.  phase 3:
 * as phase 2, for a low-rank stage run with u_rowsums set on exactly the
 * matrices with rows >= cols and rank a power of two in [8, 512]: their row
 * sums of u^2 and g_low^2 are read in place of u and g_low (the two norms of
 * compute_apollo_norms, kernels.cu:2410-2453, per channel); u_rowsums on any
 * other matrix, or phase 3 without it, reads the wrong values.  upload and
 * step_scalars as for a8_apollo_step_multi: phase 1 runs the device projection
 * schedule, phases 2 and 3 read lr, the bias factor and the SR step from the
 * block; a phase after phase 1 of the same records may pass upload == 0. */
int a8_apollo_step_multi_phase(int phase, int dtype, int stochastic, const a8_apollo_tensor* tensors,
                               int ntensors, void* table_dev, int64_t table_bytes, double beta_val, double beta1,
                               int has_m, float apollo_eps, float log_floor, int v_bits, int block_size, int m_bits,
                               int m_mode, int m_fp32, int m_block_size, int channel, float apollo_scale,
                               int scale_front, int fira, float fira_margin, float d, float lr_val, float eps2,
                               int scale_parameter, int bias_mode, float weight_decay, int wd_mode, int upload,
                               const void* step_scalars, void* stream);

/* Low-rank state and hyper-parameters of one matrix for a8_apollo_lowrank_x.
 * Coded states are AL8 (uint8) / AL16 (int16) codes with per-block scale and
 * min_log (blocks of block_size), zero codes in a fresh state. */
typedef struct a8_apollo_x_args {
  const float* g_low;      /* rows_low x cols_low, row-major (phase-1 workspace) */
  float* u;                /* out: the low-rank update, same layout */
  float* xws;              /* a8_apollo_x_workspace_floats(rows_low, cols_low) floats */
  int64_t rows_low, cols_low;
  int factorize;           /* apollo_factorize */
  int came;                /* beta3 set */
  int has_m;               /* beta1 set */
  int first_step;          /* no low-rank second moment yet (V or row / column EMA) */
  /* non-factorised V: codes (v_bits 8 / 16) or fp32 (v_bits 0), n_low values */
  void* v_q;
  float* v_scale;
  float* v_min_log;
  float* v_fp32;
  int v_bits;
  int block_size;          /* AL block of V, residual and confidence codes */
  /* factorised V: fp32 row (rows_low) and column (cols_low) EMAs */
  float* row_var;
  float* col_var;
  /* momentum: codes (m_q, m_scale) or fp32 m_fp32 (non-null selects it) */
  uint8_t* m_q;
  float* m_scale;
  float* m_fp32;
  int m_bits, m_mode, m_block_size;
  /* CAME, non-factorised: residual EMA (n_low values), codes or fp32 */
  void* res_q;
  float* res_scale;
  float* res_min_log;
  float* res_fp32;
  /* CAME, factorised: row (rows_low) and column (cols_low) confidence EMAs */
  void* crow_q;
  float* crow_scale;
  float* crow_min_log;
  float* crow_fp32;
  void* ccol_q;
  float* ccol_scale;
  float* ccol_min_log;
  float* ccol_fp32;
  int c_bits;              /* 0: fp32 residual / confidence */
  double beta_v, beta1, beta3;
  float apollo_eps, eps_sq, log_floor, eps_came, d;
  /* 1: in place of u, leave for each row i the sums of u^2 and g_low^2 (double,
   * from fp32 squares) at ((double*)u)[2 i] and [2 i + 1], for phase 3 of
   * a8_apollo_step_multi_phase; cols_low must be a power of two in [8, 512].
   * 0: write u. */
  int u_rowsums;
} a8_apollo_x_args;

/* Replaces the factorised (apollo_factorize, optimizer.py:2689-2758) and CAME
 * (beta3, optimizer.py:2800-2896) low-rank stages of _update_param_apollo, in
 * the arithmetic of its CPU branches: second-moment EMA, RMS clip (d > 0),
 * momentum EMA, residual / confidence EMAs, and the update u = update_low.
 * With neither flag, the plain stage (optimizer.py:2759-2799): V EMA, momentum
 * EMA, u = x / (sqrt(v) + apollo_eps).  block_size (coded V, residual or
 * confidence): a multiple of 128 up to 2^30; m_block_size (coded momentum): a
 * multiple of 4 in [32, 2^30]. */
int a8_apollo_lowrank_x(const a8_apollo_x_args* args, void* stream);
int64_t a8_apollo_x_workspace_floats(int64_t rows_low, int64_t cols_low);

/* The same stage for nmat matrices at once (the reference steps them one by one
 * in _update_param_apollo, optimizer.py:2587-3084): matrices that agree on every
 * flag and hyper-parameter of their records share one launch per pass, over
 * descriptor tables in table_dev (a8_apollo_x_table_bytes(nmat) bytes of device
 * memory, written on the stream when `upload` is non-zero; with upload == 0 the
 * tables of an earlier call with the same records are used, and upload != 0 on a
 * capturing stream is refused).  Each record needs its own xws.
 * step_scalars (NULL: the records' beta_v): the device block of a8_step_advance,
 * whose beta_val is the V lerp weight (the records' beta_v is then not read), so
 * that the stage can be captured in a HIP graph with the phases around it. */
int a8_apollo_lowrank_x_multi(const a8_apollo_x_args* args, int nmat, void* table_dev, int64_t table_bytes,
                              int upload, const void* step_scalars, void* stream);
int64_t a8_apollo_x_table_bytes(int nmat);

/* Replaces dequantize_log_nonneg (kernels.cu:2593-2632; called by
 * _log_dequantize_nonneg, optimizer.py:328-338): output[i] = 0 for code 0, else
 * 2^(((q-1) * scale[b]) / (L-2) + min_log[b]) with b = i / block_size, L = 256
 * (v_bits 8, uint8 codes) or 65536 (v_bits 16, int16 codes read as unsigned), in
 * the fallback's numerics (optimizer.py:340-353: division, correctly rounded
 * exp2).  output: fp32, 16-byte aligned. */
int a8_dequantize_log_nonneg(float* output, const void* q, const float* scale, const float* min_log,
                             int64_t numel, int block_size, int v_bits, void* stream);

/* Replaces dequantize_dynamic (kernels.cu:2571-2590; called by
 * _dequantize_dynamic_pytorch, optimizer.py:483-488): output[i] = qmap[q_i] *
 * scale[i / block_size] with the codebook of a8_set_qmap; m_bits 8 (one code per
 * byte) or 4 (two per byte, even element in the high nibble). */
int a8_dequantize_dynamic(float* output, const uint8_t* q, const float* scale, int64_t numel, int block_size,
                          int m_bits, void* stream);

/* Replaces _m_dequantize (optimizer.py:535-541) for every momentum codec, where
 * the reference decodes uniform codes with PyTorch ops (_dequantize_uniform_pytorch,
 * optimizer.py:522-532: (q - 128) * (s / 128), or (q - 8) * (s / 8) for 4 bits)
 * and dynamic codes as a8_dequantize_dynamic.  m_mode 0 uniform, 1 dynamic;
 * m_bits 8 or 4 (even element in the high nibble).  Used when a checkpoint's
 * momentum changes from codes to fp32 (_migrate_quantize_flag, optimizer.py:1032-1042). */
int a8_dequantize_momentum(float* output, const uint8_t* q, const float* scale, int64_t numel, int block_size,
                           int m_bits, int m_mode, void* stream);

/* Replaces _quant_v (optimizer.py:379-383, _log_quantize_nonneg 299-325) on a whole
 * fp32 tensor of non-negative values: per block of any size, l_max = log2 of the
 * largest value, l_min = log2 of the smallest non-zero one floored at log_floor
 * (the reference's default -126), l_min := l_max - 1 for a flat block, codes
 * round((log2 v - l_min) / s * (L - 2)) + 1 and 0 for zeros.  q holds
 * ceil(numel / block_size) * block_size codes (uint8, or int16 for v_bits 16) and
 * receives 0 for the padding.  Used when a checkpoint's second-moment state changes
 * from fp32 to codes (_migrate_quantize_flag, optimizer.py:976-1012). */
int a8_al_encode(void* q, float* scale, float* min_log, const float* x, int64_t numel, int block_size, int v_bits,
                 float log_floor, void* stream);

/* Replaces the SGD branch of _update_param_8bit (optimizer.py:2045-2077; beta2 and
 * beta2_decay both None), whose CUDA path calls fused_m_quantize_lerp
 * (kernels.cu:523-588) and then _apply_update_pytorch (optimizer.py:866-881).
 * Fallback arithmetic: m' = lerp(deq(m), g, 1 - beta1); u = m' / (1 - beta1), or
 * u = g without momentum; p = fma(-alpha/denom, u * s, p * decay) with
 * denom = max(1, sqrt(sum u^2) / (sqrt(numel) d)) for d > 0 and the Fira scale s
 * (1 without Fira); M is requantised from the fp32 m'.
 * mode 0: one pass, no clip, no Fira.  mode 1 (NORM): accumulates sum(u^2) into
 * *norm_buf (zeroed by the caller), writes nothing; it needs norm_parts,
 * a8_norm_parts_sgd doubles of workspace (one partial per workgroup, added in
 * index order by a second launch, so the sum has the same bits run to run).  mode 2 (APPLY): reads
 * *norm_buf, and fira = the 3-float output of a8_fira_scalar(norm_buf, prev, one,
 * apply=1) when Fira is on (else null); a non-finite norm then zeroes the update
 * (optimizer.py:797-800).  Momentum: m_q/m_scale (codes padded to whole
 * m_block_size blocks, m_bits/m_mode as in a8_fused_update_1d; m_block_size a
 * multiple of 4 in [32, 2^30]), or fp32 m, or neither.  stochastic: 16-bit params
 * written with the kernels.cu:48-87 stream. */
int a8_sgd_step(int mode, int dtype, int stochastic, void* param, const void* grad, uint8_t* m_q, float* m_scale,
                float* m, float* norm_buf, double* norm_parts, const float* fira, const float* alpha, const float* decay, int64_t numel,
                double beta1, int m_bits, int m_mode, int m_block_size, float d, float alpha_val, float decay_val,
                int has_decay, uint64_t sr_seed, uint64_t sr_step, void* stream);

typedef struct a8_tensor_sgd {
  void* param;
  const void* grad;
  uint8_t* m_q;
  float* m_scale;
  float* m;
  float* norm_buf;
  const float* fira;
  const float* alpha;
  const float* decay;
  int64_t numel;
  uint64_t sr_seed;
  double* norm_parts;      /* NORM: a8_norm_parts_sgd(numel, ...) doubles of workspace */
  const float* fira_sum;   /* APPLY with fira: Fira's finite sum of u^2 (NULL: fira + 2, the
                              layout of a one-tensor a8_fira_scalar output); fira itself is
                              read for the scale only, so a batch can point each tensor at
                              out[i] and out[2n + i] of one n-tensor a8_fira_scalar */
} a8_tensor_sgd;

/* Multi-tensor form of a8_sgd_step: one launch per group.  m_kind: 0 none,
 * 1 quantised (m_q, m_scale), 2 fp32 (m).  step_scalars (NULL: the scalar
 * arguments): the device block of a8_step_advance, whose alpha, decay (when
 * has_decay) and step replace alpha_val, decay_val and sr_step (graph capture). */
int a8_sgd_step_multi(int mode, int dtype, int stochastic, const a8_tensor_sgd* tensors, int ntensors,
                      void* table_dev, int64_t table_bytes, double beta1, int m_kind, int m_bits, int m_mode,
                      int m_block_size, float d, float alpha_val, float decay_val, int has_decay, uint64_t sr_step,
                      int upload, const void* step_scalars, void* stream);
int64_t a8_table_bytes_sgd(int ntensors);
/* Doubles of norm_parts workspace a NORM pass of the SGD step needs for one tensor
 * (m_block_size: that of coded momentum, 0 without); -1 for an invalid block size. */
int64_t a8_norm_parts_sgd(int64_t numel, int m_block_size);

/* Replaces fused_m_quantize_lerp (kernels.cu:523-588; called by
 * _m_fused_quantize_lerp, optimizer.py:563-571) with the arithmetic of its twin
 * _m_ema_pytorch (optimizer.py:690-701): m' = lerp(deq(m), x, 1 - beta) per
 * element (non-finite x read as 0), then one absmax per block and requantised
 * codes; fp32_out (optional) receives m'.  x: x_dtype (A8_F32/BF16/F16).
 * block_size: a multiple of 4 in [32, 2^30]. */
int a8_m_quantize_lerp(uint8_t* m_q, float* m_scale, const void* x, int x_dtype, float* fp32_out, double beta,
                       int block_size, int64_t numel, int m_bits, int m_mode, void* stream);

/* ---- Stand-alone primitives of the reference's module.  The reference's
 * optimizer runs its factored, CAME and APOLLO steps as sequences of these; this
 * library's own optimizer uses the fused entry points above instead.  Each keeps
 * the arithmetic of the reference's PyTorch twin where one exists. */

/* Replaces fused_log_quantize_lerp (kernels.cu:340-520; called by _fused_v_ema,
 * optimizer.py:677-685) with the arithmetic of its twin _deq_v -> lerp_ -> _quant_v
 * (optimizer.py:2232-2238): x = square_input ? x*x + eps1 : x (non-finite read as
 * 0); v' = lerp(deq(v), x, beta); per block of block_size (a multiple of 128 up to
 * 2^30) the AL range is refit from the non-zero v' with floor log_floor;
 * fp32_out (optional) receives v'.  Codes past numel in the last block become 0.
 * q: uint8 (v_bits 8) or int16 (v_bits 16) codes padded to whole blocks. */
int a8_log_quantize_lerp(void* q, float* scale, float* min_log, const void* x, int x_dtype, float* fp32_out,
                         double beta, int block_size, int square_input, float eps1, int64_t numel, float log_floor,
                         int v_bits, void* stream);

/* Arguments of a8_factored_prim; a pointer an op does not use may be null.
 * row, col: the row and column second moments (index b*rows + r, b*cols + c);
 * row_mean: their per-matrix row mean (index b); conf_*: CAME confidence
 * statistics in the same layout. */
typedef struct a8_factored_prim_args {
  void* param;
  const void* grad;
  uint8_t* m_q;
  float* m_scale;
  float* m;
  const float* row;
  const float* col;
  const float* row_mean;
  const float* conf_row;
  const float* conf_col;
  const float* conf_row_mean;
  float* row_sum;
  float* col_sum;
  float* norm_buf;
  const float* alpha;
  const float* prev_norm;
  const float* decay;
  const float* clip;
  int64_t rows;
  int64_t cols;
  int64_t numel;
  double beta1;
  float eps_came;
  float d;
  int m_bits;
  int m_mode;
  int m_block_size;
  uint64_t sr_seed;
  uint64_t sr_step;
} a8_factored_prim_args;

/* Factored element primitives over a (batch of) rows x cols matrices, with
 * inv_row = 1/sqrt(row/row_mean), inv_col = 1/sqrt(col) per element:
 *   op 0-3  fused_update_2d[_full]_{noclip,norm,apply,lag}[_sr] (kernels.cu:1523-1920;
 *           twin optimizer.py:958-970): x = lerp(m, g, 1-beta1) (m: m_q codes or fp32
 *           m, updated in place except by norm) or g; u = (x*inv_row)*inv_col;
 *           norm and lag add sum(u^2) to *norm_buf; apply divides the step by
 *           max(1, sqrt(*norm_buf)/(sqrt(numel) d)) and lag by
 *           max(1, *prev_norm/(sqrt(numel) d)) when d > 0; p = fma(-step, u, p)
 *           (stochastic: SR of fma(-step, u, p*decay)).  op 1 without momentum is
 *           compute_ut_rms (kernels.cu:1962-1999).
 *   op 4    compute_factored_sums (kernels.cu:1925-1956): row_sum[b*rows+r] and
 *           col_sum[b*cols+c] += g^2 (accumulated with atomics, as the reference).
 *   op 5    fused_came_pass1 / fused_came_full_pass1 (kernels.cu:2003-2094; twin
 *           optimizer.py:929-934): U = ((g*inv_row)*inv_col)/ *clip,
 *           M' = lerp(M, U, 1-beta1), res = (U-M')^2 + eps_came added to
 *           row_sum/col_sum; fp32 m is updated, codes are not.
 *   op 6, 7 fused_came_pass2_norm / fused_came_pass2[_sr] and fused_came_full_pass2
 *           (kernels.cu:2097-2221; twin optimizer.py:950-956): M' recomputed from
 *           the codes and U (or the fp32 m as pass 1 left it); u = (M'*inv_crow)*inv_ccol
 *           with the confidence factors; op 6 adds sum(u^2) to *norm_buf, op 7
 *           writes p = fma(-alpha, u, p) and the codes.
 * Non-finite gradients are read as 0. */
int a8_factored_prim(int op, int dtype, int stochastic, const a8_factored_prim_args* args, void* stream);

/* Replaces compute_apollo_norms (kernels.cu:2410-2455; came = 0:
 * u = m/(sqrt(v)+eps)) and apollo_came_compute_update_norms (kernels.cu:2520-2560;
 * came = 1: u = m/sqrt(max(v, eps)), elements at index >= numel skipped, gradient
 * non-finite read as 0): norm_update[c] = ||u||, norm_grad[c] = ||grad_low|| over
 * element c*stride_n + i*stride_d, i < d (sums in double). */
int a8_apollo_norms(const float* m, const float* v, const float* grad_low, float* norm_update, float* norm_grad,
                    int64_t n_channels, int64_t d, int64_t stride_n, int64_t stride_d, int64_t numel, float eps,
                    int came, void* stream);

/* Replaces compute_apollo_came_rms (kernels.cu:2457-2478): *sum_u2 +=
 * sum((g / sqrt(max(v, eps_sq)))^2), non-finite g read as 0. */
int a8_apollo_came_rms(const float* grad_low, const float* v, float* sum_u2, float eps_sq, int64_t numel,
                       void* stream);

/* Replaces apollo_came_compute_m_res (kernels.cu:2480-2518):
 * U = (g / sqrt(max(v, eps_sq))) / *clip_factor; m_out = lerp(deq(m_q_old), U, 1-beta1);
 * res_out = max(lerp(res_old, (U - m_out)^2 + eps_came, 1-beta3), FLT_MIN). */
int a8_apollo_came_m_res(const float* grad_low, const float* v, const uint8_t* m_q_old, const float* m_scale_old,
                         const float* res_old, float* m_out, float* res_out, const float* clip_factor, double beta1,
                         double beta3, float eps_came, float eps_sq, int m_block_size, int64_t numel, int m_bits,
                         int m_mode, void* stream);

/* fp32 second-moment EMA of the reference's PyTorch branch for fp32 V
 * (optimizer.py:2185-2188, taken when V is fp32 and M quantised):
 * v = v * (1 - beta_val) + (beta_val * g) * g, then + beta_val * eps_g when
 * eps_g > 0; non-finite g read as 0.  grad: grad_dtype (A8_F32/BF16/F16). */
int a8_vema_fp32(float* v, const void* grad, int grad_dtype, double beta_val, float eps_g, int64_t numel,
                 void* stream);

/* Replaces apollo_apply_{bf16_det,bf16_sr,fp16_sr} (grad fp32, grad_native = 0) and
 * apollo_apply_{bf16,fp16}_{det,sr}_native (grad of the param's type, scrubbed and
 * negated when maximize; grad_native = 1) (kernels.cu:2638-3000) on a rows x cols
 * bf16/fp16 param: s = final_scale[row] (side_right), [col], or [0] (tensor scale);
 * deterministic: p = rn(rn(p*decay) + (update_scale*g)*s); stochastic: the
 * kernels.cu:48-87 rounding of p*decay + (g*s)*update_scale.  decay may be null. */
int a8_apollo_writeback(int dtype, int grad_native, int stochastic, void* param, const void* grad,
                        const float* final_scale, const float* decay, const float* update_scale, int side_right,
                        int is_channel, int maximize, uint64_t sr_seed, uint64_t sr_step, int64_t rows, int64_t cols,
                        void* stream);

#ifdef __cplusplus
}
#endif
#endif
