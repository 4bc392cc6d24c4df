// Internal glue between the kernels and the C ABI: error state, checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/adafactor8bit_amd.h"

namespace a8 {

void set_error_msg(const char* msg);

inline int set_error(int code, const char* msg) {
  set_error_msg(msg);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof buf, "%s launch failed: %s", what, hipGetErrorString(e));
    set_error_msg(buf);
    return A8_ERR_HIP;
  }
  return 0;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Host-to-device copy of a descriptor table on stream st that does not wait for
// earlier work on the stream (staged through pinned host memory).
hipError_t upload_table(void* dst, const void* src, size_t bytes, hipStream_t st);

}  // namespace a8

namespace a8 {
// Table forms of the standalone EMAs, for callers that run one stage over many
// tensors (a8_apollo_x.hip).  x, out and dec are fp32.
struct MEmaItem {   // momentum: m' = lerp(deq(m), x, 1 - beta), re-encoded; out = m' (optional)
  uint8_t* m_q;
  float* m_scale;
  const float* x;
  float* out;
  int64_t n;
};
int64_t m_ema_table_bytes(int n);
// upload == 0 (in each of these table forms): the table from an earlier call with
// the same items is still in table_dev, and no copy is made (a captured graph's
// launches then read it as it stands)
int m_ema_multi(const MEmaItem* it, int n, void* table_dev, double beta, int block_size, int m_bits, int m_mode,
                hipStream_t st, int upload = 1);

struct CameTailItem {   // non-factorised CAME APOLLO after the RMS clip (k_came_tail)
  const float* U;         // U before the clip division
  const float* clip;      // device clip factor, or null (d = 0)
  uint8_t* m_q;           // coded momentum, or
  float* m_scale;
  float* m_fp32;          // fp32 momentum
  void* r_q;              // coded residual EMA, or
  float* r_scale;
  float* r_min_log;
  float* r_fp32;          // fp32 residual EMA
  float* u;               // out: the low-rank update, or its row sums (rs_C)
  int64_t n;
  const float* g;         // g_low, read for the row sums
  int64_t rs_C;           // row length C (> 0): row sums of u^2 and g_low^2 in u's place
};
bool came_tail_ok(int m_fp32, int m_block_size, int c_bits, int block_size);
int64_t came_tail_table_bytes(int n);
int came_tail_multi(const CameTailItem* it, int n, void* table_dev, double beta1, double beta3, float eps_came,
                    float eps_sq, int m_fp32, int m_bits, int m_mode, int m_block_size, int c_bits, int block_size,
                    hipStream_t st, int upload = 1);

struct FactTailItem {   // factorised APOLLO momentum EMA and update (k_fact_tail)
  const float* g;         // g_low
  uint8_t* m_q;           // coded momentum, or
  float* m_scale;
  float* m_fp32;          // fp32 momentum
  const float* rv;        // row / column EMAs (R, C)
  const float* cv;
  const float* rmean;     // device clamped row mean
  float* u;               // out: the low-rank update, or its row sums (rs)
  int64_t n, C;
  int rs;                 // row sums of u^2 and g_low^2 in u's place
};
int64_t fact_tail_table_bytes(int n);
int fact_tail_multi(const FactTailItem* it, int n, void* table_dev, double beta1, float apollo_eps, int m_fp32,
                    int m_bits, int m_mode, int m_block_size, hipStream_t st, int upload = 1);

// Row sums of u^2 and g^2 (double, summed from fp32 squares) over the rows of C
// elements of an n-element row-major matrix (C a power of two in [8, 512]), two
// per row at out[2 i], out[2 i + 1]; out must not overlap u or g.
int rowsum_sq(const float* u, const float* g, int64_t n, int64_t C, double* out, hipStream_t st);
bool rowsum_len_ok(int64_t C);

struct VEmaItem {   // AL state: v' = lerp(deq(v), x (or x^2 + eps1), w), re-encoded with a block refit
  void* q;
  float* scale;
  float* min_log;
  const float* x;
  float* out;       // v' before encoding (optional)
  float* dec;       // the decoded new codes (optional)
  int64_t n;
};
int64_t v_ema_table_bytes(int n);
// w_dev: the lerp weight is (float) w_dev->beta_val, read on the device, in place of w
int v_ema_multi(const VEmaItem* it, int n, void* table_dev, double w, int block_size, int square, float eps1,
                float log_floor, int v_bits, hipStream_t st, int upload = 1,
                const a8_step_scalars* w_dev = nullptr);

// Codebook upload of the factored-step translation unit (called by a8_set_qmap).
hipError_t factored_upload_qmap(const float* q8, const float* q4);
hipError_t apollo_upload_qmap(const float* q8, const float* q4);
hipError_t decode_upload_qmap(const float* q8, const float* q4);
hipError_t sgd_upload_qmap(const float* q8, const float* q4);
hipError_t prims_upload_qmap(const float* q8, const float* q4);
hipError_t update1d_k_upload_qmap(const float* q8, const float* q4);
}  // namespace a8
