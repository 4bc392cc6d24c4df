// Standalone decoders of the stored state formats (gfx950).
//
// dequantize_log_nonneg (kernels.cu:2593-2632, used by _log_dequantize_nonneg,
// optimizer.py:328-353): v = 0 for code 0, else 2^(((q - 1) * s) / (L - 2) + l_min)
// per block, with the fallback's numerics (division, then a correctly rounded
// exp2; int16 codes below zero count +65536).
// dequantize_dynamic (kernels.cu:2571-2590, used by _dequantize_dynamic_pytorch,
// optimizer.py:483-499): m = qmap[q] * s, D4 packs the even element in the high
// nibble; a8_dequantize_momentum adds the uniform codecs (optimizer.py:522-532).
// a8_al_encode writes AL codes for a whole fp32 tensor (_quant_v, optimizer.py:379-383).
// The optimizer uses these when a checkpoint's state changes between codes and fp32.
// One workgroup decodes 2048 consecutive elements, 8 per lane, with vector
// stores; AL8 blocks of >= 512 elements decode through an LDS table of the 255
// values of each block the workgroup touches.
#include "a8_common.cuh"
#include "a8_mcodec.cuh"
#include "a8_abi_impl.h"

namespace a8 {

constexpr int kDecUnit = 2048;
constexpr int kDecTab = 6;   // blocks a 2048-element range can touch with block_size >= 512

__device__ __forceinline__ float al_value(uint32_t c, float s, float lm, float lm2) {
  return c ? exp2_exact(((float)(c - 1) * s) / lm2 + lm) : 0.0f;
}

template <int VB>
__global__ __launch_bounds__(256) void k_dec_log(float* __restrict__ out, const void* __restrict__ q,
                                                 const float* __restrict__ scale, const float* __restrict__ min_log,
                                                 int64_t numel, int64_t bs, int use_tab) {
  __shared__ float tab[kDecTab * 256];
  const int lane = threadIdx.x;
  const int64_t u0 = (int64_t)blockIdx.x * kDecUnit;
  const int64_t e0 = u0 + (int64_t)lane * 8;
  constexpr float lm2 = VB == 8 ? 254.0f : 65534.0f;
  const int64_t b0 = u0 / bs;   // first block the range touches
  if (VB == 8 && use_tab) {
    const int64_t last = ((u0 + kDecUnit < numel ? u0 + kDecUnit : numel) - 1) / bs;
    const int nb = (int)(last - b0 + 1);
    for (int i = lane; i < nb * 256; i += 256) {
      const int64_t b = b0 + i / 256;
      tab[i] = al_value((uint32_t)(i & 255), gp(scale)[b], gp(min_log)[b], lm2);
    }
    __syncthreads();
  }
  if (e0 >= numel) return;
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t e = e0 + k;
    if (e >= numel) { v[k] = 0.0f; continue; }
    uint32_t c;
    if constexpr (VB == 8) c = gp(reinterpret_cast<const uint8_t*>(q))[e];
    else c = gp(reinterpret_cast<const uint16_t*>(q))[e];   // int16 < 0 reads as code + 65536
    const int64_t b = e / bs;
    if (VB == 8 && use_tab) v[k] = tab[(int)(b - b0) * 256 + (int)c];
    else v[k] = al_value(c, gp(scale)[b], gp(min_log)[b], lm2);
  }
  store8<float>(out, e0, numel, v);
}

// Momentum codes to fp32 (codec mk: 1 UF8, 2 UF4, 3 D8, 4 D4; the 4-bit forms
// keep the even element in the high nibble): UF m = (q - 128) * (s / 128) or
// (q - 8) * (s / 8) (optimizer.py:522-532), D m = qmap[q] * s (483-499).
__global__ __launch_bounds__(256) void k_dec_m(float* __restrict__ out, const uint8_t* __restrict__ q,
                                               const float* __restrict__ scale, int64_t numel, int64_t bs,
                                               int mk) {
  const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e0 >= numel) return;
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t e = e0 + k;
    if (e >= numel) { v[k] = 0.0f; continue; }
    const float s = gp(scale)[e / bs];
    uint32_t c;
    if (mk == 1 || mk == 3) {
      c = gp(q)[e];
    } else {
      const uint32_t packed = gp(q)[e >> 1];
      c = (e & 1) ? (packed & 0x0Fu) : (packed >> 4);
    }
    v[k] = m_decode(mk, c, s);
  }
  store8<float>(out, e0, numel, v);
}

// fp32 non-negative values to AL codes, as the reference's _quant_v does for a
// whole tensor (_log_quantize_nonneg, optimizer.py:299-325, 379-383): one
// workgroup per block of any size.  Pass 1 takes the block's largest value and
// its smallest non-zero one; the refit is the CPU rule (minimum over non-zero
// entries, floored, l_min := l_max - 1 for a flat block); pass 2 writes the
// codes, code 0 for zeros and for the padding beyond numel.
template <int VB>
__global__ __launch_bounds__(256) void k_al_enc(void* __restrict__ q, float* __restrict__ scale,
                                                float* __restrict__ min_log, const float* __restrict__ x,
                                                int64_t numel, int64_t bs, float floor_) {
  constexpr int LM2 = VB == 8 ? 254 : 65534;
  __shared__ float s8[8];
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t i0 = b * bs;
  const int64_t i1 = i0 + bs < numel ? i0 + bs : numel;
  float mx = 0.0f;
  uint32_t key = 0xFFFFFFFFu;   // bits(v) - 1 is monotone in v > 0; v = 0 maps to the largest key
  for (int64_t i = i0 + lane; i < i1; i += 256) {
    const float v = gp(x)[i];
    mx = fmaxf(mx, v);
    key = min(key, __float_as_uint(v) - 1u);
  }
  mx = grp_max(mx, 64);
  key = grp_umin(key, 64);
  if ((lane & 63) == 0) {
    s8[lane >> 6] = mx;
    s8[4 + (lane >> 6)] = __uint_as_float(key);
  }
  __syncthreads();
  mx = fmaxf(fmaxf(s8[0], s8[1]), fmaxf(s8[2], s8[3]));
  key = min(min(__float_as_uint(s8[4]), __float_as_uint(s8[5])), min(__float_as_uint(s8[6]), __float_as_uint(s8[7])));
  const float mnz = key == 0xFFFFFFFFu ? __builtin_inff() : __uint_as_float(key + 1u);
  const ALFit f = al_refit(mx, mnz, floor_, (float)LM2);
  for (int64_t k = lane; k < bs; k += 256) {
    const int64_t i = i0 + k;
    const float v = i < numel ? gp(x)[i] : 0.0f;
    const uint32_t code = al_finish<LM2>(v, al_round_exact<LM2>(v, f));
    if constexpr (VB == 8) gp(reinterpret_cast<uint8_t*>(q))[i] = (uint8_t)code;
    else gp(reinterpret_cast<uint16_t*>(q))[i] = (uint16_t)code;
  }
  if (lane == 0) {
    gp(scale)[b] = f.s;
    gp(min_log)[b] = f.lmin;
  }
}

hipError_t decode_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

}  // namespace a8

using namespace a8;

extern "C" {

int a8_dequantize_log_nonneg(float* output, const void* q, const float* scale, const float* min_log,
                             int64_t numel, int block_size, int v_bits, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!output || !q || !scale || !min_log) return set_error(A8_ERR_ARG, "null pointer");
  if (block_size <= 0) return set_error(A8_ERR_BLOCK, "block_size must be positive");
  if (v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  if (!aligned16(output)) return set_error(A8_ERR_ALIGN, "output must be 16-byte aligned");
  const int64_t nwg = (numel + kDecUnit - 1) / kDecUnit;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  const int use_tab = block_size >= 512 ? 1 : 0;   // then a 2048-element range touches <= kDecTab blocks
  hipStream_t st = (hipStream_t)stream;
  if (v_bits == 8)
    hipLaunchKernelGGL(k_dec_log<8>, dim3((unsigned)nwg), dim3(256), 0, st, output, q, scale, min_log, numel,
                       (int64_t)block_size, use_tab);
  else
    hipLaunchKernelGGL(k_dec_log<16>, dim3((unsigned)nwg), dim3(256), 0, st, output, q, scale, min_log, numel,
                       (int64_t)block_size, 0);
  return check_launch("k_dec_log");
}

int a8_dequantize_dynamic(float* output, const uint8_t* q, const float* scale, int64_t numel, int block_size,
                          int m_bits, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!output || !q || !scale) return set_error(A8_ERR_ARG, "null pointer");
  if (block_size <= 0) return set_error(A8_ERR_BLOCK, "block_size must be positive");
  if (m_bits != 8 && m_bits != 4) return set_error(A8_ERR_ARG, "m_bits must be 8 or 4");
  if (!aligned16(output)) return set_error(A8_ERR_ALIGN, "output must be 16-byte aligned");
  const int64_t nwg = (numel + kDecUnit - 1) / kDecUnit;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  hipLaunchKernelGGL(k_dec_m, dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream, output, q, scale, numel,
                     (int64_t)block_size, m_bits == 8 ? 3 : 4);
  return check_launch("k_dec_m");
}

int a8_dequantize_momentum(float* output, const uint8_t* q, const float* scale, int64_t numel, int block_size,
                           int m_bits, int m_mode, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!output || !q || !scale) return set_error(A8_ERR_ARG, "null pointer");
  if (block_size <= 0 || (m_bits == 4 && block_size % 2)) return set_error(A8_ERR_BLOCK, "bad m_block_size");
  if ((m_bits != 8 && m_bits != 4) || (m_mode != 0 && m_mode != 1))
    return set_error(A8_ERR_ARG, "m_bits must be 8 or 4 and m_mode 0 (uniform) or 1 (dynamic)");
  if (!aligned16(output)) return set_error(A8_ERR_ALIGN, "output must be 16-byte aligned");
  const int64_t nwg = (numel + kDecUnit - 1) / kDecUnit;
  if (nwg > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  const int mk = m_mode == 0 ? (m_bits == 8 ? 1 : 2) : (m_bits == 8 ? 3 : 4);
  hipLaunchKernelGGL(k_dec_m, dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream, output, q, scale, numel,
                     (int64_t)block_size, mk);
  return check_launch("k_dec_m");
}

int a8_al_encode(void* q, float* scale, float* min_log, const float* x, int64_t numel, int block_size, int v_bits,
                 float log_floor, void* stream) {
  if (numel < 0) return set_error(A8_ERR_SIZE, "numel < 0");
  if (numel == 0) return 0;
  if (!q || !scale || !min_log || !x) return set_error(A8_ERR_ARG, "null pointer");
  if (block_size <= 0) return set_error(A8_ERR_BLOCK, "block_size must be positive");
  if (v_bits != 8 && v_bits != 16) return set_error(A8_ERR_ARG, "v_bits must be 8 or 16");
  const int64_t nblk = (numel + block_size - 1) / block_size;
  if (nblk > 0x7FFFFFFF) return set_error(A8_ERR_SIZE, "numel too large");
  hipStream_t st = (hipStream_t)stream;
  if (v_bits == 8)
    hipLaunchKernelGGL(k_al_enc<8>, dim3((unsigned)nblk), dim3(256), 0, st, q, scale, min_log, x, numel,
                       (int64_t)block_size, log_floor);
  else
    hipLaunchKernelGGL(k_al_enc<16>, dim3((unsigned)nblk), dim3(256), 0, st, q, scale, min_log, x, numel,
                       (int64_t)block_size, log_floor);
  return check_launch("k_al_enc");
}

}  // extern "C"
