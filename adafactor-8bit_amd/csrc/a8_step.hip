// Per-step scalars on the device, for steps captured in a HIP graph.
//
// The reference forms the scalars of a step on the host from its step count
// (optimizer.py:2012-2039 bias correction, eps and weight decay; 832-856 the step
// size; the V lerp weight 1 - beta2 or t^beta2_decay).  Baked into launch
// arguments they would freeze in a captured graph, so with a8_step_advance the
// count lives in device memory: one single-lane kernel adds one to it and writes
// this step's scalars, which the multi-tensor kernels then read.  The arithmetic
// is the host planner's: double precision for powers and square roots, then
// float32 products rounded as the planner's float32 (numpy) arithmetic rounds them.
#include "a8_common.cuh"
#include "a8_abi_impl.h"

namespace a8 {

__global__ void k_step_advance(a8_step_spec sp, int64_t* counter, a8_step_scalars* out) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  const int64_t t = gp(counter)[0] + 1;
  gp(counter)[0] = t;
  const double td = (double)t;
  double beta_val = 0.0;
  if (sp.v_mode == 1) beta_val = 1.0 - sp.beta2;
  else if (sp.v_mode == 2) beta_val = pow(td, sp.beta2_decay);
  // lr_dev: the current value of a device learning rate (a tensor lr that a
  // scheduler fills between replays), read in fp32 as the reference reads a tensor lr
  const double lr = sp.lr_dev ? (double)*gp(sp.lr_dev) : sp.lr;
  const float rho = (float)(sp.relative_step ? fmin(lr, 1.0 / sqrt(td)) : lr);
  float alpha = rho;
  double eps_d = sp.adam_denom ? sp.eps1 : 0.0;
  float bias = 1.0f;
  if (sp.bias_mode == 1) {
    const double bc1 = 1.0 - pow(sp.beta1, td);
    const double bc2 = 1.0 - pow(sp.beta2, td);
    const double fac = sqrt(bc2) / bc1;
    alpha = alpha * (float)fac;
    if (sp.adam_denom) eps_d = sp.eps1 * sqrt(bc2);
    bias = (float)fac;
  } else if (sp.bias_mode == 2) {
    const double bc1 = 1.0 - pow(sp.beta1, td);
    alpha = alpha / (float)bc1;
    bias = (float)bc1;
  }
  float apollo_bias = 1.0f;   // APOLLO's bias factor (optimizer.py:3015-3023)
  if (sp.apollo_bias_mode == 1) {
    const double bc1 = 1.0 - pow(sp.beta1, td);
    apollo_bias = (float)(sqrt(1.0 - pow(sp.beta2, td)) / bc1);
  } else if (sp.apollo_bias_mode == 2) {
    apollo_bias = (float)(1.0 - pow(sp.beta1, td));
  }
  float decay = 1.0f;
  if (sp.wd_mode == 1) decay = 1.0f - alpha * sp.wd;
  else if (sp.wd_mode == 2) decay = 1.0f - rho * sp.wd;
  a8_step_scalars s{};
  s.beta_val = beta_val;
  s.eps_d = (float)eps_d;
  s.alpha = alpha;
  s.decay = decay;
  s.bias_factor = bias;
  s.rho = rho;
  s.apollo_bias = apollo_bias;
  s.step = (uint64_t)t;
  uint64_t w[sizeof(a8_step_scalars) / 8];
  __builtin_memcpy(w, &s, sizeof(s));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(a8_step_scalars) / 8); ++i) gp(reinterpret_cast<uint64_t*>(out))[i] = w[i];
}

}  // namespace a8

using namespace a8;

extern "C" int a8_step_advance(const a8_step_spec* spec, int64_t* counter, a8_step_scalars* out, void* stream) {
  if (!spec || !counter || !out) return set_error(A8_ERR_ARG, "null pointer");
  if (spec->bias_mode < 0 || spec->bias_mode > 2 || spec->wd_mode < 0 || spec->wd_mode > 2)
    return set_error(A8_ERR_ARG, "bias_mode and wd_mode must be 0..2");
  if (spec->v_mode < 0 || spec->v_mode > 2) return set_error(A8_ERR_ARG, "v_mode must be 0..2");
  if (spec->apollo_bias_mode < 0 || spec->apollo_bias_mode > 2)
    return set_error(A8_ERR_ARG, "apollo_bias_mode must be 0..2");
  hipLaunchKernelGGL(k_step_advance, dim3(1), dim3(64), 0, (hipStream_t)stream, *spec, counter, out);
  return check_launch("k_step_advance");
}
