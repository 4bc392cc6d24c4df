// The fused 1-D step under the reference kernels' AL rule (A8_AL_KERNEL_RULE):
// the KR = 1 instantiations of a8_update1d_kern.cuh, in their own translation unit
// so that they compile in parallel with the default rule's.
#include "a8_update1d_kern.cuh"

namespace a8 {

int launch_any_kernel_rule(int dtype, int sr, int vbits, int mode, const Desc1D& one, const Desc1D* table,
                           int ntab, int64_t nwg, const Hyper1D& h, hipStream_t st) {
  return launch_rule<1>(dtype, sr, vbits, mode, one, table, ntab, nwg, h, st);
}

hipError_t update1d_k_upload_qmap(const float* q8, const float* q4) { return upload_qmap_tu(q8, q4); }

}  // namespace a8
