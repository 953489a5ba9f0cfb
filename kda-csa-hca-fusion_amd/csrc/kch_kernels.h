// Internal launch interface between the C-ABI layer (abi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace kch {

// Contiguous row-major tensors; element types follow the dtype enum of the ABI.
//   q, k : [B, T, H, K]      v, o : [B, T, HV, V]
//   g    : [B, T, HV, K]     beta : [B, T, HV]
//   s0, s_out : [B, HV, K, V] fp32 (either may be null)
struct KdaParams {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* s0;
  void* o;
  float* s_out;
  int B, T, H, HV, K, V;
  float scale;
  float g_clamp_min;  // -inf disables the clamp
};

hipError_t kda_chunk_dispatch(const KdaParams& p, int dtype, hipStream_t stream);
// bf16 / fp16 inputs, K in {64, 128}, V a multiple of 64 (kda_chunk_lp.hip)
hipError_t kda_chunk_lp_dispatch(const KdaParams& p, int dtype, hipStream_t stream);
hipError_t kda_recurrent_dispatch(const KdaParams& p, int dtype, hipStream_t stream);

}  // namespace kch
