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
// Two-kernel chunk path (kda_split.hip): bf16 / fp16, K in {64,128}, V in {64,128};
// ws is 256-byte aligned and holds kda_split_ws_bytes bytes.
bool kda_split_supported(int K, int V, int dtype);
size_t kda_split_ws_bytes(int B, int T, int HV, int K, int V);
hipError_t kda_split_dispatch(const KdaParams& p, void* ws, int dtype, hipStream_t stream);

// Causal depthwise convolution, kernel 3 (kda_frontend.hip).
//   x, out : [B, T, d]   lookback : [B, 2, d] or null (zeros)
//   weight : [d, 3]      bias : [d] or null            (all of the dtype)
struct ShortConvParams {
  const void* x;
  const void* lookback;
  const void* weight;
  const void* bias;
  void* out;
  int B, T, d;
};
hipError_t short_conv_dispatch(const ShortConvParams& p, int dtype, hipStream_t stream);

// KDA activations (kda_frontend.hip). Row r = b*T + t of `proj` holds
// [q (H*K) | k (H*K) | v (HV*V) | beta logits (HV) | ...], ld_proj elements
// apart; row r of `gl` holds the HV*K gate pre-activations, ld_gl apart.
// Outputs are contiguous: q, k [B,T,H,K]; v [B,T,HV,V]; g [B,T,HV,K]; beta [B,T,HV].
struct KdaGatesParams {
  const void* proj;
  long long ld_proj;
  const void* gl;
  long long ld_gl;
  void* q;
  void* k;
  void* v;
  void* g;
  void* beta;
  int B, T, H, HV, K, V;
  float decay_scale;
};
hipError_t kda_gates_dispatch(const KdaGatesParams& p, int dtype, hipStream_t stream);

// fp32 LayerNorm of rows of d elements (kda_frontend.hip).
struct LayerNormParams {
  const void* x;
  const void* w;
  const void* b;  // may be null
  void* out;
  int rows, d;
  float eps;
};
hipError_t layer_norm_dispatch(const LayerNormParams& p, int dtype, int wdtype, hipStream_t stream);

// y[M, N] = x[M, K] w[N, K]^T for M <= 16 rows (linear_rows.hip).
struct LinearRowsParams {
  const void* x;
  const void* w;
  void* y;
  long long ldx, ldw, ldy;  // row strides in elements
  int M, N, K;
};
hipError_t linear_rows_dispatch(const LinearRowsParams& p, int dtype, hipStream_t stream);

}  // namespace kch
