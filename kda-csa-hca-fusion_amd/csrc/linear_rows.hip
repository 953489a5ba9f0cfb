// Linear map of a few rows for decode steps (gfx950):
//   y[m, n] = sum_k x[m, k] w[n, k]      (torch.nn.functional.linear, no bias)
// bf16 / fp16 in and out, fp32 accumulation, 1 <= M <= 16 rows. It serves the
// projections of a single-token decode step (the layer projections of
// /root/reference/ops_fused.py:571-581,609,713,739 and
// /root/reference/run_decoding.py:334-336,522,598,783,815), where a BLAS call
// costs more host time than its GEMM takes on the GPU.
//
// y^T = W x^T on v_mfma_f32_16x16x32: the A operand is a 16-row tile of W
// (lane: row n0 + l % 16, 8 consecutive k), the B operand x^T (lane: row
// l % 16 of x, zero past M). A workgroup of 4 waves takes one 16-column tile of
// y; the waves split the K steps (32 k each) into four contiguous ranges,
// issue their loads eight steps at a time, and sum their partial tiles in LDS.
// The kernel reads W once (2 N K bytes) and is bound by that stream.

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

template <typename T> struct Vec8;
template <> struct Vec8<bf16_t> {
  typedef bf16_t type __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mfma(type a, type b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Vec8<_Float16> {
  typedef _Float16 type __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mfma(type a, type b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kBatch = 8;  // K steps whose loads are in flight together

template <typename T>
__global__ __launch_bounds__(256) void linear_rows_kernel(LinearRowsParams p) {
  using V = Vec8<T>;
  typedef typename V::type v8;
  __shared__ float part[4][16 * 16];  // per-wave partial tile, [n][m]
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16;
  // rows past N re-read row N - 1 (their results are not stored); rows of x
  // past M read row 0 and are zeroed
  const T* wrow = static_cast<const T*>(p.w) + (size_t)min(n0 + r, p.N - 1) * p.ldw + 8 * q;
  const bool mok = r < p.M;
  const T* xrow = static_cast<const T*>(p.x) + (size_t)(mok ? r : 0) * p.ldx + 8 * q;
  const int ks = p.K / 32;
  const int per = (ks + 3) / 4;
  const int s0 = wv * per, s1 = min(ks, s0 + per);
  const v8 zero = {};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int sb = s0; sb < s1; sb += kBatch) {
    v8 a[kBatch], b[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int s = min(sb + u, s1 - 1);  // past the range: a repeated step, zeroed below
      a[u] = *reinterpret_cast<const v8*>(wrow + 32 * s);
      b[u] = *reinterpret_cast<const v8*>(xrow + 32 * s);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const bool live = mok && sb + u < s1;
      acc = V::mfma(a[u], live ? b[u] : zero, acc);
    }
  }
  // acc[e]: y^T[n0 + 4 q + e][m = r]
#pragma unroll
  for (int e = 0; e < 4; ++e) part[wv][(4 * q + e) * 16 + r] = acc[e];
  __syncthreads();
  const int t = threadIdx.x, n = t >> 4, m = t & 15;
  if (m < p.M && n0 + n < p.N) {
    const float v = part[0][t] + part[1][t] + part[2][t] + part[3][t];
    static_cast<T*>(p.y)[(size_t)m * p.ldy + n0 + n] = from_f32<T>(v);
  }
}

}  // namespace

hipError_t linear_rows_dispatch(const LinearRowsParams& p, int dtype, hipStream_t s) {
  const dim3 grid((unsigned)((p.N + 15) / 16)), block(256);
  if (dtype == DT_BF16) hipLaunchKernelGGL(linear_rows_kernel<bf16_t>, grid, block, 0, s, p);
  else hipLaunchKernelGGL(linear_rows_kernel<_Float16>, grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace kch
