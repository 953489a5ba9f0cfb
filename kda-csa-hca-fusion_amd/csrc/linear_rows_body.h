// The block-level body of the decode-step row projection (linear_rows.hip),
// shared by its own kernel and by the launch that runs it beside a cache
// append (decode_step.hip).
//
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
//
// Options for a decode step: a LayerNorm of the x rows first (the norm in
// front of a sub-layer's projections, ops_fused.py:42-60,879-955: wave w
// normalises rows w, w + 4, ... into LDS, which the B operand then reads),
// the residual add after it (y = res + y, with y rounded to the dtype first,
// as the separate add of ops_fused.py:879-955 sees it), and an increment of
// the decode step's token counter by one thread.

#pragma once

#include <type_traits>

#include "attn_common.h"
#include "kch_kernels.h"

namespace kch {

namespace rows_detail {

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

constexpr int kBatch = 16;  // K steps whose loads are in flight together

// One workgroup's 16-column tile of y (tile index blk), 256 threads.
template <typename T, typename WT>
__device__ __forceinline__ void linear_rows_block(const LinearRowsParams& p, int blk) {
  using V = Vec8<T>;
  typedef typename V::type v8;
  constexpr bool LN = !std::is_void<WT>::value;
  extern __shared__ __attribute__((aligned(16))) char xs_raw[];  // LN: M rows of K + 8
  __shared__ float part[4][16 * 16];  // per-wave partial tile, [n][m]
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, q = lane >> 4;
  const int n0 = blk * 16;
  const int ldl = p.K + 8;  // LDS row stride (elements)
  if constexpr (LN) {
    // rows of LayerNorm(x) in the dtype, as a separate norm would store them
    T* xs = reinterpret_cast<T*>(xs_raw);
    const WT* lw = static_cast<const WT*>(p.ln_w);
    const WT* lb = static_cast<const WT*>(p.ln_b);
    constexpr int G = 8;  // 8-element groups per lane: K <= 4096
    for (int m = wv; m < p.M; m += 4) {
      const T* xr = static_cast<const T*>(p.x) + (size_t)m * p.ldx;
      float v[G][8];
      float s = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int k0 = 8 * lane + 512 * g;
        if (k0 < p.K) {
          Load8<T>::run(xr + k0, v[g]);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[g][i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s += v[g][i];
      }
      const float mean = wave_sum(s) / (float)p.K;
      float ss = 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (8 * lane + 512 * g >= p.K) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float dv = v[g][i] - mean;
          ss += dv * dv;
        }
      }
      const float rstd = 1.f / sqrtf(wave_sum(ss) / (float)p.K + p.ln_eps);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int k0 = 8 * lane + 512 * g;
        if (k0 >= p.K) continue;
        float w8[8], b8[8], y8[8];
        Load8<WT>::run(lw + k0, w8);
        if (lb) {
          Load8<WT>::run(lb + k0, b8);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) b8[i] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) y8[i] = (v[g][i] - mean) * rstd * w8[i] + b8[i];
        union { T h[8]; v8 vv; } u;
#pragma unroll
        for (int i = 0; i < 8; ++i) u.h[i] = from_f32<T>(y8[i]);
        *reinterpret_cast<v8*>(xs + (size_t)m * ldl + k0) = u.vv;
      }
    }
    __syncthreads();
  }
  // rows past N re-read row N - 1 (their results are not stored); rows of x
  // past M read row 0 and are zeroed
  const T* wrow = static_cast<const T*>(p.w) + (size_t)min(n0 + r, p.N - 1) * p.ldw + 8 * q;
  const bool mok = r < p.M;
  const T* xrow = LN ? reinterpret_cast<const T*>(xs_raw) + (size_t)(mok ? r : 0) * ldl + 8 * q
                     : static_cast<const T*>(p.x) + (size_t)(mok ? r : 0) * p.ldx + 8 * q;
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
    T* yp = static_cast<T*>(p.y) + (size_t)m * p.ldy + n0 + n;
    if (p.res) {
      const float rv = to_f32(static_cast<const T*>(p.res)[(size_t)m * p.ldr + n0 + n]);
      *yp = from_f32<T>(rv + stored<T>(v));
    } else {
      *yp = from_f32<T>(v);
    }
  }
  if (p.counter && blk == 0 && t == 0) p.counter[0] = p.counter[0] + 1;
}

}  // namespace rows_detail

}  // namespace kch
