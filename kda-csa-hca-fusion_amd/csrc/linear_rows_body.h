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
  // rows past N re-read row N - 1 (their results are not stored); rows of x
  // past M read row 0 and are zeroed
  const T* wrow = static_cast<const T*>(p.w) + (size_t)min(n0 + r, p.N - 1) * p.ldw + 8 * q;
  const int ks = p.K / 32;
  const int per = (ks + 3) / 4;
  const int s0 = wv * per, s1 = min(ks, s0 + per);
  // the first batch of W is requested before the normalisation (it does not
  // depend on x), so the stream of W starts at once
  v8 a[kBatch];
  auto load_w = [&](int sb) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) a[u] = *reinterpret_cast<const v8*>(wrow + 32 * min(sb + u, s1 - 1));
  };
  if (s0 < s1) load_w(s0);
  if constexpr (LN) {
    // rows of LayerNorm(x) in the dtype, as a separate norm would store them
    // (with the KDA front: the convolution over [lookback ; LN(x)])
    T* xs = reinterpret_cast<T*>(xs_raw);
    const WT* lw = static_cast<const WT*>(p.ln_w);
    const WT* lb = static_cast<const WT*>(p.ln_b);
    if (p.K <= 2048) {
      // a thread per 8 channels, all four waves on every row, the rows two at
      // a time: the parameters, then both rows' x (and lookback) loads are in
      // flight together, and each statistic is one block reduction
      __shared__ float red2[2][4][2];
      const int tid = threadIdx.x, k0 = 8 * tid;
      const bool act = k0 < p.K;
      const int kk = act ? k0 : 0;
      float w8[8], b8[8], w3[24], cb[8];
      Load8<WT>::run(lw + kk, w8);
      if (lb) {
        Load8<WT>::run(lb + kk, b8);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) b8[i] = 0.f;
      }
      if (p.conv_w) {
#pragma unroll
        for (int u3 = 0; u3 < 3; ++u3)
          Load8<T>::run(static_cast<const T*>(p.conv_w) + 3 * kk + 8 * u3, w3 + 8 * u3);
        if (p.conv_b) {
          Load8<T>::run(static_cast<const T*>(p.conv_b) + kk, cb);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) cb[i] = 0.f;
        }
      }
      for (int m0 = 0; m0 < p.M; m0 += 2) {
        float v[2][8], l0[2][8], l1[2][8];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int m = min(m0 + rr, p.M - 1);
          Load8<T>::run(static_cast<const T*>(p.x) + (size_t)m * p.ldx + kk, v[rr]);
          if (p.conv_w) {
            const T* lk = static_cast<const T*>(p.look) + (size_t)m * 2 * p.K;
            Load8<T>::run(lk + kk, l0[rr]);
            Load8<T>::run(lk + p.K + kk, l1[rr]);
          }
        }
        float mean[2], rstd[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float sm = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) sm += v[rr][i];
          sm = wave_sum(act ? sm : 0.f);
          if (lane == 0) red2[0][wv][rr] = sm;
        }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          mean[rr] = (red2[0][0][rr] + red2[0][1][rr] + red2[0][2][rr] + red2[0][3][rr]) / (float)p.K;
          float sq = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float dv = v[rr][i] - mean[rr];
            sq += dv * dv;
          }
          sq = wave_sum(act ? sq : 0.f);
          if (lane == 0) red2[1][wv][rr] = sq;
        }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int m = m0 + rr;
          rstd[rr] = 1.f / sqrtf((red2[1][0][rr] + red2[1][1][rr] + red2[1][2][rr] + red2[1][3][rr]) /
                                     (float)p.K + p.ln_eps);
          if (m >= p.M || !act) continue;
          float y8[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) y8[i] = (v[rr][i] - mean[rr]) * rstd[rr] * w8[i] + b8[i];
          if (p.conv_w) {
            float h8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              h8[i] = stored<T>(y8[i]);
              y8[i] = fmaf(w3[3 * i + 2], h8[i], fmaf(w3[3 * i + 1], l1[rr][i], fmaf(w3[3 * i], l0[rr][i], cb[i])));
            }
            if (blk == 0 && p.h_out) {
              union { T h[8]; v8 vv; } uh;
#pragma unroll
              for (int i = 0; i < 8; ++i) uh.h[i] = from_f32<T>(h8[i]);
              *reinterpret_cast<v8*>(static_cast<T*>(p.h_out) + (size_t)m * p.K + k0) = uh.vv;
            }
          }
          union { T h[8]; v8 vv; } u;
#pragma unroll
          for (int i = 0; i < 8; ++i) u.h[i] = from_f32<T>(y8[i]);
          *reinterpret_cast<v8*>(xs + (size_t)m * ldl + k0) = u.vv;
        }
      }
      __syncthreads();
    }
    constexpr int G = 8;  // 8-element groups per lane: K <= 4096
    for (int m = p.K <= 2048 ? p.M : wv; m < p.M; m += 4) {
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
        if (p.conv_w) {
          // the LayerNorm output as the layer receives it (rounded to the
          // dtype), then out = bias + w0 look[0] + w1 look[1] + w2 h
          const T* lk = static_cast<const T*>(p.look) + (size_t)m * 2 * p.K;
          float l0[8], l1[8], w3[24], bias[8], h8[8];
          Load8<T>::run(lk + k0, l0);
          Load8<T>::run(lk + p.K + k0, l1);
#pragma unroll
          for (int u3 = 0; u3 < 3; ++u3)
            Load8<T>::run(static_cast<const T*>(p.conv_w) + 3 * k0 + 8 * u3, w3 + 8 * u3);
          if (p.conv_b) {
            Load8<T>::run(static_cast<const T*>(p.conv_b) + k0, bias);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) bias[i] = 0.f;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            h8[i] = stored<T>(y8[i]);
            y8[i] = fmaf(w3[3 * i + 2], h8[i], fmaf(w3[3 * i + 1], l1[i], fmaf(w3[3 * i], l0[i], bias[i])));
          }
          if (blk == 0 && p.h_out) {
            union { T h[8]; v8 vv; } uh;
#pragma unroll
            for (int i = 0; i < 8; ++i) uh.h[i] = from_f32<T>(h8[i]);
            *reinterpret_cast<v8*>(static_cast<T*>(p.h_out) + (size_t)m * p.K + k0) = uh.vv;
          }
        }
        union { T h[8]; v8 vv; } u;
#pragma unroll
        for (int i = 0; i < 8; ++i) u.h[i] = from_f32<T>(y8[i]);
        *reinterpret_cast<v8*>(xs + (size_t)m * ldl + k0) = u.vv;
      }
    }
    __syncthreads();
  }
  const bool mok = r < p.M;
  const T* xrow = LN ? reinterpret_cast<const T*>(xs_raw) + (size_t)(mok ? r : 0) * ldl + 8 * q
                     : static_cast<const T*>(p.x) + (size_t)(mok ? r : 0) * p.ldx + 8 * q;
  const v8 zero = {};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int sb = s0; sb < s1; sb += kBatch) {
    if (sb != s0) load_w(sb);
    v8 b[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) b[u] = *reinterpret_cast<const v8*>(xrow + 32 * min(sb + u, s1 - 1));
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const bool live = mok && sb + u < s1;  // past the range: a repeated step, zeroed
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
