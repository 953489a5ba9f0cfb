// KDA layer front-end: the causal depthwise short convolution and the fused
// q/k/v/g/beta activations that sit between the layer's projection GEMMs and
// the KDA kernels (KDAHybridLayer.forward_functional, ops_fused.py:480-581).
//
// Both kernels are HBM-bound elementwise passes in fp32 arithmetic. Where the
// reference chains several torch operations on a bf16 / fp16 tensor, every
// intermediate it stores is rounded to that dtype here too.

#include <hip/hip_runtime.h>

#include "attn_common.h"
#include "kch_kernels.h"

namespace kch {

namespace {

// Eight consecutive channels as fp32 (VEC=8) or one channel (VEC=1).
template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float* f) {
  if constexpr (VEC == 8) {
    Load8<T>::run(p, f);
  } else {
    f[0] = to_f32(*p);
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const float* f) {
  if constexpr (VEC == 8 && sizeof(T) == 2) {
    union { T h[8]; uint4 u; } r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.h[i] = from_f32<T>(f[i]);
    *reinterpret_cast<uint4*>(p) = r.u;
  } else if constexpr (VEC == 8) {
    reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
  } else {
    *p = from_f32<T>(f[0]);
  }
}

// out[b,t,c] = bias[c] + w[c,0] x[t-2] + w[c,1] x[t-1] + w[c,2] x[t], where
// x[-2], x[-1] are lookback[b,0], lookback[b,1] (zeros without a lookback).
// A thread owns VEC channels of a run of RUN tokens and slides the window,
// so every input row is read once; a wave covers 64 channel vectors of the
// same tokens (contiguous 1 KB rows for VEC=8, bf16).
template <typename T, int VEC, int RUN>
__global__ __launch_bounds__(256) void short_conv_kernel(ShortConvParams p) {
  const int nvec = p.d / VEC;
  const int runs = (p.T + RUN - 1) / RUN;
  const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
  if (id >= (long long)nvec * runs * p.B) return;
  const int cv = (int)(id % nvec);
  const long long rest = id / nvec;
  const int run = (int)(rest % runs);
  const int b = (int)(rest / runs);
  const int c0 = cv * VEC;
  const T* x = static_cast<const T*>(p.x) + (size_t)b * p.T * p.d + c0;
  const T* w = static_cast<const T*>(p.weight);
  float w0[VEC], w1[VEC], w2[VEC], bias[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    w0[i] = to_f32(w[(c0 + i) * 3 + 0]);
    w1[i] = to_f32(w[(c0 + i) * 3 + 1]);
    w2[i] = to_f32(w[(c0 + i) * 3 + 2]);
    bias[i] = p.bias ? to_f32(static_cast<const T*>(p.bias)[c0 + i]) : 0.f;
  }
  const int t0 = run * RUN;
  const int t1 = min(t0 + RUN, p.T);
  float xm2[VEC], xm1[VEC], cur[VEC], o[VEC];
  auto fetch = [&](int t, float* f) {
    if (t >= 0) {
      load_vec<T, VEC>(x + (size_t)t * p.d, f);
    } else if (p.lookback) {
      load_vec<T, VEC>(static_cast<const T*>(p.lookback) + ((size_t)b * 2 + (t + 2)) * p.d + c0, f);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) f[i] = 0.f;
    }
  };
  fetch(t0 - 2, xm2);
  fetch(t0 - 1, xm1);
  T* out = static_cast<T*>(p.out) + (size_t)b * p.T * p.d + c0;
  for (int t = t0; t < t1; ++t) {
    load_vec<T, VEC>(x + (size_t)t * p.d, cur);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      o[i] = fmaf(w2[i], cur[i], fmaf(w1[i], xm1[i], fmaf(w0[i], xm2[i], bias[i])));
      xm2[i] = xm1[i];
      xm1[i] = cur[i];
    }
    store_vec<T, VEC>(out + (size_t)t * p.d, o);
  }
}

// Workgroup (row, y) for token row `row`: y < QK_UNITS(H) -> waves take q/k
// head vectors 4y .. 4y + 3 of the 2H (silu, then per-head L2
// normalisation); higher y -> a 1024-element slice of v (silu), g (-softplus *
// decay) and beta (sigmoid). Spreading a row over several workgroups keeps a
// decode step (one row per sequence) from running on a couple of CUs.
__host__ __device__ inline int gates_qk_units(int H) { return (2 * H + 3) / 4; }

template <typename T>
__global__ __launch_bounds__(256) void kda_gates_kernel(KdaGatesParams p) {
  const long long row = blockIdx.x;
  const T* pr = static_cast<const T*>(p.proj) + row * p.ld_proj;
  const T* gr = static_cast<const T*>(p.gl) + row * p.ld_gl;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int HK = p.H * p.K;
  const int qku = gates_qk_units(p.H);
  if ((int)blockIdx.y < qku) {
    const int h = 4 * blockIdx.y + wave;
    if (h >= 2 * p.H) return;
    const T* src = pr + (size_t)h * p.K;
    // F.normalize(F.silu(proj)) on a tensor of type T (ops_fused.py:571-572):
    // silu's output, the norm and the quotient are each stored in T
    float vals[4];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      vals[j] = e < p.K ? stored<T>(silu_f(to_f32(src[e]))) : 0.f;
      ss += vals[j] * vals[j];
    }
    const float nrm = fmaxf(stored<T>(sqrtf(wave_sum(ss))), 1e-12f);
    T* dst = h < p.H ? static_cast<T*>(p.q) + (row * p.H + h) * p.K
                     : static_cast<T*>(p.k) + (row * p.H + (h - p.H)) * p.K;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      if (e < p.K) dst[e] = from_f32<T>(vals[j] / nrm);
    }
    return;
  }
  const int nv = p.HV * p.V, ng = p.HV * p.K;
  const int i0 = ((int)blockIdx.y - qku) * 1024;
  T* v = static_cast<T*>(p.v) + row * nv;
  T* g = static_cast<T*>(p.g) + row * ng;
  for (int i = i0 + threadIdx.x; i < min(nv, i0 + 1024); i += 256)
    v[i] = from_f32<T>(silu_f(to_f32(pr[2 * HK + i])));
  // -softplus(.) is stored in T before the decay scale multiplies it (ops_fused.py:579)
  for (int i = i0 + threadIdx.x; i < min(ng, i0 + 1024); i += 256)
    g[i] = from_f32<T>(-stored<T>(softplus_f(to_f32(gr[i]))) * p.decay_scale);
  if (i0 == 0) {
    T* beta = static_cast<T*>(p.beta) + row * p.HV;
    for (int i = threadIdx.x; i < p.HV; i += 256)
      beta[i] = from_f32<T>(sigmoid_f(to_f32(pr[2 * HK + nv + i])));
  }
}

// Wave per token row (4 rows per workgroup), 16-byte loads and stores: lane
// (LPH lanes per head vector, LPH = K / 8) takes 8 consecutive channels. The
// q/k head vectors go 64 / LPH per pass (the L2 norm is a reduction over the
// head's LPH lanes), then v, g and beta, the loads of four passes in flight
// together. Rounding as in kda_gates_kernel; bf16 results take the
// activations on the hardware exponential (silu_t and the like), which round
// to the same bf16 values.
template <typename T, int LPH>
__global__ __launch_bounds__(256) void kda_gates_vec_kernel(KdaGatesParams p, long long rows) {
  constexpr int U = 4;  // passes whose loads are in flight together
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const T* pr = static_cast<const T*>(p.proj) + row * p.ld_proj;
  const T* gr = static_cast<const T*>(p.gl) + row * p.ld_gl;
  const int HK = p.H * p.K;
  constexpr int HPP = 64 / LPH;  // head vectors per pass
  const int c = lane % LPH;
  for (int h0 = 0; h0 < 2 * p.H; h0 += U * HPP) {
    float f[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u)
      Load8<T>::run(pr + (size_t)min(h0 + u * HPP + lane / LPH, 2 * p.H - 1) * p.K + 8 * c, f[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int h = h0 + u * HPP + lane / LPH;
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[u][i] = stored<T>(silu_t<T>(f[u][i]));
        ss += f[u][i] * f[u][i];
      }
#pragma unroll
      for (int o = 1; o < LPH; o <<= 1) ss += __shfl_xor(ss, o);
      // (an IEEE division: quotients of two 16-bit values often sit exactly
      // on a rounding tie, where a reciprocal's ulp decides the result)
      const float nrm = fmaxf(stored<T>(sqrtf(ss)), 1e-12f);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[u][i] = f[u][i] / nrm;
      if (h < 2 * p.H) {
        T* dst = h < p.H ? static_cast<T*>(p.q) + (row * p.H + h) * p.K
                         : static_cast<T*>(p.k) + (row * p.H + (h - p.H)) * p.K;
        store_vec<T, 8>(dst + 8 * c, f[u]);
      }
    }
  }
  const int nv8 = p.HV * p.V / 8, ng8 = p.HV * p.K / 8;
  T* v = static_cast<T*>(p.v) + row * (8LL * nv8);
  T* g = static_cast<T*>(p.g) + row * (8LL * ng8);
  for (int i0 = lane; i0 < nv8; i0 += U * 64) {
    float f[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) Load8<T>::run(pr + 2 * HK + 8 * min(i0 + 64 * u, nv8 - 1), f[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[u][e] = silu_t<T>(f[u][e]);
      if (i0 + 64 * u < nv8) store_vec<T, 8>(v + 8 * (i0 + 64 * u), f[u]);
    }
  }
  // -softplus(.) is stored in T before the decay scale multiplies it (ops_fused.py:579)
  for (int i0 = lane; i0 < ng8; i0 += U * 64) {
    float f[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) Load8<T>::run(gr + 8 * min(i0 + 64 * u, ng8 - 1), f[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[u][e] = -stored<T>(softplus_t<T>(f[u][e])) * p.decay_scale;
      if (i0 + 64 * u < ng8) store_vec<T, 8>(g + 8 * (i0 + 64 * u), f[u]);
    }
  }
  T* beta = static_cast<T*>(p.beta) + row * p.HV;
  for (int i = lane; i < p.HV; i += 64) beta[i] = from_f32<T>(sigmoid_t<T>(to_f32(pr[2 * HK + 8 * nv8 + i])));
}

// One workgroup per row: the row's values stay in registers (d <= 4096), the
// mean and the biased variance come from two block reductions in fp32, then
// (x - mean) * rstd * w + b is rounded once to the output dtype.
template <typename T, typename WT>
__global__ __launch_bounds__(256) void layer_norm_kernel(LayerNormParams p) {
  constexpr int MAXV = 16;
  __shared__ float red[8];
  const long long row = blockIdx.x;
  const T* x = static_cast<const T*>(p.x) + row * p.d;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v[MAXV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int e = tid + 256 * i;
    v[i] = e < p.d ? to_f32(x[e]) : 0.f;
    s += v[i];
  }
  for (int e = tid + 256 * MAXV; e < p.d; e += 256) s += to_f32(x[e]);
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)p.d;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int e = tid + 256 * i;
    const float dv = v[i] - mean;
    ss += e < p.d ? dv * dv : 0.f;
  }
  for (int e = tid + 256 * MAXV; e < p.d; e += 256) {
    const float dv = to_f32(x[e]) - mean;
    ss += dv * dv;
  }
  ss = wave_sum(ss);
  if (lane == 0) red[4 + wave] = ss;
  __syncthreads();
  const float var = (red[4] + red[5] + red[6] + red[7]) / (float)p.d;
  const float rstd = 1.f / sqrtf(var + p.eps);
  const WT* w = static_cast<const WT*>(p.w);
  const WT* bb = static_cast<const WT*>(p.b);
  T* out = static_cast<T*>(p.out) + row * p.d;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int e = tid + 256 * i;
    if (e < p.d) {
      const float y = (v[i] - mean) * rstd * to_f32(w[e]) + (bb ? to_f32(bb[e]) : 0.f);
      out[e] = from_f32<T>(y);
    }
  }
  for (int e = tid + 256 * MAXV; e < p.d; e += 256) {
    const float y = (to_f32(x[e]) - mean) * rstd * to_f32(w[e]) + (bb ? to_f32(bb[e]) : 0.f);
    out[e] = from_f32<T>(y);
  }
}

// Wave per row (4 rows per workgroup): lane l holds 16-byte chunks
// l + 64 j (j < NC) of the row in registers, so d <= 512 NC; the mean and the
// biased variance are wave reductions in fp32 (two passes over the registers).
template <typename WT>
__device__ __forceinline__ void load_w8(const WT* w, float* f) {
  if constexpr (sizeof(WT) == 4) {
    const float4 a = reinterpret_cast<const float4*>(w)[0], b = reinterpret_cast<const float4*>(w)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    Load8<WT>::run(w, f);
  }
}

template <typename T, typename WT, int NC>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(LayerNormParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long row = (long long)blockIdx.x * 4 + wave;
  if (row >= p.rows) return;
  const T* x = static_cast<const T*>(p.x) + row * p.d;
  const int nch = p.d / 8;
  float v[NC][8];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int ch = lane + 64 * j;
    if (ch < nch) {
      Load8<T>::run(x + 8 * ch, v[j]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[j][i];
  }
  const float mean = wave_sum(s) / (float)p.d;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const bool ok = lane + 64 * j < nch;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float dv = v[j][i] - mean;
      ss += ok ? dv * dv : 0.f;
    }
  }
  const float var = wave_sum(ss) / (float)p.d;
  const float rstd = 1.f / sqrtf(var + p.eps);
  const WT* w = static_cast<const WT*>(p.w);
  const WT* bb = static_cast<const WT*>(p.b);
  T* out = static_cast<T*>(p.out) + row * p.d;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int ch = lane + 64 * j;
    if (ch < nch) {
      float wf[8], bf[8];
      load_w8<WT>(w + 8 * ch, wf);
      if (bb) {
        load_w8<WT>(bb + 8 * ch, bf);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) bf[i] = 0.f;
      }
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = (v[j][i] - mean) * rstd * wf[i] + bf[i];
      store_vec<T, 8>(out + 8 * ch, y);
    }
  }
}

template <typename T, typename WT>
hipError_t layer_norm_vec_launch(const LayerNormParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
  if (p.d <= 512) hipLaunchKernelGGL((layer_norm_vec_kernel<T, WT, 1>), grid, block, 0, s, p);
  else if (p.d <= 1024) hipLaunchKernelGGL((layer_norm_vec_kernel<T, WT, 2>), grid, block, 0, s, p);
  else if (p.d <= 2048) hipLaunchKernelGGL((layer_norm_vec_kernel<T, WT, 4>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((layer_norm_vec_kernel<T, WT, 8>), grid, block, 0, s, p);
  return hipGetLastError();
}

template <typename T>
hipError_t layer_norm_launch(const LayerNormParams& p, int wdtype, hipStream_t s) {
  // 16-byte rows of 16-bit values: the wave-per-row kernel
  const uintptr_t al = reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.out) |
                       reinterpret_cast<uintptr_t>(p.w) | reinterpret_cast<uintptr_t>(p.b);
  if constexpr (sizeof(T) == 2) {
    if (p.d % 8 == 0 && p.d <= 4096 && al % 16 == 0) {
      if (wdtype == DT_F32) return layer_norm_vec_launch<T, float>(p, s);
      if (wdtype == DT_BF16) return layer_norm_vec_launch<T, bf16_t>(p, s);
      return layer_norm_vec_launch<T, _Float16>(p, s);
    }
  }
  const dim3 grid((unsigned)p.rows), block(256);
  if (wdtype == DT_F32) hipLaunchKernelGGL((layer_norm_kernel<T, float>), grid, block, 0, s, p);
  else if (wdtype == DT_BF16) hipLaunchKernelGGL((layer_norm_kernel<T, bf16_t>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((layer_norm_kernel<T, _Float16>), grid, block, 0, s, p);
  return hipGetLastError();
}

template <typename T>
hipError_t short_conv_launch(const ShortConvParams& p, hipStream_t s) {
  constexpr int RUN = 16;
  const bool vec = (p.d % 8 == 0);
  const long long runs = (p.T + RUN - 1) / RUN;
  const long long threads = (long long)(vec ? p.d / 8 : p.d) * runs * p.B;
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  if (vec)
    hipLaunchKernelGGL((short_conv_kernel<T, 8, RUN>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((short_conv_kernel<T, 1, RUN>), grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t short_conv_dispatch(const ShortConvParams& p, int dtype, hipStream_t s) {
  if (dtype == DT_F32) return short_conv_launch<float>(p, s);
  if (dtype == DT_BF16) return short_conv_launch<bf16_t>(p, s);
  return short_conv_launch<_Float16>(p, s);
}

template <typename T>
bool gates_vec_launch(const KdaGatesParams& p, hipStream_t s) {
  const int lph = p.K / 8;
  const uintptr_t al = reinterpret_cast<uintptr_t>(p.proj) | reinterpret_cast<uintptr_t>(p.gl) |
                       reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
                       reinterpret_cast<uintptr_t>(p.v) | reinterpret_cast<uintptr_t>(p.g);
  if (p.K % 8 || lph < 1 || lph > 64 || (lph & (lph - 1)) || (p.HV * p.V) % 8 || al % 16 ||
      p.ld_proj % 8 || p.ld_gl % 8)
    return false;
  const long long rows = (long long)p.B * p.T;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  switch (lph) {
    case 1: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 1>), grid, block, 0, s, p, rows); break;
    case 2: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 2>), grid, block, 0, s, p, rows); break;
    case 4: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 4>), grid, block, 0, s, p, rows); break;
    case 8: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 8>), grid, block, 0, s, p, rows); break;
    case 16: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 16>), grid, block, 0, s, p, rows); break;
    case 32: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 32>), grid, block, 0, s, p, rows); break;
    default: hipLaunchKernelGGL((kda_gates_vec_kernel<T, 64>), grid, block, 0, s, p, rows); break;
  }
  return true;
}

hipError_t kda_gates_dispatch(const KdaGatesParams& p, int dtype, hipStream_t s) {
  // 16-byte rows of 16-bit values: the wave-per-row kernel
  if (dtype == DT_BF16 && gates_vec_launch<bf16_t>(p, s)) return hipGetLastError();
  if (dtype == DT_F16 && gates_vec_launch<_Float16>(p, s)) return hipGetLastError();
  const int slices = (max(p.HV * p.V, p.HV * p.K) + 1023) / 1024;
  const dim3 grid((unsigned)((long long)p.B * p.T), (unsigned)(gates_qk_units(p.H) + max(slices, 1))), block(256);
  if (dtype == DT_F32)
    hipLaunchKernelGGL((kda_gates_kernel<float>), grid, block, 0, s, p);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL((kda_gates_kernel<bf16_t>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((kda_gates_kernel<_Float16>), grid, block, 0, s, p);
  return hipGetLastError();
}

hipError_t layer_norm_dispatch(const LayerNormParams& p, int dtype, int wdtype, hipStream_t s) {
  if (dtype == DT_F32) return layer_norm_launch<float>(p, wdtype, s);
  if (dtype == DT_BF16) return layer_norm_launch<bf16_t>(p, wdtype, s);
  return layer_norm_launch<_Float16>(p, wdtype, s);
}

}  // namespace kch
