// Backward of the KDA layer's front end and of the hybrid stack's LayerNorm
// (the autograd backward of KDAHybridLayer's short convolution and
// activations, /root/reference/ops_fused.py:480-581, and of _Fp32LayerNorm,
// ops_fused.py:42-60). fp32 arithmetic; gradients are written in the
// tensors' own dtypes, the weight gradients accumulate in fp32 buffers.
//
// kda_gates_bwd_kernel  one workgroup per token row: q/k head vectors a wave
//   each (F.normalize(silu(a)): du = (dy - y (y.dy)) / |u|, da = du silu'(a)),
//   then v (silu), the gate pre-activation (g = -softplus(z) * decay:
//   dz = -decay sigmoid(z) dg, 1 above softplus's threshold) and beta
//   (sigmoid).
// short_conv_bwd_kernel thread per (channel, run of tokens, b): dx of the
//   run (the transposed 3-tap filter), and the run's sums for the filter taps
//   and the bias, added to fp32 buffers; the first run also writes the
//   lookback rows' gradient when asked.
// layer_norm_bwd_kernel wave per row, 8 waves per workgroup (4 above 2048
//   channels), 1 to 16 rows per wave (as many as keep about 1024 workgroups in flight): dx from the
//   recomputed mean and rstd; the rows' dy x^ and dy sums stay in registers,
//   meet in LDS across the eight waves, then add into fp32 buffers. At 4096
//   rows of 2048 one row per wave takes the kernel from 366 us (64 workgroups
//   of 16 rows per wave, one wave per CU) to the latency of a few rows.

#include <hip/hip_runtime.h>

#include "attn_common.h"
#include "kch_kernels.h"

namespace kch {

namespace {

__device__ __forceinline__ float dsilu(float a) {
  const float s = sigmoid_f(a);
  return s * (1.f + a * (1.f - s));
}

template <typename T>
__global__ __launch_bounds__(256) void kda_gates_bwd_kernel(KdaGatesBwdParams p) {
  const long long row = blockIdx.x;
  const T* pr = static_cast<const T*>(p.proj) + row * p.ld_proj;
  const T* gr = static_cast<const T*>(p.gl) + row * p.ld_gl;
  T* dpr = static_cast<T*>(p.dproj) + row * p.ld_proj;
  T* dgr = static_cast<T*>(p.dgl) + row * p.ld_gl;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int HK = p.H * p.K;
  for (int h = wave; h < 2 * p.H; h += 4) {
    const T* src = pr + (size_t)h * p.K;
    const T* dy = h < p.H ? static_cast<const T*>(p.dq) + (row * p.H + h) * p.K
                          : static_cast<const T*>(p.dk) + (row * p.H + (h - p.H)) * p.K;
    float a[4], u[4], g[4];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      a[j] = e < p.K ? to_f32(src[e]) : 0.f;
      u[j] = e < p.K ? stored<T>(silu_f(a[j])) : 0.f;
      g[j] = e < p.K ? to_f32(dy[e]) : 0.f;
      ss += u[j] * u[j];
    }
    const float n = stored<T>(sqrtf(wave_sum(ss)));
    const float nn = fmaxf(n, 1e-12f);
    float yd = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) yd += (u[j] / nn) * g[j];
    yd = wave_sum(yd);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      if (e < p.K) {
        const float du = n > 1e-12f ? (g[j] - (u[j] / nn) * yd) / nn : g[j] / nn;
        dpr[(size_t)h * p.K + e] = from_f32<T>(du * dsilu(a[j]));
      }
    }
  }
  const int nv = p.HV * p.V, ng = p.HV * p.K;
  const T* dv = static_cast<const T*>(p.dv) + row * nv;
  const T* dg = static_cast<const T*>(p.dg) + row * ng;
  const T* db = static_cast<const T*>(p.dbeta) + row * p.HV;
  for (int i = threadIdx.x; i < nv; i += 256)
    dpr[2 * HK + i] = from_f32<T>(to_f32(dv[i]) * dsilu(to_f32(pr[2 * HK + i])));
  for (int i = threadIdx.x; i < ng; i += 256) {
    const float z = to_f32(gr[i]);
    const float sp = z > 20.f ? 1.f : sigmoid_f(z);
    dgr[i] = from_f32<T>(-p.decay_scale * sp * to_f32(dg[i]));
  }
  for (int i = threadIdx.x; i < p.HV; i += 256) {
    const float s = sigmoid_f(to_f32(pr[2 * HK + nv + i]));
    dpr[2 * HK + nv + i] = from_f32<T>(to_f32(db[i]) * s * (1.f - s));
  }
}

constexpr int kConvRun = 64;

template <typename T>
__global__ __launch_bounds__(256) void short_conv_bwd_kernel(ShortConvBwdParams p) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= p.d) return;
  const int run = blockIdx.y, b = blockIdx.z;
  const int t0 = run * kConvRun, t1 = min(t0 + kConvRun, p.T);
  const T* x = static_cast<const T*>(p.x) + (size_t)b * p.T * p.d + c;
  const T* dy = static_cast<const T*>(p.dy) + (size_t)b * p.T * p.d + c;
  T* dx = static_cast<T*>(p.dx) + (size_t)b * p.T * p.d + c;
  const T* w = static_cast<const T*>(p.weight);
  const float w0 = to_f32(w[c * 3 + 0]), w1 = to_f32(w[c * 3 + 1]), w2 = to_f32(w[c * 3 + 2]);
  auto xv = [&](int t) -> float {
    if (t >= 0) return to_f32(x[(size_t)t * p.d]);
    if (p.lookback) return to_f32(static_cast<const T*>(p.lookback)[((size_t)b * 2 + (t + 2)) * p.d + c]);
    return 0.f;
  };
  auto dyv = [&](int t) -> float { return t < p.T ? to_f32(dy[(size_t)t * p.d]) : 0.f; };
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, sb = 0.f;
  float xm2 = xv(t0 - 2), xm1 = xv(t0 - 1);
  float d1 = dyv(t0 + 1), d2 = dyv(t0 + 2);
  for (int t = t0; t < t1; ++t) {
    const float d0 = t == t0 ? dyv(t0) : d1;
    if (t != t0) {
      d1 = d2;
      d2 = dyv(t + 2);
    }
    const float xc = xv(t);
    // out[t] = w0 x[t-2] + w1 x[t-1] + w2 x[t] + bias
    dx[(size_t)t * p.d] = from_f32<T>(w2 * d0 + w1 * d1 + w0 * d2);
    s0 += d0 * xm2;
    s1 += d0 * xm1;
    s2 += d0 * xc;
    sb += d0;
    xm2 = xm1;
    xm1 = xc;
  }
  atomicAdd(p.dw + c * 3 + 0, s0);
  atomicAdd(p.dw + c * 3 + 1, s1);
  atomicAdd(p.dw + c * 3 + 2, s2);
  if (p.db) atomicAdd(p.db + c, sb);
  if (p.dlookback && run == 0) {
    // x[-2] feeds out[0] through w0; x[-1] feeds out[0] through w1 and out[1]
    // through w0 (dy past T is zero)
    T* dlb = static_cast<T*>(p.dlookback) + (size_t)b * 2 * p.d + c;
    const float g0 = dyv(0), g1 = dyv(1);
    dlb[0] = from_f32<T>(w0 * g0);
    dlb[p.d] = from_f32<T>(w1 * g0 + w0 * g1);
  }
}

constexpr int kLnWaves = 8;
constexpr int kLnMaxRowsPerWave = 16;

// NJ = channels per lane (d <= 64 NJ): the rows' dy x^ and dy sums stay in
// registers; the four waves meet in LDS at the end.
template <typename T, typename WT, int NJ, int NW>
__global__ __launch_bounds__(64 * NW) void layer_norm_bwd_kernel(LayerNormBwdParams p, int rpw) {
  extern __shared__ float lds[];  // [2][d]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int d = p.d;
  const WT* w = static_cast<const WT*>(p.w);
  float aw[NJ], ab[NJ], wv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int i = lane + 64 * j;
    aw[j] = ab[j] = 0.f;
    wv[j] = i < d ? to_f32(w[i]) : 0.f;
  }
  const long long r0 = ((long long)blockIdx.x * NW + wave) * rpw;
  for (int rr = 0; rr < rpw; ++rr) {
    const long long row = r0 + rr;
    if (row >= p.rows) break;
    const T* x = static_cast<const T*>(p.x) + row * d;
    const T* dy = static_cast<const T*>(p.dy) + row * d;
    T* dx = static_cast<T*>(p.dx) + row * d;
    float xv[NJ], gv[NJ];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = lane + 64 * j;
      xv[j] = i < d ? to_f32(x[i]) : 0.f;
      gv[j] = i < d ? to_f32(dy[i]) : 0.f;
      s += xv[j];
    }
    const float mean = wave_sum(s) / d;
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = lane + 64 * j;
      const float e = i < d ? xv[j] - mean : 0.f;
      v += e * e;
    }
    const float rstd = rsqrtf(wave_sum(v) / d + p.eps);
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      xv[j] = (xv[j] - mean) * rstd;  // now x^
      const float g = gv[j] * wv[j];
      sg += g;
      sgx += g * xv[j];
    }
    sg = wave_sum(sg) / d;
    sgx = wave_sum(sgx) / d;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = lane + 64 * j;
      if (i < d) {
        dx[i] = from_f32<T>(rstd * (gv[j] * wv[j] - sg - xv[j] * sgx));
        aw[j] += gv[j] * xv[j];
        ab[j] += gv[j];
      }
    }
  }
  // the waves' sums, one wave after another into [2][d] of LDS
  for (int wv_ = 0; wv_ < NW; ++wv_) {
    if (wave == wv_) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int i = lane + 64 * j;
        if (i < d) {
          lds[i] = (wv_ ? lds[i] : 0.f) + aw[j];
          lds[d + i] = (wv_ ? lds[d + i] : 0.f) + ab[j];
        }
      }
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < d; i += 64 * NW) {
    atomicAdd(p.dw + i, lds[i]);
    if (p.db) atomicAdd(p.db + i, lds[d + i]);
  }
}

template <typename T, typename WT, int NJ, int NW>
void ln_bwd_launch(const LayerNormBwdParams& p, hipStream_t s) {
  long long rpw = (p.rows + NW * 1024 - 1) / (NW * 1024);
  rpw = rpw < 1 ? 1 : (rpw > kLnMaxRowsPerWave ? kLnMaxRowsPerWave : rpw);
  const long long per_block = NW * rpw;
  const unsigned blocks = (unsigned)((p.rows + per_block - 1) / per_block);
  const size_t lds = (size_t)2 * p.d * sizeof(float);
  hipLaunchKernelGGL((layer_norm_bwd_kernel<T, WT, NJ, NW>), dim3(blocks), dim3(64 * NW), lds, s, p,
                     (int)rpw);
}

// eight waves per workgroup up to 2048 channels; four beyond (their rows
// take twice the registers)
template <typename T, typename WT>
hipError_t ln_bwd_nj(const LayerNormBwdParams& p, hipStream_t s) {
  const int nj = (p.d + 63) / 64;
  if (nj <= 8) ln_bwd_launch<T, WT, 8, kLnWaves>(p, s);
  else if (nj <= 16) ln_bwd_launch<T, WT, 16, kLnWaves>(p, s);
  else if (nj <= 32) ln_bwd_launch<T, WT, 32, kLnWaves>(p, s);
  else ln_bwd_launch<T, WT, 64, 4>(p, s);
  return hipGetLastError();
}

template <typename T>
hipError_t ln_bwd_w(const LayerNormBwdParams& p, int wdtype, hipStream_t s) {
  if (wdtype == DT_F32) return ln_bwd_nj<T, float>(p, s);
  if (wdtype == DT_BF16) return ln_bwd_nj<T, bf16_t>(p, s);
  return ln_bwd_nj<T, _Float16>(p, s);
}

}  // namespace

hipError_t kda_gates_bwd_dispatch(const KdaGatesBwdParams& p, int dtype, hipStream_t stream) {
  const unsigned rows = (unsigned)((long long)p.B * p.T);
  if (dtype == DT_F32) hipLaunchKernelGGL(kda_gates_bwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
  else if (dtype == DT_BF16) hipLaunchKernelGGL(kda_gates_bwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  else hipLaunchKernelGGL(kda_gates_bwd_kernel<_Float16>, dim3(rows), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t short_conv_bwd_dispatch(const ShortConvBwdParams& p, int dtype, hipStream_t stream) {
  const dim3 grid((p.d + 255) / 256, (p.T + kConvRun - 1) / kConvRun, p.B);
  if (dtype == DT_F32) hipLaunchKernelGGL(short_conv_bwd_kernel<float>, grid, dim3(256), 0, stream, p);
  else if (dtype == DT_BF16) hipLaunchKernelGGL(short_conv_bwd_kernel<bf16_t>, grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL(short_conv_bwd_kernel<_Float16>, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t layer_norm_bwd_dispatch(const LayerNormBwdParams& p, int dtype, int wdtype, hipStream_t stream) {
  if (dtype == DT_F32) return ln_bwd_w<float>(p, wdtype, stream);
  if (dtype == DT_BF16) return ln_bwd_w<bf16_t>(p, wdtype, stream);
  return ln_bwd_w<_Float16>(p, wdtype, stream);
}

}  // namespace kch
