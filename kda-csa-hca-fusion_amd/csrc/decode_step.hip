// Device-driven kernels of a hybrid decode step (gfx950), one new token per
// sequence. Every count that changes from step to step -- the token's position,
// the accumulator and ring slots, whether a block completes -- is derived from
// one device counter, n_seen (tokens the caches held before this step), so the
// launches of a step are the same on every step and a captured graph of them
// replays correctly.
//
// kda_front_kernel   LayerNorm of the residual row (_Fp32LayerNorm,
//   /root/reference/ops_fused.py:42-60), the causal depthwise convolution over
//   [lookback ; h] (ops_fused.py:480-551), then lookback <- [lookback[1] ; h].
//   One workgroup per sequence; thread t owns channels 8 t + 2048 j .. + 7, so
//   it reads and rewrites its own lookback entries only.
// kda_step_kernel    the token's KDA activations (ops_fused.py:571-581):
//   q, k = normalize(silu(.)) per head, v = silu(.), g = -softplus(g_up g_down)
//   * decay, beta = sigmoid(.), each rounded to the layer dtype where the
//   reference stores it, and the recurrent update of the state
//   (ops_kda.py:175-267: S <- S e^g; S <- S + beta k (v - k^T S); o = q^T S
//   scale). Workgroup (sequence, value head, 32 value columns); thread
//   (column tid / 8, phase tid % 8) owns state rows phase + 8 i. Optionally it
//   also advances the conv lookback (the front then ran in the projection's
//   prologue: linear_rows_body.h).
// cache_step_kernel  CSADecodingCache.append_step / HCADecodingCache.append_step
//   for one token (ops_decoding_cache.py:631-782, 1200-1267): the ring-window
//   row, the accumulator row and, on the block's last token, the block's
//   compressed row (softmax over the block's positions of Z + B per channel,
//   weighting C; CSA overlaps the previous block's b-branch rows), its
//   attention key row and, for CSA, its indexer key row with the inverse norm;
//   then the b-branch rows the next CSA block overlaps with. One workgroup per
//   sequence.
// cache_step_rows_kernel  the append beside a row projection of the same step
//   (the query up-projection: linear_rows_body.h) in one launch.

#include "attn_common.h"
#include "kch_kernels.h"
#include "linear_rows_body.h"

namespace kch {

namespace {

// Block-wide sum over the 256 threads (red: 4 floats of LDS, reusable after
// the call returns in every thread).
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float* f) {
  if constexpr (sizeof(T) == 2) {
    union { T h[8]; uint4 u; } r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.h[i] = from_f32<T>(f[i]);
    *reinterpret_cast<uint4*>(p) = r.u;
  } else {
    reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
  }
}

// ---------------------------------------------------------------------------
template <typename T, typename WT>
__global__ __launch_bounds__(256) void kda_front_kernel(KdaFrontParams p) {
  constexpr int G = 2;  // 8-channel groups per thread: d <= 4096
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int d = p.d;
  const T* x = static_cast<const T*>(p.x) + (size_t)b * p.ldx;
  float v[G][8];
  float s = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int c0 = 8 * tid + 2048 * g;
    if (c0 < d) {
      Load8<T>::run(x + c0, v[g]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[g][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[g][i];
  }
  const float mean = block_sum(s, red) / (float)d;
  float ss = 0.f;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (8 * tid + 2048 * g >= d) continue;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float dv = v[g][i] - mean;
      ss += dv * dv;
    }
  }
  const float rstd = 1.f / sqrtf(block_sum(ss, red) / (float)d + p.eps);
  const WT* lw = static_cast<const WT*>(p.ln_w);
  const WT* lb = static_cast<const WT*>(p.ln_b);
  const T* cw = static_cast<const T*>(p.conv_w);
  const T* cb = static_cast<const T*>(p.conv_b);
  T* look = static_cast<T*>(p.lookback) + (size_t)b * 2 * d;
  T* out = static_cast<T*>(p.out) + (size_t)b * d;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int c0 = 8 * tid + 2048 * g;
    if (c0 >= d) continue;
    float w8[8], b8[8], h[8], l0[8], l1[8], w3[24], bias[8], o[8];
    Load8<WT>::run(lw + c0, w8);
    if (lb) {
      Load8<WT>::run(lb + c0, b8);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) b8[i] = 0.f;
    }
    Load8<T>::run(look + c0, l0);
    Load8<T>::run(look + d + c0, l1);
#pragma unroll
    for (int u = 0; u < 3; ++u) Load8<T>::run(cw + 3 * c0 + 8 * u, w3 + 8 * u);
    if (cb) {
      Load8<T>::run(cb + c0, bias);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) bias[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // the LayerNorm output as the layer receives it (rounded to the dtype)
      h[i] = stored<T>((v[g][i] - mean) * rstd * w8[i] + b8[i]);
      // out[t] = bias + w0 x[t-2] + w1 x[t-1] + w2 x[t]
      o[i] = fmaf(w3[3 * i + 2], h[i], fmaf(w3[3 * i + 1], l1[i], fmaf(w3[3 * i], l0[i], bias[i])));
    }
    store8<T>(out + c0, o);
    store8<T>(look + c0, l1);
    store8<T>(look + d + c0, h);
  }
}

// ---------------------------------------------------------------------------
template <int K, typename T>
__global__ __launch_bounds__(256) void kda_step_kernel(KdaStepParams p) {
  constexpr int RPT = K / 8;
  constexpr int KJ = (K + 63) / 64;
  __shared__ float sq[K], sk[K], sg[K], sgd[K];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvs = p.V / 32;
  const int vs = blockIdx.x % nvs;
  const int bh = blockIdx.x / nvs;
  const int hv = bh % p.HV, b = bh / p.HV;
  const int h = hv / (p.HV / p.H);
  const int col = vs * 32 + (tid >> 3), ph = tid & 7;
  const int HK = p.H * K, HVV = p.HV * p.V;
  const T* pr = static_cast<const T*>(p.proj) + (size_t)b * p.ld_proj;
  float* st = p.state + (size_t)(b * p.HV + hv) * K * p.V + col;
  if (p.look) {
    // the conv lookback advances: [look[0] ; look[1]] <- [look[1] ; h], this
    // workgroup's slice of the d channels (the projection that read the old
    // lookback has finished)
    const int nwg = p.HV * nvs, wi = hv * nvs + vs;
    const int per = ((p.d + nwg - 1) / nwg + 7) & ~7;
    const int c1 = min(p.d, (wi + 1) * per);
    T* lk = static_cast<T*>(p.look) + (size_t)b * 2 * p.d;
    const T* hh = static_cast<const T*>(p.h_in) + (size_t)b * p.d;
    for (int c = wi * per + tid; c < c1; c += 256) {
      lk[c] = lk[p.d + c];
      lk[p.d + c] = hh[c];
    }
  }

  // the state column and this thread's gate weights first: their loads
  // overlap the activations below
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = st[(size_t)(ph + 8 * i) * p.V];
  constexpr int HALF = K / 2;
  constexpr int GW = (K + 127) / 128;  // gate outputs per thread pair
  typedef T vec8 __attribute__((ext_vector_type(8)));  // held as stored (16-bit types packed)
  const int half = tid & 1;
  vec8 wg[GW][HALF / 8];
#pragma unroll
  for (int r = 0; r < GW; ++r) {
    const int i = (tid >> 1) + 128 * r;
    const T* wr = static_cast<const T*>(p.g_up) + (size_t)(hv * K + min(i, K - 1)) * K + half * HALF;
#pragma unroll
    for (int j = 0; j < HALF / 8; ++j) wg[r][j] = *reinterpret_cast<const vec8*>(wr + 8 * j);
  }
  const float vt = stored<T>(silu_f(to_f32(pr[2 * HK + hv * p.V + col])));
  const float bt = stored<T>(sigmoid_f(to_f32(pr[2 * HK + HVV + hv])));
  if (tid < K) sgd[tid] = to_f32(pr[2 * HK + HVV + p.HV + tid]);
  if (wave < 2) {
    // F.normalize(F.silu(.)) of head h of q (wave 0) or k (wave 1): silu's
    // output, the norm and the quotient are each stored in T
    const T* src = pr + wave * HK + h * K;
    float vals[KJ];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int e = lane + 64 * j;
      vals[j] = e < K ? stored<T>(silu_f(to_f32(src[e]))) : 0.f;
      ss += vals[j] * vals[j];
    }
    const float nrm = fmaxf(stored<T>(sqrtf(wave_sum(ss))), 1e-12f);
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int e = lane + 64 * j;
      if (e < K) {
        const float qk = stored<T>(vals[j] / nrm);
        if (wave == 0) sq[e] = qk * p.scale;
        else sk[e] = qk;
      }
    }
  }
  __syncthreads();
  // gate pre-activations of head hv: gl[i] = g_up[hv K + i, :] . g_down, two
  // threads per output (halves of the dot product)
  {
#pragma unroll
    for (int r = 0; r < GW; ++r) {
      const int i = (tid >> 1) + 128 * r;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < HALF; ++j) acc = fmaf(to_f32(wg[r][j / 8][j % 8]), sgd[half * HALF + j], acc);
      acc += __shfl_xor(acc, 1);
      if (half == 0 && i < K) {
        // the linear's output, -softplus and the decay product are each stored in T
        float g = stored<T>(-stored<T>(softplus_f(stored<T>(acc))) * p.decay_scale);
        g = fmaxf(g, p.g_clamp_min);
        sg[i] = expf(g);
      }
    }
  }
  __syncthreads();
  float kS = 0.f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    S[i] *= sg[ph + 8 * i];
    kS += sk[ph + 8 * i] * S[i];
  }
  kS += __shfl_xor(kS, 1);
  kS += __shfl_xor(kS, 2);
  kS += __shfl_xor(kS, 4);
  const float dlt = bt * (vt - kS);
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    S[i] += sk[ph + 8 * i] * dlt;
    o += sq[ph + 8 * i] * S[i];
  }
  o += __shfl_xor(o, 1);
  o += __shfl_xor(o, 2);
  o += __shfl_xor(o, 4);
  if (ph == 0) static_cast<T*>(p.o)[(size_t)b * HVV + hv * p.V + col] = from_f32<T>(o);
#pragma unroll
  for (int i = 0; i < RPT; ++i) st[(size_t)(ph + 8 * i) * p.V] = S[i];
}

// ---------------------------------------------------------------------------
// Softmax-weighted mean over a block's positions for one channel: rows
// j < nrow of branch a (value va(j), logit za(j) + Ba[j]) and, with `prev`, m
// rows of branch b; two passes (max, then exp-weighted sums), a before b.
template <typename VA, typename ZA, typename VB, typename ZB>
__device__ __forceinline__ float block_mean(int m, bool prev, VA va, ZA za, VB vb, ZB zb) {
  float mx = -INFINITY;
  for (int j = 0; j < m; ++j) mx = fmaxf(mx, za(j));
  if (prev)
    for (int j = 0; j < m; ++j) mx = fmaxf(mx, zb(j));
  float den = 0.f, num = 0.f;
  for (int j = 0; j < m; ++j) {
    const float e = expf(za(j) - mx);
    den += e;
    num += e * va(j);
  }
  if (prev)
    for (int j = 0; j < m; ++j) {
      const float e = expf(zb(j) - mx);
      den += e;
      num += e * vb(j);
    }
  return num / den;
}

// The append of sequence b (one workgroup of 256 threads).
template <typename T>
__device__ __forceinline__ void cache_step_block(const CacheStepParams& p, int b) {
  __shared__ float red[8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = p.n_seen[0];
  const int m = p.m, c = p.c, cI = p.cI;
  const int W = p.csa ? 4 * c + 2 * cI : 2 * c;
  const int j_cur = t % m, blk = t / m;
  const bool complete = j_cur == m - 1 && blk < p.cap;
  const T* x = static_cast<const T*>(p.proj) + (size_t)b * p.ld_proj;
  T* acc = static_cast<T*>(p.acc) + (size_t)b * m * W;

  // ring-window row: the token's C (a-branch) row, L2-normalised (wave 0)
  if (p.ring && wave == 0) {
    float v[4];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int ch = lane + 64 * u;
      v[u] = ch < c ? to_f32(x[ch]) : 0.f;
      ss += v[u] * v[u];
    }
    const float inv = p.normalize ? l2_inv(wave_sum(ss)) : 1.f;
    T* row = static_cast<T*>(p.ring) + ((size_t)b * p.win + t % p.win) * c;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int ch = lane + 64 * u;
      if (ch < c) row[ch] = from_f32<T>(v[u] * inv);
    }
  }
  if (!complete) {
    for (int e = tid; e < W; e += 256) acc[(size_t)j_cur * W + e] = x[e];
    return;
  }
  // row j of the block: the accumulator, the last one this token's projections
  auto row = [&](int j) { return j == m - 1 ? x : acc + (size_t)j * W; };
  const size_t orow = (size_t)b * p.cap + blk;
  T* prev = p.csa ? static_cast<T*>(p.prev) + (size_t)b * m * 2 * c : nullptr;
  const bool overlap = p.csa && blk > 0;
  float cval = 0.f, kval = 0.f;
  if (tid < c) {
    const int ch = tid;
    if (p.csa) {
      cval = block_mean(
          m, overlap, [&](int j) { return to_f32(row(j)[ch]); },
          [&](int j) { return to_f32(row(j)[2 * c + ch]) + p.Ba[j * c + ch]; },
          [&](int j) { return to_f32(prev[(size_t)j * 2 * c + ch]); },
          [&](int j) { return to_f32(prev[(size_t)j * 2 * c + c + ch]) + p.Bb[j * c + ch]; });
    } else {
      cval = block_mean(
          m, false, [&](int j) { return to_f32(row(j)[ch]); },
          [&](int j) { return to_f32(row(j)[c + ch]) + p.Ba[j * c + ch]; },
          [&](int j) { return 0.f; }, [&](int j) { return 0.f; });
    }
  } else if (p.csa && tid - c < cI) {
    const int ch = tid - c;
    kval = block_mean(
        m, false, [&](int j) { return to_f32(row(j)[4 * c + ch]); },
        [&](int j) { return to_f32(row(j)[4 * c + cI + ch]) + p.Bk[j * cI + ch]; },
        [&](int j) { return 0.f; }, [&](int j) { return 0.f; });
  }
  // the rows as the cache stores them (its dtype), then their norms
  const float cst = stored<T>(cval), kst = stored<T>(kval);
  const bool is_c = tid < c, is_k = p.csa && tid >= c && tid - c < cI;
  float sc = is_c ? cst * cst : 0.f, sk = is_k ? kst * kst : 0.f;
  sc = wave_sum(sc);
  sk = wave_sum(sk);
  if (lane == 0) {
    red[wave] = sc;
    red[4 + wave] = sk;
  }
  __syncthreads();  // also: every read of prev above is done
  if (is_c) {
    const float inv = p.normalize ? l2_inv(red[0] + red[1] + red[2] + red[3]) : 1.f;
    static_cast<T*>(p.c_rows)[orow * c + tid] = from_f32<T>(cval);
    static_cast<bf16_t*>(p.c_keys)[orow * c + tid] = (bf16_t)(cst * inv);
  }
  if (is_k) {
    static_cast<T*>(p.k_rows)[orow * cI + (tid - c)] = from_f32<T>(kval);
    if (tid == c) p.k_inv[orow] = 1.f / fmaxf(sqrtf(red[4] + red[5] + red[6] + red[7]), 1e-12f);
  }
  if (p.csa) {
    // the b-branch rows [Cb | Zb] of this block, for the next one
    for (int e = tid; e < m * 2 * c; e += 256) {
      const int j = e / (2 * c), r = e - j * 2 * c;
      prev[e] = row(j)[r < c ? c + r : 3 * c + (r - c)];
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void cache_step_kernel(CacheStepParams p) {
  cache_step_block<T>(p, (int)blockIdx.x);
}

// A cache append and a row projection of the same decode step in one launch:
// the first ngemv workgroups take the projection's 16-column tiles, the rest
// one sequence's append each. Both read only the step's projection row.
template <typename T>
__global__ __launch_bounds__(256) void cache_step_rows_kernel(CacheStepParams cp, LinearRowsParams lp,
                                                              int ngemv) {
  const int blk = (int)blockIdx.x;
  if (blk < ngemv) rows_detail::linear_rows_block<T, void>(lp, blk);
  else cache_step_block<T>(cp, blk - ngemv);
}

template <typename T>
hipError_t kda_front_launch(const KdaFrontParams& p, int wdtype, hipStream_t s) {
  const dim3 grid((unsigned)p.B), block(256);
  if (wdtype == DT_F32) hipLaunchKernelGGL((kda_front_kernel<T, float>), grid, block, 0, s, p);
  else if (wdtype == DT_BF16) hipLaunchKernelGGL((kda_front_kernel<T, bf16_t>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((kda_front_kernel<T, _Float16>), grid, block, 0, s, p);
  return hipGetLastError();
}

template <typename T>
hipError_t kda_step_launch(const KdaStepParams& p, hipStream_t s) {
  const dim3 grid((unsigned)(p.B * p.HV * (p.V / 32))), block(256);
  switch (p.K) {
    case 16: hipLaunchKernelGGL((kda_step_kernel<16, T>), grid, block, 0, s, p); break;
    case 32: hipLaunchKernelGGL((kda_step_kernel<32, T>), grid, block, 0, s, p); break;
    case 64: hipLaunchKernelGGL((kda_step_kernel<64, T>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((kda_step_kernel<128, T>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((kda_step_kernel<256, T>), grid, block, 0, s, p); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t kda_front_dispatch(const KdaFrontParams& p, int dtype, int wdtype, hipStream_t s) {
  if (dtype == DT_F32) return kda_front_launch<float>(p, wdtype, s);
  if (dtype == DT_BF16) return kda_front_launch<bf16_t>(p, wdtype, s);
  return kda_front_launch<_Float16>(p, wdtype, s);
}

hipError_t kda_step_dispatch(const KdaStepParams& p, int dtype, hipStream_t s) {
  if (dtype == DT_F32) return kda_step_launch<float>(p, s);
  if (dtype == DT_BF16) return kda_step_launch<bf16_t>(p, s);
  return kda_step_launch<_Float16>(p, s);
}

hipError_t cache_step_rows_dispatch(const CacheStepParams& cp, const LinearRowsParams& lp, int dtype,
                                   hipStream_t s) {
  const int ngemv = (lp.N + 15) / 16;
  const dim3 grid((unsigned)(ngemv + cp.B)), block(256);
  if (dtype == DT_BF16) hipLaunchKernelGGL(cache_step_rows_kernel<bf16_t>, grid, block, 0, s, cp, lp, ngemv);
  else hipLaunchKernelGGL(cache_step_rows_kernel<_Float16>, grid, block, 0, s, cp, lp, ngemv);
  return hipGetLastError();
}

hipError_t cache_step_dispatch(const CacheStepParams& p, int dtype, hipStream_t s) {
  const dim3 grid((unsigned)p.B), block(256);
  if (dtype == DT_F32) hipLaunchKernelGGL(cache_step_kernel<float>, grid, block, 0, s, p);
  else if (dtype == DT_BF16) hipLaunchKernelGGL(cache_step_kernel<bf16_t>, grid, block, 0, s, p);
  else hipLaunchKernelGGL(cache_step_kernel<_Float16>, grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace kch
