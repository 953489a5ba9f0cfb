// KDA per-token recurrence for gfx950 (decode steps and short sequences).
//
// Restates naive_recurrent_kda (/root/reference/ops_kda.py:175-267): per token
//   S <- S * exp(g_t)                      (per key channel, ops_kda.py:254)
//   S <- S + (beta_t k_t) (x) (v_t - k_t^T S)  (ops_kda.py:255-256)
//   o_t = (scale q_t)^T S                  (post-update state, ops_kda.py:257)
// with fp32 compute and the gate clamped at g_clamp_min (ops_kda.py:224-225);
// fp64 inputs compute in fp64 with an fp64 state, as the reference does for
// them (ops_kda.py:125-127).
//
// grid  : one workgroup per (b, hv, 32-column slice of V)
// block : 256 threads; thread (col = tid/8, phase = tid%8) owns state rows
//         phase + 8*i of column col, so k^T S and q^T S reduce over 8 lanes.
// This path is bound by the state read/write (K*V*4 bytes per head, twice).

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

template <typename AccT, typename T>
__device__ __forceinline__ AccT to_acc(T x) {
  if constexpr (sizeof(T) == 8) return (AccT)x;
  else return (AccT)to_f32(x);
}

template <int K, typename InT, typename AccT>
__global__ __launch_bounds__(256) void kda_recurrent_kernel(KdaParams p) {
  constexpr int RPT = K / 8;
  constexpr bool F64 = sizeof(AccT) == 8;
  __shared__ AccT sq[K], sk[K], sg[K];
  const int tid = threadIdx.x;
  const int nvs = (p.V + 31) / 32;
  const int vs = blockIdx.x % nvs;
  const int bh = blockIdx.x / nvs;
  const int hv = bh % p.HV;
  const int b = bh / p.HV;
  const int h = hv / (p.HV / p.H);
  const int col = vs * 32 + (tid >> 3);
  const int ph = tid & 7;
  const bool okc = col < p.V;
  const InT* gq = static_cast<const InT*>(p.q);
  const InT* gk = static_cast<const InT*>(p.k);
  const InT* gv = static_cast<const InT*>(p.v);
  const InT* gg = static_cast<const InT*>(p.g);
  const InT* gb = static_cast<const InT*>(p.beta);
  InT* go = static_cast<InT*>(p.o);
  const AccT* s0 = reinterpret_cast<const AccT*>(p.s0);
  AccT* s_out = reinterpret_cast<AccT*>(p.s_out);
  const AccT scale = F64 ? (AccT)p.scale64 : (AccT)p.scale;
  const AccT clampv = F64 ? (AccT)p.g_clamp_min64 : (AccT)p.g_clamp_min;
  const bool do_clamp = clampv > (AccT)-INFINITY;

  AccT S[RPT];
  const size_t sbase = (size_t)(b * p.HV + hv) * K * p.V;
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    S[i] = (s0 && okc) ? s0[sbase + (size_t)(ph + 8 * i) * p.V + col] : (AccT)0;

  for (int t = 0; t < p.T; ++t) {
    __syncthreads();
    if (tid < K) {
      const size_t qk = ((size_t)(b * p.T + t) * p.H + h) * K + tid;
      const size_t gi = ((size_t)(b * p.T + t) * p.HV + hv) * K + tid;
      sq[tid] = to_acc<AccT>(gq[qk]) * scale;
      sk[tid] = to_acc<AccT>(gk[qk]);
      AccT gt = to_acc<AccT>(gg[gi]);
      if (do_clamp) gt = gt > clampv ? gt : clampv;
      if constexpr (F64) sg[tid] = exp(gt);
      else sg[tid] = expf(gt);
    }
    const AccT bt = to_acc<AccT>(gb[(size_t)(b * p.T + t) * p.HV + hv]);
    const AccT vt = okc ? to_acc<AccT>(gv[((size_t)(b * p.T + t) * p.HV + hv) * p.V + col]) : (AccT)0;
    __syncthreads();
    AccT kS = 0;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] *= sg[ph + 8 * i];
      kS += sk[ph + 8 * i] * S[i];
    }
    kS += __shfl_xor(kS, 1);
    kS += __shfl_xor(kS, 2);
    kS += __shfl_xor(kS, 4);
    const AccT d = bt * (vt - kS);
    AccT o = 0;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] += sk[ph + 8 * i] * d;
      o += sq[ph + 8 * i] * S[i];
    }
    o += __shfl_xor(o, 1);
    o += __shfl_xor(o, 2);
    o += __shfl_xor(o, 4);
    if (ph == 0 && okc) {
      if constexpr (F64) go[((size_t)(b * p.T + t) * p.HV + hv) * p.V + col] = o;
      else go[((size_t)(b * p.T + t) * p.HV + hv) * p.V + col] = from_f32<InT>(o);
    }
  }
  if (s_out && okc) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) s_out[sbase + (size_t)(ph + 8 * i) * p.V + col] = S[i];
  }
}

template <int K, typename InT, typename AccT>
static hipError_t launch_rec(const KdaParams& p, hipStream_t stream) {
  const int grid = p.B * p.HV * ((p.V + 31) / 32);
  hipLaunchKernelGGL((kda_recurrent_kernel<K, InT, AccT>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <typename InT, typename AccT = float>
static hipError_t rec_by_k(const KdaParams& p, hipStream_t s) {
  switch (p.K) {
    case 16: return launch_rec<16, InT, AccT>(p, s);
    case 32: return launch_rec<32, InT, AccT>(p, s);
    case 64: return launch_rec<64, InT, AccT>(p, s);
    case 128: return launch_rec<128, InT, AccT>(p, s);
    default: return launch_rec<256, InT, AccT>(p, s);
  }
}

hipError_t kda_recurrent_dispatch(const KdaParams& p, int dtype, hipStream_t stream) {
  if (dtype == DT_F32) return rec_by_k<float>(p, stream);
  if (dtype == DT_BF16) return rec_by_k<bf16_t>(p, stream);
  return rec_by_k<_Float16>(p, stream);
}

hipError_t kda_recurrent_f64_dispatch(const KdaParams& p, hipStream_t stream) {
  return rec_by_k<double, double>(p, stream);
}

}  // namespace kch
