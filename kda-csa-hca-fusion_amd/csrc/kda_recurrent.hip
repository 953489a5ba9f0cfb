// KDA per-token recurrence for gfx950 (decode steps and short sequences).
//
// Restates naive_recurrent_kda (/root/reference/ops_kda.py:175-267): per token
//   S <- S * exp(g_t)                      (per key channel, ops_kda.py:254)
//   S <- S + (beta_t k_t) (x) (v_t - k_t^T S)  (ops_kda.py:255-256)
//   o_t = (scale q_t)^T S                  (post-update state, ops_kda.py:257)
// with fp32 compute and the gate clamped at g_clamp_min (ops_kda.py:224-225).
//
// grid  : one workgroup per (b, hv, 32-column slice of V)
// block : 256 threads; thread (col = tid/8, phase = tid%8) owns state rows
//         phase + 8*i of column col, so k^T S and q^T S reduce over 8 lanes.
// This path is bound by the state read/write (K*V*4 bytes per head, twice).

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

template <int K, typename InT>
__global__ __launch_bounds__(256) void kda_recurrent_kernel(KdaParams p) {
  constexpr int RPT = K / 8;
  __shared__ float sq[K], sk[K], sg[K];
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
  const bool do_clamp = p.g_clamp_min > -INFINITY;

  float S[RPT];
  const size_t sbase = (size_t)(b * p.HV + hv) * K * p.V;
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    S[i] = (p.s0 && okc) ? p.s0[sbase + (size_t)(ph + 8 * i) * p.V + col] : 0.f;

  for (int t = 0; t < p.T; ++t) {
    __syncthreads();
    if (tid < K) {
      const size_t qk = ((size_t)(b * p.T + t) * p.H + h) * K + tid;
      const size_t gi = ((size_t)(b * p.T + t) * p.HV + hv) * K + tid;
      sq[tid] = to_f32(gq[qk]) * p.scale;
      sk[tid] = to_f32(gk[qk]);
      float gt = to_f32(gg[gi]);
      if (do_clamp) gt = fmaxf(gt, p.g_clamp_min);
      sg[tid] = expf(gt);
    }
    const float bt = to_f32(gb[(size_t)(b * p.T + t) * p.HV + hv]);
    const float vt = okc ? to_f32(gv[((size_t)(b * p.T + t) * p.HV + hv) * p.V + col]) : 0.f;
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
    const float d = bt * (vt - kS);
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] += sk[ph + 8 * i] * d;
      o += sq[ph + 8 * i] * S[i];
    }
    o += __shfl_xor(o, 1);
    o += __shfl_xor(o, 2);
    o += __shfl_xor(o, 4);
    if (ph == 0 && okc) go[((size_t)(b * p.T + t) * p.HV + hv) * p.V + col] = from_f32<InT>(o);
  }
  if (p.s_out && okc) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) p.s_out[sbase + (size_t)(ph + 8 * i) * p.V + col] = S[i];
  }
}

template <int K, typename InT>
static hipError_t launch_rec(const KdaParams& p, hipStream_t stream) {
  const int grid = p.B * p.HV * ((p.V + 31) / 32);
  hipLaunchKernelGGL((kda_recurrent_kernel<K, InT>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <typename InT>
static hipError_t rec_by_k(const KdaParams& p, hipStream_t s) {
  switch (p.K) {
    case 16: return launch_rec<16, InT>(p, s);
    case 32: return launch_rec<32, InT>(p, s);
    case 64: return launch_rec<64, InT>(p, s);
    case 128: return launch_rec<128, InT>(p, s);
    default: return launch_rec<256, InT>(p, s);
  }
}

hipError_t kda_recurrent_dispatch(const KdaParams& p, int dtype, hipStream_t stream) {
  if (dtype == DT_F32) return rec_by_k<float>(p, stream);
  if (dtype == DT_BF16) return rec_by_k<bf16_t>(p, stream);
  return rec_by_k<_Float16>(p, stream);
}

}  // namespace kch
