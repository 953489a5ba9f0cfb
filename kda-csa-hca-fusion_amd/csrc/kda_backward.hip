// KDA recurrence backward for gfx950: the gradients of naive_recurrent_kda
// (/root/reference/ops_kda.py:175-267), the function the reference's own
// gradient tests differentiate (run_correctness.py:765-833, 1032-1092). The
// chunked form computes the same function, so its gradients are these too.
//
// Forward, per (b, hv) and token t (q^ = scale q, a = exp(max(g, clamp))):
//   Sd = diag(a) S;   u = v - Sd^T k;   d = beta u;   S' = Sd + k d^T;   o = S'^T q^
// Backward, tokens in reverse, carrying dS = dL/dS' from the later tokens:
//   dSt = dS + q^ do^T
//   dq^ = S' do;   dd = dSt^T k;   du = beta dd;   dv = du;   dbeta = dd . u
//   dk  = dSt d - Sd du
//   dSd = dSt - k du^T;   dg = rowsum(dSd * Sd)  (zero where g < clamp)
//   dS  = diag(a) dSd
// The columns of the state are independent in both directions; only dq^,
// dk, dg and dbeta sum over columns.
//
// kda_recurrent_bwd_kernel  one workgroup per (b, hv, slice of V): with PH
//   row phases per column, lane l of wave w owns rows (l / CW) + PH i of
//   column CW w + l % CW (CW = 64 / PH; slices of 4 CW columns). The sums over
//   columns, three K-vectors per token, are DPP steps within CW-lane groups;
//   the two per-column sums over rows are row rotations plus permlane swaps.
//   PH = 8 (32-column slices) when the grid has a workgroup for every CU;
//   PH = 16 (16-column slices: half the rows per thread, twice the
//   workgroups) for smaller grids, whose per-token chain is the bound. Pass 1 runs the recurrence forward and stores
//   the state at the start of every segment of SEG tokens (a checkpoint in the
//   workspace). Pass 2 walks the segments in reverse: it reloads the
//   checkpoint, recomputes the segment's decayed states Sd into registers,
//   then runs the token backward in reverse. Per token the column sums of
//   dq^, dk, dg (and dbeta) are formed within the wave by lane shuffles, the
//   four waves' sums meet in LDS, and each slice writes one partial record
//   per (b, t, hv) to the workspace.
// kda_bwd_reduce_kernel     one workgroup per (b, t, h): sums the slices'
//   partials and the value heads of a key head (q and k are shared by the
//   HV / H value heads), applies scale and the clamp mask, writes dq, dk, dg,
//   dbeta in the input dtype.
// Arithmetic is fp32 for fp32 / bf16 / fp16 inputs and fp64 for fp64 inputs,
// as in the forward (ops_kda.py:125-127).

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

template <typename AccT, typename T>
__device__ __forceinline__ AccT acc_of(T x) {
  if constexpr (sizeof(T) == 8) return (AccT)x;
  else return (AccT)to_f32(x);
}

template <typename OutT, typename AccT>
__device__ __forceinline__ OutT out_of(AccT x) {
  if constexpr (sizeof(OutT) == 8) return (OutT)x;
  else return from_f32<OutT>((float)x);
}

template <int CTRL>
__device__ __forceinline__ float dpp_acc(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_acc(double v) {
  const long long x = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(x >> 32), CTRL, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// x of lane l ^ D (D = 16 or 32) by v_permlane16_swap / v_permlane32_swap of
// x with itself: the swap leaves x[l ^ D] in the second result where l & D is
// 0 and in the first where it is set.
template <int D>
__device__ __forceinline__ unsigned swap_u32(unsigned u) {
  const bool hi = (__lane_id() & D) != 0;
  if constexpr (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return hi ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return hi ? r[0] : r[1];
  }
}
template <int D>
__device__ __forceinline__ float swap_acc(float v) {
  return __uint_as_float(swap_u32<D>(__float_as_uint(v)));
}
template <int D>
__device__ __forceinline__ double swap_acc(double v) {
  const unsigned long long x = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = swap_u32<D>((unsigned)x);
  const unsigned hi = swap_u32<D>((unsigned)(x >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// tokens per checkpoint segment: the segment's decayed states stay in
// registers (SEG * K / PH values per thread, at most 128 VGPRs), and the
// segment's rows and per-token column sums (15 K values a token) in 64 KB of
// LDS; at most 8
template <int K, typename AccT, int PH>
constexpr int seg_len() {
  constexpr int per_tok = K / PH * (int)(sizeof(AccT) / 4);
  constexpr int by_regs = 128 / per_tok;
  constexpr int by_lds = 65536 / (15 * K * (int)sizeof(AccT));
  constexpr int s = by_regs < by_lds ? by_regs : by_lds;
  return s > 8 ? 8 : s;
}

template <int K, typename InT, typename AccT, int kPh>
__global__ __launch_bounds__(256) void kda_recurrent_bwd_kernel(KdaBwdParams p) {
  constexpr int kCw = 64 / kPh, kCols = 4 * kCw;
  constexpr int RPT = K / kPh;
  constexpr int SEG = seg_len<K, AccT, kPh>();
  constexpr int PS = 3 * K + 1;  // partial record: dq^ [K] | dk [K] | dg [K] | dbeta
  constexpr bool F64 = sizeof(AccT) == 8;
  __shared__ AccT sq[SEG][K], sk[SEG][K], sa[SEG][K], sb[SEG];
  __shared__ AccT sw[SEG][4][3][K];
  __shared__ AccT sbw[SEG][4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvs = (p.V + kCols - 1) / kCols;
  const int vs = blockIdx.x % nvs;
  const int bh = blockIdx.x / nvs;
  const int hv = bh % p.HV, b = bh / p.HV, h = hv / (p.HV / p.H);
  const int cl = wave * kCw + (lane % kCw), ph = lane / kCw;
  const int col = vs * kCols + cl;
  const bool okc = col < p.V;
  const int T = p.T;
  const int nseg = (T + SEG - 1) / SEG;
  const InT* gq = static_cast<const InT*>(p.q);
  const InT* gk = static_cast<const InT*>(p.k);
  const InT* gv = static_cast<const InT*>(p.v);
  const InT* gg = static_cast<const InT*>(p.g);
  const InT* gb = static_cast<const InT*>(p.beta);
  const InT* gdo = static_cast<const InT*>(p.d_o);
  const AccT* s0 = static_cast<const AccT*>(p.s0);
  const AccT* dsT = static_cast<const AccT*>(p.ds_final);
  AccT* ds0 = static_cast<AccT*>(p.ds0);
  AccT* ck = static_cast<AccT*>(p.ck) + (size_t)blockIdx.x * nseg * K * kCols;
  AccT* part = static_cast<AccT*>(p.part);
  const AccT scale = (AccT)p.scale;
  const AccT clampv = (AccT)p.g_clamp_min;
  const bool do_clamp = p.g_clamp_min > -INFINITY;
  const size_t sbase = (size_t)(b * p.HV + hv) * K * p.V;

  auto red8 = [](AccT x) {  // over the phases of a column (lanes CW apart)
    // row_ror by CW (and 8): the lanes of the 16-lane row sharing the column
    if constexpr (kCw == 4) x += dpp_acc<0x124>(x);
    x += dpp_acc<0x128>(x);
    x += swap_acc<16>(x);
    x += swap_acc<32>(x);
    return x;
  };
  auto colsum = [](AccT x) {  // over the CW columns of a wave (CW-lane groups)
    x += dpp_acc<0xB1>(x);   // quad_perm [1,0,3,2]
    x += dpp_acc<0x4E>(x);   // quad_perm [2,3,0,1]
    if constexpr (kCw == 8) x += dpp_acc<0x141>(x);  // row_half_mirror: the other quad
    return x;
  };
  // the segment's key, decay and beta rows (and scaled q) into LDS
  auto load_seg = [&](int t0, int len, bool with_q) {
    for (int idx = tid; idx < len * K; idx += 256) {
      const int j = idx / K, c = idx % K;
      const int t = t0 + j;
      const size_t qk = ((size_t)(b * T + t) * p.H + h) * K + c;
      const size_t gi = ((size_t)(b * T + t) * p.HV + hv) * K + c;
      sk[j][c] = acc_of<AccT>(gk[qk]);
      if (with_q) sq[j][c] = acc_of<AccT>(gq[qk]) * scale;
      AccT gt = acc_of<AccT>(gg[gi]);
      if (do_clamp) gt = gt > clampv ? gt : clampv;
      if constexpr (F64) sa[j][c] = exp(gt);
      else sa[j][c] = expf(gt);
    }
    if (tid < len) sb[tid] = acc_of<AccT>(gb[(size_t)(b * T + t0 + tid) * p.HV + hv]);
  };
  auto col_val = [&](const InT* base, int t) -> AccT {
    return okc ? acc_of<AccT>(base[((size_t)(b * T + t) * p.HV + hv) * p.V + col]) : (AccT)0;
  };

  // ---- pass 1: forward, a checkpoint at the start of every segment ----
  AccT S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    S[i] = (s0 && okc) ? s0[sbase + (size_t)(ph + kPh * i) * p.V + col] : (AccT)0;
  for (int s = 0; s < nseg; ++s) {
    const int t0 = s * SEG, len = min(SEG, T - t0);
#pragma unroll
    for (int i = 0; i < RPT; ++i) ck[((size_t)s * K + ph + kPh * i) * kCols + cl] = S[i];
    __syncthreads();  // the previous segment's LDS rows are consumed
    load_seg(t0, len, false);
    AccT vv[SEG];
#pragma unroll
    for (int j = 0; j < SEG; ++j) vv[j] = j < len ? col_val(gv, t0 + j) : (AccT)0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      if (j < len) {
        AccT kS = 0;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          S[i] *= sa[j][ph + kPh * i];
          kS += sk[j][ph + kPh * i] * S[i];
        }
        kS = red8(kS);
        const AccT d = sb[j] * (vv[j] - kS);
#pragma unroll
        for (int i = 0; i < RPT; ++i) S[i] += sk[j][ph + kPh * i] * d;
      }
    }
  }
  // the checkpoints are re-read by the thread that wrote them
  __threadfence_block();

  // ---- pass 2: segments in reverse ----
  AccT dS[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    dS[i] = (dsT && okc) ? dsT[sbase + (size_t)(ph + kPh * i) * p.V + col] : (AccT)0;
  InT* gdv = static_cast<InT*>(p.dv);
  for (int s = nseg - 1; s >= 0; --s) {
    const int t0 = s * SEG, len = min(SEG, T - t0);
    __syncthreads();  // LDS of the previous segment is free
    load_seg(t0, len, true);
    AccT vv[SEG], dov[SEG], uu[SEG];
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      vv[j] = j < len ? col_val(gv, t0 + j) : (AccT)0;
      dov[j] = j < len ? col_val(gdo, t0 + j) : (AccT)0;
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) S[i] = ck[((size_t)s * K + ph + kPh * i) * kCols + cl];
    __syncthreads();
    // recompute: Sd of every token of the segment, and u
    AccT Sd[SEG][RPT];
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      uu[j] = 0;
      if (j < len) {
        AccT kS = 0;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          S[i] *= sa[j][ph + kPh * i];
          Sd[j][i] = S[i];
          kS += sk[j][ph + kPh * i] * S[i];
        }
        kS = red8(kS);
        uu[j] = vv[j] - kS;
        const AccT d = sb[j] * uu[j];
#pragma unroll
        for (int i = 0; i < RPT; ++i) S[i] += sk[j][ph + kPh * i] * d;
      }
    }
    // the token backward, last token first
#pragma unroll
    for (int jj = 0; jj < SEG; ++jj) {
      const int j = SEG - 1 - jj;
      if (j < len) {
        const AccT d = sb[j] * uu[j];
        AccT dd = 0;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          dS[i] += sq[j][ph + kPh * i] * dov[j];  // now dSt
          dd += dS[i] * sk[j][ph + kPh * i];
        }
        dd = red8(dd);
        const AccT du = sb[j] * dd;
        if (ph == 0 && okc)
          gdv[((size_t)(b * T + t0 + j) * p.HV + hv) * p.V + col] = out_of<InT>(du);
        // each row's column sums go to LDS as soon as they are formed
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          const AccT kr = sk[j][ph + kPh * i];
          const AccT P = colsum((Sd[j][i] + kr * d) * dov[j]);
          const AccT Dk = colsum(dS[i] * d - Sd[j][i] * du);
          const AccT dSd = dS[i] - kr * du;
          const AccT Gv = colsum(dSd * Sd[j][i]);
          dS[i] = sa[j][ph + kPh * i] * dSd;
          if (lane % kCw == 0) {
            sw[j][wave][0][ph + kPh * i] = P;
            sw[j][wave][1][ph + kPh * i] = Dk;
            sw[j][wave][2][ph + kPh * i] = Gv;
          }
        }
        const AccT cb = colsum(ph == 0 ? dd * uu[j] : (AccT)0);
        if (lane == 0) sbw[j][wave] = cb;
      }
    }
    __syncthreads();
    // the four waves' sums: one partial record per token of the segment
    for (int idx = tid; idx < len * PS; idx += 256) {
      const int j = idx / PS, e = idx % PS;
      AccT sum;
      if (e < 3 * K) {
        const int qn = e / K, c = e % K;
        sum = sw[j][0][qn][c] + sw[j][1][qn][c] + sw[j][2][qn][c] + sw[j][3][qn][c];
      } else {
        sum = sbw[j][0] + sbw[j][1] + sbw[j][2] + sbw[j][3];
      }
      part[(((size_t)(b * T + t0 + j) * p.HV + hv) * nvs + vs) * PS + e] = sum;
    }
  }
  if (ds0 && okc) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) ds0[sbase + (size_t)(ph + kPh * i) * p.V + col] = dS[i];
  }
}

template <typename InT, typename AccT>
__global__ __launch_bounds__(256) void kda_bwd_reduce_kernel(KdaBwdParams p, int cols) {
  const int K = p.K, PS = 3 * K + 1;
  const int nvs = (p.V + cols - 1) / cols;
  const int G = p.HV / p.H;
  const int h = blockIdx.x % p.H;
  const size_t bt = blockIdx.x / p.H;  // b * T + t
  const AccT* part = static_cast<const AccT*>(p.part);
  const InT* gg = static_cast<const InT*>(p.g);
  const AccT clampv = (AccT)p.g_clamp_min;
  const bool do_clamp = p.g_clamp_min > -INFINITY;
  for (int c = threadIdx.x; c < K; c += blockDim.x) {
    AccT dq = 0, dk = 0;
    for (int gi = 0; gi < G; ++gi) {
      const int hv = h * G + gi;
      const AccT* pp = part + (bt * p.HV + hv) * nvs * PS;
      AccT a = 0, kd = 0, gs = 0;
      for (int vs = 0; vs < nvs; ++vs) {
        a += pp[vs * PS + c];
        kd += pp[vs * PS + K + c];
        gs += pp[vs * PS + 2 * K + c];
      }
      dq += a;
      dk += kd;
      const size_t gi_idx = (bt * p.HV + hv) * K + c;
      const bool pass = !do_clamp || acc_of<AccT>(gg[gi_idx]) >= clampv;
      static_cast<InT*>(p.dg)[gi_idx] = out_of<InT>(pass ? gs : (AccT)0);
      if (c == 0) {
        AccT bs = 0;
        for (int vs = 0; vs < nvs; ++vs) bs += pp[vs * PS + 3 * K];
        static_cast<InT*>(p.dbeta)[bt * p.HV + hv] = out_of<InT>(bs);
      }
    }
    const size_t qi = (bt * p.H + h) * K + c;
    static_cast<InT*>(p.dq)[qi] = out_of<InT>(dq * (AccT)p.scale);
    static_cast<InT*>(p.dk)[qi] = out_of<InT>(dk);
  }
}

template <int K, typename InT, typename AccT>
hipError_t launch_bwd(const KdaBwdParams& p, int ph, hipStream_t s) {
  const int cols = 4 * (64 / ph);
  const int nvs = (p.V + cols - 1) / cols;
  if (ph == 16)
    hipLaunchKernelGGL((kda_recurrent_bwd_kernel<K, InT, AccT, 16>), dim3(p.B * p.HV * nvs), dim3(256), 0,
                       s, p);
  else
    hipLaunchKernelGGL((kda_recurrent_bwd_kernel<K, InT, AccT, 8>), dim3(p.B * p.HV * nvs), dim3(256), 0,
                       s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int threads = K <= 64 ? 64 : (K <= 128 ? 128 : 256);
  hipLaunchKernelGGL((kda_bwd_reduce_kernel<InT, AccT>), dim3((unsigned)((size_t)p.B * p.T * p.H)),
                     dim3(threads), 0, s, p, cols);
  return hipGetLastError();
}

template <typename InT, typename AccT>
hipError_t bwd_by_k(const KdaBwdParams& p, int ph, hipStream_t s) {
  switch (p.K) {
    case 16: return launch_bwd<16, InT, AccT>(p, ph, s);
    case 32: return launch_bwd<32, InT, AccT>(p, ph, s);
    case 64: return launch_bwd<64, InT, AccT>(p, ph, s);
    case 128: return launch_bwd<128, InT, AccT>(p, ph, s);
    default: return launch_bwd<256, InT, AccT>(p, ph, s);
  }
}

template <int K, typename AccT>
size_t ck_bytes(int B, int T, int HV, int V, int ph) {
  const int seg = ph == 16 ? seg_len<K, AccT, 16>() : seg_len<K, AccT, 8>();
  const int cols = 4 * (64 / ph);
  return (size_t)B * HV * ((V + cols - 1) / cols) * ((T + seg - 1) / seg) * K * cols * sizeof(AccT);
}

template <typename AccT>
size_t ck_bytes_by_k(int B, int T, int HV, int K, int V, int ph) {
  switch (K) {
    case 16: return ck_bytes<16, AccT>(B, T, HV, V, ph);
    case 32: return ck_bytes<32, AccT>(B, T, HV, V, ph);
    case 64: return ck_bytes<64, AccT>(B, T, HV, V, ph);
    case 128: return ck_bytes<128, AccT>(B, T, HV, V, ph);
    default: return ck_bytes<256, AccT>(B, T, HV, V, ph);
  }
}

// 16 phases (16-column slices) when 32-column slices would leave CUs idle
int phases(int B, int HV, int V) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return (long long)B * HV * ((V + 31) / 32) < cus ? 16 : 8;
}

size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

template <typename InT, typename AccT>
hipError_t reduce_only(const KdaBwdParams& p, int cols, hipStream_t s) {
  const int threads = p.K <= 64 ? 64 : (p.K <= 128 ? 128 : 256);
  hipLaunchKernelGGL((kda_bwd_reduce_kernel<InT, AccT>), dim3((unsigned)((size_t)p.B * p.T * p.H)),
                     dim3(threads), 0, s, p, cols);
  return hipGetLastError();
}

}  // namespace

hipError_t kda_bwd_reduce_launch(const KdaBwdParams& p, int cols, int dtype, hipStream_t stream) {
  if (dtype == DT_F64) return reduce_only<double, double>(p, cols, stream);
  if (dtype == DT_F32) return reduce_only<float, float>(p, cols, stream);
  if (dtype == DT_BF16) return reduce_only<bf16_t, float>(p, cols, stream);
  return reduce_only<_Float16, float>(p, cols, stream);
}

size_t kda_bwd_ws_bytes(int B, int T, int HV, int K, int V, bool f64) {
  const int ph = phases(B, HV, V);
  const int cols = 4 * (64 / ph);
  const size_t acc = f64 ? 8 : 4;
  const size_t ck = f64 ? ck_bytes_by_k<double>(B, T, HV, K, V, ph) : ck_bytes_by_k<float>(B, T, HV, K, V, ph);
  const size_t part = (size_t)B * T * HV * ((V + cols - 1) / cols) * (3 * K + 1) * acc;
  return al256(ck) + al256(part);
}

hipError_t kda_bwd_dispatch(KdaBwdParams p, int dtype, void* ws, hipStream_t stream) {
  const bool f64 = dtype == DT_F64;
  const int ph = phases(p.B, p.HV, p.V);
  const size_t ck = f64 ? ck_bytes_by_k<double>(p.B, p.T, p.HV, p.K, p.V, ph)
                        : ck_bytes_by_k<float>(p.B, p.T, p.HV, p.K, p.V, ph);
  p.ck = ws;
  p.part = static_cast<char*>(ws) + al256(ck);
  if (f64) return bwd_by_k<double, double>(p, ph, stream);
  if (dtype == DT_F32) return bwd_by_k<float, float>(p, ph, stream);
  if (dtype == DT_BF16) return bwd_by_k<bf16_t, float>(p, ph, stream);
  return bwd_by_k<_Float16, float>(p, ph, stream);
}

}  // namespace kch
