// CSA / HCA forward for the inputs the MFMA kernels do not take: float64
// (the reference computes in fp64 for fp64 inputs, ops_csa.py:229,263,510,922;
// ops_hca.py:138), head dims c or c_I above 128, more than 16 indexer heads,
// and indexer masks other than the standard block-causal one. Plain SIMT
// kernels templated on the compute type T (float or double), every sum in T.
//
//   gen_compress_kernel  one thread per (b, block, channel): the softmax-gated
//                        compression of ops_csa.py:198-305 (single branch, or
//                        overlapped: block i mixes branch a of block i with
//                        branch b of block i-1)
//   gen_l2norm_kernel    one wave per row: x / max(||x||, 1e-12) (F.normalize)
//   gen_indexer_kernel   one workgroup per (b, t): the head-weighted ReLU logits
//                        of ops_csa.py:503-536 under an arbitrary boolean mask
//                        (or the block-causal rule b < (t+1)/m, or none),
//                        then a bitonic sort of (logit, block) pairs in LDS:
//                        descending logit, ties by ascending block index;
//                        the first min(topk, n_blocks) are the selection
//                        (-1 where the logit is infinite, ops_csa.py:550-554)
//   gen_attn_kernel      one workgroup per (b, t): scores of every head against
//                        the selected compressed rows (CSA) or every causal
//                        block (HCA), then the window rows; the joint softmax
//                        with the sink (CSA: row max clamped at 0,
//                        ops_csa.py:1100-1155; HCA: the plain row max,
//                        ops_hca.py:166-186); the weighted sum of the rows.
//                        Scores and weights live in a workspace.

#include <float.h>
#include <limits.h>

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

template <typename T>
__device__ __forceinline__ T ninf() {
  return -__builtin_huge_val();
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const T u = __shfl_xor(v, o, 64);
    v = u > v ? u : v;
  }
  return v;
}

template <typename T>
__global__ __launch_bounds__(256) void gen_compress_kernel(GenCompressParams p) {
  const T* Ca = static_cast<const T*>(p.Ca);
  const T* Cb = static_cast<const T*>(p.Cb);
  const T* Za = static_cast<const T*>(p.Za);
  const T* Zb = static_cast<const T*>(p.Zb);
  const T* Ba = static_cast<const T*>(p.Ba);
  const T* Bb = static_cast<const T*>(p.Bb);
  T* out = static_cast<T*>(p.out);
  const int m = p.m, c = p.c, nb = p.T / m;
  const size_t total = (size_t)p.B * nb * c;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int ch = (int)(i % c);
    const int blk = (int)((i / c) % nb);
    const size_t b = i / ((size_t)c * nb);
    const size_t ra = (b * p.T + (size_t)blk * m) * c + ch;      // row blk*m of branch a
    const bool prev = p.overlapped && blk > 0;
    const size_t rb = prev ? ra - (size_t)m * c : 0;              // block blk-1 of branch b
    T mx = ninf<T>();
    for (int j = 0; j < m; ++j) {
      const T a = Za[ra + (size_t)j * c] + Ba[j * c + ch];
      mx = a > mx ? a : mx;
      if (prev) {
        const T bb = Zb[rb + (size_t)j * c] + Bb[j * c + ch];
        mx = bb > mx ? bb : mx;
      }
    }
    T den = 0, num = 0;
    for (int j = 0; j < m; ++j) {
      const T ea = exp(Za[ra + (size_t)j * c] + Ba[j * c + ch] - mx);
      den += ea;
      num += ea * Ca[ra + (size_t)j * c];
      if (prev) {
        const T eb = exp(Zb[rb + (size_t)j * c] + Bb[j * c + ch] - mx);
        den += eb;
        num += eb * Cb[rb + (size_t)j * c];
      }
    }
    out[i] = num / den;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gen_l2norm_kernel(const T* x, T* y, long long rows, int c,
                                                        int normalize) {
  const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const T* xr = x + (size_t)r * c;
  T* yr = y + (size_t)r * c;
  T s = 0;
  for (int d = lane; d < c; d += 64) s += xr[d] * xr[d];
  s = wave_sum(s);
  const T nrm = sqrt(s);
  const T den = normalize ? (nrm > (T)1e-12 ? nrm : (T)1e-12) : (T)1;
  for (int d = lane; d < c; d += 64) yr[d] = xr[d] / den;
}

// a before b in the selection order: larger logit first, ties by smaller index
template <typename T>
__device__ __forceinline__ bool before(T va, int ia, T vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

template <typename T>
__global__ __launch_bounds__(256) void gen_indexer_kernel(GenIndexerParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int HI = p.nIh, DI = p.cI, nb = p.nb, N = p.sortN;
  T* sq = reinterpret_cast<T*>(smem);                // [HI][DI] query rows (normalised)
  T* sw = sq + (size_t)HI * DI;                       // [HI] head weights
  T* sv = sw + HI;                                    // [N] logits
  int* si = reinterpret_cast<int*>(sv + N);           // [N] block indices
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const size_t bt = blockIdx.x;
  const int t = (int)(bt % p.T);
  const size_t b = bt / p.T;
  const T* q = static_cast<const T*>(p.q) + bt * HI * DI;
  const T* k = static_cast<const T*>(p.k) + b * nb * DI;
  for (int e = tid; e < HI * DI; e += 256) sq[e] = q[e];
  if (tid < HI) sw[tid] = p.w ? static_cast<const T*>(p.w)[bt * HI + tid] : (T)1;
  __syncthreads();
  if (p.normalize_q) {
    for (int h = wv; h < HI; h += 4) {
      T s = 0;
      for (int d = lane; d < DI; d += 64) s += sq[h * DI + d] * sq[h * DI + d];
      s = wave_sum(s);
      const T nrm = sqrt(s);
      const T den = nrm > (T)1e-12 ? nrm : (T)1e-12;
      for (int d = lane; d < DI; d += 64) sq[h * DI + d] /= den;
    }
    __syncthreads();
  }
  const T scale = (T)p.scale;
  const unsigned char* mask = static_cast<const unsigned char*>(p.mask);
  T* logits = static_cast<T*>(p.logits);
  for (int n = tid; n < N; n += 256) {
    T v = ninf<T>();
    if (n < nb) {
      const bool vis = mask ? mask[(size_t)b * p.mask_bstride + (size_t)t * p.mask_tstride + n] != 0
                            : (p.causal_m < 1 || n < (t + 1) / p.causal_m);
      const T* kr = k + (size_t)n * DI;
      T acc = 0;
      for (int h = 0; h < HI; ++h) {
        T dot = 0;
        for (int d = 0; d < DI; ++d) dot += sq[h * DI + d] * kr[d];
        dot *= scale;
        acc += sw[h] * (dot > (T)0 ? dot : (T)0);
      }
      v = vis ? acc : ninf<T>();
      if (logits) logits[bt * nb + n] = v;
    }
    sv[n] = v;
    si[n] = n < nb ? n : INT_MAX;
  }
  __syncthreads();
  // bitonic sort into selection order
  for (int kk = 2; kk <= N; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < N; i += 256) {
        const int ij = i ^ j;
        if (ij > i) {
          const bool asc = (i & kk) == 0;  // this run in selection order
          const T vi = sv[i], vj = sv[ij];
          const int ii = si[i], ji = si[ij];
          const bool swap = asc ? before(vj, ji, vi, ii) : before(vi, ii, vj, ji);
          if (swap) {
            sv[i] = vj; sv[ij] = vi;
            si[i] = ji; si[ij] = ii;
          }
        }
      }
      __syncthreads();
    }
  }
  long long* idx = static_cast<long long*>(p.idx);
  const int S = p.topk < nb ? p.topk : nb;
  for (int e = tid; e < p.topk; e += 256) {
    long long v = -1;
    if (e < S && !__builtin_isinf(sv[e])) v = si[e];
    idx[bt * p.topk + e] = v;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gen_attn_kernel(GenAttnParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nh = p.nh, c = p.c, win = p.win;
  const int nsel = p.idx ? p.topk : p.nb;  // compressed candidates
  const int K = nsel + win;
  T* sq = reinterpret_cast<T*>(smem);      // [nh][c]
  int* srow = reinterpret_cast<int*>(sq + (size_t)nh * c);  // [K] row (-1 invalid)
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const size_t bt = blockIdx.x;
  const int t = (int)(bt % p.T);
  const size_t b = bt / p.T;
  const T* q = static_cast<const T*>(p.q) + bt * nh * c;
  const T* kv = static_cast<const T*>(p.kv) + b * p.nb * c;
  const T* loc = p.local ? static_cast<const T*>(p.local) + b * p.T * c : nullptr;
  T* sc = static_cast<T*>(p.ws) + bt * nh * K;  // scores, then weights [nh][K]
  for (int e = tid; e < nh * c; e += 256) sq[e] = q[e];
  const int vis = (t + 1) / p.m;
  for (int k = tid; k < K; k += 256) {
    int r = -1;
    if (k < nsel) {
      if (p.idx) {
        const long long s = static_cast<const long long*>(p.idx)[bt * p.topk + k];
        r = s >= 0 && s < p.nb ? (int)s : -1;
      } else {
        r = k < vis ? k : -1;
      }
    } else {
      const int pos = t - win + 1 + (k - nsel);
      r = pos >= 0 ? pos : -1;
    }
    srow[k] = r;
  }
  __syncthreads();
  if (p.normalize_q) {
    for (int h = wv; h < nh; h += 4) {
      T s = 0;
      for (int d = lane; d < c; d += 64) s += sq[h * c + d] * sq[h * c + d];
      s = wave_sum(s);
      const T nrm = sqrt(s);
      const T den = nrm > (T)1e-12 ? nrm : (T)1e-12;
      for (int d = lane; d < c; d += 64) sq[h * c + d] /= den;
    }
    __syncthreads();
  }
  const T scale = (T)p.scale;
  for (int e = tid; e < nh * K; e += 256) {
    const int h = e / K, k = e % K, r = srow[k];
    T s = ninf<T>();
    if (r >= 0) {
      const T* row = k < nsel ? kv + (size_t)r * c : loc + (size_t)r * c;
      T dot = 0;
      for (int d = 0; d < c; ++d) dot += sq[h * c + d] * row[d];
      s = dot * scale;
    }
    sc[e] = s;
  }
  __syncthreads();
  // joint softmax per head, one wave per head
  const T* sink = static_cast<const T*>(p.sink);
  for (int h = wv; h < nh; h += 4) {
    T* sh = sc + (size_t)h * K;
    T mx = ninf<T>();
    for (int k = lane; k < K; k += 64) mx = sh[k] > mx ? sh[k] : mx;
    mx = wave_max(mx);
    const bool none = mx == ninf<T>();
    T ref;  // the subtracted row maximum
    if (sink) ref = p.hca ? (none ? (T)0 : mx) : (mx > (T)0 ? mx : (T)0);
    else ref = none ? (T)0 : mx;
    T den = 0;
    for (int k = lane; k < K; k += 64) den += sh[k] == ninf<T>() ? (T)0 : exp(sh[k] - ref);
    den = wave_sum(den);
    if (sink) den += exp(sink[h] - ref);
    for (int k = lane; k < K; k += 64)
      sh[k] = (none || sh[k] == ninf<T>()) ? (T)0 : exp(sh[k] - ref) / den;
  }
  __syncthreads();
  T* out = static_cast<T*>(p.out) + bt * nh * c;
  for (int e = tid; e < nh * c; e += 256) {
    const int h = e / c, d = e % c;
    const T* ph = sc + (size_t)h * K;
    T acc = 0;
    for (int k = 0; k < K; ++k) {
      const int r = srow[k];
      if (r < 0) continue;
      const T* row = k < nsel ? kv + (size_t)r * c : loc + (size_t)r * c;
      acc += ph[k] * row[d];
    }
    out[e] = acc;
  }
}

unsigned grid_for(size_t n) {
  const size_t g = (n + 255) / 256;
  return (unsigned)(g < 65536 ? (g ? g : 1) : 65536);
}

}  // namespace

int gen_sort_n(int nb) {
  int n = 1;
  while (n < nb) n <<= 1;
  return n;
}

size_t gen_indexer_smem(int nIh, int cI, int nb, bool f64) {
  const size_t e = f64 ? 8 : 4;
  const size_t n = (size_t)gen_sort_n(nb);
  return ((size_t)nIh * cI + nIh + n) * e + n * 4;
}

size_t gen_attn_smem(int nh, int c, int K, bool f64) {
  return (size_t)nh * c * (f64 ? 8 : 4) + (size_t)K * 4;
}

hipError_t gen_compress_launch(const GenCompressParams& p, bool f64, hipStream_t s) {
  const size_t total = (size_t)p.B * (p.T / p.m) * p.c;
  if (f64)
    hipLaunchKernelGGL((gen_compress_kernel<double>), dim3(grid_for(total)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gen_compress_kernel<float>), dim3(grid_for(total)), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t gen_l2norm_launch(const void* x, void* y, long long rows, int c, int normalize, bool f64,
                             hipStream_t s) {
  const unsigned g = (unsigned)((rows + 3) / 4);
  if (f64)
    hipLaunchKernelGGL((gen_l2norm_kernel<double>), dim3(g), dim3(256), 0, s,
                       static_cast<const double*>(x), static_cast<double*>(y), rows, c, normalize);
  else
    hipLaunchKernelGGL((gen_l2norm_kernel<float>), dim3(g), dim3(256), 0, s,
                       static_cast<const float*>(x), static_cast<float*>(y), rows, c, normalize);
  return hipGetLastError();
}

hipError_t gen_indexer_launch(GenIndexerParams p, bool f64, hipStream_t s) {
  p.sortN = gen_sort_n(p.nb);
  const size_t smem = gen_indexer_smem(p.nIh, p.cI, p.nb, f64);
  const dim3 g((unsigned)((size_t)p.B * p.T));
  if (f64)
    hipLaunchKernelGGL((gen_indexer_kernel<double>), g, dim3(256), smem, s, p);
  else
    hipLaunchKernelGGL((gen_indexer_kernel<float>), g, dim3(256), smem, s, p);
  return hipGetLastError();
}

hipError_t gen_attn_launch(const GenAttnParams& p, bool f64, hipStream_t s) {
  const int K = (p.idx ? p.topk : p.nb) + p.win;
  const size_t smem = gen_attn_smem(p.nh, p.c, K, f64);
  const dim3 g((unsigned)((size_t)p.B * p.T));
  if (f64)
    hipLaunchKernelGGL((gen_attn_kernel<double>), g, dim3(256), smem, s, p);
  else
    hipLaunchKernelGGL((gen_attn_kernel<float>), g, dim3(256), smem, s, p);
  return hipGetLastError();
}

}  // namespace kch
