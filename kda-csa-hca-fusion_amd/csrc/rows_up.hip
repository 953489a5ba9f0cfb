// Low-rank up-projection for prefill (gfx950):
//   Y[M, N] = X[M, K] W[N, K]^T      (torch.nn.functional.linear, no bias)
// with a short K (the query latent of CSA / HCA, dc = K <= 256) and many rows:
// q = W_UQ cQ of /root/reference/ops_hca.py:140 and ops_csa.py:923 (q_idx,
// ops_csa.py:877, likewise). The product is bound
// by writing Y (2 M N bytes; X and W are small), so the kernel is built
// around the output stream.
//
// K <= 128: weight-stationary, rows_up_ws_kernel. A persistent workgroup
// (8 waves, one per CU) owns a 256-column slice of W for the whole kernel:
// wave (rt, ch) holds columns 128 ch .. + 127 of the slice as MFMA A-operand
// fragments in registers (v_mfma_f32_16x16x32: lane (r, q) holds row r of a
// 16-row tile, k = 32 s + 8 q .. + 7), and the workgroup walks 64-row blocks
// of X (its slice's share of them): wave (rt, ch) loads row tile rt of the
// block as B-operand fragments (two blocks ahead), computes its 16 x 128
// piece of Y^T, and stages it in LDS; after a barrier the workgroup writes the
// block's 64 rows x 256 columns as 16-byte nontemporal stores. The 8 slices
// of a row block run on one XCD. W is read from L2 once per workgroup
// (instead of once per row block), X once per XCD.
// K = 256: rows_up_kernel, 64 rows of X per workgroup held in registers, W
// tiles streamed from L2 per 64-column round, the same staged output.
// Measured at M = 131072, N = 2048, K = 128 (bf16, MI355X): 99 us, against a
// 96 us floor for the store pattern alone and 183 us for hipBLASLt.

#include <algorithm>

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

template <typename T> struct UpVec;
template <> struct UpVec<bf16_t> {
  typedef bf16_t v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mfma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct UpVec<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mfma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kUpRows = 64;  // rows of X per workgroup

// TPW: 16-column tiles per wave and round (a round covers 64 TPW columns)
template <typename T, int KS, int TPW>
__global__ __launch_bounds__(256) void rows_up_kernel(RowsProjParams p) {
  using U = UpVec<T>;
  typedef typename U::v8 v8;
  constexpr int CPR = 64 * TPW;     // columns per round
  constexpr int LD = CPR + 8;       // LDS stage row stride (elements)
  constexpr int PPR = CPR / 8;      // 16-byte pieces per stage row
  __shared__ __attribute__((aligned(16))) T stage[2][kUpRows * LD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const int r = lane & 15, q = lane >> 4;
  const long long m0 = (long long)blockIdx.x * kUpRows;
  const T* x = static_cast<const T*>(p.x);
  const T* w = static_cast<const T*>(p.w);
  T* y = static_cast<T*>(p.y);
  // this lane's X fragments: row m0 + 16 mt + r (rows past M re-read row M - 1;
  // their results are not stored)
  v8 xf[4][KS];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const long long row = min(m0 + 16 * mt + r, (long long)p.M - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      xf[mt][s] = *reinterpret_cast<const v8*>(x + row * p.ldx + 32 * s + 8 * q);
  }
  const int nround = (p.N + CPR - 1) / CPR;
  // W fragments of this wave's tiles in round rd: columns CPR rd + 16 (TPW wv + j)
  // (columns past N re-read row N - 1)
  auto load_w = [&](int rd, v8 (&wf)[TPW][KS]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      const int n = min(CPR * rd + 16 * (TPW * wv + j) + r, p.N - 1);
#pragma unroll
      for (int s = 0; s < KS; ++s)
        wf[j][s] = *reinterpret_cast<const v8*>(w + (size_t)n * p.ldw + 32 * s + 8 * q);
    }
  };
  const bool vec_out = (p.N % 8) == 0;
  auto round = [&](int rd, const v8 (&wf)[TPW][KS], T* st) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = U::mfma(wf[j][s], xf[mt][s], acc);
        // acc[e] = Y[m0 + 16 mt + r][CPR rd + 16 (TPW wv + j) + 4 q + e]
        union { T h[4]; uint2 u; } o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o.h[e] = from_f32<T>(acc[e]);
        *reinterpret_cast<uint2*>(st + (16 * mt + r) * LD + 16 * (TPW * wv + j) + 4 * q) = o.u;
      }
    }
    __syncthreads();
    // the stage's rows as whole pieces: thread t takes piece t % PPR of rows
    // t / PPR + (256 / PPR) i
#pragma unroll
    for (int i = 0; i < kUpRows * PPR / 256; ++i) {
      const int idx = tid + 256 * i;
      const int lr = idx / PPR, pc = idx % PPR;
      const long long row = m0 + lr;
      const int c0 = CPR * rd + 8 * pc;
      if (row >= p.M || c0 >= p.N) continue;
      const T* src = st + lr * LD + 8 * pc;
      T* dst = y + row * p.ldy + c0;
      if (vec_out) {
        store_stream16(dst, *reinterpret_cast<const u32x4_t*>(src));
      } else {
        for (int e = 0; e < 8 && c0 + e < p.N; ++e) dst[e] = src[e];
      }
    }
  };
  v8 wa[TPW][KS], wb[TPW][KS];
  load_w(0, wa);
  // two rounds per iteration so that fragment buffers and stages have static names
  int rd = 0;
  for (; rd + 1 < nround; rd += 2) {
    load_w(rd + 1, wb);
    round(rd, wa, stage[0]);
    if (rd + 2 < nround) load_w(rd + 2, wa);
    round(rd + 1, wb, stage[1]);
  }
  if (rd < nround) round(rd, wa, stage[0]);
}

constexpr int kWsCols = 256;  // columns of W per workgroup slice
constexpr int kWsLd = kWsCols + 8;
constexpr int kWsDepth = 3;     // X blocks in flight per wave (two loaded ahead)

// Workgroup -> (slice, group) of the persistent grid. Workgroup i runs on XCD
// i % 8; with per_slice a multiple of 8 the 8 slices of one row-block group
// share an XCD, so a block of X is fetched into that XCD's L2 once for all
// slices and whole rows of Y are written from one XCD.
__device__ __forceinline__ void ws_place(int bid, int nslice, int per_slice, int& sl, int& g) {
  if (per_slice % 8 == 0) {
    const int xc = bid % 8, j = bid / 8;
    sl = j % nslice;
    g = (j / nslice) * 8 + xc;
  } else {
    sl = bid % nslice;
    g = bid / nslice;
  }
}

template <typename T, int KS>
__global__ __launch_bounds__(512) void rows_up_ws_kernel(RowsProjParams p, int nslice, int per_slice) {
  using U = UpVec<T>;
  typedef typename U::v8 v8;
  __shared__ __attribute__((aligned(16))) T stage[kUpRows * kWsLd];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(tid >> 6));
  const int rt = wv & 3, ch = wv >> 2;  // row tile of the block, column half of the slice
  const int r = lane & 15, q = lane >> 4;
  int sl, g;
  ws_place(blockIdx.x, nslice, per_slice, sl, g);
  const long long nblk = (p.M + kUpRows - 1) / kUpRows;
  if (g >= nblk) return;
  const T* x = static_cast<const T*>(p.x);
  const T* w = static_cast<const T*>(p.w);
  T* y = static_cast<T*>(p.y);
  const int cbase = kWsCols * sl + 128 * ch;  // this wave's first column
  // this wave's W fragments: 8 tiles of 16 columns (columns past N re-read N - 1)
  v8 wf[8][KS];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int n = min(cbase + 16 * j + r, p.N - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s) wf[j][s] = *reinterpret_cast<const v8*>(w + (size_t)n * p.ldw + 32 * s + 8 * q);
  }
  auto load_x = [&](long long blk, v8 (&xf)[KS]) {
    const long long row = min(blk * kUpRows + 16 * rt + r, (long long)p.M - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s) xf[s] = *reinterpret_cast<const v8*>(x + row * p.ldx + 32 * s + 8 * q);
  };
  const bool vec_out = (p.N % 8) == 0;
  constexpr int PPR = kWsCols / 8;  // 16-byte pieces per staged row
  auto block = [&](long long blk, const v8 (&xf)[KS]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = U::mfma(wf[j][s], xf[s], acc);
      // acc[e] = Y[blk 64 + 16 rt + r][cbase + 16 j + 4 q + e]
      union { T h[4]; uint2 u; } o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o.h[e] = from_f32<T>(acc[e]);
      *reinterpret_cast<uint2*>(stage + (16 * rt + r) * kWsLd + 128 * ch + 16 * j + 4 * q) = o.u;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kUpRows * PPR / 512; ++i) {
      const int idx = tid + 512 * i;
      const int lr = idx / PPR, pc = idx % PPR;
      const long long row = blk * kUpRows + lr;
      const int c0 = kWsCols * sl + 8 * pc;
      if (row >= p.M || c0 >= p.N) continue;
      const T* src = stage + lr * kWsLd + 8 * pc;
      T* dst = y + row * p.ldy + c0;
      if (vec_out) {
        store_stream16(dst, *reinterpret_cast<const u32x4_t*>(src));
      } else {
        for (int e = 0; e < 8 && c0 + e < p.N; ++e) dst[e] = src[e];
      }
    }
    __syncthreads();  // the stage is written again by the next block
  };
  // ring of kWsDepth fragment buffers, unrolled so that every index is static:
  // block b's fragments were loaded kWsDepth - 1 blocks earlier
  v8 xr[kWsDepth][KS];
#pragma unroll
  for (int i = 0; i < kWsDepth - 1; ++i)
    if (g + (long long)i * per_slice < nblk) load_x(g + (long long)i * per_slice, xr[i]);
  for (long long b0 = g; b0 < nblk; b0 += (long long)kWsDepth * per_slice) {
#pragma unroll
    for (int u = 0; u < kWsDepth; ++u) {
      const long long b = b0 + (long long)u * per_slice;
      if (b >= nblk) break;
      const long long nb = b + (long long)(kWsDepth - 1) * per_slice;
      if (nb < nblk) load_x(nb, xr[(u + kWsDepth - 1) % kWsDepth]);
      block(b, xr[u]);
    }
  }
}

int cu_count() {
  // multiprocessor count of each device, queried once
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (counts[dev] == 0) {
    int c = 256;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    counts[dev] = c;
  }
  return counts[dev];
}

template <typename T>
hipError_t rows_up_ws_launch(const RowsProjParams& p, hipStream_t s) {
  // one persistent workgroup per CU, spread evenly over the column slices;
  // per_slice is a multiple of 8 when there are enough row blocks (XCD-local
  // placement, ws_place)
  const int cus = cu_count();
  const int nslice = (p.N + kWsCols - 1) / kWsCols;
  const long long nblk = (p.M + kUpRows - 1) / kUpRows;
  int per_slice = std::max(1, cus / nslice);
  if (per_slice >= 8) per_slice -= per_slice % 8;
  if (nblk < per_slice) per_slice = (int)nblk;
  const dim3 grid((unsigned)(nslice * per_slice)), block(512);
  switch (p.K / 32) {
    case 1: hipLaunchKernelGGL((rows_up_ws_kernel<T, 1>), grid, block, 0, s, p, nslice, per_slice); break;
    case 2: hipLaunchKernelGGL((rows_up_ws_kernel<T, 2>), grid, block, 0, s, p, nslice, per_slice); break;
    default: hipLaunchKernelGGL((rows_up_ws_kernel<T, 4>), grid, block, 0, s, p, nslice, per_slice); break;
  }
  return hipGetLastError();
}

template <typename T, int TPW>
hipError_t rows_up_launch(const RowsProjParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.M + kUpRows - 1) / kUpRows)), block(256);
  switch (p.K / 32) {
    case 1: hipLaunchKernelGGL((rows_up_kernel<T, 1, TPW>), grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL((rows_up_kernel<T, 2, TPW>), grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL((rows_up_kernel<T, 4, TPW>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((rows_up_kernel<T, 8, TPW>), grid, block, 0, s, p); break;
  }
  return hipGetLastError();
}

template <typename T>
hipError_t rows_up_by_k(const RowsProjParams& p, hipStream_t s) {
  if (p.K <= 128) return rows_up_ws_launch<T>(p, s);
  return rows_up_launch<T, 1>(p, s);
}

}  // namespace

hipError_t rows_up_dispatch(const RowsProjParams& p, int dtype, hipStream_t s) {
  if (dtype == DT_BF16) return rows_up_by_k<bf16_t>(p, s);
  return rows_up_by_k<_Float16>(p, s);
}

}  // namespace kch
