// Device-side helpers shared by the gfx950 kernels of this library.
//
// * storage conversions for bf16 / fp16 / fp32 inputs,
// * the MFMA shapes used for 16x16 output tiles:
//     v_mfma_f32_16x16x32_bf16  (gfx950; A/B: 8 bf16 per lane)
//     v_mfma_f32_16x16x16_bf16  (A/B: 4 bf16 per lane)
//     v_mfma_f32_16x16x4_f32    (A/B: 1 fp32 per lane)
//   Lane l of a wave64 holds A row (l % 16) and B column (l % 16); the K
//   elements it holds are k = KPL*(l / 16) + [0, KPL). The accumulator holds
//   rows 4*(l / 16) + [0, 4) of column (l % 16).
//   One accumulation chain uses a single MFMA shape: feeding the accumulator
//   of a 16x16x32 bf16 MFMA into a 16x16x16 one gave wrong, timing-dependent
//   results on gfx950 in this library's kernels.
// * tile_mma: one 16x16 fp32 output tile from operands resident in LDS, with A
//   stored row-major [row][k] and B stored transposed [col][k].
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace kch {

typedef __bf16 bf16_t;
typedef bf16_t bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16_t bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte store of a large output stream (nontemporal: the lines are not kept
// in L2 for reuse). Writing 537 MB of MFMA results this way took 113 us
// instead of 179 us with ordinary stores from the same kernel on MI355X.
__device__ __forceinline__ void store_stream16(void* dst, u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst));
}

// Input storage types accepted by the C-ABI (dtype enum: 0 fp32, 1 bf16, 2 fp16;
// 3 fp64 where an entry point says so).
enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_F64 = 3 };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active), with
// DPP: row_shr 1, 2, 4, 8 scan each 16-lane row (a lane whose source lies
// before its row start adds 0), then row_bcast:15 adds row 0's total to row 1
// and row 2's to row 3, and row_bcast:31 the total of rows 0-1 to rows 2 and 3
// (lanes outside the row mask keep 0). No LDS traffic.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
  return x;
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return (bf16_t)x; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }

// Two consecutive elements of a storage type, converted to fp32.
template <typename T> struct Pair;
template <> struct Pair<float> {
  typedef float2 raw;
  static __device__ __forceinline__ float2 cvt(raw r) { return r; }
};
template <> struct Pair<bf16_t> {
  typedef uint32_t raw;
  static __device__ __forceinline__ float2 cvt(raw r) {
    return make_float2(__uint_as_float(r << 16), __uint_as_float(r & 0xffff0000u));
  }
};
template <> struct Pair<_Float16> {
  typedef uint32_t raw;
  static __device__ __forceinline__ float2 cvt(raw r) {
    _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(r & 0xffffu));
    _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(r >> 16));
    return make_float2((float)lo, (float)hi);
  }
};

// Three-part bf16 split of fp32 values: x = hi + mid + lo up to the rounding
// of the last part (each difference below is exact in fp32), so hi carries 8
// significant bits, mid the next 8 and lo the next 8: together the 24 bits of
// x. Dot products formed from the six leading cross products of such splits
// (hi*hi, hi*mid, mid*hi, hi*lo, lo*hi, mid*mid: every bf16 product is exact
// in fp32) carry fp32-level error (terms of 2^-24 and below dropped).
__device__ __forceinline__ void split3_bf16(const float* f, bf16x8& hi, bf16x8& mid, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16_t h = (bf16_t)f[i];
    const float r = f[i] - (float)h;
    const bf16_t md = (bf16_t)r;
    hi[i] = h;
    mid[i] = md;
    lo[i] = (bf16_t)(r - (float)md);
  }
}

// Two-part fp16 split of components of unit vectors, prescaled by 2^8:
// hi = fp16(256 x), lo = fp16(256 x - hi) (the difference is exact in fp32),
// so hi + lo carries 22 significant bits of 256 x, and for |x| <= 1 no part
// overflows or (down to |x| ~ 2^-20) leaves the normal range. A dot product
// of two such splits from hi*hi + hi*lo + lo*hi (fp16 products are exact in
// fp32) is 2^16 times the dot product, to about 2^-22 relative.
constexpr float kSplit16Scale = 256.f;
constexpr float kSplit16Unscale = 1.f / 65536.f;
__device__ __forceinline__ void split2_f16(const float* f, f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float x = f[i] * kSplit16Scale;
    const _Float16 h = (_Float16)x;
    hi[i] = h;
    lo[i] = (_Float16)(x - (float)h);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The KDA layer's activations in fp32 (torch's silu, sigmoid, and softplus
// with beta 1 and threshold 20: x above the threshold, else log1p(e^x)).
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// The same activations for results rounded to bf16 next, with the hardware
// base-2 exponential (v_exp_f32, about 1 ulp; e^x = 2^(x log2 e)) and
// logarithm in place of the library's range-reduced expf / log1pf; the IEEE
// divisions stay. Over every finite bf16 input the bf16-rounded results equal
// those of silu_f / sigmoid_f / softplus_f (checked exhaustively on gfx950,
// tests/test_hybrid_gpu.py::test_kda_gates_fast_activations_exhaustive); for
// fp16 results they do not always, so fp16 keeps the library forms. log1p(t)
// is Goldberg's t log(u) / (u - 1), u = 1 + t (exact where u rounds to 1;
// D. Goldberg, "What every computer scientist should know about
// floating-point arithmetic", 1991, Theorem 4); below x = -80, where e^x
// leaves the normal range, the library exponential keeps the denormal tail.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float silu_bf(float x) { return x / (1.f + exp_hw(-x)); }
__device__ __forceinline__ float sigmoid_bf(float x) { return 1.f / (1.f + exp_hw(-x)); }
__device__ __forceinline__ float softplus_bf(float x) {
  if (x > 20.f) return x;
  const float t = x < -80.f ? expf(x) : exp_hw(x);
  const float u = 1.f + t, d = u - 1.f;
  return d == 0.f ? t : (__builtin_amdgcn_logf(u) * 0.6931471805599453f) * t / d;
}
// The activations a kernel with 16-bit results of type T uses.
template <typename T> __device__ __forceinline__ float silu_t(float x) {
  if constexpr (std::is_same<T, bf16_t>::value) return silu_bf(x); else return silu_f(x);
}
template <typename T> __device__ __forceinline__ float sigmoid_t(float x) {
  if constexpr (std::is_same<T, bf16_t>::value) return sigmoid_bf(x); else return sigmoid_f(x);
}
template <typename T> __device__ __forceinline__ float softplus_t(float x) {
  if constexpr (std::is_same<T, bf16_t>::value) return softplus_bf(x); else return softplus_f(x);
}

// The value a tensor of type T stores for x (identity for fp32): each torch
// operation of the reference writes its result in the layer's dtype, and the
// next one reads it back from there.
template <typename T>
__device__ __forceinline__ float stored(float x) {
  if constexpr (sizeof(T) == 2) return to_f32(from_f32<T>(x));
  return x;
}

// Orders LDS traffic of one wave: every lane's earlier LDS writes are visible to
// every lane's later LDS reads. Waves are not synchronised with each other.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ---------------------------------------------------------------------------
// 16x16 output tile: acc += A[16 x kd] * B[kd x 16]
//   A: LDS, row-major, row stride lda (elements); A[r][k] at A[r*lda + k]
//   B: LDS, transposed, row stride ldb;            B[k][n] at B[n*ldb + k]
// kd must be a multiple of 16 (bf16) or 4 (fp32).
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 tile_mma(f32x4 acc, const float* A, int lda,
                                          const float* B, int ldb, int kd) {
  const int l = lane_id();
  const int r = l & 15;
  const int kq = l >> 4;
  const float* a = A + r * lda + kq;
  const float* b = B + r * ldb + kq;
  for (int k = 0; k < kd; k += 4)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[k], b[k], acc, 0, 0, 0);
  return acc;
}

// Row index (within a 16x16 tile) of accumulator element e held by this lane.
__device__ __forceinline__ int acc_row(int e) { return ((lane_id() >> 4) << 2) + e; }
__device__ __forceinline__ int acc_col() { return lane_id() & 15; }

}  // namespace kch
