// Device helpers shared by the KDA chunk kernels (kda_chunk_lp.hip, kda_split.hip).
#pragma once

#include <type_traits>

#include "kch_device.h"

namespace kch {
namespace kda_detail {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRange2 = 80.f * kLog2e;  // |G - G_a| bound of the anchored path (log2 units)
constexpr float kPos2 = 25.f * kLog2e;    // bound under which clamp(max=50) cannot bind

// j-th lower-triangular 16x16 tile (row-major order) of a 64x64 chunk matrix.
__device__ __forceinline__ int lower_tile_row(int j) { return (j >= 1) + (j >= 3) + (j >= 6); }
__device__ __forceinline__ int lower_tile_col(int j) {
  const int r = lower_tile_row(j);
  return j - r * (r + 1) / 2;
}

template <typename InT> __device__ __forceinline__ float h2f(uint32_t bits16);
template <> __device__ __forceinline__ float h2f<bf16_t>(uint32_t u) { return __uint_as_float(u << 16); }
template <> __device__ __forceinline__ float h2f<_Float16>(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)u);
}
// element j (0 = low half) of a packed pair of 16-bit values
template <typename InT> __device__ __forceinline__ float elem(uint32_t w, int j) {
  return h2f<InT>(j ? (w >> 16) : (w & 0xffffu));
}

// Per-lane raw storage of CPL consecutive 16-bit values (4 -> 8 bytes, 2 -> 4 bytes).
template <int CPL> struct RawT;
template <> struct RawT<4> {
  typedef uint2 type;
  static __device__ __forceinline__ uint32_t word(const uint2& r, int j) { return j ? r.y : r.x; }
};
template <> struct RawT<2> {
  typedef uint32_t type;
  static __device__ __forceinline__ uint32_t word(const uint32_t& r, int) { return r; }
};

// DPP move (gfx9 encodings): row_shr:n = 0x110+n, row_share:n = 0x150+n, quad_perm = 0x00-0xff.
template <int CTRL, bool ZERO_FILL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, ZERO_FILL));
}
// Inclusive prefix sum over the 16 lanes of each DPP row.
__device__ __forceinline__ float row_prefix_sum(float v) {
  v += dpp<0x111, true>(v);
  v += dpp<0x112, true>(v);
  v += dpp<0x114, true>(v);
  v += dpp<0x118, true>(v);
  return v;
}

__device__ __forceinline__ void st_bf16x4(bf16_t* dst, float a, float b, float c, float d) {
  bf16x4 o = {(bf16_t)a, (bf16_t)b, (bf16_t)c, (bf16_t)d};
  *reinterpret_cast<bf16x4*>(dst) = o;
}

// acc += A[16 x KD] B[KD x 16]; A row-major (stride lda), B stored [n][k]
// (stride ldb). All fragments are read before the MFMA chain starts. A chain
// uses one MFMA shape only: 16x16x32 steps when KD is a multiple of 32, else
// 16x16x16 steps throughout.
template <int KD>
__device__ __forceinline__ f32x4 mma16(f32x4 acc, const bf16_t* A, int lda, const bf16_t* B,
                                       int ldb) {
  const int l = lane_id();
  const bf16_t* a = A + (l & 15) * lda;
  const bf16_t* b = B + (l & 15) * ldb;
  const int q = l >> 4;
  if constexpr (KD % 32 == 0) {
    constexpr int N = KD / 32;
    bf16x8 fa[N], fb[N];
#pragma unroll
    for (int s = 0; s < N; ++s) {
      fa[s] = *reinterpret_cast<const bf16x8*>(a + 32 * s + 8 * q);
      fb[s] = *reinterpret_cast<const bf16x8*>(b + 32 * s + 8 * q);
    }
#pragma unroll
    for (int s = 0; s < N; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[s], fb[s], acc, 0, 0, 0);
  } else {
    constexpr int N = KD / 16;
    bf16x4 fa[N], fb[N];
#pragma unroll
    for (int s = 0; s < N; ++s) {
      fa[s] = *reinterpret_cast<const bf16x4*>(a + 16 * s + 4 * q);
      fb[s] = *reinterpret_cast<const bf16x4*>(b + 16 * s + 4 * q);
    }
#pragma unroll
    for (int s = 0; s < N; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(fa[s], fb[s], acc, 0, 0, 0);
  }
  return acc;
}

// Two products sharing the A operand: acc0 += A B0, acc1 += A B1.
template <int KD>
__device__ __forceinline__ void mma16x2(f32x4& acc0, f32x4& acc1, const bf16_t* A, int lda,
                                        const bf16_t* B0, const bf16_t* B1, int ldb) {
  static_assert(KD % 32 == 0, "full 32-wide steps");
  constexpr int N32 = KD / 32;
  const int l = lane_id();
  const int q = l >> 4;
  const bf16_t* a = A + (l & 15) * lda;
  const bf16_t* b0 = B0 + (l & 15) * ldb;
  const bf16_t* b1 = B1 + (l & 15) * ldb;
  bf16x8 fa[N32], f0[N32], f1[N32];
#pragma unroll
  for (int s = 0; s < N32; ++s) {
    fa[s] = *reinterpret_cast<const bf16x8*>(a + 32 * s + 8 * q);
    f0[s] = *reinterpret_cast<const bf16x8*>(b0 + 32 * s + 8 * q);
    f1[s] = *reinterpret_cast<const bf16x8*>(b1 + 32 * s + 8 * q);
  }
#pragma unroll
  for (int s = 0; s < N32; ++s) {
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[s], f0[s], acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[s], f1[s], acc1, 0, 0, 0);
  }
}

template <int V> using IC = std::integral_constant<int, V>;


}  // namespace kda_detail
}  // namespace kch
