// Device building blocks shared by the CSA / HCA prefill and decode kernels.
//
// * Wave-level reductions (sum / max over 64 lanes, over lane groups).
// * L2 row normalisation: x / max(||x||_2, 1e-12), the F.normalize semantics
//   used throughout the reference (ops_csa.py:523-525,929,950,1110-1112;
//   ops_hca.py:135,141,154).
// * MqaWave: one wave computes the joint-softmax MQA output of ONE query
//   (up to 16 heads of head dim HD) over a list of shared key/value rows,
//   fed 16 keys at a time. Scores, masking, the running max / sum and the
//   sink follow ops_csa.py:1126-1149 / ops_hca.py:166-186:
//       p_i = exp(s_i) / (sum_valid exp(s_j) + exp(sink))   (sink present)
//       p_i = softmax over the valid keys                   (no sink)
//   and an output of 0 when no key is valid.
//
// MQA layout (lane l, q = l >> 4, n = l & 15):
//   S^T = K Q^T with v_mfma_f32_16x16x32_bf16: A = 16 key rows (row-major, the
//   lane reads 8 dims of key n), B = Q stored [head][dim]. The accumulator holds
//   keys 4q..4q+3 of head n, which is exactly the B operand layout of the
//   16x16x16 MFMA in O^T = V^T P^T (k = keys), so P never leaves the lane.
//   V^T fragments (4 keys of one dim) are read from a wave-private LDS copy of
//   the 16 rows with the transposing LDS read (one instruction per tile).
//   O^T tile t holds dims 16t + 4q..4q+3 of head n.
// Softmax reference: M (per head) trails the running max by at most 8 in
// log2 units; o and L are rescaled only when a chunk exceeds that, and the
// final o / L (with the sink term taken relative to the same M) is the same
// quotient.
#pragma once

#include "kch_device.h"

namespace kch {

constexpr float kLog2eF = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.f;  // MqaWave: slack of the softmax reference point
// Initial reference point of the query-tile kernel: finite, so exp2(s - M) of a
// masked score (-inf) is 0 without a guard; any finite score exceeds it by far
// more than kRescaleLog2, so the first valid key always resets M.
constexpr float kMFloor = -1e30f;

// max without NaN canonicalisation (operands are never NaN here)
__device__ __forceinline__ float fmax_nc(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, INFINITY); }

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
// sum / max over the 4 lanes {n, n+16, n+32, n+48} (all lanes active), with
// the gfx950 row swaps: permlane16_swap(v, v) leaves rows (0,0,2,2) in one
// result and (1,1,3,3) in the other, permlane32_swap(v, v) halves (lo,lo) and
// (hi,hi), so combining the two results pairs every lane with its partner.
__device__ __forceinline__ float colq_sum(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float colq_max(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float l2_inv(float sumsq) { return 1.f / fmaxf(sqrtf(sumsq), 1e-12f); }

template <typename T> __device__ __forceinline__ float ld_f32(const T* p) { return to_f32(*p); }

// 8 consecutive values of type T (16 / 32 bytes) converted to fp32.
template <typename T> struct Load8;
template <> struct Load8<bf16_t> {
  static __device__ __forceinline__ void run(const bf16_t* p, float* f) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <> struct Load8<_Float16> {
  static __device__ __forceinline__ void run(const _Float16* p, float* f) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const h8 r = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)r[i];
  }
};
template <> struct Load8<float> {
  static __device__ __forceinline__ void run(const float* p, float* f) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

__device__ __forceinline__ bf16x8 to_bf16x8(const float* f) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16_t)f[i];
  return r;
}

// One wave, one query, up to 16 heads of head dim HD (64 or 128).
template <int HD>
struct MqaWave {
  static constexpr int NS = HD / 32;   // 32-wide k steps of S^T
  static constexpr int NT = HD / 16;   // O^T tiles
  static constexpr int LDS_LD = HD + 8;  // staging row stride (bf16)
  static constexpr int STAGE_BYTES = 16 * LDS_LD * 2;

  bf16x8 qf[NS];  // Q fragments: head n, dims 8q + 32s
  f32x4 o[NT];
  float M, L;     // softmax reference point (log2 units) and sum of head n
  float qscale2;  // score scale * log2(e)

  // q_row: this lane's head row (nullptr for a padding head -> zeros);
  // normalise: L2-normalise each head row (4 lanes share a head).
  template <typename QT>
  __device__ __forceinline__ void init(const QT* q_row, bool normalise, float scale) {
    const int q = lane_id() >> 4;
    float f[NS][8];
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (q_row) Load8<QT>::run(q_row + 32 * s + 8 * q, f[s]);
      else {
#pragma unroll
        for (int i = 0; i < 8; ++i) f[s][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += f[s][i] * f[s][i];
    }
    float inv = 1.f;
    if (normalise) inv = l2_inv(colq_sum(ss));
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[s][i] *= inv;
      qf[s] = to_bf16x8(f[s]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    M = -INFINITY;
    L = 0.f;
    qscale2 = scale * kLog2eF;
  }

  // As init, for the query-tile kernel: the row is always readable (`keep`
  // false, for a padding head or query, zeroes it after the load, so the load
  // is not conditional); the sign of `scale` is folded into the fragments so
  // that qscale2 >= 0; M starts at a finite floor (kMFloor) instead of -inf.
  template <typename QT>
  __device__ __forceinline__ void init_always(const QT* q_row, bool keep, bool normalise, float scale) {
    const int q = lane_id() >> 4;
    float f[NS][8];
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      Load8<QT>::run(q_row + 32 * s + 8 * q, f[s]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[s][i] = keep ? f[s][i] : 0.f;
        ss += f[s][i] * f[s][i];
      }
    }
    float inv = 1.f;
    if (normalise) inv = l2_inv(colq_sum(ss));
    if (scale < 0.f) inv = -inv;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[s][i] *= inv;
      qf[s] = to_bf16x8(f[s]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    M = kMFloor;
    L = 0.f;
    qscale2 = fabsf(scale) * kLog2eF;
  }

  // Fragments of 16 key rows: this lane's key row (key n = lane & 15) at dims
  // 32s + 8q .. 32s + 8q + 7.
  struct Frag {
    bf16x8 k[NS];
  };
  __device__ __forceinline__ static void load(Frag& f, const bf16_t* row) {
    const int q = lane_id() >> 4;
#pragma unroll
    for (int s = 0; s < NS; ++s) f.k[s] = *reinterpret_cast<const bf16x8*>(row + 32 * s + 8 * q);
  }

  // Consume 16 keys. `row` is this lane's key row (key n = lane & 15), valid
  // for every lane (point invalid keys at any readable row); `valid16` has bit
  // k set when key k of the chunk is valid. `stage` is this wave's LDS buffer.
  __device__ __forceinline__ void chunk(const bf16_t* row, unsigned valid16, bf16_t* stage) {
    Frag f;
    load(f, row);
    chunk(f, valid16, stage);
  }

  // Consume 16 keys already loaded into registers.
  __device__ __forceinline__ void chunk(const Frag& f, unsigned valid16, bf16_t* stage) {
    const int l = lane_id();
    const int q = l >> 4, n = l & 15;
    // previous chunk's V^T reads by this wave are complete before the overwrite
    wave_lds_sync();
#pragma unroll
    for (int s = 0; s < NS; ++s) *reinterpret_cast<bf16x8*>(stage + n * LDS_LD + 32 * s + 8 * q) = f.k[s];
    f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.k[s], qf[s], st, 0, 0, 0);
    float sv[4];
    float cm = -INFINITY;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = (valid16 >> (4 * q + e)) & 1u;
      sv[e] = ok ? st[e] * qscale2 : -INFINITY;
      cm = fmaxf(cm, sv[e]);
    }
    cm = colq_max(cm);
    // M is a reference point, not necessarily the running max: o and L are
    // rescaled only when some head's chunk max exceeds its M by more than 8
    // (log2 units), so p <= 2^8 and most chunks skip the rescale.
    if (__ballot(cm > M + kRescaleLog2)) {
      const float mnew = fmaxf(M, cm);
      const float alpha = mnew == -INFINITY ? 1.f : fast_exp2(M - mnew);  // M = -inf -> 0
      L = L * alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] *= alpha;
      M = mnew;
    }
    float p[4];
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[e] = sv[e] == -INFINITY ? 0.f : fast_exp2(sv[e] - M);  // M is finite when sv is
      ps += p[e];
    }
    L += colq_sum(ps);
    bf16x4 pb = {(bf16_t)p[0], (bf16_t)p[1], (bf16_t)p[2], (bf16_t)p[3]};
    wave_lds_sync();  // staged rows visible to the whole wave
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // V^T fragment: rows 4q .. 4q + 3, column 16t + n. The gfx950 transposing
      // read does it in one instruction: the 16 lanes of a row group each read
      // 8 bytes (row 4q + n / 4, columns 16t + 4 (n % 4) .. + 3) and lane n
      // receives column 16t + n of the 4 rows.
      typedef short s16x4 __attribute__((ext_vector_type(4)));
      const bf16_t* src = stage + (4 * q + (n >> 2)) * LDS_LD + 16 * t + 4 * (n & 3);
      const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(src));
      const bf16x4 va = __builtin_bit_cast(bf16x4, r);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, o[t], 0, 0, 0);
    }
  }

  // Final normalisation. Returns the multiplier for o (0 when nothing valid).
  __device__ __forceinline__ float finish(bool has_sink, float sink) const {
    float denom = L;
    if (has_sink) denom += fast_exp2(sink * kLog2eF - M);  // M = -inf -> +inf
    return (L > 0.f) ? 1.f / denom : 0.f;
  }
};

}  // namespace kch
