// Device building blocks shared by the CSA / HCA prefill and decode kernels.
//
// * Wave-level reductions (sum / max over 64 lanes, over lane groups).
// * L2 row normalisation: x / max(||x||_2, 1e-12), the F.normalize semantics
//   used throughout the reference (ops_csa.py:523-525,929,950,1110-1112;
//   ops_hca.py:135,141,154).
// * MqaWave: one wave computes the joint-softmax MQA output of ONE query
//   (up to 16 heads of head dim HD) over a list of shared key/value rows,
//   fed 32 keys at a time. Scores, masking, the running max / sum and the
//   sink follow ops_csa.py:1126-1149 / ops_hca.py:166-186:
//       p_i = exp(s_i) / (sum_valid exp(s_j) + exp(sink))   (sink present)
//       p_i = softmax over the valid keys                   (no sink)
//   and an output of 0 when no key is valid.
//
// MQA layout (lane l, q = l >> 4, n = l & 15):
//   S^T = K Q^T with v_mfma_f32_16x16x32_bf16 per 16 keys: A = 16 key rows
//   (the lane reads 8 dims of key n), B = Q stored [head][dim]. The
//   accumulator holds keys 4q..4q+3 of head n. O^T = V^T P^T takes 32 keys per
//   v_mfma_f32_16x16x32_bf16 (the 16x16x16 form runs at half its rate on
//   gfx950): k slot 8q + i holds key 4q + i (i < 4) of the first 16 keys and
//   key 16 + 4q + i - 4 (i >= 4) of the second, which is where the two S^T
//   accumulators leave them, so P never leaves the lane. V^T fragments are
//   read with the gfx950 transposing LDS read from a swizzled LDS copy of the
//   rows (tile_swz), two reads per O^T tile. O^T tile t holds dims
//   16t + 4q..4q+3 of head n.
// Softmax reference: M (per head) starts at a finite floor and trails the
// running max by at most 8 in log2 units: o and L are rescaled only when a
// score exceeds M + 8 (a compare against a threshold on the raw score), so
// p = exp2(s - M) <= 2^8 and a masked score (-inf) gives p = 0 without a
// guard. Each lane sums its own keys' p; finalize() totals the four lanes of a
// head. The final o / L (with the sink term taken relative to the same M) is
// the same quotient as with the exact running max.
#pragma once

#include "kch_device.h"

namespace kch {

constexpr float kLog2eF = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.f;  // MqaWave: slack of the softmax reference point
// Initial reference point of MqaWave: finite, so exp2(s - M) of a masked score
// (-inf) is 0 without a guard; any finite score exceeds it by far more than
// kRescaleLog2, so the first valid key always resets M.
constexpr float kMFloor = -1e30f;

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

// LDS tiles of rows of HD bf16 (row stride HD, no padding): the 16-byte chunk
// c of row r sits at chunk c ^ tile_swz(r % 16). gfx950 serves a 16-byte LDS
// read 16 lanes at a time over 64 banks (the lanes 4a .. 4a+3 of a 32-lane half
// with the same parity of popcount(a)), a 16-byte write 8 consecutive lanes at
// a time over 32 banks, and the 8-byte transposing read 32 lanes at a time over
// 64 banks. The swizzle keeps all four patterns on a tile free of bank
// conflicts: key-fragment reads (lane: row n = lane % 16, chunk 4s + lane / 16),
// V^T reads (row 4 (lane / 16) + n / 4, half-chunk 2 (2t + n / 2 % 2) + n % 2:
// rows 0..7 and 8..15 each need distinct tile_swz / 2 within a 256-byte bank
// sweep), fragment-layout writes (rows 0..7 need distinct tile_swz % 8 in a
// 128-byte sweep) and row writes (consecutive lanes on one row's chunks).
template <int HD>
__device__ __forceinline__ int tile_swz(int r) {
  if constexpr (HD == 128) return ((r & 7) << 1) | ((r >> 2) & 1);
  else return r & 7;  // 128-byte rows: two rows per 256-byte bank sweep
}

// This lane's element offsets into a 16-row slice of a swizzled tile. Key
// fragment s (row n, chunk 4s + q) sits at chunk
// (4s + q) ^ swz(n) = 4 (s ^ (swz >> 2)) + (q ^ (swz & 3)); V^T read t (row
// 4q + n / 4, half-chunk 2t + (n % 4) / 2) at chunk
// (2t + h) ^ swz = 2 (t ^ (swz >> 1)) + (h ^ (swz & 1)). The s and t terms only
// flip bits of their own, so the offsets are kbase ^ (s << 5), vbase ^ (t << 4).
template <int HD>
struct TileOffsets {
  int kbase, vbase;
  __device__ __forceinline__ TileOffsets() {
    const int l = lane_id(), q = l >> 4, n = l & 15;
    const int ksw = tile_swz<HD>(n);
    const int vr = 4 * q + (n >> 2);
    const int vsw = tile_swz<HD>(vr);
    kbase = n * HD + 8 * (q ^ (ksw & 3)) + 32 * (ksw >> 2);
    vbase = vr * HD + 8 * (((n >> 1) & 1) ^ (vsw & 1)) + 16 * (vsw >> 1) + 4 * (n & 1);
  }
  __device__ __forceinline__ int key(int s) const { return kbase ^ (s << 5); }
  __device__ __forceinline__ int vt(int t) const { return vbase ^ (t << 4); }
};

template <typename T> struct Store4;
template <> struct Store4<float> {
  static __device__ __forceinline__ void run(float* p, f32x4 v, float f) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0] * f, v[1] * f, v[2] * f, v[3] * f);
  }
};
template <> struct Store4<bf16_t> {
  static __device__ __forceinline__ void run(bf16_t* p, f32x4 v, float f) {
    const bf16x4 r = {(bf16_t)(v[0] * f), (bf16_t)(v[1] * f), (bf16_t)(v[2] * f), (bf16_t)(v[3] * f)};
    *reinterpret_cast<bf16x4*>(p) = r;
  }
};
template <> struct Store4<_Float16> {
  static __device__ __forceinline__ void run(_Float16* p, f32x4 v, float f) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 r = {(_Float16)(v[0] * f), (_Float16)(v[1] * f), (_Float16)(v[2] * f), (_Float16)(v[3] * f)};
    *reinterpret_cast<h4*>(p) = r;
  }
};

// Stores o * f of one query (heads [0, nh), row-major [nh][HD] of OT at out)
// as whole rows: the wave writes its 16 x HD block to `buf` (its own LDS, at
// least 16 * HD * sizeof(OT) bytes, 16-byte aligned), 16-byte chunk c of head
// row r at chunk c ^ (r % CPR), then each lane stores 16-byte chunks.
template <int HD, typename OT>
__device__ __forceinline__ void store_rows(const f32x4 (&o)[HD / 16], float f, OT* out, int nh,
                                           void* buf) {
  constexpr int CPR = HD * (int)sizeof(OT) / 16;  // 16-byte chunks per row
  constexpr int EPC = 16 / (int)sizeof(OT);       // elements per chunk
  const int l = lane_id(), q = l >> 4, n = l & 15;
  OT* sb = static_cast<OT*>(buf);
#pragma unroll
  for (int t = 0; t < HD / 16; ++t) {
    const int e0 = 16 * t + 4 * q;                 // first of the lane's 4 dims
    const int c = e0 / EPC;
    Store4<OT>::run(sb + n * HD + EPC * (c ^ (n & (CPR - 1))) + e0 % EPC, o[t], f);
  }
  wave_lds_sync();
#pragma unroll
  for (int i = 0; i < 16 * CPR / 64; ++i) {
    const int r = i * (64 / CPR) + l / CPR, c = l % CPR;
    if (r < nh)
      *reinterpret_cast<uint4*>(out + r * HD + EPC * c) =
          *reinterpret_cast<const uint4*>(sb + r * HD + EPC * (c ^ (r & (CPR - 1))));
  }
}

// One wave, one query, up to 16 heads of head dim HD (64 or 128).
template <int HD>
struct MqaWave {
  static constexpr int NS = HD / 32;          // 32-wide k steps of S^T
  static constexpr int NT = HD / 16;          // O^T tiles
  static constexpr int STAGE_ELEMS = 32 * HD;  // bf16 of a 32-row stage (chunk2)

  bf16x8 qf[NS];  // Q fragments: head n, dims 8q + 32s (sign of the scale folded in)
  f32x4 o[NT];
  float M;        // softmax reference point of head n (log2 units), finite
  float L;        // sum of p over this lane's keys (finalize(): over the head)
  float qscale2;  // |score scale| * log2(e), > 0
  float thr;      // (M + kRescaleLog2) / qscale2: a raw score above it moves M

  // q_row: this lane's head row (nullptr for a padding head -> zeros);
  // normalise: L2-normalise each head row (4 lanes share a head).
  template <typename QT>
  __device__ __forceinline__ void init(const QT* q_row, bool normalise, float scale) {
    const int q = lane_id() >> 4;
    float f[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (q_row) Load8<QT>::run(q_row + 32 * s + 8 * q, f[s]);
      else {
#pragma unroll
        for (int i = 0; i < 8; ++i) f[s][i] = 0.f;
      }
    }
    setup(f, normalise, scale);
  }
  // As init, for a row that is always readable: `keep` false (a padding head
  // or query) zeroes it after the load, so that the load is not conditional.
  template <typename QT>
  __device__ __forceinline__ void init_always(const QT* q_row, bool keep, bool normalise, float scale) {
    const int q = lane_id() >> 4;
    float f[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      Load8<QT>::run(q_row + 32 * s + 8 * q, f[s]);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[s][i] = keep ? f[s][i] : 0.f;
    }
    setup(f, normalise, scale);
  }
  __device__ __forceinline__ void setup(float (&f)[NS][8], bool normalise, float scale) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += f[s][i] * f[s][i];
    float inv = 1.f;
    if (normalise) inv = l2_inv(colq_sum(ss));
    if (scale < 0.f) inv = -inv;  // scores times |scale| from here on
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
    qscale2 = fmaxf(fabsf(scale) * kLog2eF, 1e-30f);  // -inf * qscale2 stays -inf
    thr = (M + kRescaleLog2) / qscale2;
  }

  // S^T accumulator of 16 key rows whose fragments are k (row n of the lane).
  __device__ __forceinline__ f32x4 scores(const bf16x8 (&k)[NS]) const {
    f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k[s], qf[s], st, 0, 0, 0);
    return st;
  }

  // Softmax step over 32 keys: sc = this lane's raw scores of keys 4q..4q+3
  // and 16+4q..16+4q+3 (-inf = masked). Rescales o and L when a score moves
  // M, adds the keys' p to L and returns p as the B operand of the O^T update.
  __device__ __forceinline__ bf16x8 softmax32(const float (&sc)[8]) {
    bool up = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) up |= sc[e] > thr;
    if (__ballot(up)) {
      float mx = sc[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sc[e]);
      const float mnew = fmaxf(M, colq_max(mx) * qscale2);
      const float alpha = fast_exp2(M - mnew);
      L *= alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] *= alpha;
      M = mnew;
      thr = (mnew + kRescaleLog2) / qscale2;
    }
    typedef float f32x8 __attribute__((ext_vector_type(8)));
    f32x8 pe;
    const float nm = -M;
#pragma unroll
    for (int e = 0; e < 8; ++e) pe[e] = fast_exp2(fmaf(sc[e], qscale2, nm));
    L += ((pe[0] + pe[1]) + (pe[2] + pe[3])) + ((pe[4] + pe[5]) + (pe[6] + pe[7]));
    return __builtin_convertvector(pe, bf16x8);
  }

  // V^T fragment t (16 dims x 32 keys) of 32 key rows in a swizzled LDS tile:
  // column 16t + n of rows 4q .. 4q + 3 of each 16-row slice, one transposing
  // read per slice.
  __device__ __forceinline__ static bf16x8 vt_frag(const bf16_t* rows, const TileOffsets<HD>& to,
                                                   int t) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const int vo = to.vt(t);
    const s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(rows + vo));
    const s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(rows + 16 * HD + vo));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // Softmax step and O^T update over 32 keys whose rows (the V^T source) are
  // in a swizzled LDS tile visible to this wave.
  __device__ __forceinline__ void accumulate32(const float (&sc)[8], const bf16_t* rows,
                                               const TileOffsets<HD>& to) {
    const bf16x8 pb = softmax32(sc);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt_frag(rows, to, t), pb, o[t], 0, 0, 0);
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

  // Consume 32 keys already in registers: fa keys 0..15, fb keys 16..31; bit
  // k of valid32 set when key k is valid. `stage` is this wave's LDS buffer of
  // STAGE_ELEMS (the V^T source).
  __device__ __forceinline__ void chunk2(const Frag& fa, const Frag& fb, unsigned valid32,
                                         bf16_t* stage, const TileOffsets<HD>& to) {
    const int q = lane_id() >> 4;
    wave_lds_sync();  // the previous step's V^T reads are done before the overwrite
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      *reinterpret_cast<bf16x8*>(stage + to.key(s)) = fa.k[s];
      *reinterpret_cast<bf16x8*>(stage + 16 * HD + to.key(s)) = fb.k[s];
    }
    const f32x4 sa = scores(fa.k), sb = scores(fb.k);
    float sc[8] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
    if (valid32 != 0xffffffffu) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!((valid32 >> (4 * q + e)) & 1u)) sc[e] = -INFINITY;
        if (!((valid32 >> (16 + 4 * q + e)) & 1u)) sc[4 + e] = -INFINITY;
      }
    }
    wave_lds_sync();  // staged rows visible to the whole wave
    accumulate32(sc, stage, to);
  }

  // Row-major gathers of 32 key rows: a wave load instruction covers RPI whole
  // rows (TPR lanes of 16 bytes per row), so it touches 2 RPI cache lines
  // instead of the 16 half-lines of a fragment-layout load. Load i of a step
  // holds rows i * RPI + lane / TPR, 16-byte chunk lane % TPR.
  static constexpr int TPR = HD / 8;        // lanes (16-byte chunks) per row
  static constexpr int RPI = 64 / TPR;      // rows per load instruction
  static constexpr int NLI = 32 / RPI;      // load instructions per 32 rows
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct Rows {
    u32x4 v[NLI];
  };
  // Consume 32 keys gathered row-major (row r of the step = key r); bit r of
  // valid32 set when key r is valid. The rows go to this wave's swizzled stage
  // (STAGE_ELEMS), from which both the key fragments and V^T are read.
  __device__ __forceinline__ void chunk_rows(const Rows& rr, unsigned valid32, bf16_t* stage,
                                             const TileOffsets<HD>& to) {
    const int l = lane_id(), q = l >> 4;
    wave_lds_sync();  // the previous step's reads of the stage are done before the overwrite
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      const int r = i * RPI + l / TPR, c = l % TPR;
      *reinterpret_cast<u32x4*>(stage + r * HD + 8 * (c ^ tile_swz<HD>(r & 15))) = rr.v[i];
    }
    wave_lds_sync();  // staged rows visible to the whole wave
    f32x4 sa, sb;
    {
      bf16x8 kf[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) kf[s] = *reinterpret_cast<const bf16x8*>(stage + to.key(s));
      sa = scores(kf);
#pragma unroll
      for (int s = 0; s < NS; ++s) kf[s] = *reinterpret_cast<const bf16x8*>(stage + 16 * HD + to.key(s));
      sb = scores(kf);
    }
    float sc[8] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
    if (valid32 != 0xffffffffu) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!((valid32 >> (4 * q + e)) & 1u)) sc[e] = -INFINITY;
        if (!((valid32 >> (16 + 4 * q + e)) & 1u)) sc[4 + e] = -INFINITY;
      }
    }
    accumulate32(sc, stage, to);
  }

  // Score-layout gathers of 32 key rows. Lane group q = lane / 16 loads the
  // rows whose scores it holds after the S^T MFMAs: slot k (0..7) is row
  // row_sl(k, q) = 4q + k (k < 4) or 16 + 4q + k - 4, the key of sc[k]. So
  // each lane knows the validity of its own scores from the row indices it
  // loaded (no ballots, no mask bits to assemble). A load instruction still
  // covers whole rows: with TPR = 16 (HD 128) load i is slot i of every lane
  // (rows i, 4 + i, 8 + i, 12 + i for i < 4); with TPR = 8 (HD 64) the two
  // 8-lane halves of a group take slots i and 4 + i.
  __device__ __forceinline__ static int row_sl(int k, int q) { return 4 * q + k + (k >= 4 ? 12 : 0); }
  __device__ __forceinline__ static int slot_sl(int i) {
    return TPR == 16 ? i : i + 4 * ((lane_id() >> 3) & 1);
  }
  // full: every row of the step is valid (ok is not read).
  __device__ __forceinline__ void chunk_sl(const Rows& rr, const bool (&ok)[8], bf16_t* stage,
                                           const TileOffsets<HD>& to, bool full = false) {
    const int l = lane_id(), q = l >> 4, c = l % TPR;
    wave_lds_sync();  // the previous step's reads of the stage are done before the overwrite
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      const int r = row_sl(slot_sl(i), q);
      *reinterpret_cast<u32x4*>(stage + r * HD + 8 * (c ^ tile_swz<HD>(r & 15))) = rr.v[i];
    }
    wave_lds_sync();  // staged rows visible to the whole wave
    f32x4 sa, sb;
    {
      bf16x8 kf[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) kf[s] = *reinterpret_cast<const bf16x8*>(stage + to.key(s));
      sa = scores(kf);
#pragma unroll
      for (int s = 0; s < NS; ++s) kf[s] = *reinterpret_cast<const bf16x8*>(stage + 16 * HD + to.key(s));
      sb = scores(kf);
    }
    float sc[8] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
    if (!full) {
#pragma unroll
      for (int k = 0; k < 8; ++k) sc[k] = ok[k] ? sc[k] : -INFINITY;
    }
    accumulate32(sc, stage, to);
  }

  // Totals L over the 4 lanes of each head; call once, after the last step.
  __device__ __forceinline__ void finalize() { L = colq_sum(L); }

  // Final normalisation (after finalize). Returns the multiplier for o (0 when
  // nothing is valid).
  __device__ __forceinline__ float finish(bool has_sink, float sink) const {
    float denom = L;
    if (has_sink) denom += fast_exp2(sink * kLog2eF - M);
    return (L > 0.f) ? 1.f / denom : 0.f;
  }
};

}  // namespace kch
