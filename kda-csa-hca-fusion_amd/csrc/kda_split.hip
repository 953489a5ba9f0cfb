// KDA chunked prefill as two kernels (bf16 / fp16 inputs, K in {64,128}, V in {64,128}).
//
// Restates the chunkwise WY/UT form of naive_chunk_kda
// (/root/reference/ops_kda.py:340-536). The state-independent part of every
// chunk is computed by a fully parallel kernel; a second kernel carries the
// fp32 state through the chunks with four small MFMA products per chunk.
//
// Per chunk of C = 64 tokens (G = in-chunk cumsum of the clamped gate, log2
// units internally; G_l = G at the last token):
//   L[i][j]   = beta_i sum_ch k_i e(G_i - G_j) k_j      (j <  i)
//   Aqk[i][j] = scale  sum_ch q_i e(G_i - G_j) k_j      (j <= i)
//   X  = (I + L)^{-1}
//   W' = X (beta k e(G)),   U = X (beta v)             (= w, u of ops_kda.py:418-424)
//   qg = scale q e(G),      kd = k e(G_l - G),   el = e(G_l)
// and, sequentially over the chunks (ops_kda.py:515-535):
//   v_new = U - W' S;   o = qg S + Aqk v_new;   S = diag(el) S + kd^T v_new
//
// kda_prep_kernel   one workgroup (4 waves) per (b, hv, chunk); wave w owns
//   token tile w. q/k/g/v are loaded straight into MFMA fragment layout
//   (lane = token, 8 consecutive channels per 32-channel step); the gate cumsum
//   is a DPP row scan plus a cross-wave carry. L and Aqk use decay factors
//   anchored at token 31 (e(G - G_a), e(G_a - G)) when every |G - G_a| <= 80
//   nats; otherwise they are formed exactly, one exponential per
//   (i, j, channel), with the reference's clamp(max=50) on the exponent.
//   Transposes of elementwise data (beta k e(G), k e(G_l - G), beta v) are
//   MFMA products with a 0/1 selector matrix, exact in fp32 accumulation.
// kda_state_kernel  one workgroup per (b, hv, 64-, 32- or 16-column slice of V); sibling
//   slices of one head sit on the same XCD so the shared per-chunk operands
//   are read from HBM once. The state lives in MFMA accumulators; the operands
//   of chunk n+2 are prefetched into registers while chunk n is processed.
//
// Workspace records (one per (b, hv, chunk), bf16 unless noted). Every matrix
// is stored as 16x16x32 MFMA A-operand fragments, 16 bytes per lane, so a wave
// reads one fragment with one coalesced 1 KB load:
//   wp  [C][K]  W' (row tile, k step) fragments, "packed" channel order
//   qg  [C][K]  qg fragments, packed channel order
//   kdt [K][C]  kd^T fragments, packed token order
//   aqk [C][C]  Aqk fragments, packed token order
//   u   [C][V]  U in accumulator layout (4 values per lane per 16x16 tile)
//   el  [K]     fp32
// Natural order: lane quad q of a 32-wide k step holds k = 8q .. 8q+7. Packed
// order: it holds k = 4q .. 4q+3 of the first 16 and 16+4q .. 16+4q+3 of the
// second 16 — the layout an accumulator tile has after a transpose, so
// products written by MFMAs need no shuffle. Both operands of every product
// use the same order.

#include <utility>

#include "kch_device.h"
#include "kch_kernels.h"
#include "kda_common.h"

namespace kch {

namespace {

using namespace kda_detail;

constexpr int C = 64;
constexpr float kCap2 = 50.f * kLog2e;  // clamp(max=50) of ops_kda.py:414,516, log2 units

struct SplitPtrs {
  bf16_t* wp;
  bf16_t* qg;
  bf16_t* kdt;
  bf16_t* aqk;
  bf16_t* u;
  float* el;
};

template <typename InT>
__device__ __forceinline__ void unpack8(const uint4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = elem<InT>(w[i], 0);
    f[2 * i + 1] = elem<InT>(w[i], 1);
  }
}

__device__ __forceinline__ bf16x8 pack8(const float* f) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16_t)f[i];
  return r;
}

__device__ __forceinline__ bf16x8 cat4(bf16x4 a, bf16x4 b) {
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ bf16x4 to_bf16x4(const f32x4& v) {
  return bf16x4{(bf16_t)v[0], (bf16_t)v[1], (bf16_t)v[2], (bf16_t)v[3]};
}

// out[i] = value of lane i of this lane's 16-lane DPP row (row_share:i), i < 8
template <int... I>
__device__ __forceinline__ void row_bcast8(float v, float* out, std::integer_sequence<int, I...>) {
  ((out[I] = dpp<0x150 + I, false>(v)), ...);
}

__device__ __forceinline__ f32x4 mfma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int K, int V>
struct PrepLayout {
  static constexpr int KS = K / 32;
  static constexpr int LDC = C + 8;  // bf16 row stride of [*][64] buffers
  static constexpr int LDY = 32 + 8;
  static constexpr int LDD = 20;
  static constexpr int cmax(int a, int b) { return a > b ? a : b; }
  // R0: sB fragment exchange [4][KS][64] x 16 B; then L (bf16) + fp32 diagonal
  //     blocks; in the exact path first the fp32 gate cumsum of 64 channels
  static constexpr int SZ_XB = 4 * KS * 64 * 16;
  static constexpr int SZ_LOP = C * LDC * 2;
  static constexpr int SZ_LD = 4 * 16 * LDD * 4;
  static constexpr int SZ_R0 = cmax(cmax(SZ_XB, SZ_LOP + SZ_LD), C * 64 * 4);
  static constexpr int OFF_XB = 0, OFF_LOP = 0, OFF_LD = SZ_LOP, OFF_EG = 0;
  // R1: X and X^T; in the exact path first k and q (bf16 [64][64] each)
  static constexpr int OFF_X = SZ_R0;
  static constexpr int OFF_XT = OFF_X + C * LDC * 2;
  static constexpr int OFF_EK = OFF_X, OFF_EQ = OFF_X + C * 64 * 2;
  // also in R1, during the factor stage: qg staged row-major [64][K + 8]
  static constexpr int OFF_QGS = OFF_X, LDQ = K + 8;
  static_assert(C * LDQ * 2 <= 2 * C * LDC * 2, "qg staging fits in R1");
  // R2: per-wave tile sums of the gate [4][K] fp32; then the inverse's Y scratch
  static constexpr int OFF_R2 = OFF_XT + C * LDC * 2;
  static constexpr int SZ_R2 = cmax(4 * K * 4, (2 * 16 * LDY + 32 * LDY) * 2);
  static constexpr int OFF_TS = OFF_R2, OFF_Y1 = OFF_R2, OFF_Y2 = OFF_R2 + 2 * 16 * LDY * 2;
  // R3: (beta k e(G))^T [K][LDC];  R4: (beta v)^T [V][LDC]
  static constexpr int OFF_KGT = OFF_R2 + SZ_R2;
  static constexpr int OFF_VBT = OFF_KGT + K * LDC * 2;
  static constexpr int OFF_BETA = OFF_VBT + V * LDC * 2;
  static constexpr int OFF_FLAG = OFF_BETA + C * 4;
  static constexpr int BYTES = OFF_FLAG + 16;
  static_assert(OFF_EQ + C * 64 * 2 <= OFF_R2, "exact-path k, q fit in R1");
  static_assert(BYTES <= 80 * 1024, "two workgroups per CU");
};

template <int K, int V, typename InT>
__global__ __launch_bounds__(256, 2) void kda_prep_kernel(KdaParams p, SplitPtrs ws) {
  using L = PrepLayout<K, V>;
  constexpr int KS = K / 32, VS = V / 32, KT = K / 16, VT = V / 16;
  constexpr int LDC = L::LDC, LDY = L::LDY, LDD = L::LDD;
  __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
  bf16x8* sXB = reinterpret_cast<bf16x8*>(smem + L::OFF_XB);
  bf16_t* sLop = reinterpret_cast<bf16_t*>(smem + L::OFF_LOP);
  float* sLd = reinterpret_cast<float*>(smem + L::OFF_LD);
  bf16_t* sX = reinterpret_cast<bf16_t*>(smem + L::OFF_X);
  bf16_t* sXt = reinterpret_cast<bf16_t*>(smem + L::OFF_XT);
  float* sTs = reinterpret_cast<float*>(smem + L::OFF_TS);
  bf16_t* sY1 = reinterpret_cast<bf16_t*>(smem + L::OFF_Y1);
  bf16_t* sY2t = reinterpret_cast<bf16_t*>(smem + L::OFF_Y2);
  bf16_t* sKgT = reinterpret_cast<bf16_t*>(smem + L::OFF_KGT);
  bf16_t* sVbT = reinterpret_cast<bf16_t*>(smem + L::OFF_VBT);
  float* sBeta = reinterpret_cast<float*>(smem + L::OFF_BETA);
  int* sFlag = reinterpret_cast<int*>(smem + L::OFF_FLAG);
  float* sEG = reinterpret_cast<float*>(smem + L::OFF_EG);
  bf16_t* sEK = reinterpret_cast<bf16_t*>(smem + L::OFF_EK);
  bf16_t* sEQ = reinterpret_cast<bf16_t*>(smem + L::OFF_EQ);
  bf16_t* sQgs = reinterpret_cast<bf16_t*>(smem + L::OFF_QGS);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15, q4 = lane >> 4;
  const int T = p.T;
  const int NT = (T + C - 1) / C;
  const int n = blockIdx.x % NT;
  const int bh = blockIdx.x / NT;
  const int hv = bh % p.HV;
  const int b = bh / p.HV;
  const int h = hv / (p.HV / p.H);
  const size_t rec = blockIdx.x;  // (b * HV + hv) * NT + n
  const int tk = 16 * wave + r;   // token of this lane within the chunk
  const int t = n * C + tk;
  const bool valid = t < T;
  const int tl = valid ? t : T - 1;

  // ---- loads straight into fragment layout ----
  const InT* qrow = static_cast<const InT*>(p.q) + ((size_t)(b * T + tl) * p.H + h) * K;
  const InT* krow = static_cast<const InT*>(p.k) + ((size_t)(b * T + tl) * p.H + h) * K;
  const InT* grow = static_cast<const InT*>(p.g) + ((size_t)(b * T + tl) * p.HV + hv) * K;
  const InT* vrow = static_cast<const InT*>(p.v) + ((size_t)(b * T + tl) * p.HV + hv) * V;
  // Issued in the order they are consumed (the gate scan, beta, the factor
  // stage's k and q, then v): memory waits count in issue order, so a value
  // needed early must not sit behind loads needed later.
  uint4 rq[KS], rk[KS], rg[KS], rv[VS];
#pragma unroll
  for (int s = 0; s < KS; ++s) rg[s] = *reinterpret_cast<const uint4*>(grow + 32 * s + 8 * q4);
  const float bt =
      valid ? to_f32(static_cast<const InT*>(p.beta)[(size_t)(b * T + tl) * p.HV + hv]) : 0.f;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    rk[s] = *reinterpret_cast<const uint4*>(krow + 32 * s + 8 * q4);
    rq[s] = *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * q4);
  }
#pragma unroll
  for (int s = 0; s < VS; ++s) rv[s] = *reinterpret_cast<const uint4*>(vrow + 32 * s + 8 * q4);
  if (tid == 0) sFlag[0] = 0;

  // ---- gate: clamp, log2 units, in-tile inclusive scan over the 16 tokens of the row ----
  const float clampv = p.g_clamp_min;
  float G[KS][8];
  float gmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    float f[8];
    unpack8<InT>(rg[s], f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // padded tokens carry g = 0 before the clamp, as the reference pads (ops_kda.py:375-382)
      const float gv = fmaxf(valid ? f[i] : 0.f, clampv);
      gmax = fmaxf(gmax, gv);
      G[s][i] = row_prefix_sum(gv * kLog2e);
    }
  }
  if (r == 15) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      float* dst = sTs + wave * K + 32 * s + 8 * q4;
      *reinterpret_cast<float4*>(dst) = make_float4(G[s][0], G[s][1], G[s][2], G[s][3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(G[s][4], G[s][5], G[s][6], G[s][7]);
    }
  }
  if (q4 == 0) sBeta[tk] = bt;
  __syncthreads();  // ---- B1: tile sums ----

  // ---- carry, anchors, factors ----
  const float scale = p.scale;
  float dmax = 0.f;
  bf16x8 fa[KS], fq[KS], fb[KS];
  bf16x8 sel[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int i = 0; i < 8; ++i) sel[hh][i] = (bf16_t)((8 * q4 + i == 16 * hh + r) ? 1.f : 0.f);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

  // carry from the earlier token tiles of the chunk (wave-uniform 0/1 weights)
  const float m1 = wave > 0 ? 1.f : 0.f, m2 = wave > 1 ? 1.f : 0.f, m3 = wave > 2 ? 1.f : 0.f;
  bf16_t* const qg_out = ws.qg + rec * (C * K);
  bf16x4* const kdt_out = reinterpret_cast<bf16x4*>(ws.kdt + rec * (K * C));
  // Padded tokens (t >= T) read token T-1 and carry beta = 0: every product that
  // reaches a stored output then vanishes (their L rows, U rows, W' rows and
  // k-weighted state updates are zero), so their q, k, v need no masking.
  auto emit_qkd = [&](int s, const float* qg8, const float* kg8, const float* kd8) {
    // qg leaves in packed channel order (the order of W'): staged through this
    // wave's own rows of LDS
    bf16_t* qrow_s = sQgs + tk * L::LDQ + 32 * s;
    *reinterpret_cast<bf16x8*>(qrow_s + 8 * q4) = pack8(qg8);
    wave_lds_sync();
    reinterpret_cast<bf16x8*>(qg_out)[(wave * KS + s) * 64 + lane] =
        cat4(*reinterpret_cast<const bf16x4*>(qrow_s + 4 * q4),
             *reinterpret_cast<const bf16x4*>(qrow_s + 16 + 4 * q4));
    wave_lds_sync();
    const bf16x8 kg = pack8(kg8), kd = pack8(kd8);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      // lane: channel 32s + 16hh + r, tokens 16 wave + 4 q4 + e
      const f32x4 tg = mfma32(kg, sel[hh], z4);
      *reinterpret_cast<bf16x4*>(sKgT + (32 * s + 16 * hh + r) * LDC + 16 * wave + 4 * q4) =
          to_bf16x4(tg);
      const f32x4 td = mfma32(kd, sel[hh], z4);
      const int rt = 2 * s + hh;  // channel tile = row tile of kd^T
      kdt_out[((rt * 2 + (wave >> 1)) * 64 + lane) * 2 + (wave & 1)] = to_bf16x4(td);
    }
  };
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    // G - G_a = (in-tile prefix) + off, with the carry of the earlier tiles and
    // the anchor G_a = T_0 + T_1 (tile sums T_w) folded into one offset per
    // channel: -(T_0 + T_1), -T_1, 0, T_2 for waves 0..3
    float off[8];
    {
      auto tile8 = [&](int w, float (&f)[8]) {
        const float4 a = *reinterpret_cast<const float4*>(sTs + w * K + 32 * s + 8 * q4);
        const float4 c = *reinterpret_cast<const float4*>(sTs + w * K + 32 * s + 8 * q4 + 4);
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = c.x; f[5] = c.y; f[6] = c.z; f[7] = c.w;
      };
      float t1[8];
      if (wave == 0) {
        float t0[8];
        tile8(0, t0);
        tile8(1, t1);
#pragma unroll
        for (int i = 0; i < 8; ++i) off[i] = -(t0[i] + t1[i]);
      } else if (wave == 1) {
        tile8(1, t1);
#pragma unroll
        for (int i = 0; i < 8; ++i) off[i] = -t1[i];
      } else if (wave == 2) {
#pragma unroll
        for (int i = 0; i < 8; ++i) off[i] = 0.f;
      } else {
        tile8(2, off);
      }
    }
    // Per-channel constants e(G_a) and e(G_l - G_a): lane r of the row evaluates
    // them for channel 32s + 8q4 + (r & 7) and row_share broadcasts them. With
    // |G - G_a| <= 80 nats every product below stays finite; a factor that
    // underflows belongs to a term below bf16 resolution of the output.
    float cA[8], cL[8];
    {
      const int ch = 32 * s + 8 * q4 + (r & 7);
      const float ga = sTs[ch] + sTs[K + ch];
      const float gl = ga + sTs[2 * K + ch] + sTs[3 * K + ch];
      row_bcast8(fast_exp2(ga), cA, std::make_integer_sequence<int, 8>());
      row_bcast8(fast_exp2(gl - ga), cL, std::make_integer_sequence<int, 8>());
    }
    float kf[8], qf[8];
    unpack8<InT>(rk[s], kf);
    unpack8<InT>(rq[s], qf);
    float a8[8], q8[8], b8[8], qg8[8], kg8[8], kd8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float d = G[s][i] + off[i];
      dmax = fmaxf(dmax, fabsf(d));
      const float R = fast_exp2(d), Ci = fast_exp2(-d);
      a8[i] = kf[i] * R;              // k e(G - G_a)
      q8[i] = scale * qf[i] * R;      // scale q e(G - G_a)
      b8[i] = kf[i] * Ci;             // k e(G_a - G)
      qg8[i] = q8[i] * cA[i];         // scale q e(G)
      kg8[i] = bt * a8[i] * cA[i];    // beta k e(G)
      kd8[i] = b8[i] * cL[i];         // k e(G_l - G)
    }
    fa[s] = pack8(a8);
    fq[s] = pack8(q8);
    fb[s] = pack8(b8);
    sXB[(wave * KS + s) * 64 + lane] = fb[s];
    emit_qkd(s, qg8, kg8, kd8);
    if (wave == 0 && r == 0) {
      float* e = ws.el + rec * K + 32 * s + 8 * q4;
      *reinterpret_cast<float4*>(e) =
          make_float4(cA[0] * cL[0], cA[1] * cL[1], cA[2] * cL[2], cA[3] * cL[3]);
      *reinterpret_cast<float4*>(e + 4) =
          make_float4(cA[4] * cL[4], cA[5] * cL[5], cA[6] * cL[6], cA[7] * cL[7]);
    }
  }
  if (__builtin_amdgcn_ballot_w64(dmax > kRange2)) {
    // Some element of this wave lies outside the anchored range (the chunk takes
    // the exact L / Aqk path): the factored products may overflow, so qg, kg and
    // kd are evaluated again with direct exponentials and rewritten.
    // (q, k and g are reloaded and the gate scan redone, so that nothing of the
    // main loop stays live for this rare pass)
#pragma unroll 1
    for (int s = 0; s < KS; ++s) {
      float kf[8], qf[8], gf[8], qg8[8], kg8[8], kd8[8];
      unpack8<InT>(*reinterpret_cast<const uint4*>(krow + 32 * s + 8 * q4), kf);
      unpack8<InT>(*reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * q4), qf);
      unpack8<InT>(*reinterpret_cast<const uint4*>(grow + 32 * s + 8 * q4), gf);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int ch = 32 * s + 8 * q4 + i;
        const float t0 = sTs[ch], t1 = sTs[K + ch], t2 = sTs[2 * K + ch], t3 = sTs[3 * K + ch];
        const float Gi = row_prefix_sum(fmaxf(valid ? gf[i] : 0.f, clampv) * kLog2e) +
                         fmaf(m1, t0, fmaf(m2, t1, m3 * t2));
        const float eG = fast_exp2(Gi);
        qg8[i] = scale * qf[i] * eG;
        kg8[i] = bt * kf[i] * eG;
        kd8[i] = kf[i] * fast_exp2(t0 + t1 + t2 + t3 - Gi);
      }
      emit_qkd(s, qg8, kg8, kd8);
    }
  }
#pragma unroll
  for (int s = 0; s < VS; ++s) {
    float vf[8];
    unpack8<InT>(rv[s], vf);
#pragma unroll
    for (int i = 0; i < 8; ++i) vf[i] = bt * vf[i];
    const bf16x8 vb = pack8(vf);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const f32x4 tv = mfma32(vb, sel[hh], z4);
      *reinterpret_cast<bf16x4*>(sVbT + (32 * s + 16 * hh + r) * LDC + 16 * wave + 4 * q4) =
          to_bf16x4(tv);
    }
  }
  {
    // the wave's flags, OR-ed by ballots: one LDS atomic per wave (the lanes'
    // own atomics on one word serialise, and the outer token tiles, far from
    // the anchor, set the range flag on most lanes)
    const int fl = (__builtin_amdgcn_ballot_w64(dmax > kRange2) ? 1 : 0) |
                   (__builtin_amdgcn_ballot_w64(gmax > 0.f) ? 2 : 0) |
                   (__builtin_amdgcn_ballot_w64(dmax > kPos2) ? 4 : 0);
    if (fl && lane == 0) atomicOr(sFlag, fl);
  }
  __syncthreads();  // ---- B2: sB exchange, kg^T, (beta v)^T, flags ----

  const int flag = sFlag[0];
  const bool exact = (flag & 1) || ((flag & 2) && (flag & 4));
  bf16x4* aqk_out = reinterpret_cast<bf16x4*>(ws.aqk + rec * (C * C));
  if (!exact) {
    // L^T and Aqk^T tiles (j tile tj, i tile = wave): A = sB[tj], B = sA / sQ of this wave
    f32x4 lt[4], at[4];
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      lt[tj] = z4;
      at[tj] = z4;
      if (tj <= wave) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 xb = (tj == wave) ? fb[s] : sXB[(tj * KS + s) * 64 + lane];
          lt[tj] = mfma32(xb, fa[s], lt[tj]);
          at[tj] = mfma32(xb, fq[s], at[tj]);
        }
      }
    }
    // lane: L / Aqk row i = tk, columns j = 16 tj + 4 q4 + e
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      f32x4 av;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 16 * tj + 4 * q4 + e;
        av[e] = (tj <= wave && j <= tk) ? at[tj][e] : 0.f;
        lt[tj][e] = (tj <= wave && j < tk) ? lt[tj][e] * bt : 0.f;
      }
      aqk_out[((wave * 2 + (tj >> 1)) * 64 + lane) * 2 + (tj & 1)] = to_bf16x4(av);
    }
    __syncthreads();  // ---- B3: the sB exchange is dead; R0 becomes L ----
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      if (tj <= wave)
        *reinterpret_cast<bf16x4*>(sLop + tk * LDC + 16 * tj + 4 * q4) = to_bf16x4(lt[tj]);
      if (tj == wave) {
        // fp32 diagonal block, columns stored permuted: c -> (c & 3) * 4 + (c >> 2)
        float* d = sLd + (wave * 16 + r) * LDD;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e * 4 + q4] = lt[tj][e];
      }
    }
  } else {
    // ---- exact L / Aqk: one exponential per (i, j, channel), 64 channels per pass ----
    const int i = tid >> 2, jg = tid & 3;
    float lacc[16], aacc[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) lacc[u] = aacc[u] = 0.f;
#pragma unroll
    for (int half = 0; half < K / 64; ++half) {
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        // reload this lane's k, q, g and redo the gate scan (the tile sums are still in sTs)
        const int ch0 = 64 * half + 32 * ss + 8 * q4;
        float kf[8], qf[8], gf[8];
        unpack8<InT>(*reinterpret_cast<const uint4*>(krow + ch0), kf);
        unpack8<InT>(*reinterpret_cast<const uint4*>(qrow + ch0), qf);
        unpack8<InT>(*reinterpret_cast<const uint4*>(grow + ch0), gf);
        const int c0 = 32 * ss + 8 * q4;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float carry = 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w)
            if (w < wave) carry += sTs[w * K + ch0 + e];
          const float gl = row_prefix_sum(fmaxf(valid ? gf[e] : 0.f, clampv) * kLog2e) + carry;
          sEG[tk * 64 + c0 + e] = gl;
          sEK[tk * 64 + c0 + e] = (bf16_t)(valid ? kf[e] : 0.f);
          sEQ[tk * 64 + c0 + e] = (bf16_t)(valid ? qf[e] : 0.f);
        }
      }
      __syncthreads();
      for (int ch = 0; ch < 64; ++ch) {
        const float gi = sEG[i * 64 + ch];
        const float ki = (float)sEK[i * 64 + ch];
        const float qi = (float)sEQ[i * 64 + ch];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int j = jg + 4 * u;
          const float e = fast_exp2(fminf(gi - sEG[j * 64 + ch], kCap2));
          const float kj = (float)sEK[j * 64 + ch];
          lacc[u] += ki * kj * e;
          aacc[u] += qi * kj * e;
        }
      }
      __syncthreads();
    }
    const float bi = sBeta[i];
    bf16_t* aq = ws.aqk + rec * (C * C);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int j = jg + 4 * u;
      const float lv = j < i ? bi * lacc[u] : 0.f;
      const float av = j <= i ? scale * aacc[u] : 0.f;
      sLop[i * LDC + j] = (bf16_t)lv;
      if ((i >> 4) == (j >> 4)) {
        const int jj = j & 15;
        sLd[((i >> 4) * 16 + (i & 15)) * LDD + (jj & 3) * 4 + (jj >> 2)] = lv;
      }
      const int fl = (i & 15) + 16 * ((j & 15) >> 2);
      aq[(((i >> 4) * 2 + (j >> 5)) * 64 + fl) * 8 + ((j >> 4) & 1) * 4 + (j & 3)] = (bf16_t)av;
    }
  }
  __syncthreads();  // ---- B_LA ----

  // ============ inverse of I + L: 16x16 diagonal blocks in fp32, wave d -> block d ============
  {
    const int blk = wave;
    const int cc = lane >> 2;   // column of the block inverse
    const int part = lane & 3;  // this lane sums the terms k = 4j + part
    float Lr[16][4];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float4 v = *reinterpret_cast<const float4*>(sLd + (blk * 16 + rr) * LDD + part * 4);
      Lr[rr][0] = v.x; Lr[rr][1] = v.y; Lr[rr][2] = v.z; Lr[rr][3] = v.w;
    }
    float xs[4] = {0.f, 0.f, 0.f, 0.f};  // x[4j + part] of column cc
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float sacc = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * j < rr) sacc += Lr[rr][j] * xs[j];
      sacc += dpp<0xb1, false>(sacc);  // quad_perm [1,0,3,2]
      sacc += dpp<0x4e, false>(sacc);  // quad_perm [2,3,0,1]
      const float xr = (rr < cc) ? 0.f : ((rr == cc) ? 1.f : -sacc);
      if ((rr & 3) == part) xs[rr >> 2] = xr;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = 4 * j + part;
      sX[(16 * blk + rr) * LDC + 16 * blk + cc] = (bf16_t)xs[j];
      sXt[(16 * blk + cc) * LDC + 16 * blk + rr] = (bf16_t)xs[j];
    }
  }
  __syncthreads();  // ---- B_I0 ----
  // level 1: X[2w+1][2w] = -X[2w+1][2w+1] L[2w+1][2w] X[2w][2w]
  if (wave < 2) {
    const int d0 = 2 * wave, d1 = 2 * wave + 1;
    bf16_t* y = sY1 + wave * 16 * LDY;
    f32x4 acc = mma16<16>(z4, sLop + 16 * d1 * LDC + 16 * d0, LDC, sXt + 16 * d0 * LDC + 16 * d0, LDC);
    st_bf16x4(y + acc_col() * LDY + acc_row(0), acc[0], acc[1], acc[2], acc[3]);
    wave_lds_sync();
    acc = mma16<16>(z4, sX + 16 * d1 * LDC + 16 * d1, LDC, y, LDY);
#pragma unroll
    for (int e = 0; e < 4; ++e) sX[(16 * d1 + acc_row(e)) * LDC + 16 * d0 + acc_col()] = (bf16_t)(-acc[e]);
    st_bf16x4(sXt + (16 * d0 + acc_col()) * LDC + 16 * d1 + acc_row(0), -acc[0], -acc[1], -acc[2],
              -acc[3]);
  }
  __syncthreads();  // ---- B_I1 ----
  // level 2: Y2 = L[32:,:32] X[:32,:32]
  {
    const int i = wave >> 1, j = wave & 1;
    f32x4 acc = z4;
    if (j == 0)
      acc = mma16<32>(acc, sLop + (32 + 16 * i) * LDC, LDC, sXt, LDC);
    else
      acc = mma16<16>(acc, sLop + (32 + 16 * i) * LDC + 16, LDC, sXt + 16 * LDC + 16, LDC);
    st_bf16x4(sY2t + (16 * j + acc_col()) * LDY + 16 * i + acc_row(0), acc[0], acc[1], acc[2], acc[3]);
  }
  __syncthreads();  // ---- B_I2 ----
  // X[32:,:32] = -X[32:,32:] Y2
  {
    const int i = wave >> 1, j = wave & 1;
    f32x4 acc = z4;
    if (i == 0)
      acc = mma16<16>(acc, sX + 32 * LDC + 32, LDC, sY2t + 16 * j * LDY, LDY);
    else
      acc = mma16<32>(acc, sX + 48 * LDC + 32, LDC, sY2t + 16 * j * LDY, LDY);
#pragma unroll
    for (int e = 0; e < 4; ++e) sX[(32 + 16 * i + acc_row(e)) * LDC + 16 * j + acc_col()] = (bf16_t)(-acc[e]);
    st_bf16x4(sXt + (16 * j + acc_col()) * LDC + 32 + 16 * i + acc_row(0), -acc[0], -acc[1], -acc[2],
              -acc[3]);
  }
  __syncthreads();  // ---- B_I3 ----

  // ============ W'^T = kg^T X^T and U = X (beta v), written as fragments ============
  bf16x4* wp_out = reinterpret_cast<bf16x4*>(ws.wp + rec * (C * K));
  bf16x4* u_out = reinterpret_cast<bf16x4*>(ws.u + rec * (C * V));
  auto wtile = [&](int wt, auto BI_) {
    constexpr int bi = decltype(BI_)::value;
    const f32x4 acc = mma16<16 * (bi + 1)>(z4, sKgT + 16 * wt * LDC, LDC, sX + 16 * bi * LDC, LDC);
    // lane: channels 16 wt + 4 q4 + e of token 16 bi + r -> packed half (wt & 1) of k step wt / 2
    wp_out[((bi * KS + (wt >> 1)) * 64 + lane) * 2 + (wt & 1)] = to_bf16x4(acc);
  };
  auto utile = [&](int ct, auto TT_) {
    constexpr int tt = decltype(TT_)::value;
    const f32x4 acc = mma16<16 * (tt + 1)>(z4, sX + 16 * tt * LDC, LDC, sVbT + 16 * ct * LDC, LDC);
    u_out[(tt * VT + ct) * 64 + lane] = to_bf16x4(acc);
  };
#pragma unroll
  for (int j = 0; j < KT / 4; ++j) {
    const int wt = wave * (KT / 4) + j;
    wtile(wt, IC<0>());
    wtile(wt, IC<1>());
    wtile(wt, IC<2>());
    wtile(wt, IC<3>());
  }
#pragma unroll
  for (int j = 0; j < VT / 4; ++j) {
    const int ct = wave * (VT / 4) + j;
    utile(ct, IC<0>());
    utile(ct, IC<1>());
    utile(ct, IC<2>());
    utile(ct, IC<3>());
  }
}

template <int K, int BV, typename OutT>
__global__ __launch_bounds__(256, 1) void kda_state_kernel(KdaParams p, SplitPtrs ws) {
  constexpr int KS = K / 32, CT = BV / 16, RT = K / 64;
  constexpr int LDO = BV + 8;  // sO row stride: row = token
  // sS (row = value column, K channels) and sVn (row = value column, C tokens)
  // hold each 32-element block in packed order, element 4a + i (a, i < 4) at
  // 8a + i and element 16 + 4a + i at 8a + 4 + i, so an MFMA fragment of the
  // block (packed k = 4q .. 4q+3, 16+4q .. 16+4q+3) is one 16-byte read. The
  // 16-byte chunks of a row are XOR-swizzled by the row (swz_s, swz_v): every
  // fragment read and every 16-byte state write is free of bank conflicts (a
  // 16-byte LDS read is served 16 lanes at a time, lanes 4a .. 4a+3 of a
  // 32-lane half grouped by the parity of a; 16-byte writes 8 lanes at a
  // time). Pairs of 8-byte reads would be merged into ds_read2_b64, which
  // moves a quarter of the bytes per cycle of ds_read_b128.
  __shared__ __attribute__((aligned(16))) bf16_t sS[BV * K];
  __shared__ __attribute__((aligned(16))) bf16_t sVn[BV * C];
  __shared__ __attribute__((aligned(16))) OutT sO[C * LDO];
  // 256-byte rows (K = 128): chunk ^ (row % 16); 128-byte rows: chunk ^ (row / 2 % 8)
  auto swz_s = [](int row) { return K == 128 ? (row & 15) : ((row >> 1) & 7); };
  auto swz_v = [](int row) { return (row >> 1) & 7; };

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15, q4 = lane >> 4;
  const int V = p.V, VT = V / 16;
  const int nslice = V / BV;
  const int total = p.B * p.HV * nslice;
  int wid = blockIdx.x;
  if ((total & 7) == 0) wid = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int vs = wid % nslice;
  const int bh = wid / nslice;
  const int hv = bh % p.HV;
  const int b = bh / p.HV;
  const int T = p.T;
  const int NT = (T + C - 1) / C;
  const size_t rec0 = (size_t)bh * NT;

  struct Pf {
    bf16x8 wp[KS], qg[KS], aq[2], kd[RT][2];
    bf16x4 u[CT];
    float4 el[RT];
  };
  // part 0: the state products' operands (needed first); part 1: the rest
  auto load = [&](Pf& f, int n, int part) {
    const size_t rec = rec0 + n;
    const bf16x8* W = reinterpret_cast<const bf16x8*>(ws.wp + rec * (C * K));
    const bf16x8* Q = reinterpret_cast<const bf16x8*>(ws.qg + rec * (C * K));
    const bf16x8* A = reinterpret_cast<const bf16x8*>(ws.aqk + rec * (C * C));
    const bf16x8* Kd = reinterpret_cast<const bf16x8*>(ws.kdt + rec * (K * C));
    const bf16x4* U = reinterpret_cast<const bf16x4*>(ws.u + rec * ((size_t)C * V));
    if (part == 0) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        f.wp[s] = W[(wave * KS + s) * 64 + lane];
        f.qg[s] = Q[(wave * KS + s) * 64 + lane];
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) f.u[ct] = U[(wave * VT + vs * CT + ct) * 64 + lane];
      return;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) f.aq[s] = A[(wave * 2 + s) * 64 + lane];
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int rt = RT * wave + j;
#pragma unroll
      for (int s = 0; s < 2; ++s) f.kd[j][s] = Kd[(rt * 2 + s) * 64 + lane];
      f.el[j] = *reinterpret_cast<const float4*>(ws.el + rec * K + 16 * rt + 4 * q4);
    }
  };

  // state: rows 16 rt + 4 q4 + e (rt = RT wave + j), column 16 ct + r of this slice
  const size_t sbase = (size_t)(b * p.HV + hv) * K * V;
  f32x4 S[RT][CT];
#pragma unroll
  for (int j = 0; j < RT; ++j)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (RT * wave + j) + 4 * q4 + e;
        S[j][ct][e] = p.s0 ? p.s0[sbase + (size_t)row * V + vs * BV + 16 * ct + r] : 0.f;
      }
  auto write_state = [&]() {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int row = 16 * ct + r;
      if constexpr (RT == 2) {
        // channels 32 wave + 4 q4 + e (j = 0) and 32 wave + 16 + 4 q4 + e (j = 1):
        // packed positions 8 q4 .. 8 q4 + 7 of block `wave`, one chunk
        *reinterpret_cast<bf16x8*>(sS + row * K + 8 * ((4 * wave + q4) ^ swz_s(row))) =
            cat4(to_bf16x4(S[0][ct]), to_bf16x4(S[1][ct]));
      } else {
        // channels 16 wave + 4 q4 + e: half (wave & 1) of chunk q4 of block wave / 2
        *reinterpret_cast<bf16x4*>(sS + row * K + 8 * ((4 * (wave >> 1) + q4) ^ swz_s(row)) +
                                   4 * (wave & 1)) = to_bf16x4(S[0][ct]);
      }
    }
  };
  OutT* go = static_cast<OutT*>(p.o) + ((size_t)b * T * p.HV + hv) * V + vs * BV;
  const size_t ostride = (size_t)p.HV * V;
  auto store_o = [&](int n) {
    constexpr int SEG = BV / 8 * (int)sizeof(OutT) / 2;  // 16-byte segments per token row
    constexpr int EPS = 16 / (int)sizeof(OutT);          // elements per segment
#pragma unroll
    for (int k = 0; k < (C * SEG + 255) / 256; ++k) {
      const int idx = tid + 256 * k;
      if (idx < C * SEG) {
        const int tok = idx / SEG, sg = idx % SEG;
        const int t = n * C + tok;
        if (t < T)
          *reinterpret_cast<uint4*>(go + (size_t)t * ostride + EPS * sg) =
              *reinterpret_cast<const uint4*>(sO + tok * LDO + EPS * sg);
      }
    }
  };

  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  // operands of chunk n+2 are requested while chunk n is processed
  auto chunk = [&](int n, Pf& cur, Pf& nxt) {
    __syncthreads();  // state copy and the previous chunk's output are in LDS
    if (n > 0) store_o(n - 1);
    // (past the last chunk the requests repeat the last record: no branch, so the
    // loads share a scheduling region with the products and interleave with them)
    const int npf = min(n + 2, NT - 1);
    load(nxt, npf, 0);
    // va: W' S tiles (tokens x columns); oa: o^T tiles (columns x tokens), formed
    // with the operands swapped (S^T qg^T) so that a lane holds 4 consecutive
    // output columns of one token
    f32x4 va[CT], oa[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) va[ct] = oa[ct] = z4;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int row = 16 * ct + r;
        const bf16x8 sf =
            *reinterpret_cast<const bf16x8*>(sS + row * K + 8 * ((4 * s + q4) ^ swz_s(row)));
        va[ct] = mfma32(cur.wp[s], sf, va[ct]);
        oa[ct] = mfma32(sf, cur.qg[s], oa[ct]);
      }
    }
    // (the compiler's own order of these reads, products and requests is as
    // fast as a forced interleave of two reads, two products and one request)
    load(nxt, npf, 1);
    // v_new = U - W' S (lane: tokens 16 wave + 4 q4 + e of column 16 ct + r)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f32x4 vn;
#pragma unroll
      for (int e = 0; e < 4; ++e) vn[e] = (float)cur.u[ct][e] - va[ct][e];
      // tokens 16 wave + 4 q4 + e: half (wave & 1) of chunk q4 of block wave / 2
      const int row = 16 * ct + r;
      *reinterpret_cast<bf16x4*>(sVn + row * C + 8 * ((4 * (wave >> 1) + q4) ^ swz_v(row)) +
                                 4 * (wave & 1)) = to_bf16x4(vn);
    }
    __syncthreads();  // v_new visible; every read of sS is done
    bf16x8 vf[2][CT];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int row = 16 * ct + r;
        vf[s][ct] = *reinterpret_cast<const bf16x8*>(sVn + row * C + 8 * ((4 * s + q4) ^ swz_v(row)));
      }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      // o^T += v_new^T Aqk^T
      oa[ct] = mfma32(vf[0][ct], cur.aq[0], oa[ct]);
      if (wave >= 2) oa[ct] = mfma32(vf[1][ct], cur.aq[1], oa[ct]);
    }
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        S[j][ct][0] *= cur.el[j].x;
        S[j][ct][1] *= cur.el[j].y;
        S[j][ct][2] *= cur.el[j].z;
        S[j][ct][3] *= cur.el[j].w;
        S[j][ct] = mfma32(cur.kd[j][0], vf[0][ct], S[j][ct]);
        S[j][ct] = mfma32(cur.kd[j][1], vf[1][ct], S[j][ct]);
      }
    // lane: token 16 wave + r, columns 16 ct + 4 q4 + e
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      OutT ov[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = from_f32<OutT>(oa[ct][e]);
      *reinterpret_cast<uint2*>(sO + (16 * wave + r) * LDO + 16 * ct + 4 * q4) =
          *reinterpret_cast<const uint2*>(ov);
    }
    write_state();
  };

  write_state();
  Pf f0, f1, f2;
  load(f0, 0, 0);
  load(f0, 0, 1);
  if (NT > 1) {
    load(f1, 1, 0);
    load(f1, 1, 1);
  }
  // The loop body is three unconditional chunks and the tail is peeled: with a
  // branch between the chunks the compiler's wait counts lose track at the
  // join and it waits for nearly every outstanding load (memory counts are
  // in issue order, so that includes the operands fetched for later chunks).
  int n = 0;
  for (; n + 3 <= NT; n += 3) {
    chunk(n, f0, f2);
    chunk(n + 1, f1, f0);
    chunk(n + 2, f2, f1);
  }
  if (n < NT) chunk(n, f0, f2);
  if (n + 1 < NT) chunk(n + 1, f1, f0);
  __syncthreads();
  store_o(NT - 1);
  if (p.s_out) {
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * (RT * wave + j) + 4 * q4 + e;
          p.s_out[sbase + (size_t)row * V + vs * BV + 16 * ct + r] = S[j][ct][e];
        }
  }
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct SplitSizes {
  size_t wp, qg, kdt, aqk, u, el, total;
};

SplitSizes split_sizes(int B, int T, int HV, int K, int V) {
  const size_t R = (size_t)B * HV * ((T + C - 1) / C);
  SplitSizes z;
  z.wp = align256(R * C * K * 2);
  z.qg = align256(R * C * K * 2);
  z.kdt = align256(R * K * C * 2);
  z.aqk = align256(R * C * C * 2);
  z.u = align256(R * C * V * 2);
  z.el = align256(R * K * 4);
  z.total = z.wp + z.qg + z.kdt + z.aqk + z.u + z.el;
  return z;
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

template <int K, int V, typename InT>
hipError_t launch_split(const KdaParams& p, SplitPtrs w, hipStream_t s) {
  const int NT = (p.T + C - 1) / C;
  hipLaunchKernelGGL((kda_prep_kernel<K, V, InT>), dim3(p.B * p.HV * NT), dim3(256), 0, s, p, w);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // 32-column V slices when 64-column ones would leave more than half of the
  // CUs without a state workgroup, 16-column ones when 32-column ones would
  // (the chain of one chunk is then half as long, and every CU has a head's
  // slice: the C4 prefill's B = 2)
  const long long heads = (long long)p.B * p.HV;
  if (V == 128 && 2LL * heads * (V / 32) <= cu_count())
    hipLaunchKernelGGL((kda_state_kernel<K, 16, InT>), dim3(p.B * p.HV * (V / 16)), dim3(256), 0, s, p, w);
  else if (V == 128 && 2LL * heads * (V / 64) <= cu_count())
    hipLaunchKernelGGL((kda_state_kernel<K, 32, InT>), dim3(p.B * p.HV * (V / 32)), dim3(256), 0, s, p, w);
  else
    hipLaunchKernelGGL((kda_state_kernel<K, 64, InT>), dim3(p.B * p.HV * (V / 64)), dim3(256), 0, s, p, w);
  return hipGetLastError();
}

}  // namespace

bool kda_split_supported(int K, int V, int dtype) {
  return (dtype == DT_BF16 || dtype == DT_F16) && (K == 64 || K == 128) && (V == 64 || V == 128);
}

size_t kda_split_ws_bytes(int B, int T, int HV, int K, int V) {
  return split_sizes(B, T, HV, K, V).total;
}

hipError_t kda_split_dispatch(const KdaParams& p, void* ws, int dtype, hipStream_t stream) {
  const SplitSizes z = split_sizes(p.B, p.T, p.HV, p.K, p.V);
  char* base = static_cast<char*>(ws);
  SplitPtrs w;
  w.wp = reinterpret_cast<bf16_t*>(base);
  w.qg = reinterpret_cast<bf16_t*>(base + z.wp);
  w.kdt = reinterpret_cast<bf16_t*>(base + z.wp + z.qg);
  w.aqk = reinterpret_cast<bf16_t*>(base + z.wp + z.qg + z.kdt);
  w.u = reinterpret_cast<bf16_t*>(base + z.wp + z.qg + z.kdt + z.aqk);
  w.el = reinterpret_cast<float*>(base + z.wp + z.qg + z.kdt + z.aqk + z.u);
  const bool bf = dtype == DT_BF16;
  if (p.K == 128) {
    if (p.V == 128) return bf ? launch_split<128, 128, bf16_t>(p, w, stream)
                              : launch_split<128, 128, _Float16>(p, w, stream);
    return bf ? launch_split<128, 64, bf16_t>(p, w, stream) : launch_split<128, 64, _Float16>(p, w, stream);
  }
  if (p.V == 128) return bf ? launch_split<64, 128, bf16_t>(p, w, stream)
                            : launch_split<64, 128, _Float16>(p, w, stream);
  return bf ? launch_split<64, 64, bf16_t>(p, w, stream) : launch_split<64, 64, _Float16>(p, w, stream);
}

}  // namespace kch
