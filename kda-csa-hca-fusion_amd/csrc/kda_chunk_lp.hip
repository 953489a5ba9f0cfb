// KDA chunked prefill for bf16 / fp16 inputs on gfx950 (the configs[1] hot path).
//
// Restates the chunkwise WY/UT form of the reference
// (/root/reference/ops_kda.py:340-536, naive_chunk_kda) as one fused kernel.
//
//   grid  : one workgroup per (batch b, value head hv, 64-column slice of V);
//           sibling slices of one head are placed on the same XCD
//   block : 512 threads = 8 wave64s, 64-token chunks processed in sequence
//   state : the fp32 K x 64 state slice lives in MFMA accumulators; wave w owns
//           column tile (w & 3) and half (w >> 2) of the K rows
//
// Notation per chunk (G = in-chunk cumsum of the clamped gate, a = token 31 is
// the anchor, e(x) = exp(x) per key channel):
//   R  = e(G - G_a),  Ci = e(G_a - G)                     [64 x K]
//   sA = k R,  sQ = scale q R,  sB = k Ci
//   L[r][c]   = beta_r sum_ch sA[r] sB[c]     (c <  r)   -- beta_r sum k_r e(G_r-G_c) k_c
//   Aqk[r][c] = sum_ch sQ[r] sB[c]            (c <= r)   -- scale sum q_r e(G_r-G_c) k_c
//   X  = (I + L)^{-1}                        (fp32 16x16 diagonal blocks, then
//                                             two levels of bf16 MFMA block products)
//   S' = diag(e(G_a)) S                       (state rows pre-scaled by the anchor decay)
//   W' = X (beta sA),   U = X (beta v)
//   v_new = U - W' S'                         (= u - w S of ops_kda.py:518)
//   o     = sQ S' + Aqk v_new                 (= (q e^G) S + Aqk v_new, ops_kda.py:519)
//   S     = diag(e(G_last)) S + diag(e(G_last - G_a)) sB^T v_new   (ops_kda.py:520-535)
// (I+L)^{-1} diag(beta) equals (solve_triangular(I-A, A) + I) diag(beta) of
// ops_kda.py:418-421 with A = -L.
//
// Several products are formed transposed (e.g. L^T = sB sA^T) so that each lane
// holds 4 consecutive elements of an LDS row and stores them with one 8-byte write.
//
// Range guard. Every factor above is a normal bf16/fp32 number when
// |G - G_a| <= 80 and G_a >= -80 (nats); with a gate g <= 0 the clamp(max=50) of
// ops_kda.py:414,516 never binds. A chunk outside that range, or with a positive
// gate and |G - G_a| > 25, is flagged and processed instead by the exact
// per-token recurrence (ops_kda.py:253-258) on the same register-resident state.
//
// Padding (ops_kda.py:375-382): tokens t >= T load as zeros (k = beta = g = 0),
// which leaves the state unchanged; their outputs are not stored.

#include <type_traits>

#include "kch_device.h"
#include "kch_kernels.h"
#include "kda_common.h"

namespace kch {

namespace {

using namespace kda_detail;

template <int K>
struct LpLayout {
  static constexpr int C = 64, BV = 64;
  static constexpr int LDK = K + 8;   // bf16 row stride of [64][K] buffers
  static constexpr int LDC = C + 8;   // bf16 row stride of [*][64] buffers
  static constexpr int LDY = 32 + 8;  // Y scratch of the inverse
  static constexpr int LDD = 20;      // fp32 row stride of the diagonal L blocks
  static constexpr int KT = K / 16;   // channel tiles
  static constexpr int CPL = K / 32;  // channels per lane in the elementwise stage
  static constexpr int RTW = KT / 2;  // state row tiles per wave
  static constexpr int SZ_ROWK = C * LDK * 2;
  static constexpr int SZ_TK = K * LDC * 2;
  static constexpr int SZ_CC = C * LDC * 2;
  static constexpr int OFF_A = 0;                     // sA  [64][LDK]   -> later W'
  static constexpr int OFF_B = OFF_A + SZ_ROWK;       // sB  [64][LDK]   -> later Y scratch
  static constexpr int OFF_Q = OFF_B + SZ_ROWK;       // sQ  [64][LDK]
  static constexpr int OFF_ABT = OFF_Q + SZ_ROWK;     // (beta sA)^T [K][LDC] -> later v_new^T
  static constexpr int OFF_BT = OFF_ABT + SZ_TK;      // sB^T [K][LDC]
  static constexpr int OFF_VBT = OFF_BT + SZ_TK;      // (beta v)^T [64][LDC]
  static constexpr int OFF_LD = OFF_VBT + SZ_CC;      // fp32 diagonal L blocks [4][16][LDD]
  static constexpr int OFF_LOP = OFF_LD + 4 * 16 * LDD * 4;  // L bf16 [64][LDC]
  static constexpr int OFF_AQK = OFF_LOP + SZ_CC;     // Aqk bf16 [64][LDC]
  static constexpr int OFF_X = OFF_AQK + SZ_CC;       // X row-major [64][LDC] (also o staging)
  static constexpr int OFF_XT = OFF_X + SZ_CC;        // X^T [64][LDC]
  static constexpr int OFF_ST = OFF_XT + SZ_CC;       // S'^T [64 cols][LDK]
  static constexpr int OFF_SM = OFF_ST + BV * LDK * 2;
  // small fp32 arrays: e(G_a)[K], e(G_last)[K], e(G_last-G_a)[K], beta[64],
  // fallback reductions [4][64], flags[2]
  static constexpr int OFF_EA = OFF_SM;
  static constexpr int OFF_EL = OFF_EA + K * 4;
  static constexpr int OFF_ELA = OFF_EL + K * 4;
  static constexpr int OFF_BETA = OFF_ELA + K * 4;
  static constexpr int OFF_RED = OFF_BETA + 64 * 4;
  static constexpr int OFF_FLAG = OFF_RED + 4 * 64 * 4;
  static constexpr int BYTES = OFF_FLAG + 16;
  // exact-recurrence fallback buffers (alias the dead fast-path buffers)
  static constexpr int OFF_FQ = 0;                    // q raw [64][K] (input type)
  static constexpr int OFF_FK = OFF_FQ + C * K * 2;   // k raw
  static constexpr int OFF_FG = OFF_FK + C * K * 2;   // clamped gate, log2 units, fp32 [64][K]
  static constexpr int OFF_FV = OFF_FG + C * K * 4;   // v raw [64][64]
  static constexpr int OFF_FB = OFF_FV + C * BV * 2;  // beta fp32 [64]
  static_assert(OFF_FB + 64 * 4 <= OFF_VBT, "fallback buffers alias dead fast-path buffers");
  static_assert(OFF_B + 2 * 16 * LDY * 2 + 32 * LDY * 2 <= OFF_Q, "inverse scratch fits in sB");
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

}  // namespace

template <int K, typename InT>
__global__ __launch_bounds__(512) void kda_chunk_lp_kernel(KdaParams p) {
  using L = LpLayout<K>;
  constexpr int C = L::C, BV = L::BV, LDK = L::LDK, LDC = L::LDC, LDY = L::LDY, LDD = L::LDD;
  constexpr int KT = L::KT, CPL = L::CPL, RTW = L::RTW;
  using Raw = RawT<CPL>;
  typedef typename Raw::type raw_t;

  __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
  bf16_t* sA = reinterpret_cast<bf16_t*>(smem + L::OFF_A);
  bf16_t* sW = sA;
  bf16_t* sB = reinterpret_cast<bf16_t*>(smem + L::OFF_B);
  bf16_t* sY1 = sB;                        // [2 waves][16][LDY] level-1 scratch (Y^T)
  bf16_t* sY2t = sB + 2 * 16 * LDY;        // Y2^T [32][LDY]
  bf16_t* sQ = reinterpret_cast<bf16_t*>(smem + L::OFF_Q);
  bf16_t* sAbT = reinterpret_cast<bf16_t*>(smem + L::OFF_ABT);
  bf16_t* sVnT = sAbT;
  bf16_t* sBT = reinterpret_cast<bf16_t*>(smem + L::OFF_BT);
  bf16_t* sVbT = reinterpret_cast<bf16_t*>(smem + L::OFF_VBT);
  float* sLd = reinterpret_cast<float*>(smem + L::OFF_LD);
  bf16_t* sLop = reinterpret_cast<bf16_t*>(smem + L::OFF_LOP);
  bf16_t* sAqk = reinterpret_cast<bf16_t*>(smem + L::OFF_AQK);
  bf16_t* sX = reinterpret_cast<bf16_t*>(smem + L::OFF_X);
  bf16_t* sO = sX;
  bf16_t* sXt = reinterpret_cast<bf16_t*>(smem + L::OFF_XT);
  bf16_t* sST = reinterpret_cast<bf16_t*>(smem + L::OFF_ST);
  float* sEa = reinterpret_cast<float*>(smem + L::OFF_EA);
  float* sEl = reinterpret_cast<float*>(smem + L::OFF_EL);
  float* sEla = reinterpret_cast<float*>(smem + L::OFF_ELA);
  float* sBeta = reinterpret_cast<float*>(smem + L::OFF_BETA);
  float* sRed = reinterpret_cast<float*>(smem + L::OFF_RED);
  int* sFlag = reinterpret_cast<int*>(smem + L::OFF_FLAG);
  InT* sFq = reinterpret_cast<InT*>(smem + L::OFF_FQ);
  InT* sFk = reinterpret_cast<InT*>(smem + L::OFF_FK);
  float* sFg = reinterpret_cast<float*>(smem + L::OFF_FG);
  InT* sFv = reinterpret_cast<InT*>(smem + L::OFF_FV);
  float* sFb = reinterpret_cast<float*>(smem + L::OFF_FB);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63;

  // ---- workgroup -> (b, hv, slice) ----
  const int nslice = p.V / BV;
  const int total = p.B * p.HV * nslice;
  int wid = blockIdx.x;
  if ((total & 7) == 0) wid = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int vs = wid % nslice;
  const int bh = wid / nslice;
  const int hv = bh % p.HV;
  const int b = bh / p.HV;
  const int h = hv / (p.HV / p.H);
  const int T = p.T;

  // per-workgroup base pointers; token t is at base + t * stride (32-bit offsets,
  // the host guarantees T * stride < 2^31)
  const int qk_stride = p.H * K, g_stride = p.HV * K, v_stride = p.HV * p.V, b_stride = p.HV;
  const InT* __restrict__ gq = static_cast<const InT*>(p.q) + ((size_t)b * T * p.H + h) * K;
  const InT* __restrict__ gk = static_cast<const InT*>(p.k) + ((size_t)b * T * p.H + h) * K;
  const InT* __restrict__ gg = static_cast<const InT*>(p.g) + ((size_t)b * T * p.HV + hv) * K;
  const InT* __restrict__ gv =
      static_cast<const InT*>(p.v) + ((size_t)b * T * p.HV + hv) * p.V + vs * BV;
  const InT* __restrict__ gbeta = static_cast<const InT*>(p.beta) + (size_t)b * T * p.HV + hv;
  InT* __restrict__ go = static_cast<InT*>(p.o) + ((size_t)b * T * p.HV + hv) * p.V + vs * BV;

  // ---- elementwise mapping: lane -> tokens 4*tg..4*tg+3 (tg = lane & 15) and
  //      CPL channels from chb (channel quad cq = lane >> 4); wave -> K/8 channels ----
  const int tg = lane & 15;
  const int cq = lane >> 4;
  const int chb = (K / 8) * wave + CPL * cq;
  const int vcb = 8 * wave + 2 * cq;  // two V columns

  // Prefetch registers: issued one chunk ahead and consumed only in stage P
  // (tokens t >= T read token T-1 and are zeroed at use).
  raw_t rq[4], rk[4], rg[4];
  uint32_t rv[4], rb[4];
  auto load_chunk = [&](int n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int t = n * C + 4 * tg + i;
      t = t < T ? t : T - 1;
      rq[i] = *reinterpret_cast<const raw_t*>(gq + t * qk_stride + chb);
      rk[i] = *reinterpret_cast<const raw_t*>(gk + t * qk_stride + chb);
      rg[i] = *reinterpret_cast<const raw_t*>(gg + t * g_stride + chb);
      rv[i] = *reinterpret_cast<const uint32_t*>(gv + t * v_stride + vcb);
      rb[i] = *reinterpret_cast<const unsigned short*>(gbeta + t * b_stride);
    }
  };

  // ---- state: wave owns column tile ct, row tiles [RTW*half, RTW*half + RTW) ----
  const int ct = wave & 3;
  const int half = wave >> 2;
  const int scol = vs * BV + 16 * ct + acc_col();
  const size_t sbase = (size_t)(b * p.HV + hv) * K * p.V;
  f32x4 S[RTW];
#pragma unroll
  for (int i = 0; i < RTW; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * (RTW * half + i) + acc_row(e);
      S[i][e] = p.s0 ? p.s0[sbase + (size_t)row * p.V + scol] : 0.f;
    }

  if (tid < 2) sFlag[tid] = 0;
  __syncthreads();
  const float clampv = p.g_clamp_min;  // -inf disables the clamp
  const float scale = p.scale;
  const int nchunks = (T + C - 1) / C;
  bool pending_o = false;  // sO holds the previous chunk's output
  int pending_n = 0;

  auto store_o = [&](int n) {
    // 64 tokens x 64 columns, one 16-byte segment per thread
    const int tok = tid >> 3, cb = tid & 7;
    const int t = n * C + tok;
    if (t < T) {
      const uint4 val = *reinterpret_cast<const uint4*>(sO + tok * LDC + 8 * cb);
      InT* dst = go + t * v_stride + 8 * cb;
      if constexpr (std::is_same<InT, bf16_t>::value) {
        *reinterpret_cast<uint4*>(dst) = val;
      } else {
        const bf16_t* sv = reinterpret_cast<const bf16_t*>(&val);
        InT tmp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) tmp[i] = (InT)(float)sv[i];
        *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(tmp);
      }
    }
  };

  load_chunk(0);

  for (int n = 0; n < nchunks; ++n) {
    // ============ stage P: gate cumsum and decay-scaled operands ============
    {
      const int t0 = n * C + 4 * tg;
      float bt[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) bt[i] = (t0 + i < T) ? h2f<InT>(rb[i]) : 0.f;
      float gmax = -INFINITY, dmax = 0.f, amin = 0.f;
      float a[4][CPL], qq[4][CPL], bb[4][CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        float G[4];
        float run = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float g = (t0 + i < T) ? elem<InT>(Raw::word(rg[i], c >> 1), c & 1) : 0.f;
          g = fmaxf(g, clampv);
          gmax = fmaxf(gmax, g);
          run += g * kLog2e;
          G[i] = run;
        }
        const float incl = row_prefix_sum(run);    // sum over token groups <= tg
        const float excl = incl - run;
        const float Ga = dpp<0x157, false>(incl);  // token 31: group 7, last
        const float Gl = dpp<0x15f, false>(incl);  // token 63: group 15, last
        amin = fminf(amin, Ga);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float d = G[i] + excl - Ga;
          dmax = fmaxf(dmax, fabsf(d));
          const float R = fast_exp2(d);
          const float Ci = fast_exp2(-d);
          const float kk = (t0 + i < T) ? elem<InT>(Raw::word(rk[i], c >> 1), c & 1) : 0.f;
          const float qv = (t0 + i < T) ? elem<InT>(Raw::word(rq[i], c >> 1), c & 1) : 0.f;
          a[i][c] = kk * R;
          qq[i][c] = qv * R * scale;
          bb[i][c] = kk * Ci;
        }
        if (tg == 0) {
          sEa[chb + c] = fast_exp2(Ga);
          sEl[chb + c] = fast_exp2(Gl);
          sEla[chb + c] = fast_exp2(Gl - Ga);
        }
      }
      const bool bad = !(dmax <= kRange2) || !(amin >= -kRange2);
      const int fl = (bad ? 1 : 0) | (gmax > 0.f ? 2 : 0) | (dmax > kPos2 ? 4 : 0);
      // OR-ed over the active lanes by ballots: one LDS atomic per wave, from its
      // first active lane (the lanes' own atomics on one word serialise)
      {
        const int wf = (__builtin_amdgcn_ballot_w64((fl & 1) != 0) ? 1 : 0) |
                       (__builtin_amdgcn_ballot_w64((fl & 2) != 0) ? 2 : 0) |
                       (__builtin_amdgcn_ballot_w64((fl & 4) != 0) ? 4 : 0);
        const int first = __ffsll((long long)__builtin_amdgcn_ballot_w64(true)) - 1;
        if (wf && (int)(threadIdx.x & 63) == first) atomicOr(&sFlag[n & 1], wf);
      }
      // row-major operands [token][channel]: CPL channels per token
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (4 * tg + i) * LDK + chb;
        if constexpr (CPL == 4) {
          st_bf16x4(sA + row, a[i][0], a[i][1], a[i][2], a[i][3]);
          st_bf16x4(sQ + row, qq[i][0], qq[i][1], qq[i][2], qq[i][3]);
          st_bf16x4(sB + row, bb[i][0], bb[i][1], bb[i][2], bb[i][3]);
        } else {
          typedef bf16_t bf16x2_t __attribute__((ext_vector_type(2)));
          *reinterpret_cast<bf16x2_t*>(sA + row) = bf16x2_t{(bf16_t)a[i][0], (bf16_t)a[i][1]};
          *reinterpret_cast<bf16x2_t*>(sQ + row) = bf16x2_t{(bf16_t)qq[i][0], (bf16_t)qq[i][1]};
          *reinterpret_cast<bf16x2_t*>(sB + row) = bf16x2_t{(bf16_t)bb[i][0], (bf16_t)bb[i][1]};
        }
      }
      // transposed operands [channel][token]: 4 tokens per channel
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int row = (chb + c) * LDC + 4 * tg;
        st_bf16x4(sAbT + row, a[0][c] * bt[0], a[1][c] * bt[1], a[2][c] * bt[2], a[3][c] * bt[3]);
        st_bf16x4(sBT + row, bb[0][c], bb[1][c], bb[2][c], bb[3][c]);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float vv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) vv[i] = (t0 + i < T) ? elem<InT>(rv[i], j) * bt[i] : 0.f;
        st_bf16x4(sVbT + (vcb + j) * LDC + 4 * tg, vv[0], vv[1], vv[2], vv[3]);
      }
      if (wave == 0 && cq == 0)
        *reinterpret_cast<float4*>(sBeta + 4 * tg) = make_float4(bt[0], bt[1], bt[2], bt[3]);
    }
    __syncthreads();  // ---- B_P: operands, flag, decay vectors visible ----

    const int flag = sFlag[n & 1];
    const bool exact = (flag & 1) || ((flag & 2) && (flag & 4));
    if (tid == 0) sFlag[(n + 1) & 1] = 0;

    if (!exact) {
      if (n + 1 < nchunks) load_chunk(n + 1);
      // ============ stage LA: L^T, Aqk^T, S'^T, store of the previous output ============
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int job = wave + 8 * jj;
        if (job < 10) {
          const int ti = lower_tile_row(job), tj = lower_tile_col(job);
          f32x4 lt = {0.f, 0.f, 0.f, 0.f}, at = {0.f, 0.f, 0.f, 0.f};
          // L^T tile = sB[tj] sA[ti]^T, Aqk^T tile = sB[tj] sQ[ti]^T
          mma16x2<K>(lt, at, sB + 16 * tj * LDK, LDK, sA + 16 * ti * LDK, sQ + 16 * ti * LDK, LDK);
          // lane holds key tokens c0..c0+3 of query token r
          const int r = 16 * ti + acc_col();
          const int c0 = 16 * tj + acc_row(0);
          const float br = sBeta[r];
          float lv[4], av[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            lv[e] = (c0 + e < r) ? lt[e] * br : 0.f;
            av[e] = (c0 + e <= r) ? at[e] : 0.f;
          }
          st_bf16x4(sLop + r * LDC + c0, lv[0], lv[1], lv[2], lv[3]);
          st_bf16x4(sAqk + r * LDC + c0, av[0], av[1], av[2], av[3]);
          if (ti == tj) {
            // fp32 diagonal block, columns stored permuted: c -> (c & 3) * 4 + (c >> 2)
            float* d = sLd + (ti * 16 + acc_col()) * LDD;
            const int cl4 = acc_row(0) >> 2;
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e * 4 + cl4] = lv[e];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < RTW; ++i) {
        const int row0 = 16 * (RTW * half + i) + acc_row(0);
        const float4 ea = *reinterpret_cast<const float4*>(sEa + row0);
        st_bf16x4(sST + (16 * ct + acc_col()) * LDK + row0, S[i][0] * ea.x, S[i][1] * ea.y,
                  S[i][2] * ea.z, S[i][3] * ea.w);
      }
      if (pending_o) store_o(pending_n);
      __syncthreads();  // ---- B_LA ----

      // ============ inverse: 16x16 diagonal blocks in fp32, wave d -> block d ============
      if (wave < 4) {
        const int blk = wave;
        const int cc = lane >> 2;   // column of the block inverse
        const int part = lane & 3;  // this lane sums the terms k = 4j + part
        float Lr[16][4];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float4 v = *reinterpret_cast<const float4*>(sLd + (blk * 16 + r) * LDD + part * 4);
          Lr[r][0] = v.x; Lr[r][1] = v.y; Lr[r][2] = v.z; Lr[r][3] = v.w;
        }
        float xs[4] = {0.f, 0.f, 0.f, 0.f};  // x[4j + part] of column cc
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float s = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (4 * j < r) s += Lr[r][j] * xs[j];
          s += dpp<0xb1, false>(s);  // quad_perm [1,0,3,2]
          s += dpp<0x4e, false>(s);  // quad_perm [2,3,0,1]
          const float xr = (r < cc) ? 0.f : ((r == cc) ? 1.f : -s);
          if ((r & 3) == part) xs[r >> 2] = xr;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * j + part;
          sX[(16 * blk + r) * LDC + 16 * blk + cc] = (bf16_t)xs[j];
          sXt[(16 * blk + cc) * LDC + 16 * blk + r] = (bf16_t)xs[j];
        }
      }
      __syncthreads();  // ---- B_I0 ----
      // ============ level 1: X[2w+1][2w] = -X[2w+1][2w+1] L[2w+1][2w] X[2w][2w] ============
      if (wave < 2) {
        const int d0 = 2 * wave, d1 = 2 * wave + 1;
        bf16_t* y = sY1 + wave * 16 * LDY;
        // Y = L[d1][d0] X[d0][d0], stored transposed
        f32x4 acc = mma16<16>(f32x4{0.f, 0.f, 0.f, 0.f}, sLop + 16 * d1 * LDC + 16 * d0, LDC,
                              sXt + 16 * d0 * LDC + 16 * d0, LDC);
        st_bf16x4(y + acc_col() * LDY + acc_row(0), acc[0], acc[1], acc[2], acc[3]);
        wave_lds_sync();
        acc = mma16<16>(f32x4{0.f, 0.f, 0.f, 0.f}, sX + 16 * d1 * LDC + 16 * d1, LDC, y, LDY);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sX[(16 * d1 + acc_row(e)) * LDC + 16 * d0 + acc_col()] = (bf16_t)(-acc[e]);
        st_bf16x4(sXt + (16 * d0 + acc_col()) * LDC + 16 * d1 + acc_row(0), -acc[0], -acc[1],
                  -acc[2], -acc[3]);
      }
      __syncthreads();  // ---- B_I1 ----
      // ============ level 2: Y2 = L[32:,:32] X[:32,:32] ============
      if (wave < 4) {
        const int i = wave >> 1, j = wave & 1;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (j == 0)
          acc = mma16<32>(acc, sLop + (32 + 16 * i) * LDC, LDC, sXt, LDC);
        else
          acc = mma16<16>(acc, sLop + (32 + 16 * i) * LDC + 16, LDC, sXt + 16 * LDC + 16, LDC);
        st_bf16x4(sY2t + (16 * j + acc_col()) * LDY + 16 * i + acc_row(0), acc[0], acc[1], acc[2],
                  acc[3]);
      }
      __syncthreads();  // ---- B_I2 ----
      // ============ X[32:,:32] = -X[32:,32:] Y2 ============
      if (wave < 4) {
        const int i = wave >> 1, j = wave & 1;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (i == 0)
          acc = mma16<16>(acc, sX + 32 * LDC + 32, LDC, sY2t + 16 * j * LDY, LDY);
        else
          acc = mma16<32>(acc, sX + 48 * LDC + 32, LDC, sY2t + 16 * j * LDY, LDY);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sX[(32 + 16 * i + acc_row(e)) * LDC + 16 * j + acc_col()] = (bf16_t)(-acc[e]);
        st_bf16x4(sXt + (16 * j + acc_col()) * LDC + 32 + 16 * i + acc_row(0), -acc[0], -acc[1],
                  -acc[2], -acc[3]);
      }
      __syncthreads();  // ---- B_I3 ----

      // ============ U = X (beta v),  W'^T = (beta sA)^T X^T ============
      f32x4 U[2];
      auto u_stage = [&](auto HF_) {
        constexpr int HF = decltype(HF_)::value;
        U[0] = mma16<16 * (2 * HF + 1)>(f32x4{0.f, 0.f, 0.f, 0.f}, sX + 16 * (2 * HF) * LDC, LDC,
                                         sVbT + 16 * ct * LDC, LDC);
        U[1] = mma16<16 * (2 * HF + 2)>(f32x4{0.f, 0.f, 0.f, 0.f}, sX + 16 * (2 * HF + 1) * LDC,
                                         LDC, sVbT + 16 * ct * LDC, LDC);
      };
      if (half == 0) u_stage(IC<0>());
      else u_stage(IC<1>());
      auto wtile = [&](int wt, auto BI_) {
        constexpr int bi = decltype(BI_)::value;
        f32x4 acc = mma16<16 * (bi + 1)>(f32x4{0.f, 0.f, 0.f, 0.f}, sAbT + 16 * wt * LDC, LDC,
                                         sX + 16 * bi * LDC, LDC);
        // lane: channels 16wt + acc_row(0..3) of token 16bi + acc_col()
        st_bf16x4(sW + (16 * bi + acc_col()) * LDK + 16 * wt + acc_row(0), acc[0], acc[1], acc[2],
                  acc[3]);
      };
      if constexpr (KT == 8) {
        wtile(wave, IC<0>());
        wtile(wave, IC<1>());
        wtile(wave, IC<2>());
        wtile(wave, IC<3>());
      } else {
        if (half == 0) {
          wtile(wave & 3, IC<0>());
          wtile(wave & 3, IC<1>());
        } else {
          wtile(wave & 3, IC<2>());
          wtile(wave & 3, IC<3>());
        }
      }
      __syncthreads();  // ---- B_WU: W' visible; sAbT free for v_new^T ----

      // ============ v_new = U - W' S' ============
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int bi = 2 * half + j;
        f32x4 acc = mma16<K>(f32x4{0.f, 0.f, 0.f, 0.f}, sW + 16 * bi * LDK, LDK,
                             sST + 16 * ct * LDK, LDK);
        st_bf16x4(sVnT + (16 * ct + acc_col()) * LDC + 16 * bi + acc_row(0), U[j][0] - acc[0],
                  U[j][1] - acc[1], U[j][2] - acc[2], U[j][3] - acc[3]);
      }
      __syncthreads();  // ---- B_VN ----

      // ============ o^T = S'^T sQ^T + v_new^T Aqk^T;  S update ============
      auto o_stage = [&](auto HF_) {
        constexpr int HF = decltype(HF_)::value;
        f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
        mma16x2<K>(o0, o1, sST + 16 * ct * LDK, LDK, sQ + 16 * (2 * HF) * LDK,
                   sQ + 16 * (2 * HF + 1) * LDK, LDK);
        // intra-chunk terms in their own accumulators (one MFMA shape per chain)
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        const f32x4 i0 =
            mma16<16 * (2 * HF + 1)>(z, sVnT + 16 * ct * LDC, LDC, sAqk + 16 * (2 * HF) * LDC, LDC);
        const f32x4 i1 = mma16<16 * (2 * HF + 2)>(z, sVnT + 16 * ct * LDC, LDC,
                                                  sAqk + 16 * (2 * HF + 1) * LDC, LDC);
        o0 += i0;
        o1 += i1;
        // lane: V columns 16ct + acc_row(0..3) of token 16bi + acc_col()
        st_bf16x4(sO + (16 * (2 * HF) + acc_col()) * LDC + 16 * ct + acc_row(0), o0[0], o0[1],
                  o0[2], o0[3]);
        st_bf16x4(sO + (16 * (2 * HF + 1) + acc_col()) * LDC + 16 * ct + acc_row(0), o1[0], o1[1],
                  o1[2], o1[3]);
      };
      if (half == 0) o_stage(IC<0>());
      else o_stage(IC<1>());
#pragma unroll
      for (int i = 0; i < RTW; ++i) {
        const int rt = RTW * half + i;
        f32x4 acc = mma16<C>(f32x4{0.f, 0.f, 0.f, 0.f}, sBT + 16 * rt * LDC, LDC,
                             sVnT + 16 * ct * LDC, LDC);
        const int row0 = 16 * rt + acc_row(0);
        const float4 el = *reinterpret_cast<const float4*>(sEl + row0);
        const float4 ela = *reinterpret_cast<const float4*>(sEla + row0);
        S[i][0] = el.x * S[i][0] + ela.x * acc[0];
        S[i][1] = el.y * S[i][1] + ela.y * acc[1];
        S[i][2] = el.z * S[i][2] + ela.z * acc[2];
        S[i][3] = el.w * S[i][3] + ela.w * acc[3];
      }
      pending_o = true;
      pending_n = n;
    } else {
      // ============ exact per-token recurrence for a flagged chunk ============
      if (pending_o) store_o(pending_n);
      pending_o = false;
      {
        const int t0 = n * C + 4 * tg;
        // raw operands of this chunk, from the registers that still hold it
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = t0 + i < T;
          const int row = (4 * tg + i) * K + chb;
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            const uint32_t wq = Raw::word(rq[i], c >> 1), wk = Raw::word(rk[i], c >> 1);
            const uint32_t wg = Raw::word(rg[i], c >> 1);
            sFq[row + c] = (InT)(ok ? elem<InT>(wq, c & 1) : 0.f);
            sFk[row + c] = (InT)(ok ? elem<InT>(wk, c & 1) : 0.f);
            sFg[row + c] = ok ? fmaxf(elem<InT>(wg, c & 1), clampv) * kLog2e : 0.f;
          }
#pragma unroll
          for (int j = 0; j < 2; ++j)
            sFv[(4 * tg + i) * BV + vcb + j] = (InT)(ok ? elem<InT>(rv[i], j) : 0.f);
          if (wave == 0 && cq == 0) sFb[4 * tg + i] = ok ? h2f<InT>(rb[i]) : 0.f;
        }
      }
      if (n + 1 < nchunks) load_chunk(n + 1);
      __syncthreads();
      const int tend = min(C, T - n * C);
      const int col = 16 * ct + acc_col();
      for (int t = 0; t < tend; ++t) {
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < RTW; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = 16 * (RTW * half + i) + acc_row(e);
            S[i][e] *= fast_exp2(sFg[t * K + row]);
            part += to_f32(sFk[t * K + row]) * S[i][e];
          }
        part += __shfl_xor(part, 16);
        part += __shfl_xor(part, 32);
        if (lane < 16) sRed[half * 64 + col] = part;
        __syncthreads();
        const float kS = sRed[col] + sRed[64 + col];
        const float d = sFb[t] * (to_f32(sFv[t * BV + col]) - kS);
        float po = 0.f;
#pragma unroll
        for (int i = 0; i < RTW; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = 16 * (RTW * half + i) + acc_row(e);
            S[i][e] += to_f32(sFk[t * K + row]) * d;
            po += to_f32(sFq[t * K + row]) * S[i][e];
          }
        po += __shfl_xor(po, 16);
        po += __shfl_xor(po, 32);
        if (lane < 16) sRed[128 + half * 64 + col] = po;
        __syncthreads();
        if (half == 0 && lane < 16) {
          const float o = (sRed[128 + col] + sRed[192 + col]) * scale;
          go[(n * C + t) * v_stride + col] = (InT)o;
        }
      }
    }
    __syncthreads();  // ---- B_END: every read of this chunk's buffers is complete ----
  }
  if (pending_o) store_o(pending_n);

  if (p.s_out) {
#pragma unroll
    for (int i = 0; i < RTW; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (RTW * half + i) + acc_row(e);
        p.s_out[sbase + (size_t)row * p.V + scol] = S[i][e];
      }
  }
}

template <int K, typename InT>
static hipError_t launch_lp(const KdaParams& p, hipStream_t stream) {
  const int total = p.B * p.HV * (p.V / 64);
  hipLaunchKernelGGL((kda_chunk_lp_kernel<K, InT>), dim3(total), dim3(512), 0, stream, p);
  return hipGetLastError();
}

hipError_t kda_chunk_lp_dispatch(const KdaParams& p, int dtype, hipStream_t stream) {
  if (dtype == DT_BF16) {
    if (p.K == 128) return launch_lp<128, bf16_t>(p, stream);
    return launch_lp<64, bf16_t>(p, stream);
  }
  if (p.K == 128) return launch_lp<128, _Float16>(p, stream);
  return launch_lp<64, _Float16>(p, stream);
}

}  // namespace kch
