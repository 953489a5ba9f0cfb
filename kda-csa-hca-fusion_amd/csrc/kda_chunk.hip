// KDA chunked prefill for fp32 inputs on gfx950 (bf16 / fp16: kda_chunk_lp.hip).
//
// Restates the chunkwise WY/UT form of the reference
// (/root/reference/ops_kda.py:340-536, naive_chunk_kda) as one fused kernel:
//
//   grid  : one workgroup per (batch b, value head hv, 64-column slice of V)
//   block : 256 threads = 4 wave64s
//   loop  : sequential over chunks of C tokens; the fp32 state slice
//           S[:, slice] (K x 64) lives in MFMA accumulators across chunks,
//           wave w owning columns [16w, 16w+16) of the slice.
//
// Per chunk (G = in-chunk cumsum of the clamped gate, in log2 units):
//   L[r][c]   = beta_r * sum_k k_r e^{G_r-G_c} k_c          (c <  r)
//   Aqk[r][c] = scale  * sum_k q_r e^{G_r-G_c} k_c          (c <= r)
//   X         = (I + L)^{-1}                                  (fp32 diagonal blocks,
//                                                             MFMA block substitution)
//   w = X (beta * k * e^{G}),  u = X (beta * v)
//   v_new = u - w S;  o = (scale q e^{G}) S + Aqk v_new
//   S     = e^{G_last} * S + (k e^{G_last - G})^T v_new
// which is (I+L)^{-1} diag(beta) = (solve_triangular(I-A, A) + I) diag(beta)
// of ops_kda.py:418-421 with A = -L.
//
// Decay factors. e^{G_r - G_c} is split as e^{G_r - G_a} * e^{G_a - G_c} with
// the anchor a = row C/2-1, so both MFMA operands stay inside the fp32/bf16
// exponent range. A chunk where |G_r - G_a| could leave that range, or where a
// positive gate could make clamp(max=50) of ops_kda.py:414,516 bind, takes an
// exact elementwise path for L and Aqk instead (flagged per chunk).
//
// Padding (ops_kda.py:375-382): rows t >= T load as zeros (k = beta = g = 0),
// which leaves the state unchanged and produces outputs that are not stored.

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

constexpr float LOG2E = 1.4426950408889634f;

template <int K, int C, typename OpT>
struct KdaChunkLayout {
  static constexpr int BV = 64;                       // V columns per workgroup
  static constexpr int NB = C / 16;                   // 16-row blocks per chunk
  static constexpr int KT = K / 16;                   // 16-channel tiles
  static constexpr int NTOK = C * K / 512;            // tokens per elementwise thread
  static constexpr int NGRP = C / NTOK;               // token groups
  static constexpr int NCP = K / 2;                   // channel pairs
  static constexpr int AGRP = (C / 2) / NTOK;         // groups before the anchor row
  static constexpr int VR = C / 8;                    // rows per v-loading thread
  static constexpr int PADO = sizeof(OpT) == 2 ? 8 : 4;
  static constexpr int LDK = K + PADO;                // [*][K] operand rows
  static constexpr int LDC = C + PADO;                // [*][C] operand rows
  static constexpr int LDF = C + 4;                   // fp32 [C][C]
  static constexpr int LDY = 16 + PADO;
  static constexpr int SO = sizeof(OpT);

  static constexpr int P_FAST = 3 * C * LDK * SO;
  static constexpr int P_INV = C * LDF * 4 + 3 * C * LDC * SO + (C - 16) * LDY * SO;
  static constexpr int P_STATE = 4 * 16 * LDK * SO + 4 * 16 * LDC * SO;
  static constexpr int P_SLOW = C * K * 4;
  static constexpr int cmax(int a, int b) { return a > b ? a : b; }
  static constexpr int round16(int x) { return (x + 15) & ~15; }
  static constexpr int SZ_P = round16(cmax(cmax(P_FAST, P_INV), cmax(P_STATE, P_SLOW)));
  static constexpr int SZ_Q = round16(C * LDK * SO);                 // sQE
  static constexpr int SZ_R = round16(K * LDC * SO);                 // sKdT
  static constexpr int SZ_S = round16(cmax((K + BV) * LDC * SO, C * LDK * SO));  // sKEt+sVt / sW
  static constexpr int SZ_T = round16(C * LDC * SO);                 // sAqk
  static constexpr int SZ_M = round16(NGRP * K * 4 + K * 4 + C * 4 + 16);
  static constexpr int OFF_Q = SZ_P;
  static constexpr int OFF_R = OFF_Q + SZ_Q;
  static constexpr int OFF_S = OFF_R + SZ_R;
  static constexpr int OFF_T = OFF_S + SZ_S;
  static constexpr int OFF_M = OFF_T + SZ_T;
  static constexpr int BYTES = OFF_M + SZ_M;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
  static_assert(NTOK >= 2 && (C / 2) % NTOK == 0, "token grouping");
};

template <typename OpT>
__device__ __forceinline__ void store2(OpT* dst, float a, float b) {
  dst[0] = from_f32<OpT>(a);
  dst[1] = from_f32<OpT>(b);
}

// Contiguous store of N values (N in {2,4,8,16}) into OpT storage.
template <typename OpT, int N>
__device__ __forceinline__ void store_row(OpT* dst, const float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) dst[i] = from_f32<OpT>(v[i]);
}

}  // namespace

template <int K, int C, typename InT, typename OpT>
__global__ __launch_bounds__(256) void kda_chunk_kernel(KdaParams p) {
  using L = KdaChunkLayout<K, C, OpT>;
  using PR = Pair<InT>;
  constexpr int BV = L::BV, NB = L::NB, KT = L::KT, NTOK = L::NTOK, NGRP = L::NGRP;
  constexpr int NCP = L::NCP, AGRP = L::AGRP, VR = L::VR;
  constexpr int LDK = L::LDK, LDC = L::LDC, LDF = L::LDF, LDY = L::LDY;
  constexpr int WT = KT / 4;  // w-part column tiles per wave in the RHS product

  __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
  OpT* sA = reinterpret_cast<OpT*>(smem);
  OpT* sQ = sA + C * LDK;
  OpT* sB = sQ + C * LDK;
  float* sL = reinterpret_cast<float*>(smem);
  OpT* sLop = reinterpret_cast<OpT*>(smem + C * LDF * 4);
  OpT* sX = sLop + C * LDC;
  OpT* sXt = sX + C * LDC;
  OpT* sYt = sXt + C * LDC;
  OpT* sSt = reinterpret_cast<OpT*>(smem);
  OpT* sVn = sSt + 4 * 16 * LDK;
  float* sG = reinterpret_cast<float*>(smem);
  OpT* sQE = reinterpret_cast<OpT*>(smem + L::OFF_Q);
  OpT* sKdT = reinterpret_cast<OpT*>(smem + L::OFF_R);
  OpT* sKEt = reinterpret_cast<OpT*>(smem + L::OFF_S);
  OpT* sVt = sKEt + K * LDC;
  OpT* sW = reinterpret_cast<OpT*>(smem + L::OFF_S);
  OpT* sAqk = reinterpret_cast<OpT*>(smem + L::OFF_T);
  float* sTot = reinterpret_cast<float*>(smem + L::OFF_M);
  float* sGl = sTot + NGRP * K;
  float* sBeta = sGl + K;
  int* sFlag = reinterpret_cast<int*>(sBeta + C);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;

  // ---- workgroup -> (b, hv, slice); sibling slices share an XCD ----
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

  const InT* __restrict__ gq = static_cast<const InT*>(p.q);
  const InT* __restrict__ gk = static_cast<const InT*>(p.k);
  const InT* __restrict__ gv = static_cast<const InT*>(p.v);
  const InT* __restrict__ gg = static_cast<const InT*>(p.g);
  const InT* __restrict__ gbeta = static_cast<const InT*>(p.beta);
  InT* __restrict__ go = static_cast<InT*>(p.o);

  // elementwise mapping: channel pair cp, token group tg
  const int cp = tid % NCP;
  const int tg = tid / NCP;
  const int ch0 = 2 * cp;
  const int r0 = tg * NTOK;
  // v mapping: column pair vp, row group vg
  const int vp = tid & 31;
  const int vg = tid >> 5;

  typename PR::raw rq[NTOK], rk[NTOK], rgt[NTOK], rv[VR];
  float rb[NTOK], rbv[VR];

  auto load_chunk = [&](int n) {
    const int t0 = n * C;
#pragma unroll
    for (int i = 0; i < NTOK; ++i) {
      const int t = t0 + r0 + i;
      const bool ok = t < T;
      const size_t qk = ((size_t)(b * T + t) * p.H + h) * K + ch0;
      const size_t gi = ((size_t)(b * T + t) * p.HV + hv) * K + ch0;
      typename PR::raw z{};
      rq[i] = ok ? *reinterpret_cast<const typename PR::raw*>(gq + qk) : z;
      rk[i] = ok ? *reinterpret_cast<const typename PR::raw*>(gk + qk) : z;
      rgt[i] = ok ? *reinterpret_cast<const typename PR::raw*>(gg + gi) : z;
      rb[i] = ok ? to_f32(gbeta[(size_t)(b * T + t) * p.HV + hv]) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int t = t0 + vg * VR + i;
      const bool ok = t < T;
      typename PR::raw z{};
      rv[i] = ok ? *reinterpret_cast<const typename PR::raw*>(
                       gv + ((size_t)(b * T + t) * p.HV + hv) * p.V + vs * BV + 2 * vp)
                 : z;
      rbv[i] = ok ? to_f32(gbeta[(size_t)(b * T + t) * p.HV + hv]) : 0.f;
    }
  };

  // ---- state slice in accumulators: tile kt covers channels [16kt,16kt+16) ----
  f32x4 Sacc[KT];
  const int scol = vs * BV + 16 * wave + acc_col();
  const size_t sbase = (size_t)(b * p.HV + hv) * K * p.V;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      Sacc[kt][e] = p.s0 ? p.s0[sbase + (size_t)(16 * kt + acc_row(e)) * p.V + scol] : 0.f;

  if (tid == 0) { sFlag[0] = 0; sFlag[1] = 0; }
  const float clampv = p.g_clamp_min;
  const bool do_clamp = clampv > -INFINITY;
  const float scale = p.scale;
  const int nchunks = (T + C - 1) / C;
  load_chunk(0);

  for (int n = 0; n < nchunks; ++n) {
    // ---------------- stage 1: gate cumsum (log2 units) ----------------
    float2 G[NTOK];
    bool anypos = false;
    {
      float2 run = make_float2(0.f, 0.f);
#pragma unroll
      for (int i = 0; i < NTOK; ++i) {
        float2 gv2 = PR::cvt(rgt[i]);
        if (do_clamp) { gv2.x = fmaxf(gv2.x, clampv); gv2.y = fmaxf(gv2.y, clampv); }
        anypos |= (gv2.x > 0.f) | (gv2.y > 0.f);
        run.x += gv2.x * LOG2E;
        run.y += gv2.y * LOG2E;
        G[i] = run;
      }
      sTot[tg * K + ch0] = run.x;
      sTot[tg * K + ch0 + 1] = run.y;
    }
    __syncthreads();  // B1: totals visible; previous chunk's state phase is done
    float2 off = make_float2(0.f, 0.f), anc = make_float2(0.f, 0.f), last = make_float2(0.f, 0.f);
#pragma unroll
    for (int j = 0; j < NGRP; ++j) {
      const float tx = sTot[j * K + ch0], ty = sTot[j * K + ch0 + 1];
      if (j < tg) { off.x += tx; off.y += ty; }
      if (j < AGRP) { anc.x += tx; anc.y += ty; }
      last.x += tx; last.y += ty;
    }
    int flag = anypos ? 2 : 0;
#pragma unroll
    for (int i = 0; i < NTOK; ++i) {
      G[i].x += off.x;  // G relative to the chunk start
      G[i].y += off.y;
      const float dx = fabsf(G[i].x - anc.x), dy = fabsf(G[i].y - anc.y);
      const float dm = fmaxf(dx, dy);
      if (dm > 120.f) flag |= 1;
      if (dm > 25.f * LOG2E) flag |= 4;
    }
    // OR-ed over the active lanes by ballots: one LDS atomic per wave, from its
    // first active lane (the lanes' own atomics on one word serialise)
    {
      const int wf = (__builtin_amdgcn_ballot_w64((flag & 1) != 0) ? 1 : 0) |
                     (__builtin_amdgcn_ballot_w64((flag & 2) != 0) ? 2 : 0) |
                     (__builtin_amdgcn_ballot_w64((flag & 4) != 0) ? 4 : 0);
      const int first = __ffsll((long long)__builtin_amdgcn_ballot_w64(true)) - 1;
      if (wf && (int)(threadIdx.x & 63) == first) atomicOr(&sFlag[n & 1], wf);
    }
    if (cp == 0) {
#pragma unroll
      for (int i = 0; i < NTOK; ++i) sBeta[r0 + i] = rb[i];
    }
    if (tg == 0) { sGl[ch0] = fast_exp2(last.x); sGl[ch0 + 1] = fast_exp2(last.y); }
    __syncthreads();  // B2: flag complete
    const int fl = sFlag[n & 1];
    const bool slow = (fl & 1) || ((fl & 2) && (fl & 4));
    if (tid == 0) sFlag[(n + 1) & 1] = 0;

    // ---------------- stage 2: decay-scaled operands ----------------
    {
      float kEb[2][NTOK], kd[2][NTOK];
      const float eax = fast_exp2(anc.x), eay = fast_exp2(anc.y);
      const float dlx = fast_exp2(last.x - anc.x), dly = fast_exp2(last.y - anc.y);
#pragma unroll
      for (int i = 0; i < NTOK; ++i) {
        const int r = r0 + i;
        const float2 kk = PR::cvt(rk[i]);
        const float2 qq = PR::cvt(rq[i]);
        const float br = rb[i];
        float qEx, qEy;
        if (!slow) {
          const float Rx = fast_exp2(G[i].x - anc.x), Ry = fast_exp2(G[i].y - anc.y);
          const float Cx = fast_exp2(anc.x - G[i].x), Cy = fast_exp2(anc.y - G[i].y);
          store2(sA + r * LDK + ch0, kk.x * Rx, kk.y * Ry);
          store2(sQ + r * LDK + ch0, qq.x * Rx * scale, qq.y * Ry * scale);
          store2(sB + r * LDK + ch0, kk.x * Cx, kk.y * Cy);
          qEx = qq.x * (Rx * eax) * scale;
          qEy = qq.y * (Ry * eay) * scale;
          kEb[0][i] = kk.x * (Rx * eax) * br;
          kEb[1][i] = kk.y * (Ry * eay) * br;
          kd[0][i] = kk.x * (Cx * dlx);
          kd[1][i] = kk.y * (Cy * dly);
        } else {
          const float Ex = fast_exp2(G[i].x), Ey = fast_exp2(G[i].y);
          sG[r * K + ch0] = G[i].x;
          sG[r * K + ch0 + 1] = G[i].y;
          qEx = qq.x * Ex * scale;
          qEy = qq.y * Ey * scale;
          kEb[0][i] = kk.x * Ex * br;
          kEb[1][i] = kk.y * Ey * br;
          kd[0][i] = kk.x * fast_exp2(last.x - G[i].x);
          kd[1][i] = kk.y * fast_exp2(last.y - G[i].y);
        }
        store2(sQE + r * LDK + ch0, qEx, qEy);
      }
      store_row<OpT, NTOK>(sKEt + ch0 * LDC + r0, kEb[0]);
      store_row<OpT, NTOK>(sKEt + (ch0 + 1) * LDC + r0, kEb[1]);
      store_row<OpT, NTOK>(sKdT + ch0 * LDC + r0, kd[0]);
      store_row<OpT, NTOK>(sKdT + (ch0 + 1) * LDC + r0, kd[1]);
      float vx[VR], vy[VR];
#pragma unroll
      for (int i = 0; i < VR; ++i) {
        const float2 vv = PR::cvt(rv[i]);
        vx[i] = vv.x * rbv[i];
        vy[i] = vv.y * rbv[i];
      }
      store_row<OpT, VR>(sVt + (2 * vp) * LDC + vg * VR, vx);
      store_row<OpT, VR>(sVt + (2 * vp + 1) * LDC + vg * VR, vy);
    }
    // prefetch the next chunk while this one is processed
    if (n + 1 < nchunks) load_chunk(n + 1);
    __syncthreads();  // B3: operands ready

    // ---------------- stage 3: L and Aqk ----------------
    if (!slow) {
      // sL / sLop alias the sA / sQ / sB operands: every wave finishes its
      // products (held in registers) before any wave stores a result.
      constexpr int NTILE = NB * NB;
      constexpr int JPW = (2 * NTILE) / 4;  // jobs per wave
      f32x4 tacc[JPW];
#pragma unroll
      for (int jj = 0; jj < JPW; ++jj) {
        const int job = wave + 4 * jj;
        const int mat = job / NTILE;
        const int ti = (job % NTILE) / NB;
        const int tj = (job % NTILE) % NB;
        tacc[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (tj <= ti)
          tacc[jj] = tile_mma(tacc[jj], (mat == 0 ? sA : sQ) + 16 * ti * LDK, LDK,
                              sB + 16 * tj * LDK, LDK, K);
      }
      __syncthreads();  // all reads of sA / sQ / sB done
#pragma unroll
      for (int jj = 0; jj < JPW; ++jj) {
        const int job = wave + 4 * jj;
        const int mat = job / NTILE;
        const int ti = (job % NTILE) / NB;
        const int tj = (job % NTILE) % NB;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 16 * ti + acc_row(e), c = 16 * tj + acc_col();
          if (mat == 0) {
            const float val = (r > c) ? tacc[jj][e] * sBeta[r] : 0.f;
            sL[r * LDF + c] = val;
            sLop[r * LDC + c] = from_f32<OpT>(val);
          } else {
            sAqk[r * LDC + c] = from_f32<OpT>((c <= r) ? tacc[jj][e] : 0.f);
          }
        }
      }
    } else {
      // exact elementwise path: clamp(max=50) on the decay exponent as the reference
      constexpr int TPR = 256 / C;      // threads per row
      constexpr int CPT = C / TPR;      // columns per thread
      const int r = tid / TPR;
      const int cbase = (tid % TPR) * CPT;
      const int tr = n * C + r;
      float accL[CPT], accA[CPT];
#pragma unroll
      for (int j = 0; j < CPT; ++j) { accL[j] = 0.f; accA[j] = 0.f; }
      if (tr < T) {
        const size_t rowr = ((size_t)(b * T + tr) * p.H + h) * K;
        for (int ch = 0; ch < K; ++ch) {
          const float gr = sG[r * K + ch];
          const float kr = to_f32(gk[rowr + ch]);
          const float qr = to_f32(gq[rowr + ch]);
#pragma unroll
          for (int j = 0; j < CPT; ++j) {
            const int c = cbase + j;
            const int tc = n * C + c;
            if (c <= r && tc < T) {
              const float e = fast_exp2(fminf(gr - sG[c * K + ch], 50.f * LOG2E));
              const float kc = to_f32(gk[((size_t)(b * T + tc) * p.H + h) * K + ch]);
              accL[j] += kr * e * kc;
              accA[j] += qr * e * kc;
            }
          }
        }
      }
      __syncthreads();  // sG no longer read (it aliases sL / sLop)
      const float br = sBeta[r];
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        const int c = cbase + j;
        const float lv = (c < r) ? accL[j] * br : 0.f;
        sL[r * LDF + c] = lv;
        sLop[r * LDC + c] = from_f32<OpT>(lv);
        sAqk[r * LDC + c] = from_f32<OpT>((c <= r) ? accA[j] * scale : 0.f);
      }
    }
    __syncthreads();  // B4: L, Aqk ready

    // ---------------- stage 4a: inverses of the 16x16 diagonal blocks ----------------
    if (wave < NB && (tid & 63) < 16) {
      const int blk = wave;
      const int cc = tid & 15;
      const float* Lb = sL + (16 * blk) * LDF + 16 * blk;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float s = 0.f;
#pragma unroll
        for (int kx = 0; kx < r; ++kx) s += Lb[r * LDF + kx] * x[kx];
        x[r] = (r < cc) ? 0.f : ((r == cc) ? 1.f : -s);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) sX[(16 * blk + r) * LDC + 16 * blk + cc] = from_f32<OpT>(x[r]);
      store_row<OpT, 16>(sXt + (16 * blk + cc) * LDC + 16 * blk, x);
    }
    __syncthreads();

    // ---------------- stage 4b: off-diagonal blocks of X ----------------
#pragma unroll
    for (int bi = 1; bi < NB; ++bi) {
      if (wave < bi) {
        const int jt = wave;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mma(acc, sLop + 16 * bi * LDC + 16 * jt, LDC, sXt + 16 * jt * LDC + 16 * jt, LDC,
                       16 * (bi - jt));
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sYt[(16 * jt + acc_col()) * LDY + acc_row(e)] = from_f32<OpT>(acc[e]);
      }
      __syncthreads();
      if (wave < bi) {
        const int jt = wave;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mma(acc, sX + 16 * bi * LDC + 16 * bi, LDC, sYt + 16 * jt * LDY, LDY, 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const OpT val = from_f32<OpT>(-acc[e]);
          sX[(16 * bi + acc_row(e)) * LDC + 16 * jt + acc_col()] = val;
          sXt[(16 * jt + acc_col()) * LDC + 16 * bi + acc_row(e)] = val;
        }
      }
      __syncthreads();
    }

    // ---------------- stage 5: w = X (beta k e^G), u = X (beta v) ----------------
    f32x4 Wacc[NB][WT > 0 ? WT : 1];
    f32x4 Uacc[NB];
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
      const int kd_ = 16 * (bi + 1);
#pragma unroll
      for (int j = 0; j < WT; ++j) {
        const int ct = wave + 4 * j;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        Wacc[bi][j] = tile_mma(acc, sX + 16 * bi * LDC, LDC, sKEt + 16 * ct * LDC, LDC, kd_);
      }
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      Uacc[bi] = tile_mma(acc, sX + 16 * bi * LDC, LDC, sVt + 16 * wave * LDC, LDC, kd_);
    }
    __syncthreads();  // sKEt / sVt / sX reads complete: sW may overwrite them
#pragma unroll
    for (int bi = 0; bi < NB; ++bi)
#pragma unroll
      for (int j = 0; j < WT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          sW[(16 * bi + acc_row(e)) * LDK + 16 * (wave + 4 * j) + acc_col()] =
              from_f32<OpT>(Wacc[bi][j][e]);
    __syncthreads();  // sW visible

    // ---------------- state phase (wave-local: columns [16w, 16w+16)) ----------------
    OpT* myS = sSt + wave * 16 * LDK;   // S^T slice: [col][channel]
    OpT* myVn = sVn + wave * 16 * LDC;  // v_new^T slice: [col][token]
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        myS[acc_col() * LDK + 16 * kt + acc_row(e)] = from_f32<OpT>(Sacc[kt][e]);
    wave_lds_sync();
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = tile_mma(acc, sW + 16 * bi * LDK, LDK, myS, LDK, K);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        myVn[acc_col() * LDC + 16 * bi + acc_row(e)] = from_f32<OpT>(Uacc[bi][e] - acc[e]);
    }
    wave_lds_sync();
#pragma unroll
    for (int bi = 0; bi < NB; ++bi) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = tile_mma(acc, sQE + 16 * bi * LDK, LDK, myS, LDK, K);
      acc = tile_mma(acc, sAqk + 16 * bi * LDC, LDC, myVn, LDC, 16 * (bi + 1));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = n * C + 16 * bi + acc_row(e);
        if (t < T) go[((size_t)(b * T + t) * p.HV + hv) * p.V + scol] = from_f32<InT>(acc[e]);
      }
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) Sacc[kt][e] *= sGl[16 * kt + acc_row(e)];
      Sacc[kt] = tile_mma(Sacc[kt], sKdT + 16 * kt * LDC, LDC, myVn, LDC, C);
    }
  }

  if (p.s_out) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        p.s_out[sbase + (size_t)(16 * kt + acc_row(e)) * p.V + scol] = Sacc[kt][e];
  }
}

template <int K, int C, typename InT, typename OpT>
static hipError_t launch_chunk(const KdaParams& p, hipStream_t stream) {
  const int total = p.B * p.HV * (p.V / 64);
  hipLaunchKernelGGL((kda_chunk_kernel<K, C, InT, OpT>), dim3(total), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t kda_chunk_dispatch(const KdaParams& p, int dtype, hipStream_t stream) {
  const int K = p.K;
  if (dtype == DT_F32) {
    if (K == 128) return launch_chunk<128, 32, float, float>(p, stream);
    return launch_chunk<64, 32, float, float>(p, stream);
  }
  // bf16 / fp16: the 8-wave kernel of kda_chunk_lp.hip
  return kda_chunk_lp_dispatch(p, dtype, stream);
}

}  // namespace kch
