// KDA chunked backward for gfx950: the gradients of naive_chunk_kda
// (/root/reference/ops_kda.py:340-536, which the reference differentiates with
// autograd; its tests pin them to the recurrent ones, run_correctness.py:
// 1032-1092) in the chunk form, for bf16 / fp16 / fp32 inputs, K and V in
// {64, 128}, chunks of 64 tokens. Arithmetic is fp32; every matrix product
// is an MFMA product of two-part bf16 splits (x = hi + lo; hi*hi + hi*lo +
// lo*hi, about 2^-16 relative per product).
//
// Per chunk (q^ = scale q, G = in-chunk cumsum of the clamped gate, natural
// log units, G_l = G at the chunk's last token):
//   M[i][j]   = beta_i sum_ch k_i k_j e^(G_i - G_j)     (j < i)
//   Aqk[i][j] = sum_ch q^_i k_j e^(G_i - G_j)           (j <= i)
//   X = (I + M)^-1,   Bk = beta k e^G,   Bv = beta v
//   W = X Bk,   U = X Bv,   Qg = q^ e^G,   Kd = k e^(G_l - G),   el = e^(G_l)
//   v_n = U - W S_n;   o = Qg S_n + Aqk v_n;   S_n+1 = el S_n + Kd^T v_n
// with the exponents of M and Aqk clamped at 50 (ops_kda.py:414,516).
// Backward, dS' = dL/dS_n+1:
//   dv_n = Aqk^T dO + Kd dS'          dS_n = Qg^T dO + el dS' - W^T dv_n
//   dBv  = X^T dv_n                   (dU = dv_n)
//   dBk  = -dBv S_n^T                 (= X^T dW with dW = -dv_n S_n^T)
//   dM   = -dBv v_n^T, strictly lower (= -X^T dX X^T: dX = dv_n v_n^T (I + M)^T
//                                      because (I + M) v_n = Bv - Bk S_n)
//   dAqk = dO v_n^T (j <= i),  dQg = dO S_n^T,  dKd = v_n dS'^T,
//   del  = rowsum(S_n * dS')
// then the elementwise chains back to q, k, v, g and beta; dg is the in-chunk
// suffix sum of dG plus the gradient of G_l.
//
// Kernels (one launch each):
//   cb_prep_kernel  per (b, hv, chunk): M, Aqk, X, W, U, Qg, Kd, el -> workspace
//                   (8 waves, two per SIMD, sharing one LDS allocation)
//   cb_fwd_kernel   per (b, hv, 64 columns of V), chunks in order: S_n, v_n
//   cb_bwd_kernel   per (b, hv, 64 columns of V), chunks in reverse: dS', dv_n, dS_0
//   cb_grad_kernel  per (b, hv, chunk): dq, dk, dv, dg, dbeta (or per-value-head
//                   partials that kda_bwd_reduce_launch sums when HV > H)
// The state kernels keep the state in MFMA accumulators; the operands shared
// by the waves sit in LDS, the rest is read straight from L2 in fragment form.
// The decay-weighted products (M, Aqk and their gradients) factor as
// e^(G_i - G_a) e^(G_a - G_j) around token a = 31 and run on MFMA when every
// gate of the chunk (or channel block) is <= 0 and every |G - G_a| <= 60 nats:
// the factors then stay in fp32 range with normal low parts, and no exponent
// reaches the clamp. Otherwise they are formed exactly, one exponential per
// (i, j, channel), with the clamp and its zero gradient.

#include <type_traits>

#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

constexpr int C = 64;
constexpr int kAnc = 31;
constexpr float kLn2Inv = 1.4426950408889634f;
constexpr float kCap = 50.f;
constexpr float kAncRange = 60.f;

__device__ __forceinline__ float ex(float x) { return __builtin_amdgcn_exp2f(x * kLn2Inv); }

struct Sp {
  bf16x8 hi, lo;
};

__device__ __forceinline__ Sp sp8(const float* f) {
  Sp s;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16_t h = (bf16_t)f[i];
    s.hi[i] = h;
    s.lo[i] = (bf16_t)(f[i] - (float)h);
  }
  return s;
}

__device__ __forceinline__ f32x4 mm3(const Sp& a, const Sp& b, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, acc, 0, 0, 0);
}

// 8 consecutive fp32 values (16-byte aligned)
__device__ __forceinline__ void ld8c(const float* p, float* f) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// 8 fp32 values ld apart
__device__ __forceinline__ void ld8s(const float* p, int ld, float* f) {
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = p[i * ld];
}

// 8 consecutive input values (16-byte aligned), as fp32
template <typename T>
__device__ __forceinline__ void ld8g(const T* p, float* f) {
  if constexpr (sizeof(T) == 4) {
    ld8c(reinterpret_cast<const float*>(p), f);
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 x = Pair<T>::cvt(w[i]);
      f[2 * i] = x.x;
      f[2 * i + 1] = x.y;
    }
  }
}

__device__ __forceinline__ void zero8(float* f) {
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = 0.f;
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// sum over the 16 lanes of a DPP row (every lane receives it)
__device__ __forceinline__ float row16_sum(float v) {
  v += dppf<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dppf<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dppf<0x141>(v);  // row_half_mirror
  v += dppf<0x140>(v);  // row_mirror
  return v;
}

// sum over the four lanes of a quad
__device__ __forceinline__ float quad_sum(float v) {
  v += dppf<0xB1>(v);
  return v + dppf<0x4E>(v);
}

// Workspace record of one (b, hv, chunk), fp32, row-major:
//   W [C][K] | Kd [C][K] | Qg [C][K] | U [C][V] | Aqk^T [C][C] | X^T [C][C] | el [K]
template <int K, int V>
struct Rec {
  static constexpr int W = 0, KD = C * K, QG = 2 * C * K, U = 3 * C * K, AQK = U + C * V,
                       XT = AQK + C * C, EL = XT + C * C, RS = (EL + K + 63) / 64 * 64;
};

struct CbWs {
  float* rec;   // [B*HV*NT][RS]
  float* sn;    // [B*HV*NT][K][V]   state at the start of each chunk
  float* dsn;   // [B*HV*NT][K][V]   dL/dS after each chunk
  float* vn;    // [B*HV*NT][C][V]   v_n
  float* dvn;   // [B*HV*NT][C][V]   dL/dv_n
  float* part;  // [B,T,HV,3K+1] per-value-head partials (HV > H), else null
  int nt;
};

constexpr int NTH = 512;  // threads of the per-chunk kernels: 8 waves, two per SIMD

// sum over the eight lanes of a half DPP row
__device__ __forceinline__ float oct_sum(float v) {
  v = quad_sum(v);
  return v + dppf<0x141>(v);  // row_half_mirror
}

// In-place inclusive prefix sums down the C = 64 rows of columns [0, NCOL) of
// an LDS matrix with row stride ld (Rev: suffix sums, from the last row up),
// plus init[column] when init is given, by all NTH threads: column
// tid % NCOL, a segment of C / (NTH / NCOL) rows each; the segment totals
// meet in tot [NTH]. Ends with a barrier.
template <int NCOL, bool Rev>
__device__ __forceinline__ void col_scan(float* m, int ld, float* tot, const float* init) {
  constexpr int NSEG = NTH / NCOL, SL = C / NSEG;
  const int col = threadIdx.x % NCOL, seg = threadIdx.x / NCOL;
  const int r0 = Rev ? (NSEG - 1 - seg) * SL : seg * SL;
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < SL; ++r) {
    const int row = Rev ? r0 + SL - 1 - r : r0 + r;
    s += m[row * ld + col];
    m[row * ld + col] = s;
  }
  tot[seg * NCOL + col] = s;
  __syncthreads();
  float off = init ? init[col] : 0.f;
  for (int q = 0; q < seg; ++q) off += tot[q * NCOL + col];
#pragma unroll
  for (int r = 0; r < SL; ++r) m[(r0 + r) * ld + col] += off;
  __syncthreads();
}

// ---------------------------------------------------------------------------
// cb_prep_kernel: one workgroup (8 waves) per (b, hv, chunk)
// ---------------------------------------------------------------------------
template <int K, int V, typename InT>
__global__ __launch_bounds__(NTH) void cb_prep_kernel(KdaBwdParams p, CbWs w) {
  using R = Rec<K, V>;
  constexpr int LK = K + 4, LC = C + 4, LV = V + 4;
  constexpr int SQ = C * LK > C * LV ? C * LK : C * LV;
  __shared__ float sk[C * LK], sG[C * LK], sq[SQ], sM[C * LC], sX[C * LC], sb[C], stot[NTH];
  __shared__ int sflag;
  float* const sv = sq;  // v [C][LV] once q^ is consumed

  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, r16 = l & 15, kq = l >> 4;
  const int nt = w.nt;
  const int n = blockIdx.x % nt, bh = blockIdx.x / nt;
  const int hv = bh % p.HV, b = bh / p.HV, h = hv / (p.HV / p.H);
  const int T = p.T, t0 = n * C;
  const float scale = (float)p.scale;
  const bool clampg = p.g_clamp_min > -INFINITY;
  const float gmin = (float)p.g_clamp_min;
  float* rec = w.rec + (size_t)blockIdx.x * R::RS;

  if (tid == 0) sflag = 1;
  __syncthreads();
  bool pos = false;
  for (int it = tid; it < C * (K / 8); it += NTH) {
    const int c = it / (K / 8), c8 = (it % (K / 8)) * 8, t = t0 + c;
    float fq[8], fk[8], fg[8];
    if (t < T) {
      const size_t qk = ((size_t)(b * T + t) * p.H + h) * K + c8;
      ld8g(static_cast<const InT*>(p.q) + qk, fq);
      ld8g(static_cast<const InT*>(p.k) + qk, fk);
      ld8g(static_cast<const InT*>(p.g) + ((size_t)(b * T + t) * p.HV + hv) * K + c8, fg);
    } else {
      zero8(fq); zero8(fk); zero8(fg);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float gc = clampg ? fmaxf(fg[i], gmin) : fg[i];
      pos |= gc > 0.f;
      sq[c * LK + c8 + i] = scale * fq[i];
      sk[c * LK + c8 + i] = fk[i];
      sG[c * LK + c8 + i] = gc;
    }
  }
  if (pos) sflag = 0;
  if (tid < C) {
    const int t = t0 + tid;
    sb[tid] = t < T ? to_f32(static_cast<const InT*>(p.beta)[(size_t)(b * T + t) * p.HV + hv]) : 0.f;
  }
  __syncthreads();
  col_scan<K, false>(sG, LK, stot, nullptr);
  if (tid < K) {
    const float ga = sG[kAnc * LK + tid];
    if (sG[tid] - ga > kAncRange || ga - sG[(C - 1) * LK + tid] > kAncRange) sflag = 0;
  }
  __syncthreads();
  const bool anchored = sflag != 0;

  // M and Aqk: wave wv owns column tile wv & 3 (j) of row tiles rt0, rt0 + 1 (i)
  {
    const int rt0 = 2 * (wv >> 2), jc = 16 * (wv & 3) + r16;
    f32x4 am[2], aa[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) am[u] = aa[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (anchored) {
#pragma unroll 1
      for (int ks = 0; ks < K; ks += 32) {
        const int ch = ks + 8 * kq;
        float fb[8], gj[8], ga[8];
        ld8c(&sk[jc * LK + ch], fb);
        ld8c(&sG[jc * LK + ch], gj);
        ld8c(&sG[kAnc * LK + ch], ga);
#pragma unroll
        for (int i = 0; i < 8; ++i) fb[i] *= ex(ga[i] - gj[i]);
        const Sp bs = sp8(fb);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i0 = 16 * (rt0 + u) + r16;
          float fk[8], fq[8], gi[8];
          ld8c(&sk[i0 * LK + ch], fk);
          ld8c(&sq[i0 * LK + ch], fq);
          ld8c(&sG[i0 * LK + ch], gi);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float P = ex(gi[i] - ga[i]);
            fk[i] *= P;
            fq[i] *= P;
          }
          am[u] = mm3(sp8(fk), bs, am[u]);
          aa[u] = mm3(sp8(fq), bs, aa[u]);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 16 * (rt0 + u) + 4 * kq + e;
          float m = 0.f, a = 0.f;
          if (jc <= i) {
            for (int ch = 0; ch < K; ++ch) {
              const float x = ex(fminf(sG[i * LK + ch] - sG[jc * LK + ch], kCap)) * sk[jc * LK + ch];
              m += sk[i * LK + ch] * x;
              a += sq[i * LK + ch] * x;
            }
          }
          am[u][e] = m;
          aa[u][e] = a;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * (rt0 + u) + 4 * kq + e;
        sM[i * LC + jc] = jc < i ? sb[i] * am[u][e] : 0.f;
        rec[R::AQK + jc * C + i] = jc <= i ? aa[u][e] : 0.f;  // stored transposed
      }
  }
  // Qg, Kd, el
  for (int it = tid; it < C * K; it += NTH) {
    const int c = it / K, ch = it % K;
    const float G = sG[c * LK + ch];
    rec[R::QG + it] = sq[c * LK + ch] * ex(G);
    rec[R::KD + it] = sk[c * LK + ch] * ex(sG[(C - 1) * LK + ch] - G);
  }
  if (tid < K) rec[R::EL + tid] = ex(sG[(C - 1) * LK + tid]);
  __syncthreads();

  // v -> LDS (over q^); X = (I + M)^-1, column cc by the eight lanes of a half row
  for (int it = tid; it < C * (V / 8); it += NTH) {
    const int c = it / (V / 8), c8 = (it % (V / 8)) * 8, t = t0 + c;
    float fv[8];
    if (t < T)
      ld8g(static_cast<const InT*>(p.v) + ((size_t)(b * T + t) * p.HV + hv) * V + c8, fv);
    else
      zero8(fv);
#pragma unroll
    for (int i = 0; i < 8; ++i) sv[c * LV + c8 + i] = fv[i];
  }
  {
    const int cc = tid >> 3, part = tid & 7;
    float xr[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) xr[jj] = 0.f;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      float s = 0.f;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        if (8 * jj < i) {
          const int j = 8 * jj + part;
          if (j < i) s += sM[i * LC + j] * xr[jj];
        }
      }
      s = oct_sum(s);
      const float xi = (i == cc ? 1.f : 0.f) - s;
      if (part == (i & 7)) xr[i >> 3] = xi;
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = 8 * jj + part;
      sX[j * LC + cc] = xr[jj];
      rec[R::XT + cc * C + j] = xr[jj];
    }
  }
  __syncthreads();

  // W^T = Bk^T X^T and U^T = Bv^T X^T, one row tile (of K, then of V) at a
  // time over the four column tiles of the chunk; stored row-major as W [C][K]
  // and U [C][V]
#pragma unroll 1
  for (int rtg = wv; rtg < K / 16 + V / 16; rtg += NTH / 64) {
    const bool isw = rtg < K / 16;
    const int r = 16 * (isw ? rtg : rtg - K / 16) + r16;
    f32x4 acc[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < C; ks += 32) {
      const int j0 = ks + 8 * kq;
      float fa[8];
      if (isw) {
        float gj[8];
        ld8s(&sk[j0 * LK + r], LK, fa);
        ld8s(&sG[j0 * LK + r], LK, gj);
#pragma unroll
        for (int i = 0; i < 8; ++i) fa[i] *= sb[j0 + i] * ex(gj[i]);
      } else {
        ld8s(&sv[j0 * LV + r], LV, fa);
#pragma unroll
        for (int i = 0; i < 8; ++i) fa[i] *= sb[j0 + i];
      }
      const Sp as = sp8(fa);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        float fb[8];
        ld8c(&sX[(16 * ct + r16) * LC + j0], fb);
        acc[ct] = mm3(as, sp8(fb), acc[ct]);
      }
    }
    const int r4 = r - r16 + 4 * kq;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      float* dst = isw ? &rec[R::W + (16 * ct + r16) * K + r4] : &rec[R::U + (16 * ct + r16) * V + r4];
      *reinterpret_cast<float4*>(dst) = make_float4(acc[ct][0], acc[ct][1], acc[ct][2], acc[ct][3]);
    }
  }
}

// (slice of V, head) of a state-kernel workgroup. Workgroups are dealt to the
// 8 XCDs round-robin; with two slices per head, blocks g and g + 8 of every
// 16 take the two slices of one head, so they share an XCD and its L2 and the
// head's per-chunk operands are read from HBM once.
template <int NVS>
__device__ __forceinline__ void slice_of(int& vs, int& bh) {
  const int g = blockIdx.x;
  if (NVS == 2 && (gridDim.x % 16) == 0) {
    vs = (g >> 3) & 1;
    bh = (g >> 4) * 8 + (g & 7);
  } else {
    vs = g % NVS;
    bh = g / NVS;
  }
}

// ---------------------------------------------------------------------------
// cb_fwd_kernel: one workgroup per (b, hv, 64 columns of V); S^T in
// accumulators (rows v, columns K), wave wv owning columns [K/4 wv, K/4 (wv+1)).
// The operands of chunk n+1 read from L2 in fragment form (W rows, U, el) are
// loaded into registers while chunk n runs; Kd, transposed into LDS, is
// loaded at the start of its own chunk and stored after the v_n product.
// ---------------------------------------------------------------------------
template <int K, int V>
__global__ __launch_bounds__(256) void cb_fwd_kernel(KdaBwdParams p, CbWs w) {
  using R = Rec<K, V>;
  constexpr int VS = 64, NVS = V / VS, LK = K + 4, LC = C + 4, KT = K / 64, KS = K / 32;
  constexpr int NKD = C * K / 4 / 256;
  __shared__ float sST[VS * LK], sVT[VS * LC], sKT[K * LC];
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, r16 = l & 15, kq = l >> 4;
  int vs, bh;
  slice_of<NVS>(vs, bh);
  const int v0 = vs * VS;
  const int nt = w.nt;
  const int cw = 16 * wv + r16;  // this lane's token row of the v_n^T column tile
  const float* s0 = static_cast<const float*>(p.s0);

  f32x4 S[4][KT];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int a = 0; a < KT; ++a) {
      const int kch = 16 * (wv * KT + a) + r16, vr = 16 * rt + 4 * kq;
      if (s0) {
        const float4 x = *reinterpret_cast<const float4*>(&s0[((size_t)bh * K + kch) * V + v0 + vr]);
        S[rt][a] = f32x4{x.x, x.y, x.z, x.w};
      } else {
        S[rt][a] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) sST[(vr + e) * LK + kch] = S[rt][a][e];
    }

  float wb[KS][8];
  float4 ub[4];
  float elb[KT];
  auto prefetch = [&](int n) {
    const float* rec = w.rec + ((size_t)bh * nt + n) * R::RS;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) ld8c(&rec[R::W + cw * K + 32 * ks + 8 * kq], wb[ks]);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
      ub[rt] = *reinterpret_cast<const float4*>(&rec[R::U + cw * V + v0 + 16 * rt + 4 * kq]);
#pragma unroll
    for (int a = 0; a < KT; ++a) elb[a] = rec[R::EL + 16 * (wv * KT + a) + r16];
  };
  prefetch(0);
  __syncthreads();

#pragma unroll 1
  for (int n = 0; n < nt; ++n) {
    const size_t ci = (size_t)bh * nt + n;
    const float* rec = w.rec + ci * R::RS;
    // Kd of this chunk: lane-consecutive rows c, so the transposed LDS
    // stores below hit distinct banks
    float4 kd[NKD];
#pragma unroll
    for (int i = 0; i < NKD; ++i) {
      const int it = tid + 256 * i, c = it % C, k4 = (it / C) * 4;
      kd[i] = *reinterpret_cast<const float4*>(&rec[R::KD + c * K + k4]);
    }
    float* sn = w.sn + ci * K * V;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kch = 16 * (wv * KT + a) + r16;
        *reinterpret_cast<float4*>(&sn[(size_t)kch * V + v0 + 16 * rt + 4 * kq]) =
            make_float4(S[rt][a][0], S[rt][a][1], S[rt][a][2], S[rt][a][3]);
      }
    // v_n^T = U^T - S^T W^T: wave wv owns column tile wv (tokens)
    f32x4 vn[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) vn[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const Sp bs = sp8(wb[ks]);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float fa[8];
        ld8c(&sST[(16 * rt + r16) * LK + 32 * ks + 8 * kq], fa);
        vn[rt] = mm3(sp8(fa), bs, vn[rt]);
      }
    }
    float* vng = w.vn + ci * C * V;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int vr = 16 * rt + 4 * kq;
      const float4 x = make_float4(ub[rt].x - vn[rt][0], ub[rt].y - vn[rt][1], ub[rt].z - vn[rt][2],
                                   ub[rt].w - vn[rt][3]);
      *reinterpret_cast<float4*>(&vng[cw * V + v0 + vr]) = x;
      sVT[(vr + 0) * LC + cw] = x.x;
      sVT[(vr + 1) * LC + cw] = x.y;
      sVT[(vr + 2) * LC + cw] = x.z;
      sVT[(vr + 3) * LC + cw] = x.w;
    }
    float el[KT];
#pragma unroll
    for (int a = 0; a < KT; ++a) el[a] = elb[a];
    if (n + 1 < nt) prefetch(n + 1);
#pragma unroll
    for (int i = 0; i < NKD; ++i) {
      const int it = tid + 256 * i, c = it % C, k4 = (it / C) * 4;
      sKT[(k4 + 0) * LC + c] = kd[i].x;
      sKT[(k4 + 1) * LC + c] = kd[i].y;
      sKT[(k4 + 2) * LC + c] = kd[i].z;
      sKT[(k4 + 3) * LC + c] = kd[i].w;
    }
    __syncthreads();
    // S_n+1^T = el S^T + v_n^T Kd
#pragma unroll
    for (int a = 0; a < KT; ++a)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) S[rt][a] *= el[a];
#pragma unroll
    for (int ks = 0; ks < C; ks += 32) {
      const int c0 = ks + 8 * kq;
      Sp bs[KT];
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        float fb[8];
        ld8c(&sKT[(16 * (wv * KT + a) + r16) * LC + c0], fb);
        bs[a] = sp8(fb);
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float fa[8];
        ld8c(&sVT[(16 * rt + r16) * LC + c0], fa);
        const Sp as = sp8(fa);
#pragma unroll
        for (int a = 0; a < KT; ++a) S[rt][a] = mm3(as, bs[a], S[rt][a]);
      }
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kch = 16 * (wv * KT + a) + r16;
#pragma unroll
        for (int e = 0; e < 4; ++e) sST[(16 * rt + 4 * kq + e) * LK + kch] = S[rt][a][e];
      }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// cb_bwd_kernel: one workgroup per (b, hv, 64 columns of V), chunks in
// reverse; dS^T in accumulators, wave wv owning columns [K/4 wv, K/4 (wv+1)).
// Aqk^T and Kd rows (fragments), el and the dO slice of chunk n-1 are loaded
// while chunk n runs (dO^T into the other of two LDS buffers); Qg and W,
// transposed into LDS, are loaded at the start of their own chunk and stored
// after the dv_n product.
// ---------------------------------------------------------------------------
template <int K, int V, typename InT>
__global__ __launch_bounds__(256) void cb_bwd_kernel(KdaBwdParams p, CbWs w) {
  using R = Rec<K, V>;
  constexpr int VS = 64, NVS = V / VS, LK = K + 4, LC = C + 4, KT = K / 64, KS = K / 32;
  constexpr int NKD = C * K / 4 / 256;
  constexpr int NDO = C * VS / 8 / 256;
  __shared__ float sdST[VS * LK], sDOT[2][VS * LC], sdVT[VS * LC], sQT[K * LC], sWT[K * LC];
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, r16 = l & 15, kq = l >> 4;
  int vs, bh;
  slice_of<NVS>(vs, bh);
  const int v0 = vs * VS;
  const int hv = bh % p.HV, b = bh / p.HV;
  const int nt = w.nt, T = p.T;
  const int cw = 16 * wv + r16;
  const float* dsf = static_cast<const float*>(p.ds_final);
  const InT* dO = static_cast<const InT*>(p.d_o);

  f32x4 D[4][KT];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int a = 0; a < KT; ++a) {
      const int kch = 16 * (wv * KT + a) + r16, vr = 16 * rt + 4 * kq;
      if (dsf) {
        const float4 x = *reinterpret_cast<const float4*>(&dsf[((size_t)bh * K + kch) * V + v0 + vr]);
        D[rt][a] = f32x4{x.x, x.y, x.z, x.w};
      } else {
        D[rt][a] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) sdST[(vr + e) * LK + kch] = D[rt][a][e];
    }

  float ab[2][8], kb[KS][8], elb[KT], dob[NDO][8];
  auto prefetch = [&](int n) {
    const float* rec = w.rec + ((size_t)bh * nt + n) * R::RS;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) ld8c(&rec[R::AQK + cw * C + 32 * ks + 8 * kq], ab[ks]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) ld8c(&rec[R::KD + cw * K + 32 * ks + 8 * kq], kb[ks]);
#pragma unroll
    for (int a = 0; a < KT; ++a) elb[a] = rec[R::EL + 16 * (wv * KT + a) + r16];
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      const int it = tid + 256 * i, c = it % C, v8 = (it / C) * 8, t = n * C + c;
      if (t < T)
        ld8g(dO + ((size_t)(b * T + t) * p.HV + hv) * V + v0 + v8, dob[i]);
      else
        zero8(dob[i]);
    }
  };
  auto store_dot = [&](float* dst) {
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      const int it = tid + 256 * i, c = it % C, v8 = (it / C) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[(v8 + j) * LC + c] = dob[i][j];
    }
  };
  prefetch(nt - 1);
  store_dot(sDOT[(nt - 1) & 1]);
  __syncthreads();

#pragma unroll 1
  for (int n = nt - 1; n >= 0; --n) {
    const size_t ci = (size_t)bh * nt + n;
    const float* rec = w.rec + ci * R::RS;
    const float* sdo = sDOT[n & 1];
    float4 qr[NKD], wr[NKD];
#pragma unroll
    for (int i = 0; i < NKD; ++i) {
      const int it = tid + 256 * i, c = it % C, k4 = (it / C) * 4;
      qr[i] = *reinterpret_cast<const float4*>(&rec[R::QG + c * K + k4]);
      wr[i] = *reinterpret_cast<const float4*>(&rec[R::W + c * K + k4]);
    }
    float* dsn = w.dsn + ci * K * V;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kch = 16 * (wv * KT + a) + r16;
        *reinterpret_cast<float4*>(&dsn[(size_t)kch * V + v0 + 16 * rt + 4 * kq]) =
            make_float4(D[rt][a][0], D[rt][a][1], D[rt][a][2], D[rt][a][3]);
      }
    // dv_n^T = dO^T Aqk + dS^T Kd^T (B operands: rows c of Aqk^T and of Kd);
    // wave wv owns column tile wv (tokens)
    f32x4 dv[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) dv[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const Sp bs = sp8(ab[ks]);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float fa[8];
        ld8c(&sdo[(16 * rt + r16) * LC + 32 * ks + 8 * kq], fa);
        dv[rt] = mm3(sp8(fa), bs, dv[rt]);
      }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const Sp bs = sp8(kb[ks]);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float fa[8];
        ld8c(&sdST[(16 * rt + r16) * LK + 32 * ks + 8 * kq], fa);
        dv[rt] = mm3(sp8(fa), bs, dv[rt]);
      }
    }
    float* dvg = w.dvn + ci * C * V;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int vr = 16 * rt + 4 * kq;
      *reinterpret_cast<float4*>(&dvg[cw * V + v0 + vr]) =
          make_float4(dv[rt][0], dv[rt][1], dv[rt][2], dv[rt][3]);
#pragma unroll
      for (int e = 0; e < 4; ++e) sdVT[(vr + e) * LC + cw] = dv[rt][e];
    }
    float el[KT];
#pragma unroll
    for (int a = 0; a < KT; ++a) el[a] = elb[a];
    if (n > 0) prefetch(n - 1);
#pragma unroll
    for (int i = 0; i < NKD; ++i) {
      const int it = tid + 256 * i, c = it % C, k4 = (it / C) * 4;
      sQT[(k4 + 0) * LC + c] = qr[i].x; sQT[(k4 + 1) * LC + c] = qr[i].y;
      sQT[(k4 + 2) * LC + c] = qr[i].z; sQT[(k4 + 3) * LC + c] = qr[i].w;
      sWT[(k4 + 0) * LC + c] = wr[i].x; sWT[(k4 + 1) * LC + c] = wr[i].y;
      sWT[(k4 + 2) * LC + c] = wr[i].z; sWT[(k4 + 3) * LC + c] = wr[i].w;
    }
    __syncthreads();
    // dS_n^T = el dS^T + dO^T Qg - dv_n^T W
#pragma unroll
    for (int a = 0; a < KT; ++a)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) D[rt][a] *= el[a];
#pragma unroll
    for (int ks = 0; ks < C; ks += 32) {
      const int c0 = ks + 8 * kq;
      Sp bq[KT], bw[KT];
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kch = 16 * (wv * KT + a) + r16;
        float fb[8];
        ld8c(&sQT[kch * LC + c0], fb);
        bq[a] = sp8(fb);
        ld8c(&sWT[kch * LC + c0], fb);
        bw[a] = sp8(fb);
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float fa[8], fd[8];
        ld8c(&sdo[(16 * rt + r16) * LC + c0], fa);
        ld8c(&sdVT[(16 * rt + r16) * LC + c0], fd);
#pragma unroll
        for (int i = 0; i < 8; ++i) fd[i] = -fd[i];
        const Sp as = sp8(fa), ds = sp8(fd);
#pragma unroll
        for (int a = 0; a < KT; ++a) {
          D[rt][a] = mm3(as, bq[a], D[rt][a]);
          D[rt][a] = mm3(ds, bw[a], D[rt][a]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kch = 16 * (wv * KT + a) + r16;
#pragma unroll
        for (int e = 0; e < 4; ++e) sdST[(16 * rt + 4 * kq + e) * LK + kch] = D[rt][a][e];
      }
    if (n > 0) store_dot(sDOT[(n - 1) & 1]);
    __syncthreads();
  }
  if (p.ds0) {
    float* ds0 = static_cast<float*>(p.ds0);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int a = 0; a < KT; ++a) {
        const int kch = 16 * (wv * KT + a) + r16;
        *reinterpret_cast<float4*>(&ds0[((size_t)bh * K + kch) * V + v0 + 16 * rt + 4 * kq]) =
            make_float4(D[rt][a][0], D[rt][a][1], D[rt][a][2], D[rt][a][3]);
      }
  }
}

// Exact decay-weighted gradient terms of row i, channel chl of a block of 64
// held in LDS with row stride 68: one exponential per (i, j), with the clamp
// at 50 and its zero gradient in dG. Returns the additions to (dk, dq^, dG,
// dbeta).
__device__ __forceinline__ float4 exact_decay_terms(const float* sG, const float* sk, const float* sq,
                                                 const float* sdM, const float* sdA, const float* sb,
                                                 int chl, int i) {
  constexpr int LC = C + 4, LH = 64 + 4;
  const float Gi = sG[i * LH + chl], ki = sk[i * LH + chl], qi = sq[i * LH + chl], bi = sb[i];
  float r1 = 0.f, r2 = 0.f, r1g = 0.f, r2g = 0.f;
  for (int j = 0; j <= i; ++j) {
    const float d = Gi - sG[j * LH + chl];
    const float x = ex(fminf(d, kCap)) * sk[j * LH + chl];
    const float gm = d > kCap ? 0.f : 1.f;
    const float m = sdM[i * LC + j] * x, a = sdA[i * LC + j] * x;
    r1 += m;
    r2 += a;
    r1g += gm * m;
    r2g += gm * a;
  }
  float c1 = 0.f, c1g = 0.f;
  for (int r = i; r < C; ++r) {
    const float d = sG[r * LH + chl] - Gi;
    const float x = ex(fminf(d, kCap));
    const float gm = d > kCap ? 0.f : 1.f;
    const float m = (sb[r] * sdM[r * LC + i] * sk[r * LH + chl] + sdA[r * LC + i] * sq[r * LH + chl]) * x;
    c1 += m;
    c1g += gm * m;
  }
  return make_float4(bi * r1 + c1, r2, bi * ki * r1g + qi * r2g - ki * c1g, ki * r1);
}

// ---------------------------------------------------------------------------
// cb_grad_kernel: one workgroup (8 waves) per (b, hv, chunk)
// ---------------------------------------------------------------------------
template <int K, int V, typename InT>
__global__ __launch_bounds__(NTH) void cb_grad_kernel(KdaBwdParams p, CbWs w) {
  using R = Rec<K, V>;
  constexpr int LC = C + 4, LV = V + 4, KH = 64, LH = KH + 4;
  constexpr int RG = 3 * C * LH > C * LV ? 3 * C * LH : C * LV;
  constexpr int NCT1 = V / 16, RT1 = 4 * NCT1 / (NTH / 64);
  __shared__ float sdBv[C * LV], sdA[C * LC], sdM[C * LC], sR[RG], sb[C], sbeta[C], sext[KH],
      stot[NTH];
  __shared__ int sflag;
  float* const sV = sR;  // dv_n [C][LV] (phase 1)
  float* const sk = sR;  // channel block: k, q^, G [C][LH]; q^ then dG
  float* const sq = sR + C * LH;
  float* const sG = sR + 2 * C * LH;

  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6, r16 = l & 15, kq = l >> 4;
  const int nt = w.nt;
  const int n = blockIdx.x % nt, bh = blockIdx.x / nt;
  const int hv = bh % p.HV, b = bh / p.HV, h = hv / (p.HV / p.H);
  const int T = p.T, t0 = n * C, HV = p.HV;
  const float scale = (float)p.scale;
  const bool clampg = p.g_clamp_min > -INFINITY;
  const float gmin = (float)p.g_clamp_min;
  const bool direct = w.part == nullptr;
  const size_t ci = blockIdx.x;
  const float* rec = w.rec + ci * R::RS;
  const float* Sn = w.sn + ci * K * V;
  const float* dSn = w.dsn + ci * K * V;
  const float* vng = w.vn + ci * C * V;
  const float* dvg = w.dvn + ci * C * V;
  const InT* dO = static_cast<const InT*>(p.d_o) + ((size_t)b * T * HV + hv) * V;  // row t at t*HV*V
  const InT* vin = static_cast<const InT*>(p.v) + ((size_t)b * T * HV + hv) * V;
  const size_t rs = (size_t)HV * V;
  // phases 2 and 3: wave wv owns column tile ct of row tiles rt0, rt0 + 1
  const int ct = wv & 3, rt0 = 2 * (wv >> 2);

  // phase 1: dBv = X^T dv_n; dv = beta dBv; dbeta += v . dBv
  for (int it = tid; it < C * V / 4; it += NTH) {
    const int c = it / (V / 4), v4 = (it % (V / 4)) * 4;
    *reinterpret_cast<float4*>(&sV[c * LV + v4]) = *reinterpret_cast<const float4*>(&dvg[c * V + v4]);
  }
  if (tid < C) {
    const int t = t0 + tid;
    sb[tid] = t < T ? to_f32(static_cast<const InT*>(p.beta)[(size_t)(b * T + t) * HV + hv]) : 0.f;
    sbeta[tid] = 0.f;
  }
  __syncthreads();
  {
    const int ct1 = wv % NCT1, r1 = (wv / NCT1) * RT1, vv = 16 * ct1 + r16;
    f32x4 acc[RT1];
#pragma unroll
    for (int u = 0; u < RT1; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < C; ks += 32) {
      const int j0 = ks + 8 * kq;
      float fb[8];
      ld8s(&sV[j0 * LV + vv], LV, fb);
      const Sp bs = sp8(fb);
#pragma unroll
      for (int u = 0; u < RT1; ++u) {
        float fa[8];
        ld8c(&rec[R::XT + (16 * (r1 + u) + r16) * C + j0], fa);
        acc[u] = mm3(sp8(fa), bs, acc[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < RT1; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = 16 * (r1 + u) + 4 * kq + e, t = t0 + c;
        const float x = acc[u][e];
        sdBv[c * LV + vv] = x;
        float s = 0.f;
        if (t < T) {
          const size_t o = (size_t)t * rs + vv;
          static_cast<InT*>(p.dv)[((size_t)b * T * HV + hv) * V + o] = from_f32<InT>(sb[c] * x);
          s = to_f32(vin[o]) * x;
        }
        s = row16_sum(s);
        if (r16 == 0) atomicAdd(&sbeta[c], s);
      }
  }
  __syncthreads();

  // phase 2: dAqk = dO v_n^T (j <= i), dM = -dBv v_n^T (j < i)
  {
    f32x4 a1[2], a2[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) a1[u] = a2[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (int ks = 0; ks < V; ks += 32) {
      const int v0 = ks + 8 * kq;
      float fb[8];
      ld8c(&vng[(16 * ct + r16) * V + v0], fb);
      const Sp bs = sp8(fb);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = 16 * (rt0 + u) + r16;
        float fa[8], fd[8];
        if (t0 + c < T)
          ld8g(dO + (size_t)(t0 + c) * rs + v0, fa);
        else
          zero8(fa);
        ld8c(&sdBv[c * LV + v0], fd);
        a1[u] = mm3(sp8(fa), bs, a1[u]);
        a2[u] = mm3(sp8(fd), bs, a2[u]);
      }
    }
    const int j = 16 * ct + r16;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * (rt0 + u) + 4 * kq + e;
        sdA[i * LC + j] = j <= i ? a1[u][e] : 0.f;
        sdM[i * LC + j] = j < i ? -a2[u][e] : 0.f;
      }
  }
  __syncthreads();

  // phase 3: channel blocks of 64 (lane: channel 16 ct + r16 of the block,
  // rows 16 (rt0 + u) + 4 kq + e)
  float dbeta[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) dbeta[u][e] = 0.f;
  const int chl = 16 * ct + r16;
#pragma unroll 1
  for (int ch0 = 0; ch0 < K; ch0 += KH) {
    const int chg = ch0 + chl;
    if (tid == 0) sflag = 1;
    __syncthreads();
    bool pos = false;
    for (int it = tid; it < C * (KH / 8); it += NTH) {
      const int c = it / (KH / 8), c8 = (it % (KH / 8)) * 8, t = t0 + c;
      float fq[8], fk[8], fg[8];
      if (t < T) {
        const size_t qk = ((size_t)(b * T + t) * p.H + h) * K + ch0 + c8;
        ld8g(static_cast<const InT*>(p.q) + qk, fq);
        ld8g(static_cast<const InT*>(p.k) + qk, fk);
        ld8g(static_cast<const InT*>(p.g) + ((size_t)(b * T + t) * HV + hv) * K + ch0 + c8, fg);
      } else {
        zero8(fq); zero8(fk); zero8(fg);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float gc = clampg ? fmaxf(fg[i], gmin) : fg[i];
        pos |= gc > 0.f;
        sq[c * LH + c8 + i] = scale * fq[i];
        sk[c * LH + c8 + i] = fk[i];
        sG[c * LH + c8 + i] = gc;
      }
    }
    if (pos) sflag = 0;
    __syncthreads();
    col_scan<KH, false>(sG, LH, stot, nullptr);
    if (tid < KH) {
      const float ga = sG[kAnc * LH + tid];
      if (sG[tid] - ga > kAncRange || ga - sG[(C - 1) * LH + tid] > kAncRange) sflag = 0;
    }
    {
      // el * del for the block's channels: eight lanes per channel
      const int cl = tid >> 3, part = tid & 7;
      const float* s1 = Sn + (size_t)(ch0 + cl) * V + part * (V / 8);
      const float* s2 = dSn + (size_t)(ch0 + cl) * V + part * (V / 8);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < V / 8; i += 4) {
        const float4 x = *reinterpret_cast<const float4*>(s1 + i);
        const float4 y = *reinterpret_cast<const float4*>(s2 + i);
        s += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
      }
      s = oct_sum(s);
      if (part == 0) sext[cl] = ex(sG[(C - 1) * LH + cl]) * s;
    }
    __syncthreads();
    const bool anchored = sflag != 0;

    float dq[2][4], dk[2][4], dg[2][4];
    {
      // dQg = dO S^T, dBk = -dBv S^T, dKd = v_n dS'^T
      f32x4 x1[2], x2[2], x3[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) x1[u] = x2[u] = x3[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
      for (int ks = 0; ks < V; ks += 32) {
        const int v0 = ks + 8 * kq;
        float fb[8];
        ld8c(&Sn[(size_t)chg * V + v0], fb);
        const Sp b1 = sp8(fb);
        ld8c(&dSn[(size_t)chg * V + v0], fb);
        const Sp b3 = sp8(fb);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int c = 16 * (rt0 + u) + r16;
          float fa[8];
          if (t0 + c < T)
            ld8g(dO + (size_t)(t0 + c) * rs + v0, fa);
          else
            zero8(fa);
          x1[u] = mm3(sp8(fa), b1, x1[u]);
          ld8c(&sdBv[c * LV + v0], fa);
#pragma unroll
          for (int i = 0; i < 8; ++i) fa[i] = -fa[i];
          x2[u] = mm3(sp8(fa), b1, x2[u]);
          ld8c(&vng[c * V + v0], fa);
          x3[u] = mm3(sp8(fa), b3, x3[u]);
        }
      }
      const float Gl = sG[(C - 1) * LH + chl];
      float colsum = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 16 * (rt0 + u) + 4 * kq + e;
          const float G = sG[c * LH + chl], kk = sk[c * LH + chl], qq = sq[c * LH + chl], bb = sb[c];
          const float eG = ex(G), ed = ex(Gl - G);
          const float y1 = x1[u][e], y2 = x2[u][e], y3 = x3[u][e];
          dq[u][e] = eG * y1;
          dk[u][e] = ed * y3 + bb * eG * y2;
          dg[u][e] = qq * eG * y1 - kk * ed * y3 + bb * kk * eG * y2;
          colsum += kk * ed * y3;
          dbeta[u][e] += kk * eG * y2;
        }
      atomicAdd(&sext[chl], colsum);
    }

    if (anchored) {
      // R1' = dM KN, R2 = dAqk KN, C1 = (beta dM)^T KP, C2 = dAqk^T QP with
      // KN = k e^(G_a - G), KP = k e^(G - G_a), QP = q^ e^(G - G_a)
      f32x4 r1[2], r2[2], c1[2], c2[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) r1[u] = r2[u] = c1[u] = c2[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float Ga = sG[kAnc * LH + chl];
#pragma unroll
      for (int ks = 0; ks < C; ks += 32) {
        const int j0 = ks + 8 * kq;
        float kj[8], gj[8], qj[8], fN[8], fP[8], fQ[8];
        ld8s(&sk[j0 * LH + chl], LH, kj);
        ld8s(&sG[j0 * LH + chl], LH, gj);
        ld8s(&sq[j0 * LH + chl], LH, qj);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float P = ex(gj[i] - Ga), N = ex(Ga - gj[i]);
          fN[i] = kj[i] * N;
          fP[i] = kj[i] * P;
          fQ[i] = qj[i] * P;
        }
        const Sp bN = sp8(fN), bP = sp8(fP), bQ = sp8(fQ);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int i0 = 16 * (rt0 + u) + r16;
          float fa[8];
          ld8c(&sdM[i0 * LC + j0], fa);
          r1[u] = mm3(sp8(fa), bN, r1[u]);
          ld8c(&sdA[i0 * LC + j0], fa);
          r2[u] = mm3(sp8(fa), bN, r2[u]);
          ld8s(&sdM[j0 * LC + i0], LC, fa);
#pragma unroll
          for (int i = 0; i < 8; ++i) fa[i] *= sb[j0 + i];
          c1[u] = mm3(sp8(fa), bP, c1[u]);
          ld8s(&sdA[j0 * LC + i0], LC, fa);
          c2[u] = mm3(sp8(fa), bQ, c2[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 16 * (rt0 + u) + 4 * kq + e;
          const float G = sG[c * LH + chl], kk = sk[c * LH + chl], qq = sq[c * LH + chl], bb = sb[c];
          const float P = ex(G - Ga), N = ex(Ga - G);
          const float y1 = P * r1[u][e], y2 = P * r2[u][e], yc = N * (c1[u][e] + c2[u][e]);
          dk[u][e] += bb * y1 + yc;
          dq[u][e] += y2;
          dg[u][e] += bb * kk * y1 + qq * y2 - kk * yc;
          dbeta[u][e] += kk * y1;
        }
    } else {
      // one row at a time (a rolled loop keeps the slow path's registers
      // few); the sums land in the row's registers through an unrolled select
#pragma unroll 1
      for (int ue = 0; ue < 8; ++ue) {
        const float4 x = exact_decay_terms(sG, sk, sq, sdM, sdA, sb, chl,
                                           16 * (rt0 + (ue >> 2)) + 4 * kq + (ue & 3));
#pragma unroll
        for (int z = 0; z < 8; ++z)
          if (z == ue) {
            dk[z >> 2][z & 3] += x.x;
            dq[z >> 2][z & 3] += x.y;
            dg[z >> 2][z & 3] += x.z;
            dbeta[z >> 2][z & 3] += x.w;
          }
      }
    }
    __syncthreads();  // every read of q^ (sq) done, sext complete
    // dG -> LDS (over q^); suffix sums over the chunk plus the G_l gradient
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) sq[(16 * (rt0 + u) + 4 * kq + e) * LH + chl] = dg[u][e];
    __syncthreads();
    col_scan<KH, true>(sq, LH, stot, sext);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = 16 * (rt0 + u) + 4 * kq + e, t = t0 + c;
        if (t >= T) continue;
        const float dgv = sq[c * LH + chl];
        if (direct) {
          const size_t qi = ((size_t)(b * T + t) * p.H + h) * K + chg;
          const size_t gi = ((size_t)(b * T + t) * HV + hv) * K + chg;
          static_cast<InT*>(p.dq)[qi] = from_f32<InT>(scale * dq[u][e]);
          static_cast<InT*>(p.dk)[qi] = from_f32<InT>(dk[u][e]);
          const bool pass = !clampg || to_f32(static_cast<const InT*>(p.g)[gi]) >= gmin;
          static_cast<InT*>(p.dg)[gi] = from_f32<InT>(pass ? dgv : 0.f);
        } else {
          float* pr = w.part + ((size_t)(b * T + t) * HV + hv) * (3 * K + 1);
          pr[chg] = dq[u][e];
          pr[K + chg] = dk[u][e];
          pr[2 * K + chg] = dgv;
        }
      }
    __syncthreads();  // before the next block overwrites sR and sext
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float s = row16_sum(dbeta[u][e]);
      if (r16 == 0) atomicAdd(&sbeta[16 * (rt0 + u) + 4 * kq + e], s);
    }
  __syncthreads();
  if (tid < C && t0 + tid < T) {
    const int t = t0 + tid;
    if (direct)
      static_cast<InT*>(p.dbeta)[(size_t)(b * T + t) * HV + hv] = from_f32<InT>(sbeta[tid]);
    else
      w.part[((size_t)(b * T + t) * HV + hv) * (3 * K + 1) + 3 * K] = sbeta[tid];
  }
}

size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

size_t rec_floats(int K, int V) {
  const int el = 3 * C * K + C * V + 2 * C * C;
  return (size_t)((el + K + 63) / 64 * 64);
}

template <int K, int V, typename InT>
hipError_t cb_launch(const KdaBwdParams& p, const CbWs& w, hipStream_t s) {
  constexpr int dt = sizeof(InT) == 4 ? DT_F32 : (std::is_same<InT, bf16_t>::value ? DT_BF16 : DT_F16);
  const unsigned chunks = (unsigned)((size_t)p.B * p.HV * w.nt);
  const unsigned heads = (unsigned)((size_t)p.B * p.HV * (V / 64));
  hipLaunchKernelGGL((cb_prep_kernel<K, V, InT>), dim3(chunks), dim3(NTH), 0, s, p, w);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((cb_fwd_kernel<K, V>), dim3(heads), dim3(256), 0, s, p, w);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((cb_bwd_kernel<K, V, InT>), dim3(heads), dim3(256), 0, s, p, w);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((cb_grad_kernel<K, V, InT>), dim3(chunks), dim3(NTH), 0, s, p, w);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (w.part) {
    KdaBwdParams q = p;
    q.part = w.part;
    return kda_bwd_reduce_launch(q, V, dt, s);
  }
  return hipSuccess;
}

template <typename InT>
hipError_t cb_by_shape(const KdaBwdParams& p, const CbWs& w, hipStream_t s) {
  if (p.K == 128 && p.V == 128) return cb_launch<128, 128, InT>(p, w, s);
  if (p.K == 128 && p.V == 64) return cb_launch<128, 64, InT>(p, w, s);
  if (p.K == 64 && p.V == 128) return cb_launch<64, 128, InT>(p, w, s);
  return cb_launch<64, 64, InT>(p, w, s);
}

}  // namespace

static_assert(Rec<128, 128>::RS % 64 == 0 && Rec<64, 64>::RS % 64 == 0, "record alignment");

bool kda_chunk_bwd_supported(int K, int V, int dtype) {
  return dtype != DT_F64 && (K == 64 || K == 128) && (V == 64 || V == 128);
}

size_t kda_chunk_bwd_ws_bytes(int B, int T, int H, int HV, int K, int V) {
  const size_t nt = (size_t)(T + C - 1) / C;
  const size_t chunks = (size_t)B * HV * nt;
  size_t total = al256(chunks * rec_floats(K, V) * 4);
  total += 2 * al256(chunks * K * V * 4);
  total += 2 * al256(chunks * C * V * 4);
  if (HV != H) total += al256((size_t)B * T * HV * (3 * K + 1) * 4);
  return total;
}

hipError_t kda_chunk_bwd_dispatch(KdaBwdParams p, int dtype, void* ws, hipStream_t stream) {
  const int nt = (p.T + C - 1) / C;
  const size_t chunks = (size_t)p.B * p.HV * nt;
  char* base = static_cast<char*>(ws);
  CbWs w;
  w.nt = nt;
  w.rec = reinterpret_cast<float*>(base);
  base += al256(chunks * rec_floats(p.K, p.V) * 4);
  w.sn = reinterpret_cast<float*>(base);
  base += al256(chunks * p.K * p.V * 4);
  w.dsn = reinterpret_cast<float*>(base);
  base += al256(chunks * p.K * p.V * 4);
  w.vn = reinterpret_cast<float*>(base);
  base += al256(chunks * C * p.V * 4);
  w.dvn = reinterpret_cast<float*>(base);
  base += al256(chunks * C * p.V * 4);
  w.part = p.HV != p.H ? reinterpret_cast<float*>(base) : nullptr;
  if (dtype == DT_F32) return cb_by_shape<float>(p, w, stream);
  if (dtype == DT_BF16) return cb_by_shape<bf16_t>(p, w, stream);
  return cb_by_shape<_Float16>(p, w, stream);
}

}  // namespace kch
