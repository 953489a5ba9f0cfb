// Attention backward on MFMA for gfx950: the gradients of the joint
// softmax over compressed rows (HCA: every causal block; CSA: the selected
// blocks), window rows and the sink, with L2-normalised queries and keys
// (normalize_qk=True, |score| <= scale). Same algebra as the SIMT kernels of
// hca_backward.hip (ops_hca.py:132-194, ops_csa.py:869-1155 under autograd):
//   s = scale qn.k,  p = exp(s - lse),  dp = dout.k,  D = sum p dp,
//   ds = p (dp - D),  dqn = scale sum ds k,  dk += scale ds qn + p dout.
//
// Every product is a two-part bf16 split x = hi + lo (2^-16 relative) with
// three MFMAs, hi*hi + hi*lo + lo*hi, accumulated in fp32; the split rows
// (queries, dout, keys) are written once by split_rows_kernel.
//
// attn_bwd_q_kernel  one wave per query (4 per workgroup), all 16 heads as the
//   MFMA columns (MQA: every key row is shared by the heads). The query's keys
//   (selected or causal blocks, then window rows) are gathered 32 rows a step
//   into the wave's LDS stage (hi and lo tiles, swizzled as the forward's):
//   S^T = K Qn^T and dP^T = K dout^T per 16 rows. Pass 1: lse and D with a
//   running maximum; pass 2: ds, and dqn^T += K^T ds^T (K^T fragments from the
//   transposing LDS read, ds^T from the accumulators, as the forward's
//   O^T = V^T P^T). Writes dq (after the L2-norm backward), lse, D, and for
//   CSA each selected slot's gradient dotted with its row and their sum gsum.
// attn_bwd_k_kernel  one workgroup per 64 key rows (16 per wave) and chunk of
//   queries, key fragments held in registers; queries are taken in pairs: the
//   pair's qn and dout rows (32 rows of (query, head)) are staged in LDS once
//   for the four waves (double-buffered), S = Qn K^T and dP = dout K^T per
//   query, then dk += ds^T Qn + p^T dout with (query, head) as the
//   contraction (the accumulators of the two queries' S are the A operand in
//   the packed order of the transposing read of Qn / dout). Writes per-chunk
//   partials of the compressed rows and the window rows' gradient.
// The L2-norm and compression backwards are hca_backward.hip's block and
// window kernels on these partials (mfma_parts).

#include "attn_common.h"
#include "kch_csa.h"
#include "kch_kernels.h"

namespace kch {

namespace {

constexpr int KQC = 512;  // queries per chunk of the key pass (compressed rows)
constexpr int KTR = 64;   // key rows per key-pass workgroup

__device__ __forceinline__ bf16_t lo_of(float x) { return (bf16_t)(x - (float)(bf16_t)x); }

// acc + a * b with b exactly bf16 (its low part zero): al*bh + ah*bh
__device__ __forceinline__ f32x4 mfma2a(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}
// acc + a * b with a exactly bf16: ah*bl + ah*bh
__device__ __forceinline__ f32x4 mfma2b(const bf16x8& ah, const bf16x8& bh, const bf16x8& bl, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                       const bf16x8& bl, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}

// Four consecutive elements at element offset off of a row stored in dt
// (DT_F32 / DT_BF16 / DT_F16), as fp32, and the rounded store of four.
__device__ __forceinline__ float4 load4(const void* base, long long off, int dt) {
  if (dt == DT_F32) return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
  const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
  if (dt == DT_BF16)
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                       __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 h = __builtin_bit_cast(h4, r);
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}
__device__ __forceinline__ void store4(void* base, long long off, float4 v, int dt) {
  if (dt == DT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + off) = v;
  } else if (dt == DT_BF16) {
    bf16x4 h = {(bf16_t)v.x, (bf16_t)v.y, (bf16_t)v.z, (bf16_t)v.w};
    *reinterpret_cast<bf16x4*>(static_cast<bf16_t*>(base) + off) = h;
  } else {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    *reinterpret_cast<h4*>(static_cast<_Float16*>(base) + off) = h;
  }
}

// Rows of HD values, grouped nin to a group, into bf16 hi / lo rows grouped nout
// to a group (rows nin .. nout-1 of a group zero): x * f = hi + lo, f = 1 /
// max(|row|, 1e-12) with normalize (written to rinv per output row), else 1.
// Each lane splits 8 consecutive values (16-byte stores of hi and lo), HD / 8
// lanes per row; input in T (the rows as given: fp32, bf16 or fp16).
template <int HD, typename T>
__global__ __launch_bounds__(256) void split_rows_kernel(const T* x, long long ngroups, int nin,
                                                         int nout, bf16_t* hi, bf16_t* lo, float* rinv,
                                                         int normalize) {
  constexpr int LPR = HD / 8;  // lanes per row
  constexpr int RPB = 256 / LPR;
  const long long orow = (long long)blockIdx.x * RPB + threadIdx.x / LPR;
  const int lc = threadIdx.x % LPR;
  const bool act = orow < ngroups * nout;  // no early return: the row sum shuffles
  const long long g = act ? orow / nout : 0;
  const int r = act ? (int)(orow - g * nout) : nin;
  float v[8];
  if (r < nin) {
    Load8<T>::run(x + (g * nin + r) * HD + 8 * lc, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.f;
  }
  float f = 1.f;
  if (normalize) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
    f = r < nin ? l2_inv(ss) : 0.f;
  }
  if (!act) return;
  bf16x8 h, l;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = v[i] * f;
    h[i] = (bf16_t)y;
    l[i] = (bf16_t)(y - (float)h[i]);
  }
  *reinterpret_cast<bf16x8*>(hi + orow * HD + 8 * lc) = h;
  *reinterpret_cast<bf16x8*>(lo + orow * HD + 8 * lc) = l;
  if (rinv && lc == 0) rinv[orow] = f;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// sum over the 16 lanes of a DPP row; every lane of the row gets the total
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror: the other quad of the 8
  v += dpp_f<0x140>(v);  // row_mirror: the other 8 of the row
  return v;
}

template <int HD>
struct QWave {
  static constexpr int NS = HD / 32, NT = HD / 16;
  static constexpr int TPR = HD / 8, RPI = 64 / TPR, NLI = 32 / RPI;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct Rows {
    u32x4 h[NLI], l[NLI];
  };
};

// ---------------------------------------------------------------- query pass
// DL0: dout is exactly bf16 (bf16 input; its split's low part is zero), so
// the products with it take two MFMAs instead of three.
template <int HD, bool SPARSE, bool DL0>
__global__ __launch_bounds__(256, 2) void attn_bwd_q_kernel(HcaBwdParams p) {
  using W = QWave<HD>;
  constexpr int NS = W::NS, NT = W::NT, TPR = W::TPR, RPI = W::RPI, NLI = W::NLI;
  constexpr int TILE = 32 * HD;  // bf16 per 32-row tile
  __shared__ __attribute__((aligned(16))) bf16_t lds[4 * 2 * TILE];
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, q = lane >> 4, n = lane & 15;
  bf16_t* sth = lds + wv * 2 * TILE;  // this wave's hi and lo tiles
  bf16_t* stl = sth + TILE;
  const int tiles_per_b = (p.T + 3) / 4;
  const int b = blockIdx.x / tiles_per_b;
  const int t = (blockIdx.x - b * tiles_per_b) * 4 + wv;
  if (t >= p.T) return;  // whole waves: no workgroup barrier below
  const size_t bt = (size_t)b * p.T + t;
  const TileOffsets<HD> to;

  // B operands: qn and dout of head n, dims 32s + 8q .. (16 heads, padded rows zero)
  bf16x8 qh[NS], ql[NS], dh[NS], dl[NS];
  {
    const size_t ro = (bt * 16 + n) * HD + 8 * q;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qh[s] = *reinterpret_cast<const bf16x8*>(p.qs_hi + ro + 32 * s);
      ql[s] = *reinterpret_cast<const bf16x8*>(p.qs_lo + ro + 32 * s);
      dh[s] = *reinterpret_cast<const bf16x8*>(p.ds_hi + ro + 32 * s);
      dl[s] = DL0 ? bf16x8{} : *reinterpret_cast<const bf16x8*>(p.ds_lo + ro + 32 * s);
    }
  }
  const int nsel = SPARSE ? p.topk : min((t + 1) / p.m2, p.nb);
  const int i0 = p.win > 0 ? max(0, p.win - 1 - t) : 0;
  const int nwin = p.win > 0 ? p.win - i0 : 0;
  const int wpos0 = t - p.win + 1 + i0;
  // The compressed rows are padded to whole 32-row steps (masked), so that a
  // step reads only compressed or only window rows, each through a buffer
  // resource over this batch row's rows (hi and lo planes): an offset past its
  // end reads zeros, so a row address is one multiply-add and masked slots
  // need no readable default. Rows are taken in the score layout of
  // MqaWave::chunk_sl: slot k of lane group q is row row_sl(k, q) of the
  // step, whose scores the lane holds, so each lane masks its own scores
  // from the indices it loaded.
  using MW = MqaWave<HD>;
  constexpr int ROWB = HD * 2;
  const int nsel_pad = p.nb > 0 ? (nsel + 31) & ~31 : 0;
  const int nsteps = (nsel_pad + nwin + 31) / 32;
  const int lane_off = 16 * (lane % TPR);
  const int hmask = (TPR == 8 && ((lane >> 3) & 1)) ? -1 : 0;  // HD 64: slot i + 4
  auto rsrc = [](const bf16_t* base, long long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), 0, (int)bytes, 0x00020000);
  };
  const long long cbytes = (long long)p.nb * ROWB, wbytes = nwin > 0 ? (long long)p.T * ROWB : 0;
  const __amdgpu_buffer_rsrc_t rs_ch = rsrc(p.kc_hi + (size_t)b * p.nb * HD, cbytes);
  const __amdgpu_buffer_rsrc_t rs_cl = rsrc(p.kc_lo + (size_t)b * p.nb * HD, cbytes);
  const __amdgpu_buffer_rsrc_t rs_wh = rsrc(nwin > 0 ? p.kl_hi + (size_t)b * p.T * HD : p.kc_hi, wbytes);
  const __amdgpu_buffer_rsrc_t rs_wl = rsrc(nwin > 0 ? p.kl_lo + (size_t)b * p.T * HD : p.kc_lo, wbytes);
  const bool has_idx = SPARSE && nsel > 0;
  const __amdgpu_buffer_rsrc_t rs_idx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int*>(has_idx ? p.idx + bt * p.topk : nullptr), 0, has_idx ? nsel * 4 : 0, 0x00020000);
  const bool idx16 = (nsel & 3) == 0;  // 16-byte index loads never straddle the end
  const float sc = p.scale * kLog2eF;  // raw score -> log2 units

  // the row indices of step m: selected or causal block, or window position
  struct Sel {
    int v[8];
  };
  auto load_sel = [&](int m, Sel& sl) {
    const int j0 = 32 * m;
    if (__builtin_amdgcn_readfirstlane(j0 < nsel_pad ? 1 : 0)) {
      if (SPARSE) {
        if (idx16) {
          typedef int i32x4 __attribute__((ext_vector_type(4)));
          const i32x4 x = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, (j0 + 4 * q) * 4, 0, 0));
          const i32x4 y = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, (j0 + 16 + 4 * q) * 4, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sl.v[e] = x[e];
            sl.v[4 + e] = y[e];
          }
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k)
            sl.v[k] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_idx, (j0 + MW::row_sl(k, q)) * 4, 0, 0);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) sl.v[k] = j0 + MW::row_sl(k, q);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) sl.v[k] = wpos0 + (j0 - nsel_pad) + MW::row_sl(k, q);
    }
  };
  // gather the 32 rows of step m (hi and lo planes); ok[k]: slot k is a key
  auto gather = [&](int m, const Sel& sl, typename W::Rows& rr, bool (&ok)[8]) {
    const int j0 = 32 * m;
    const int ms = __builtin_amdgcn_readfirstlane(j0 < nsel_pad ? 1 : 0);
    const __amdgpu_buffer_rsrc_t rh = ms ? rs_ch : rs_wh;
    const __amdgpu_buffer_rsrc_t rl = ms ? rs_cl : rs_wl;
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      // (a select of values, not an indexed read: that would put sl in scratch memory)
      const int v = TPR == 8 ? sl.v[i] ^ ((sl.v[i] ^ sl.v[(i + 4) & 7]) & hmask) : sl.v[i];
      const int off = (int)((unsigned)v * ROWB + lane_off);
      rr.h[i] = __builtin_amdgcn_raw_buffer_load_b128(rh, off, 0, 0);
      rr.l[i] = __builtin_amdgcn_raw_buffer_load_b128(rl, off, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = j0 + MW::row_sl(k, q);
      const bool okc = (j < nsel) & ((unsigned)sl.v[k] < (unsigned)p.nb);
      const bool okw = j - nsel_pad < nwin;
      ok[k] = ms ? okc : okw;
    }
  };
  auto stage = [&](const typename W::Rows& rr) {
    wave_lds_sync();  // the previous step's reads are done
#pragma unroll
    for (int i = 0; i < NLI; ++i) {
      const int r = MW::row_sl(MW::slot_sl(i), q), c = lane % TPR;
      const int off = r * HD + 8 * (c ^ tile_swz<HD>(r & 15));
      *reinterpret_cast<typename W::u32x4*>(sth + off) = rr.h[i];
      *reinterpret_cast<typename W::u32x4*>(stl + off) = rr.l[i];
    }
    wave_lds_sync();
  };
  // S^T (log2 units) and dP^T of the staged 32 rows: sc8 / dp8 for keys 4q+e, 16+4q+e of head n
  auto scores = [&](const bool (&ok)[8], float (&s8)[8], float (&d8)[8]) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bf16x8 kh = *reinterpret_cast<const bf16x8*>(sth + 16 * HD * half + to.key(s));
        const bf16x8 kl = *reinterpret_cast<const bf16x8*>(stl + 16 * HD * half + to.key(s));
        sa = mfma3(kh, kl, qh[s], ql[s], sa);
        da = DL0 ? mfma2a(kh, kl, dh[s], da) : mfma3(kh, kl, dh[s], dl[s], da);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s8[4 * half + e] = ok[4 * half + e] ? sa[e] * sc : -INFINITY;
        d8[4 * half + e] = da[e];
      }
    }
  };

  // ---- pass 1: lse (log2 units) and D = sum p dp, running maximum per head ----
  float m = -INFINITY, l = 0.f, ad = 0.f;
  {
    typename W::Rows rr;
    Sel sl;
    bool okn[8];
    if (nsteps > 0) {
      load_sel(0, sl);
      gather(0, sl, rr, okn);
      load_sel(1, sl);
    }
    for (int st = 0; st < nsteps; ++st) {
      stage(rr);
      bool ok[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) ok[k] = okn[k];
      if (st + 1 < nsteps) {
        gather(st + 1, sl, rr, okn);
        load_sel(st + 2, sl);
      }
      float s8[8], d8[8];
      scores(ok, s8, d8);
      float mx = s8[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = fmaxf(mx, s8[e]);
      const float mn = fmaxf(m, colq_max(mx));
      if (mn > m) {
        const float a = fast_exp2(m - mn);  // m = -inf: a = 0
        l *= a;
        ad *= a;
        m = mn;
      }
      if (m > -INFINITY) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = fast_exp2(s8[e] - m);  // masked: 0
          l += pe;
          ad += pe * d8[e];
        }
      }
    }
  }
  l = colq_sum(l);
  ad = colq_sum(ad);
  float sk2 = -INFINITY;
  if (p.sink && n < p.nh) sk2 = p.sink[n] * kLog2eF;
  if (sk2 > -INFINITY) {
    const float mn = fmaxf(m, sk2);
    const float a = fast_exp2(m - mn);
    l = l * a + fast_exp2(sk2 - mn);
    ad *= a;
    m = mn;
  }
  const bool live = n < p.nh && l > 0.f;
  const float lse2 = live ? m + __log2f(l) : INFINITY;
  const float D = live ? ad / l : 0.f;

  // ---- pass 2: ds, dqn^T += K^T ds^T, the slot terms ----
  f32x4 dq[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) dq[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float psel = 0.f, dssel = 0.f;  // sums over the selected slots (gsum)
  {
    typename W::Rows rr;
    Sel sl;
    bool okn[8];
    if (nsteps > 0) {
      load_sel(0, sl);
      gather(0, sl, rr, okn);
      load_sel(1, sl);
    }
    for (int st = 0; st < nsteps; ++st) {
      stage(rr);
      bool ok[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) ok[k] = okn[k];
      if (st + 1 < nsteps) {
        gather(st + 1, sl, rr, okn);
        load_sel(st + 2, sl);
      }
      float s8[8], d8[8];
      scores(ok, s8, d8);
      float pe[8], dse[8];
      bf16x8 bh, bl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pe[e] = fast_exp2(s8[e] - lse2);  // masked or dead head: 0
        dse[e] = pe[e] * (d8[e] - D) * p.scale;
        bh[e] = (bf16_t)dse[e];
        bl[e] = lo_of(dse[e]);
      }
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        const bf16x8 vh = MqaWave<HD>::vt_frag(sth, to, tt);
        const bf16x8 vl = MqaWave<HD>::vt_frag(stl, to, tt);
        dq[tt] = mfma3(vh, vl, bh, bl, dq[tt]);
      }
      if constexpr (SPARSE) {
        // the selected rows: sum over the heads of p ((dp - D) s + dp) (the row's
        // gradient dotted with the row) per slot, and this head's p and ds sums
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * st + 16 * (e >> 2) + 4 * q + (e & 3);
          const bool selk = j < nsel;
          const float sraw = s8[e] > -INFINITY ? s8[e] / kLog2eF : 0.f;  // scale qn.k
          float g = selk ? pe[e] * ((d8[e] - D) * sraw + d8[e]) : 0.f;
          g = row16_sum(g);
          if (selk) {
            psel += pe[e];
            dssel += dse[e];
          }
          // (added: calls for further groups of heads add theirs; one wave owns the slot)
          if (n == 0 && selk && p.slot_grad) p.slot_grad[bt * p.topk + j] += g;
        }
      }
    }
  }

  // ---- dq: the L2-norm backward of qn (lane: head n, dims 16 tt + 4q + e) ----
  {
    const float rq = p.rq[bt * 16 + n];
    float qv[NT][4];
    float yd = 0.f;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (n < p.nh) x = load4(p.q, (bt * p.nh + n) * HD + 16 * tt + 4 * q, p.qdt);
      qv[tt][0] = x.x * rq; qv[tt][1] = x.y * rq; qv[tt][2] = x.z * rq; qv[tt][3] = x.w * rq;
#pragma unroll
      for (int e = 0; e < 4; ++e) yd += qv[tt][e] * dq[tt][e];
    }
    yd = colq_sum(yd);
    if (n < p.nh) {
      // rq = 1 / max(|q|, eps): for |q| <= eps the norm is the constant eps
      const bool big = rq < 1e12f;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (big ? dq[tt][e] - qv[tt][e] * yd : dq[tt][e]) * rq;
        store4(p.dq, (bt * p.nh + n) * HD + 16 * tt + 4 * q, make_float4(o[0], o[1], o[2], o[3]), p.qdt);
      }
    }
    if (q == 0) {
      p.lse[bt * 16 + n] = lse2;
      p.dval[bt * 16 + n] = D;
      if (p.sink_part && n < p.nh) p.sink_part[bt * p.nh + n] = p.sink ? fast_exp2(sk2 - lse2) * D : 0.f;
    }
  }
  if constexpr (SPARSE) {
    if (p.gsum) {
      // gsum = sum over the heads of dssel qn + psel dout (dims 32s + 8q + i)
      psel = colq_sum(psel);
      dssel = colq_sum(dssel);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        float gv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float qv = (float)qh[s][i] + (float)ql[s][i];
          const float dv = (float)dh[s][i] + (float)dl[s][i];
          gv[i] = row16_sum(dssel * qv + psel * dv);
        }
        if (n == 0) {
          float* dst = p.gsum + bt * HD + 32 * s + 8 * q;
          *reinterpret_cast<float4*>(dst) = make_float4(gv[0], gv[1], gv[2], gv[3]);
          *reinterpret_cast<float4*>(dst + 4) = make_float4(gv[4], gv[5], gv[6], gv[7]);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ key pass
// MODE 0: compressed rows (HCA: visible when n < (t+1) / m2; CSA: selected),
// chunk ci of KQC queries; MODE 1: window rows (row u seen by t in [u, u + win)).
template <int HD, int MODE, bool DL0>
__global__ __launch_bounds__(256, 2) void attn_bwd_k_kernel(HcaBwdParams p, int nchunk) {
  constexpr int NS = HD / 32, NT = HD / 16;
  constexpr int TILE = 32 * HD;
  constexpr int CPR = HD / 8;                 // 16-byte chunks per row
  constexpr int LPT = 4 * TILE / 8 / 256;     // 16-byte pieces per thread per pair
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][4 * TILE];  // q hi, q lo, d hi, d lo
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, q = lane >> 4, n = lane & 15;
  const int b = blockIdx.y;
  const int nrows = MODE == 0 ? p.nb : p.T;
  const int tile = MODE == 0 ? blockIdx.x / nchunk : blockIdx.x;
  const int ci = MODE == 0 ? blockIdx.x - tile * nchunk : 0;
  const int r0 = tile * KTR;
  int tlo, thi;
  if constexpr (MODE == 0) {
    tlo = max(ci * KQC, (r0 + 1) * p.m2 - 1);
    thi = min(p.T, (ci + 1) * KQC);
  } else {
    tlo = r0;
    thi = min(p.T, r0 + KTR + p.win - 1);
  }
  if (tlo >= thi) return;  // no row of the tile is seen by this chunk (nothing to write)
  const int rk = r0 + 16 * wv + n;  // this lane's key row (B operand column)
  const bool rk_ok = rk < nrows;
  const TileOffsets<HD> to;

  // key fragments (B operand of S = Qn K^T): row rk, dims 32s + 8q ..
  bf16x8 kh[NS], kl[NS];
  {
    const bf16_t* bh = MODE == 0 ? p.kc_hi + (size_t)b * p.nb * HD : p.kl_hi + (size_t)b * p.T * HD;
    const bf16_t* bl = MODE == 0 ? p.kc_lo + (size_t)b * p.nb * HD : p.kl_lo + (size_t)b * p.T * HD;
    const size_t ro = (size_t)(rk_ok ? rk : 0) * HD + 8 * q;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      kh[s] = *reinterpret_cast<const bf16x8*>(bh + ro + 32 * s);
      kl[s] = *reinterpret_cast<const bf16x8*>(bl + ro + 32 * s);
      if (!rk_ok) kh[s] = kl[s] = bf16x8{};
    }
  }
  f32x4 dk[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) dk[tt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // staging of a query pair (t, t + 1): 4 tiles of 32 rows (query, head), row
  // 16 i + h = head h of query t + i; piece k of the thread: tile k / (LPT / 4)
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  auto fetch = [&](int tp, u32x4 (&v)[LPT]) {
#pragma unroll
    for (int k = 0; k < LPT; ++k) {
      const int pc = tid + 256 * k;              // piece index within the 4 tiles
      const int tl = pc / (TILE / 8);            // tile 0..3
      const int w = pc - tl * (TILE / 8);
      const int row = w / CPR, c = w % CPR;      // row 0..31
      const int tq = min(tp + (row >> 4), p.T - 1);
      const bf16_t* src = tl == 0 ? p.qs_hi : tl == 1 ? p.qs_lo : tl == 2 ? p.ds_hi : p.ds_lo;
      v[k] = *reinterpret_cast<const u32x4*>(src + (((size_t)b * p.T + tq) * 16 + (row & 15)) * HD + 8 * c);
    }
  };
  auto put = [&](bf16_t* buf, const u32x4 (&v)[LPT]) {
#pragma unroll
    for (int k = 0; k < LPT; ++k) {
      const int pc = tid + 256 * k;
      const int tl = pc / (TILE / 8);
      const int w = pc - tl * (TILE / 8);
      const int row = w / CPR, c = w % CPR;
      *reinterpret_cast<u32x4*>(buf + tl * TILE + row * HD + 8 * (c ^ tile_swz<HD>(row & 15))) = v[k];
    }
  };
  const int nw = (p.nb + 31) / 32;
  auto visible = [&](int tq) -> bool {
    if (tq >= thi || !rk_ok) return false;  // (the pair's second query may lie past the chunk)
    if constexpr (MODE == 1) return tq >= rk && tq < rk + p.win;
    if (p.sel) return (p.sel[((size_t)b * p.T + tq) * nw + (rk >> 5)] >> (rk & 31)) & 1u;
    return rk < (tq + 1) / p.m2;
  };

  u32x4 pv[LPT];
  fetch(tlo, pv);
  put(lds[0], pv);
  __syncthreads();
  int buf = 0;
  for (int tp = tlo; tp < thi; tp += 2) {
    const bool more = tp + 2 < thi;
    if (more) fetch(tp + 2, pv);
    const bf16_t* qs_h = lds[buf];
    const bf16_t* qs_l = lds[buf] + TILE;
    const bf16_t* ds_h = lds[buf] + 2 * TILE;
    const bf16_t* ds_l = lds[buf] + 3 * TILE;
    bf16x8 ash, asl, aph, apl;  // ds^T and p^T: key n, slots (query i, heads 4q .. 4q+3)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int tq = tp + i;
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, da = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int ko = 16 * HD * i + to.key(s);
        const bf16x8 xh = *reinterpret_cast<const bf16x8*>(qs_h + ko);
        const bf16x8 xl = *reinterpret_cast<const bf16x8*>(qs_l + ko);
        const bf16x8 yh = *reinterpret_cast<const bf16x8*>(ds_h + ko);
        sa = mfma3(xh, xl, kh[s], kl[s], sa);
        if constexpr (DL0) {
          da = mfma2b(yh, kh[s], kl[s], da);
        } else {
          const bf16x8 yl = *reinterpret_cast<const bf16x8*>(ds_l + ko);
          da = mfma3(yh, yl, kh[s], kl[s], da);
        }
      }
      // lane: heads 4q .. 4q+3 of query tq, key rk
      const bool vis = visible(tq);
      const size_t li = ((size_t)b * p.T + min(tq, p.T - 1)) * 16 + 4 * q;
      const float4 L4 = *reinterpret_cast<const float4*>(p.lse + li);
      const float4 D4 = *reinterpret_cast<const float4*>(p.dval + li);
      const float Ls[4] = {L4.x, L4.y, L4.z, L4.w}, Ds[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pe = vis ? fast_exp2(sa[e] * p.scale * kLog2eF - Ls[e]) : 0.f;
        const float dse = pe * (da[e] - Ds[e]) * p.scale;
        ash[4 * i + e] = (bf16_t)dse;
        asl[4 * i + e] = lo_of(dse);
        aph[4 * i + e] = (bf16_t)pe;
        apl[4 * i + e] = lo_of(pe);
      }
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const bf16x8 bqh = MqaWave<HD>::vt_frag(qs_h, to, tt);
      const bf16x8 bql = MqaWave<HD>::vt_frag(qs_l, to, tt);
      const bf16x8 bdh = MqaWave<HD>::vt_frag(ds_h, to, tt);
      dk[tt] = mfma3(ash, asl, bqh, bql, dk[tt]);
      if constexpr (DL0) {
        dk[tt] = mfma2a(aph, apl, bdh, dk[tt]);
      } else {
        const bf16x8 bdl = MqaWave<HD>::vt_frag(ds_l, to, tt);
        dk[tt] = mfma3(aph, apl, bdh, bdl, dk[tt]);
      }
    }
    if (more) put(lds[buf ^ 1], pv);
    __syncthreads();
    buf ^= 1;
  }
  // dk tile tt: rows (keys) 16 wv + 4q + e of the tile, column (dim) 16 tt + n
  float* out = MODE == 0 ? p.part_b + (((size_t)b * nchunk + ci) * p.nb) * HD
                         : p.part_w + (size_t)b * p.T * HD;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = r0 + 16 * wv + 4 * q + e;
    if (r < nrows) {
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) out[(size_t)r * HD + 16 * tt + n] = dk[tt][e];
    }
  }
}

}  // namespace

bool attn_bwd_mfma_supported(const HcaBwdParams& p) {
  return p.normalize && (p.c == 64 || p.c == 128) && p.nh >= 1 && p.nh <= 16;
}

static size_t al256m(size_t x) { return (x + 255) & ~size_t(255); }

size_t attn_bwd_mfma_ws_bytes(int B, int T, int c, int m2, int win, int topk) {
  const size_t BT = (size_t)B * T;
  const int nb = T / m2;
  const int nchunk = (T + KQC - 1) / KQC;
  size_t z = 3 * al256m(BT * 16 * 4);                  // lse, D, 1/|q| (16 heads)
  z += 4 * al256m(BT * 16 * c * 2);                     // qn, dout hi / lo
  z += 2 * al256m((size_t)B * nb * c * 2);              // compressed rows hi / lo
  if (win > 0) z += 2 * al256m(BT * c * 2);             // window rows hi / lo
  z += al256m((size_t)B * nchunk * nb * c * 4);         // compressed-row partials
  if (win > 0) z += al256m(BT * c * 4);                 // window-row gradients
  if (topk > 0) z += al256m(BT * ((nb + 31) / 32) * 4);  // selection bitmap
  return z;
}

hipError_t sel_bitmap_launch(const int* idx, uint32_t* sel, long long nq, int topk, int nw, hipStream_t s);
hipError_t hca_bwd_finish_launch(const HcaBwdParams& p, int nchunk, hipStream_t s);

hipError_t attn_bwd_mfma_dispatch(HcaBwdParams p, void* ws, hipStream_t s) {
  const int HD = p.c;
  const size_t BT = (size_t)p.B * p.T;
  const int nchunk = (p.T + KQC - 1) / KQC;
  char* w = static_cast<char*>(ws);
  auto take = [&](size_t bytes) {
    char* r = w;
    w += al256m(bytes);
    return r;
  };
  p.lse = reinterpret_cast<float*>(take(BT * 16 * 4));
  p.dval = reinterpret_cast<float*>(take(BT * 16 * 4));
  p.rq = reinterpret_cast<float*>(take(BT * 16 * 4));
  p.qs_hi = reinterpret_cast<bf16_t*>(take(BT * 16 * HD * 2));
  p.qs_lo = reinterpret_cast<bf16_t*>(take(BT * 16 * HD * 2));
  p.ds_hi = reinterpret_cast<bf16_t*>(take(BT * 16 * HD * 2));
  p.ds_lo = reinterpret_cast<bf16_t*>(take(BT * 16 * HD * 2));
  p.kc_hi = reinterpret_cast<bf16_t*>(take((size_t)p.B * p.nb * HD * 2));
  p.kc_lo = reinterpret_cast<bf16_t*>(take((size_t)p.B * p.nb * HD * 2));
  p.kl_hi = p.kl_lo = nullptr;
  if (p.win > 0) {
    p.kl_hi = reinterpret_cast<bf16_t*>(take(BT * HD * 2));
    p.kl_lo = reinterpret_cast<bf16_t*>(take(BT * HD * 2));
  }
  p.part_b = reinterpret_cast<float*>(take((size_t)p.B * nchunk * p.nb * HD * 4));
  p.part_w = p.win > 0 ? reinterpret_cast<float*>(take(BT * HD * 4)) : nullptr;
  p.sel = nullptr;
  if (p.idx && p.topk > 0) {
    const int nw = (p.nb + 31) / 32;
    uint32_t* sel = reinterpret_cast<uint32_t*>(take(BT * nw * 4));
    hipError_t e = fill_u32(sel, (long long)BT * nw, 0u, s);
    if (e != hipSuccess) return e;
    e = sel_bitmap_launch(p.idx, sel, (long long)BT, p.topk, nw, s);
    if (e != hipSuccess) return e;
    p.sel = sel;
  }
  p.mfma_parts = 1;
  p.part_qc = KQC;
  // split_rows_kernel: 256 / (HD / 8) rows per workgroup
  auto grid_rows = [](long long rows, int hd) {
    const long long rpb = 256 / (hd / 8);
    return dim3((unsigned)((rows + rpb - 1) / rpb));
  };
#define KCH_SPLIT_Q(HDV, QT)                                                                       \
  do {                                                                                             \
    hipLaunchKernelGGL((split_rows_kernel<HDV, QT>), grid_rows((long long)BT * 16, HDV), dim3(256), 0, \
                       s, static_cast<const QT*>(p.q), (long long)BT, p.nh, 16, p.qs_hi, p.qs_lo, p.rq, 1); \
    hipLaunchKernelGGL((split_rows_kernel<HDV, QT>), grid_rows((long long)BT * 16, HDV), dim3(256), 0, \
                       s, static_cast<const QT*>(p.dout), (long long)BT, p.nh, 16, p.ds_hi, p.ds_lo,  \
                       (float*)nullptr, 0);                                                        \
  } while (0)
#define KCH_SPLIT(HDV)                                                                              \
  do {                                                                                              \
    if (p.qdt == DT_BF16)                                                                           \
      KCH_SPLIT_Q(HDV, bf16_t);                                                                     \
    else if (p.qdt == DT_F16)                                                                       \
      KCH_SPLIT_Q(HDV, _Float16);                                                                   \
    else                                                                                            \
      KCH_SPLIT_Q(HDV, float);                                                                      \
    if (p.nb > 0)                                                                                   \
      hipLaunchKernelGGL((split_rows_kernel<HDV, float>), grid_rows((long long)p.B * p.nb, HDV),    \
                         dim3(256), 0, s, p.kc, (long long)p.B * p.nb, 1, 1, p.kc_hi, p.kc_lo,      \
                         (float*)nullptr, 0);                                                       \
    if (p.win > 0)                                                                                  \
      hipLaunchKernelGGL((split_rows_kernel<HDV, float>), grid_rows((long long)BT, HDV), dim3(256), \
                         0, s, p.kl, (long long)BT, 1, 1, p.kl_hi, p.kl_lo, (float*)nullptr, 0);    \
  } while (0)
#define KCH_PASSES_D(HDV, DL)                                                                      \
  do {                                                                                             \
    const unsigned qg = (unsigned)(p.B * ((p.T + 3) / 4));                                         \
    if (p.sparse)                                                                                  \
      hipLaunchKernelGGL((attn_bwd_q_kernel<HDV, true, DL>), dim3(qg), dim3(256), 0, s, p);        \
    else                                                                                           \
      hipLaunchKernelGGL((attn_bwd_q_kernel<HDV, false, DL>), dim3(qg), dim3(256), 0, s, p);       \
    if (p.nb > 0 && !(p.sparse && p.topk == 0)) {                                                  \
      const int ntile = (p.nb + KTR - 1) / KTR;                                                    \
      hipLaunchKernelGGL((attn_bwd_k_kernel<HDV, 0, DL>), dim3(ntile * nchunk, p.B), dim3(256), 0, s, \
                         p, nchunk);                                                               \
    }                                                                                              \
    if (p.win > 0)                                                                                 \
      hipLaunchKernelGGL((attn_bwd_k_kernel<HDV, 1, DL>), dim3((p.T + KTR - 1) / KTR, p.B), dim3(256), \
                         0, s, p, nchunk);                                                         \
  } while (0)
#define KCH_PASSES(HDV)                                                                            \
  do {                                                                                             \
    if (p.qdt == DT_BF16)                                                                          \
      KCH_PASSES_D(HDV, true);                                                                     \
    else                                                                                           \
      KCH_PASSES_D(HDV, false);                                                                    \
  } while (0)
  if (HD == 64) {
    KCH_SPLIT(64);
    KCH_PASSES(64);
  } else {
    KCH_SPLIT(128);
    KCH_PASSES(128);
  }
#undef KCH_SPLIT
#undef KCH_SPLIT_Q
#undef KCH_PASSES
#undef KCH_PASSES_D
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.nb > 0 && p.sparse && p.topk == 0) {
    // no selection: the compressed rows receive nothing
    e = fill_u32(p.part_b, (long long)p.B * nchunk * p.nb * HD, 0u, s);
    if (e != hipSuccess) return e;
  }
  return hca_bwd_finish_launch(p, nchunk, s);
}

}  // namespace kch
