// HCA attention backward for gfx950: the gradients of hca_core
// (/root/reference/ops_hca.py:132-194, differentiated by autograd in the
// reference) with respect to the queries, the compression inputs C, Z,
// B_pos, the window rows and the sink logits. fp32 throughout.
//
// Forward per query (b, t) and head h: qn = q / |q|; keys (= values) are the
// L2-normalised compressed rows kc_n of the blocks the query sees
// (n < (t+1) / m2) and the L2-normalised window rows kl_u (t-w < u <= t);
// p = softmax over scale qn.k and the sink logit; out = sum p_j k_j.
// Backward: dp_j = dout . k_j, D = sum p_j dp_j, ds_j = p_j (dp_j - D),
//   dqn = scale sum ds_j k_j,   dk_j += scale ds_j qn + p_j dout,
//   dsink = -sum p_sink D;
// then the L2-norm backward (dx = (dy - y (y.dy)) / |x|) and the compression
// backward (w = softmax over the block's tokens of Z + B_pos, per channel;
// dC = w dr, dZ = w (C - r) dr).
//
// hca_bwd_query_kernel  one workgroup per (b, t); thread (head, 8-channel
//   group). Pass A over the query's keys: running max, sum and sum p dp
//   (lse and D); pass B: dqn, then dq. Writes lse, D, 1/|q| per (t, h), and
//   for CSA the selected slots' row gradients: each one dotted with its row
//   (slot_grad) and their sum over the slots (gsum: per head the selected
//   p and ds sums times dout and qn, summed over the heads in LDS).
// hca_bwd_key_kernel    one workgroup per (tile of NBT key rows, chunk of up
//   to QC queries, b): each query row (q, dout, lse, D) is read once for the
//   NBT keys; the heads' sums meet in LDS; one partial gradient per key row
//   and chunk. Mode 0: compressed rows (queries from (n+1) m2 - 1 on);
//   mode 1: window rows (queries u .. u + w - 1).
// hca_bwd_block_kernel  one workgroup per (b, block): sums the chunks, the
//   L2-norm backward of the compressed row, the compression backward.
// hca_bwd_window_kernel one workgroup per (b, token): the window row's
//   L2-norm backward, added to dC (or written to dlocal).

#include "kch_csa.h"
#include "kch_device.h"
#include "kch_kernels.h"

namespace kch {

namespace {

constexpr int NBT = 8;    // key rows per key-kernel tile
constexpr int QC = 512;   // queries per key-kernel chunk
constexpr float kEps = 1e-12f;

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// sum over the L lanes of a head group (L = 8 or 16, aligned); every lane of
// the group gets the total
template <int L>
__device__ __forceinline__ float hsum(float v) {
  v += dppf<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dppf<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dppf<0x141>(v);  // row_half_mirror: the other quad of the 8
  if constexpr (L == 16) v += dppf<0x140>(v);  // row_mirror: the other 8 of the row
  return v;
}

__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <int HD>
__global__ __launch_bounds__(256) void hca_bwd_query_kernel(HcaBwdParams p) {
  constexpr int LPH = HD / 8;
  const int tid = threadIdx.x, h = tid / LPH, lc = tid % LPH;
  const bool act = h < p.nh;
  const int hh = act ? h : 0;
  const size_t bt = blockIdx.x;
  const int b = (int)(bt / p.T), t = (int)(bt % p.T);
  const size_t qoff = (bt * p.nh + hh) * HD + 8 * lc;
  float qn[8], dv[8];
  load8(static_cast<const float*>(p.q) + qoff, qn);
  load8(static_cast<const float*>(p.dout) + qoff, dv);
  if (!act) {
#pragma unroll
    for (int e = 0; e < 8; ++e) qn[e] = dv[e] = 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += qn[e] * qn[e];
  const float nrm = sqrtf(hsum<LPH>(ss));
  const float rq = p.normalize ? 1.f / fmaxf(nrm, kEps) : 1.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) qn[e] *= rq;

  // keys: the selected blocks (CSA; the selection's -1 slots are skipped) or
  // every block the query sees (HCA), then the window rows
  const int* sel_row = p.idx ? p.idx + bt * p.topk : nullptr;
  const int nvis = p.sparse ? p.topk : min((t + 1) / p.m2, p.nb);
  const int i0 = p.win > 0 ? max(0, p.win - 1 - t) : 0;
  const int nwin = p.win > 0 ? p.win - i0 : 0;
  const int nk = nvis + nwin;
  const int wpos0 = t - p.win + 1 + i0;  // first window position
  // (an unused selection slot points at row 0 and is masked by kvalid)
  auto kblock = [&](int j) { return sel_row ? max(sel_row[j], 0) : j; };
  auto kvalid = [&](int j) { return j >= nvis || !sel_row || sel_row[j] >= 0; };
  auto krow = [&](int j) -> const float* {
    return j < nvis ? p.kc + ((size_t)b * p.nb + kblock(j)) * HD + 8 * lc
                    : p.kl + ((size_t)b * p.T + wpos0 + (j - nvis)) * HD + 8 * lc;
  };
  auto score = [&](const float* k, float& s, float& dp) {
    float a = 0.f, c = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a += qn[e] * k[e];
      c += dv[e] * k[e];
    }
    s = hsum<LPH>(a) * p.scale;
    dp = hsum<LPH>(c);
  };

  // pass A: lse and D = sum p dp (the sink's value is zero). Key rows are
  // requested PD steps ahead (a ring of PD registers sets).
  constexpr int PD = 4;
  float m = -INFINITY, l = 0.f, ad = 0.f;
  float kb[PD][8];
#pragma unroll
  for (int u = 0; u < PD; ++u)
    if (u < nk) load8(krow(u), kb[u]);
  for (int j0 = 0; j0 < nk; j0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int j = j0 + u;
      if (j < nk) {
        float s, dp;
        score(kb[u], s, dp);
        if (j + PD < nk) load8(krow(j + PD), kb[u]);
        if (kvalid(j)) {
          const float mn = fmaxf(m, s);
          const float a = expf(m - mn), e1 = expf(s - mn);
          l = l * a + e1;
          ad = ad * a + e1 * dp;
          m = mn;
        }
      }
    }
  }
  float sk = 0.f;
  if (p.sink) {
    sk = p.sink[hh];
    const float mn = fmaxf(m, sk);
    const float a = expf(m - mn);
    l = l * a + expf(sk - mn);
    ad *= a;
    m = mn;
  }
  const float lse = l > 0.f ? m + logf(l) : INFINITY;
  const float D = l > 0.f ? ad / l : 0.f;

  // pass B: dqn = scale sum ds_j k_j
  float dq[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dq[e] = 0.f;
  float psel = 0.f, dssel = 0.f;  // sums over the selected slots of p and scale p (dp - D)
#pragma unroll
  for (int u = 0; u < PD; ++u)
    if (u < nk) load8(krow(u), kb[u]);
  for (int j0 = 0; j0 < nk; j0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int j = j0 + u;
      if (j < nk) {
        float s, dp;
        score(kb[u], s, dp);
        const float pj = kvalid(j) ? expf(s - lse) : 0.f;
        const float ds = pj * (dp - D) * p.scale;
#pragma unroll
        for (int e = 0; e < 8; ++e) dq[e] += ds * kb[u][e];
        if (j + PD < nk) load8(krow(j + PD), kb[u]);
        // the selected row's gradient dotted with the row, this head's share:
        // (scale p (dp - D) qn + p dout) . k = p ((dp - D) s + dp); the heads
        // add into slot_grad (zeroed by the caller)
        if (p.slot_grad && act && lc == 0 && j < nvis && kvalid(j))
          atomicAdd(p.slot_grad + bt * p.topk + j, pj * ((dp - D) * s + dp));
        if (j < nvis && kvalid(j)) {
          psel += pj;
          dssel += ds;
        }
      }
    }
  }
  if (p.gsum) {
    // sum over the selected slots of the rows' gradients, scale ds_j qn + p_j dout,
    // over all heads: sum_h (dssel_h qn_h + psel_h dout_h)
    __shared__ float gs[HD];
    for (int i = tid; i < HD; i += 256) gs[i] = 0.f;
    __syncthreads();
    if (act) {
#pragma unroll
      for (int e = 0; e < 8; ++e) atomicAdd(&gs[8 * lc + e], dssel * qn[e] + psel * dv[e]);
    }
    __syncthreads();
    for (int i = tid; i < HD; i += 256) p.gsum[bt * HD + i] = gs[i];
  }
  // L2-norm backward of the query row
  float yd = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) yd += qn[e] * dq[e];
  yd = hsum<LPH>(yd);
  if (act) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = p.normalize ? (nrm > kEps ? dq[e] - qn[e] * yd : dq[e]) * rq : dq[e];
    float* dst = static_cast<float*>(p.dq) + qoff;
    *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
    if (lc == 0) {
      const size_t i = bt * p.nh + h;
      p.lse[i] = lse;
      p.dval[i] = D;
      p.rq[i] = rq;
      if (p.sink_part) p.sink_part[i] = p.sink ? expf(sk - lse) * D : 0.f;
    }
  }
}

template <int HD>
__global__ __launch_bounds__(256) void hca_bwd_key_kernel(HcaBwdParams p, int mode, int nchunk, int ntile) {
  constexpr int LPH = HD / 8;
  constexpr int HS = 256 / LPH;  // head slots
  __shared__ float red[NBT][HS][HD];
  const int tid = threadIdx.x, h = tid / LPH, lc = tid % LPH;
  const bool act = h < p.nh;
  const int hh = act ? h : 0;
  const int b = blockIdx.y;
  const int tile = blockIdx.x / nchunk, ci = blockIdx.x % nchunk;
  const int r0 = tile * NBT;
  const int nrows = mode == 0 ? p.nb : p.T;
  const int rl = min(r0 + NBT, nrows) - 1;
  auto lo = [&](int r) { return mode == 0 ? (r + 1) * p.m2 - 1 : r; };
  auto hi = [&](int r) { return mode == 0 ? p.T : min(p.T, r + p.win); };
  const int tlo = lo(r0) + ci * QC;
  const int thi = min(hi(rl), tlo + QC);
  float* out = (mode == 0 ? p.part_b : p.part_w) + (((size_t)b * ntile + tile) * nchunk + ci) * NBT * HD;
  if (tlo >= thi) {
    for (int i = tid; i < NBT * HD; i += 256) out[i] = 0.f;
    return;
  }
  float k[NBT][8], acc[NBT][8];
#pragma unroll
  for (int i = 0; i < NBT; ++i) {
    const int r = r0 + i;
    if (r < nrows) {
      load8((mode == 0 ? p.kc + ((size_t)b * p.nb + r) * HD : p.kl + ((size_t)b * p.T + r) * HD) + 8 * lc,
            k[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) k[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
  }
  const int nw = (p.nb + 31) / 32;  // selection bitmap words per query
  // the next query's row, scalars and selection word are requested while the
  // current one is processed
  struct QRow {
    float q[8], d[8];
    float rq, lse, D;
    uint32_t sel;
  };
  auto fetch = [&](int t, QRow& r) {
    const size_t i0 = ((size_t)b * p.T + t) * p.nh + hh;
    load8(static_cast<const float*>(p.q) + i0 * HD + 8 * lc, r.q);
    load8(static_cast<const float*>(p.dout) + i0 * HD + 8 * lc, r.d);
    r.rq = p.rq[i0];
    r.lse = p.lse[i0];
    r.D = p.dval[i0];
    r.sel = 0xffffffffu;
    if (mode == 0 && p.sel) {
      // CSA: the tile's rows this query selected (NBT consecutive bits of one word)
      r.sel = p.sel[((size_t)b * p.T + t) * nw + (r0 >> 5)] >> (r0 & 31);
    }
  };
  QRow nx;
  fetch(tlo, nx);
  for (int t = tlo; t < thi; ++t) {
    const QRow cur = nx;
    if (t + 1 < thi) fetch(t + 1, nx);
    const uint32_t selbits = cur.sel;
    float qn[8], dv[8];
    const float lse = cur.lse, D = cur.D;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qn[e] = act ? cur.q[e] * cur.rq : 0.f;
      dv[e] = act ? cur.d[e] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NBT; ++i) {
      // (the same for every lane: a row this query did not select costs nothing)
      if (!((selbits >> i) & 1u)) continue;
      const int r = r0 + i;
      const bool valid = act && r < nrows && t >= lo(r) && t < hi(r);
      float a = 0.f, c = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a += qn[e] * k[i][e];
        c += dv[e] * k[i][e];
      }
      const float s = hsum<LPH>(a) * p.scale, dp = hsum<LPH>(c);
      const float pj = valid ? expf(s - lse) : 0.f;
      const float ds = pj * (dp - D) * p.scale;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[i][e] += ds * qn[e] + pj * dv[e];
    }
  }
  // the heads' sums
#pragma unroll
  for (int i = 0; i < NBT; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[i][h][8 * lc + e] = acc[i][e];
  __syncthreads();
  for (int o = tid; o < NBT * HD; o += 256) {
    const int i = o / HD, c = o % HD;
    float s = 0.f;
    for (int hs = 0; hs < p.nh; ++hs) s += red[i][hs][c];
    out[o] = s;
  }
}

// block reduction over the first HD threads (HD <= 256, a multiple of 64)
template <int HD>
__device__ __forceinline__ float block_sum(float v, float* sh) {
  const int tid = threadIdx.x;
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  if ((tid & 63) == 0) sh[tid >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < HD / 64; ++w) s += sh[w];
  __syncthreads();
  return s;
}

template <int HD>
__global__ __launch_bounds__(HD) void hca_bwd_block_kernel(HcaBwdParams p, int nchunk, int ntile) {
  __shared__ float sh[4];
  const int n = blockIdx.x, b = blockIdx.y, c = threadIdx.x;
  const int tile = n / NBT, i = n % NBT;
  float dk = 0.f;
  if (p.mfma_parts) {
    // the chunks from the first one that holds a query seeing block n
    for (int ci = ((n + 1) * p.m2 - 1) / p.part_qc; ci < nchunk; ++ci)
      dk += p.part_b[(((size_t)b * nchunk + ci) * p.nb + n) * HD + c];
  } else {
    for (int ci = 0; ci < nchunk; ++ci)
      dk += p.part_b[((((size_t)b * ntile + tile) * nchunk + ci) * NBT + i) * HD + c];
  }
  const size_t ri = ((size_t)b * p.nb + n) * HD + c;
  const float y = p.kc[ri], r = p.raw[ri];
  const float yd = block_sum<HD>(y * dk, sh);
  const float nrm = sqrtf(block_sum<HD>(r * r, sh));
  const float dr = !p.normalize ? dk : (nrm > kEps ? (dk - y * yd) / nrm : dk / kEps);
  const int m2 = p.m2;
  if (p.Cb) {
    // overlapped: block n mixes Ca of its own tokens with Cb of block n-1's,
    // one softmax over the 2 m logits (block 0 has no second branch)
    auto la = [&](int j) { return p.Z[((size_t)b * p.T + (size_t)n * m2 + j) * HD + c] + p.Bpos[j * HD + c]; };
    auto lb = [&](int j) {
      return p.Zb[((size_t)b * p.T + (size_t)(n - 1) * m2 + j) * HD + c] + p.Bb[j * HD + c];
    };
    float mx = -INFINITY;
    for (int j = 0; j < m2; ++j) mx = fmaxf(mx, la(j));
    if (n > 0)
      for (int j = 0; j < m2; ++j) mx = fmaxf(mx, lb(j));
    float den = 0.f;
    for (int j = 0; j < m2; ++j) den += expf(la(j) - mx);
    if (n > 0)
      for (int j = 0; j < m2; ++j) den += expf(lb(j) - mx);
    for (int j = 0; j < m2; ++j) {
      const size_t ti = ((size_t)b * p.T + (size_t)n * m2 + j) * HD + c;
      const float w = expf(la(j) - mx) / den;
      const float dz = w * (p.C[ti] - r) * dr;
      p.dC[ti] = w * dr;
      p.dZ[ti] = dz;
      p.dBp[(((size_t)b * p.nb + n) * m2 + j) * HD + c] = dz;
    }
    for (int j = 0; j < m2; ++j) {
      float dz = 0.f;
      if (n > 0) {
        const size_t ti = ((size_t)b * p.T + (size_t)(n - 1) * m2 + j) * HD + c;
        const float w = expf(lb(j) - mx) / den;
        dz = w * (p.Cb[ti] - r) * dr;
        p.dCb[ti] = w * dr;
        p.dZb[ti] = dz;
      }
      p.dBbp[(((size_t)b * p.nb + n) * m2 + j) * HD + c] = dz;
    }
    return;
  }
  // softmax over the block's m2 tokens of Z + B_pos (this channel)
  float mx = -INFINITY;
  for (int j = 0; j < m2; ++j) {
    const size_t ti = ((size_t)b * p.T + (size_t)n * m2 + j) * HD + c;
    mx = fmaxf(mx, p.Z[ti] + p.Bpos[j * HD + c]);
  }
  float den = 0.f;
  for (int j = 0; j < m2; ++j) {
    const size_t ti = ((size_t)b * p.T + (size_t)n * m2 + j) * HD + c;
    den += expf(p.Z[ti] + p.Bpos[j * HD + c] - mx);
  }
  for (int j = 0; j < m2; ++j) {
    const size_t ti = ((size_t)b * p.T + (size_t)n * m2 + j) * HD + c;
    const float w = expf(p.Z[ti] + p.Bpos[j * HD + c] - mx) / den;
    const float dz = w * (p.C[ti] - r) * dr;
    p.dC[ti] = w * dr;
    p.dZ[ti] = dz;
    p.dBp[(((size_t)b * p.nb + n) * m2 + j) * HD + c] = dz;
  }
}

template <int HD>
__global__ __launch_bounds__(HD) void hca_bwd_window_kernel(HcaBwdParams p, int nchunk, int ntile) {
  __shared__ float sh[4];
  const int u = blockIdx.x, b = blockIdx.y, c = threadIdx.x;
  const int tile = u / NBT, i = u % NBT;
  float dk = 0.f;
  if (p.mfma_parts) {
    dk = p.part_w[((size_t)b * p.T + u) * HD + c];
  } else {
    for (int ci = 0; ci < nchunk; ++ci)
      dk += p.part_w[((((size_t)b * ntile + tile) * nchunk + ci) * NBT + i) * HD + c];
  }
  const size_t ri = ((size_t)b * p.T + u) * HD + c;
  const float y = p.kl[ri], x = p.lsrc[ri];
  const float yd = block_sum<HD>(y * dk, sh);
  const float nrm = sqrtf(block_sum<HD>(x * x, sh));
  const float dx = !p.normalize ? dk : (nrm > kEps ? (dk - y * yd) / nrm : dk / kEps);
  if (p.dlocal) p.dlocal[ri] = dx;
  else p.dC[ri] += dx;
}

// bit n of word (b, t, n / 32) set when query (b, t) selected block n
__global__ __launch_bounds__(256) void sel_bitmap_kernel(const int* idx, uint32_t* sel, long long nq,
                                                         int topk, int nw) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= nq * topk) return;
  const long long q = i / topk;
  const int n = idx[i];
  if (n >= 0) atomicOr(sel + q * nw + (n >> 5), 1u << (n & 31));
}

struct Plan {
  int ntile_b, nchunk_b, ntile_w, nchunk_w;
  size_t part_b, part_w;  // floats
};

Plan plan(int B, int T, int nb, int win, int HD) {
  Plan z;
  z.ntile_b = (nb + NBT - 1) / NBT;
  z.nchunk_b = (T + QC - 1) / QC;
  z.ntile_w = win > 0 ? (T + NBT - 1) / NBT : 0;
  z.nchunk_w = win > 0 ? (NBT - 1 + win + QC - 1) / QC : 0;
  z.part_b = (size_t)B * z.ntile_b * z.nchunk_b * NBT * HD;
  z.part_w = (size_t)B * z.ntile_w * z.nchunk_w * NBT * HD;
  return z;
}

size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

template <int HD>
hipError_t launch_hca_bwd(const HcaBwdParams& p, const Plan& z, hipStream_t s) {
  if (p.idx && p.topk > 0) {
    const long long n = (long long)p.B * p.T * p.topk;
    hipLaunchKernelGGL(sel_bitmap_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p.idx,
                       const_cast<uint32_t*>(p.sel), (long long)p.B * p.T, p.topk, (p.nb + 31) / 32);
  }
  hipLaunchKernelGGL((hca_bwd_query_kernel<HD>), dim3((unsigned)((size_t)p.B * p.T)), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.nb > 0) {
    if (p.sparse && p.topk == 0) {
      // no selection: the compressed rows receive nothing
      e = fill_u32(p.part_b, (long long)(z.part_b), 0u, s);
      if (e != hipSuccess) return e;
    } else {
      hipLaunchKernelGGL((hca_bwd_key_kernel<HD>), dim3(z.ntile_b * z.nchunk_b, p.B), dim3(256), 0, s, p,
                         0, z.nchunk_b, z.ntile_b);
    }
    hipLaunchKernelGGL((hca_bwd_block_kernel<HD>), dim3(p.nb, p.B), dim3(HD), 0, s, p, z.nchunk_b, z.ntile_b);
  }
  if (p.win > 0) {
    hipLaunchKernelGGL((hca_bwd_key_kernel<HD>), dim3(z.ntile_w * z.nchunk_w, p.B), dim3(256), 0, s, p, 1,
                       z.nchunk_w, z.ntile_w);
    hipLaunchKernelGGL((hca_bwd_window_kernel<HD>), dim3(p.T, p.B), dim3(HD), 0, s, p, z.nchunk_w, z.ntile_w);
  }
  return hipGetLastError();
}

// ---- the STE surrogate's backward (ops_csa.py:1033-1099, topk_columns) ----
// soft = softmax over the visible blocks n of the indexer logits
//   lg_n = sum_h w_h relu(a_hn),  a_hn = scale qn_h . k_n
// (ops_csa.py:503-572); the selected columns of soft receive dsel (the slot
// gradients, scattered densely: 0 off the selection). Backward:
//   D = sum_n soft_n dsel_n,  dl_n = soft_n (dsel_n - D),
//   dw_h = sum_n dl_n relu(a_hn),  dqn_h = sum_n dl_n w_h [a_hn > 0] scale k_n,
//   dk_n = sum_t sum_h dl_tn w_th [a > 0] scale qn_th,
// then the L2-norm and compression backwards of the indexer keys (the block
// kernel above, single-branch). A wave holds one query's NIH heads: lane
// (h = lane / LPH, lane % LPH) takes CPL consecutive channels, LPH = 64 / NIH.

template <int W>
__device__ __forceinline__ float xsum_from(float v) {  // over lanes W, 2W, .. 32 apart
#pragma unroll
  for (int o = W; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}
template <int L>
__device__ __forceinline__ float xsum_below(float v) {  // within aligned groups of L lanes
#pragma unroll
  for (int o = 1; o < L; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

template <int NIH, int CPL>
__global__ __launch_bounds__(256) void ste_bwd_query_kernel(SteBwdParams p) {
  constexpr int LPH = 64 / NIH, CI = LPH * CPL;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long bt = (long long)blockIdx.x * 4 + wave;
  if (bt >= (long long)p.B * p.T) return;  // whole waves only: shuffles stay within a wave
  const int b = (int)(bt / p.T), t = (int)(bt % p.T);
  const int h = lane / LPH, lc = lane % LPH;
  float qn[CPL], k[CPL], dq[CPL];
  const float* qrow = p.qi + ((size_t)bt * NIH + h) * CI + lc * CPL;
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    qn[e] = qrow[e];
    ss += qn[e] * qn[e];
    dq[e] = 0.f;
  }
  const float nrm = sqrtf(xsum_below<LPH>(ss));
  const float rq = p.normalize ? 1.f / fmaxf(nrm, kEps) : 1.f;
#pragma unroll
  for (int e = 0; e < CPL; ++e) qn[e] *= rq;
  const float wh = p.w[bt * NIH + h];
  const int nvis = min((t + 1) / p.m, p.nb);
  const float* dsel = p.dsel + (size_t)bt * p.nb;
  auto logit = [&](int n, float& a) {
    const float* kr = p.kc + ((size_t)b * p.nb + n) * CI + lc * CPL;
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      k[e] = kr[e];
      d += qn[e] * k[e];
    }
    a = xsum_below<LPH>(d) * p.scale;
    // a and w_h are the same on every lane of a head group: the sum over the
    // lanes LPH apart (one per head) gives every lane the logit
    return xsum_from<LPH>(wh * fmaxf(a, 0.f));
  };
  float m = -INFINITY, l = 0.f, ad = 0.f;
  for (int n = 0; n < nvis; ++n) {
    float a;
    const float lg = logit(n, a);
    const float mn = fmaxf(m, lg);
    const float sc = expf(m - mn), e1 = expf(lg - mn);
    l = l * sc + e1;
    ad = ad * sc + e1 * dsel[n];
    m = mn;
  }
  const float lse = l > 0.f ? m + logf(l) : INFINITY;
  const float D = l > 0.f ? ad / l : 0.f;
  float dwh = 0.f;
  for (int n = 0; n < nvis; ++n) {
    float a;
    const float lg = logit(n, a);
    const float dl = expf(lg - lse) * (dsel[n] - D);
    dwh += dl * fmaxf(a, 0.f);
    const float coef = a > 0.f ? dl * wh * p.scale : 0.f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) dq[e] += coef * k[e];
  }
  // L2-norm backward of the query row
  float yd = 0.f;
#pragma unroll
  for (int e = 0; e < CPL; ++e) yd += qn[e] * dq[e];
  yd = xsum_below<LPH>(yd);
  float* dst = p.dqi + ((size_t)bt * NIH + h) * CI + lc * CPL;
#pragma unroll
  for (int e = 0; e < CPL; ++e)
    dst[e] = p.normalize ? (nrm > kEps ? dq[e] - qn[e] * yd : dq[e]) * rq : dq[e];
  if (lc == 0) {
    p.dw[bt * NIH + h] = dwh;
    p.rq[bt * NIH + h] = rq;
  }
  if (lane == 0) {
    p.lse[bt] = lse;
    p.dval[bt] = D;
  }
}

template <int NIH, int CPL>
__global__ __launch_bounds__(256) void ste_bwd_key_kernel(SteBwdParams p, int nchunk, int ntile) {
  constexpr int LPH = 64 / NIH, CI = LPH * CPL;
  __shared__ float red[4][NBT][CI];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = lane / LPH, lc = lane % LPH;
  const int b = blockIdx.y;
  const int tile = blockIdx.x / nchunk, ci = blockIdx.x % nchunk;
  const int r0 = tile * NBT;
  const int tlo = (r0 + 1) * p.m - 1 + ci * QC;
  const int thi = min(p.T, tlo + QC);
  float* out = p.part + (((size_t)b * ntile + tile) * nchunk + ci) * NBT * CI;
  if (tlo >= thi) {
    for (int i = threadIdx.x; i < NBT * CI; i += 256) out[i] = 0.f;
    return;
  }
  float k[NBT][CPL], acc[NBT][CPL];
#pragma unroll
  for (int i = 0; i < NBT; ++i)
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      k[i][e] = r0 + i < p.nb ? p.kc[((size_t)b * p.nb + r0 + i) * CI + lc * CPL + e] : 0.f;
      acc[i][e] = 0.f;
    }
  for (int t = tlo + wave; t < thi; t += 4) {
    const size_t bt = (size_t)b * p.T + t;
    const float rq = p.rq[bt * NIH + h], wh = p.w[bt * NIH + h];
    const float lse = p.lse[bt], D = p.dval[bt];
    float qn[CPL];
    const float* qrow = p.qi + (bt * NIH + h) * CI + lc * CPL;
#pragma unroll
    for (int e = 0; e < CPL; ++e) qn[e] = qrow[e] * rq;
#pragma unroll
    for (int i = 0; i < NBT; ++i) {
      const int n = r0 + i;
      const bool valid = n < p.nb && t >= (n + 1) * p.m - 1;
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) d += qn[e] * k[i][e];
      const float a = xsum_below<LPH>(d) * p.scale;
      const float lg = xsum_from<LPH>(wh * fmaxf(a, 0.f));
      const float ds = valid ? p.dsel[bt * p.nb + n] : 0.f;
      const float dl = valid ? expf(lg - lse) * (ds - D) : 0.f;
      const float coef = a > 0.f ? dl * wh * p.scale : 0.f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) acc[i][e] += coef * qn[e];
    }
  }
  // the heads' sums (lanes LPH apart), then the four waves'
#pragma unroll
  for (int i = 0; i < NBT; ++i)
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      const float v = xsum_from<LPH>(acc[i][e]);
      if (h == 0) red[wave][i][lc * CPL + e] = v;
    }
  __syncthreads();
  for (int o = threadIdx.x; o < NBT * CI; o += 256) {
    const int i = o / CI, c = o % CI;
    out[o] = red[0][i][c] + red[1][i][c] + red[2][i][c] + red[3][i][c];
  }
}

template <int NIH, int CPL>
hipError_t launch_ste(SteBwdParams p, const Plan& z, HcaBwdParams bp, hipStream_t s) {
  const unsigned rows = (unsigned)(((long long)p.B * p.T + 3) / 4);
  hipLaunchKernelGGL((ste_bwd_query_kernel<NIH, CPL>), dim3(rows), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.nb == 0) return hipSuccess;
  hipLaunchKernelGGL((ste_bwd_key_kernel<NIH, CPL>), dim3(z.ntile_b * z.nchunk_b, p.B), dim3(256), 0, s,
                     p, z.nchunk_b, z.ntile_b);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // compression and L2-norm backward of the indexer keys
  if (p.cI == 64)
    hipLaunchKernelGGL((hca_bwd_block_kernel<64>), dim3(p.nb, p.B), dim3(64), 0, s, bp, z.nchunk_b, z.ntile_b);
  else
    hipLaunchKernelGGL((hca_bwd_block_kernel<128>), dim3(p.nb, p.B), dim3(128), 0, s, bp, z.nchunk_b,
                       z.ntile_b);
  return hipGetLastError();
}

}  // namespace

hipError_t sel_bitmap_launch(const int* idx, uint32_t* sel, long long nq, int topk, int nw, hipStream_t s) {
  const long long n = nq * topk;
  hipLaunchKernelGGL(sel_bitmap_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, idx, sel, nq,
                     topk, nw);
  return hipGetLastError();
}

// The L2-norm and compression backward of the compressed rows and the window
// rows' L2-norm backward, from MFMA-path partials (p.mfma_parts).
hipError_t hca_bwd_finish_launch(const HcaBwdParams& p, int nchunk, hipStream_t s) {
  if (p.nb > 0) {
    if (p.c == 64)
      hipLaunchKernelGGL((hca_bwd_block_kernel<64>), dim3(p.nb, p.B), dim3(64), 0, s, p, nchunk, 0);
    else
      hipLaunchKernelGGL((hca_bwd_block_kernel<128>), dim3(p.nb, p.B), dim3(128), 0, s, p, nchunk, 0);
  }
  if (p.win > 0) {
    if (p.c == 64)
      hipLaunchKernelGGL((hca_bwd_window_kernel<64>), dim3(p.T, p.B), dim3(64), 0, s, p, 0, 0);
    else
      hipLaunchKernelGGL((hca_bwd_window_kernel<128>), dim3(p.T, p.B), dim3(128), 0, s, p, 0, 0);
  }
  return hipGetLastError();
}

size_t hca_bwd_ws_bytes(int B, int T, int nh, int c, int m2, int win, int topk) {
  const Plan z = plan(B, T, T / m2, win, c);
  const size_t sel = topk > 0 ? al256((size_t)B * T * ((T / m2 + 31) / 32) * 4) : 0;
  const size_t simt = 3 * al256((size_t)B * T * nh * 4) + al256(z.part_b * 4) + al256(z.part_w * 4) + sel;
  // the MFMA path (normalised rows) needs its own regions; the larger of the two
  const size_t mfma = nh <= 16 ? attn_bwd_mfma_ws_bytes(B, T, c, m2, win, topk) : 0;
  return simt > mfma ? simt : mfma;
}

hipError_t hca_bwd_dispatch(HcaBwdParams p, void* ws, hipStream_t stream) {
  if (attn_bwd_mfma_supported(p)) return attn_bwd_mfma_dispatch(p, ws, stream);
  if (p.qdt != DT_F32) return hipErrorInvalidValue;  // the SIMT kernels read fp32 rows
  const Plan z = plan(p.B, p.T, p.nb, p.win, p.c);
  char* w = static_cast<char*>(ws);
  const size_t per = al256((size_t)p.B * p.T * p.nh * 4);
  p.lse = reinterpret_cast<float*>(w);
  p.dval = reinterpret_cast<float*>(w + per);
  p.rq = reinterpret_cast<float*>(w + 2 * per);
  p.part_b = reinterpret_cast<float*>(w + 3 * per);
  p.part_w = reinterpret_cast<float*>(w + 3 * per + al256(z.part_b * 4));
  p.sel = nullptr;
  if (p.idx && p.topk > 0) {
    uint32_t* sel = reinterpret_cast<uint32_t*>(w + 3 * per + al256(z.part_b * 4) + al256(z.part_w * 4));
    // cleared by the fill kernel (no memset node under graph capture)
    hipError_t e = fill_u32(sel, (long long)p.B * p.T * ((p.nb + 31) / 32), 0u, stream);
    if (e != hipSuccess) return e;
    p.sel = sel;
  }
  return p.c == 64 ? launch_hca_bwd<64>(p, z, stream) : launch_hca_bwd<128>(p, z, stream);
}

size_t ste_bwd_ws_bytes(int B, int T, int nIh, int cI, int m) {
  const Plan z = plan(B, T, T / m, 0, cI);
  return 2 * al256((size_t)B * T * 4) + al256((size_t)B * T * nIh * 4) + al256(z.part_b * 4);
}

hipError_t ste_bwd_dispatch(SteBwdParams p, HcaBwdParams bp, void* ws, hipStream_t stream) {
  const Plan z = plan(p.B, p.T, p.nb, 0, p.cI);
  char* w = static_cast<char*>(ws);
  const size_t per = al256((size_t)p.B * p.T * 4);
  p.lse = reinterpret_cast<float*>(w);
  p.dval = reinterpret_cast<float*>(w + per);
  p.rq = reinterpret_cast<float*>(w + 2 * per);
  p.part = reinterpret_cast<float*>(w + 2 * per + al256((size_t)p.B * p.T * p.nIh * 4));
  bp.part_b = p.part;
  const int cpl = p.cI * p.nIh / 64;
#define KCH_STE(NIH, CPL) \
  if (p.nIh == NIH && cpl == CPL) return launch_ste<NIH, CPL>(p, z, bp, stream);
  // nIh * cI <= 512 (one wave per query), cI in {64, 128}
  KCH_STE(1, 1) KCH_STE(1, 2) KCH_STE(2, 2) KCH_STE(2, 4) KCH_STE(4, 4) KCH_STE(4, 8)
  KCH_STE(8, 8)
#undef KCH_STE
  return hipErrorInvalidValue;
}

}  // namespace kch
