// CSA / HCA prefill kernels for gfx950: KV compression and joint-softmax MQA.
//
// compress_kernel  csa_compress_kv            (/root/reference/ops_csa.py:198-234)
//                  csa_compress_kv_overlapped (/root/reference/ops_csa.py:237-305)
//   one wave per (batch, compressed block); lane j owns channels j and j + 64.
//   Per channel: softmax over the m (or 2m) gate logits Z + B_pos, weighted sum
//   of C. Overlapped: block i mixes Ca_i with Cb_{i-1} (block 0: the b-branch
//   logits are -inf and its values zero). Optional outputs: the raw fp32 block,
//   the attention key row (L2-normalised or raw, bf16 or fp32), and the per-token
//   window keys L2norm(C) (or raw C) of the block's source tokens.
//
// hca_attn_kernel  naive_hca core (/root/reference/ops_hca.py:132-194): query t
//   attends to the compressed blocks b < (t+1)//m (ops_csa.py:179-195) and to
//   the window positions [t-win+1, t] (ops_csa.py:151-176), in one softmax with
//   the sink in the denominator.
// csa_attn_kernel  naive_csa core (/root/reference/ops_csa.py:959-1155): query t
//   attends to the indexer-selected compressed blocks (-1 = unused slot) and to
//   the same window, in one softmax with the sink.
// Both: one wave per query (all heads at once, MqaWave), 4 waves per workgroup.

#include "attn_common.h"
#include "kch_csa.h"

namespace kch {

namespace {

template <typename T> __device__ __forceinline__ void st_val(T* p, float v) { *p = from_f32<T>(v); }

}  // namespace

template <typename InT, bool OVERLAP>
__global__ __launch_bounds__(256) void compress_kernel(CompressParams p) {
  const int wave = (blockIdx.x * 4) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int nb = p.T / p.m;
  if (wave >= p.B * nb) return;
  const int b = wave / nb, blk = wave - b * nb;
  const int m = p.m, c = p.c;
  const InT* Ca = static_cast<const InT*>(p.Ca);
  const InT* Za = static_cast<const InT*>(p.Za);
  const InT* Cb = static_cast<const InT*>(p.Cb);
  const InT* Zb = static_cast<const InT*>(p.Zb);
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int ch = lane + 64 * u;
    if (ch >= c) continue;
    // pass 1: max of the logits; pass 2: exp-weighted sums (torch.softmax order)
    float mx = -INFINITY;
    const size_t ta = (size_t)b * p.T + (size_t)blk * m;
    for (int j = 0; j < m; ++j)
      mx = fmaxf(mx, to_f32(Za[(ta + j) * p.ldZa + ch]) + p.Ba[j * c + ch]);
    const bool prev = OVERLAP && blk > 0;
    const size_t tb = ta - m;
    if (prev)
      for (int j = 0; j < m; ++j)
        mx = fmaxf(mx, to_f32(Zb[(tb + j) * p.ldZb + ch]) + p.Bb[j * c + ch]);
    float den = 0.f, num = 0.f;
    for (int j = 0; j < m; ++j) {
      const float e = expf(to_f32(Za[(ta + j) * p.ldZa + ch]) + p.Ba[j * c + ch] - mx);
      den += e;
      num += e * to_f32(Ca[(ta + j) * p.ldCa + ch]);
    }
    if (prev)
      for (int j = 0; j < m; ++j) {
        const float e = expf(to_f32(Zb[(tb + j) * p.ldZb + ch]) + p.Bb[j * c + ch] - mx);
        den += e;
        num += e * to_f32(Cb[(tb + j) * p.ldCb + ch]);
      }
    acc[u] = num / den;
  }
  const size_t orow = (size_t)b * nb + blk;
  if (p.out_raw) {
    for (int u = 0; u < 2; ++u)
      if (lane + 64 * u < c) p.out_raw[orow * c + lane + 64 * u] = acc[u];
  }
  if (p.out_key) {
    float inv = 1.f;
    if (p.normalize) inv = l2_inv(wave_sum(acc[0] * acc[0] + acc[1] * acc[1]));
    for (int u = 0; u < 2; ++u) {
      if (lane + 64 * u >= c) continue;
      const size_t o = orow * c + lane + 64 * u;
      if (p.key_f32) static_cast<float*>(p.out_key)[o] = acc[u] * inv;
      else static_cast<bf16_t*>(p.out_key)[o] = (bf16_t)(acc[u] * inv);
    }
  }
  if (p.local) {
    // window keys of the block's m source tokens (from the a-branch values)
    for (int j = 0; j < m; ++j) {
      const size_t t = (size_t)b * p.T + (size_t)blk * m + j;
      float v[2];
      for (int u = 0; u < 2; ++u) v[u] = (lane + 64 * u < c) ? to_f32(Ca[t * p.ldCa + lane + 64 * u]) : 0.f;
      float inv = 1.f;
      if (p.normalize) inv = l2_inv(wave_sum(v[0] * v[0] + v[1] * v[1]));
      for (int u = 0; u < 2; ++u)
        if (lane + 64 * u < c) p.local[t * c + lane + 64 * u] = (bf16_t)(v[u] * inv);
    }
  }
}

hipError_t compress_dispatch(const CompressParams& p, int dtype, hipStream_t stream) {
  const int nwaves = p.B * (p.T / p.m);
  const dim3 grid((nwaves + 3) / 4), block(256);
  if (p.overlap) {
    if (dtype == DT_F32) hipLaunchKernelGGL((compress_kernel<float, true>), grid, block, 0, stream, p);
    else if (dtype == DT_BF16) hipLaunchKernelGGL((compress_kernel<bf16_t, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((compress_kernel<_Float16, true>), grid, block, 0, stream, p);
  } else {
    if (dtype == DT_F32) hipLaunchKernelGGL((compress_kernel<float, false>), grid, block, 0, stream, p);
    else if (dtype == DT_BF16) hipLaunchKernelGGL((compress_kernel<bf16_t, false>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((compress_kernel<_Float16, false>), grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Joint-softmax MQA prefill. Key tables are bf16 rows of head dim HD.
// ---------------------------------------------------------------------------

template <int HD, typename QT, typename OT, bool SPARSE>
__global__ __launch_bounds__(256) void attn_prefill_kernel(AttnParams p) {
  using W = MqaWave<HD>;
  __shared__ __attribute__((aligned(16))) bf16_t stage_all[4][16 * W::LDS_LD];
  const int wv = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  bf16_t* stage = stage_all[wv];
  const int T = p.T;
  // query index: consecutive queries of one batch row per workgroup
  const long long qi = (long long)blockIdx.x * 4 + wv;
  if (qi >= (long long)p.B * T) return;
  const int b = (int)(qi / T), t = (int)(qi - (long long)b * T);

  const QT* qrow = static_cast<const QT*>(p.q) + ((size_t)qi * p.nh + n) * HD;
  W w;
  w.template init<QT>(n < p.nh ? qrow : nullptr, p.normalize_q != 0, p.scale);

  const bf16_t* kv = p.kv_comp + (size_t)b * (p.kv_bstride ? p.kv_bstride : (long long)p.nb * HD);
  if (SPARSE) {
    // selected compressed blocks; -1 marks an unused slot
    const int* idx = p.idx + (size_t)qi * p.topk;
    for (int j0 = 0; j0 < p.topk; j0 += 16) {
      const int j = j0 + n;
      const int id = (j < p.topk) ? idx[j] : -1;
      const bool ok = id >= 0 && id < p.nb;
      const unsigned valid = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
      if (valid == 0) continue;
      w.chunk(kv + (size_t)(ok ? id : 0) * HD, valid, stage);
    }
  } else {
    // dense: compressed blocks b < (t + 1) // m
    const int nvis = min(p.nb, (p.pos0 + t + 1) / p.m);
    for (int j0 = 0; j0 < nvis; j0 += 16) {
      const int j = j0 + n;
      const bool ok = j < nvis;
      const unsigned valid = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
      w.chunk(kv + (size_t)(ok ? j : 0) * HD, valid, stage);
    }
  }
  if (p.kv_local && p.local_count >= 0) {
    // window = the first local_count rows (a ring buffer, order irrelevant)
    const bf16_t* loc =
        p.kv_local + (size_t)b * (p.local_bstride ? p.local_bstride : (long long)T * HD);
    for (int j0 = 0; j0 < p.local_count; j0 += 16) {
      const int j = j0 + n;
      const bool ok = j < p.local_count;
      const unsigned valid = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
      w.chunk(loc + (size_t)(ok ? j : 0) * HD, valid, stage);
    }
  } else if (p.win > 0 && p.kv_local) {
    // window positions t - win + 1 .. t (those >= 0)
    const bf16_t* loc =
        p.kv_local + (size_t)b * (p.local_bstride ? p.local_bstride : (long long)T * HD);
    const int lo = t - p.win + 1;
    for (int j0 = lo; j0 <= t; j0 += 16) {
      const int j = j0 + n;
      const bool ok = j >= 0 && j <= t;
      const unsigned valid = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
      if (valid == 0) continue;
      w.chunk(loc + (size_t)(ok ? j : 0) * HD, valid, stage);
    }
  }
  const float f = w.finish(p.sink != nullptr, (p.sink && n < p.nh) ? p.sink[n] : 0.f);
  if (n < p.nh) {
    OT* out = static_cast<OT*>(p.out) + ((size_t)qi * p.nh + n) * HD;
    const int q4 = 4 * (lane >> 4);
#pragma unroll
    for (int tt = 0; tt < W::NT; ++tt)
#pragma unroll
      for (int e = 0; e < 4; ++e) st_val<OT>(out + 16 * tt + q4 + e, w.o[tt][e] * f);
  }
}

template <int HD, bool SPARSE>
static hipError_t launch_attn(const AttnParams& p, int qdtype, int odtype, hipStream_t s) {
  const long long nq = (long long)p.B * p.T;
  const dim3 grid((unsigned)((nq + 3) / 4)), block(256);
#define KCH_ATTN_LAUNCH(QT, OT) \
  hipLaunchKernelGGL((attn_prefill_kernel<HD, QT, OT, SPARSE>), grid, block, 0, s, p)
  if (qdtype == DT_BF16) {
    if (odtype == DT_F32) KCH_ATTN_LAUNCH(bf16_t, float);
    else KCH_ATTN_LAUNCH(bf16_t, bf16_t);
  } else if (qdtype == DT_F32) {
    if (odtype == DT_F32) KCH_ATTN_LAUNCH(float, float);
    else KCH_ATTN_LAUNCH(float, bf16_t);
  } else {
    if (odtype == DT_F32) KCH_ATTN_LAUNCH(_Float16, float);
    else KCH_ATTN_LAUNCH(_Float16, _Float16);
  }
#undef KCH_ATTN_LAUNCH
  return hipGetLastError();
}

hipError_t attn_dispatch(const AttnParams& p, bool sparse, int qdtype, int odtype, hipStream_t s) {
  if (p.hd == 128) return sparse ? launch_attn<128, true>(p, qdtype, odtype, s)
                                 : launch_attn<128, false>(p, qdtype, odtype, s);
  return sparse ? launch_attn<64, true>(p, qdtype, odtype, s)
                : launch_attn<64, false>(p, qdtype, odtype, s);
}

}  // namespace kch
