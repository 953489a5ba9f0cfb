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
__global__ __launch_bounds__(256, 3) void attn_prefill_kernel(AttnParams p) {
  using W = MqaWave<HD>;
  __shared__ __attribute__((aligned(16))) bf16_t stage_all[4][16 * W::LDS_LD];
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
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

  // The rows of this query: n_main compressed rows (the selected blocks, -1 =
  // unused slot; or the causally visible blocks), then n_win window rows (the
  // first local_count rows of a ring, or positions max(t - win + 1, 0) .. t).
  const bf16_t* kv = p.kv_comp + (size_t)b * (p.kv_bstride ? p.kv_bstride : (long long)p.nb * HD);
  const int n_main = SPARSE ? p.topk : max(0, min(p.nb, (p.pos0 + t + 1) / p.m));
  const bf16_t* loc = nullptr;
  int n_win = 0, wbase = 0;
  if (p.kv_local && p.local_count >= 0) {
    loc = p.kv_local + (size_t)b * (p.local_bstride ? p.local_bstride : (long long)T * HD);
    n_win = p.local_count;
  } else if (p.win > 0 && p.kv_local) {
    loc = p.kv_local + (size_t)b * (p.local_bstride ? p.local_bstride : (long long)T * HD);
    wbase = max(t - p.win + 1, 0);
    n_win = t - wbase + 1;
  }
  const int n_tot = (p.nb > 0 ? n_main : 0) + n_win;
  if (n_tot > 0) {
    const int nm = p.nb > 0 ? n_main : 0;
    // rows of padding lanes must be readable: a compressed row when any exists
    const bf16_t* dflt = p.nb > 0 ? kv : loc;
    // Selected block indices come 64 at a time, one per lane, from a load issued
    // a group ahead of its use (so that waiting for it never waits for the row
    // loads issued after it); loads are clamped, read entries are only those of
    // rows below n_main. Without indices a readable word is loaded.
    const bool has_idx = SPARSE && nm > 0;
    const int* ip = has_idx ? p.idx + (size_t)qi * p.topk : reinterpret_cast<const int*>(dflt);
    const int ilim = has_idx ? nm : 1;
    auto idx_group = [&](int g) { return ip[min(64 * g + lane, ilim - 1)]; };
    auto row_of = [&](int c, int ig, bool& ok) {
      const int j = 16 * c + n;
      const int sel = SPARSE ? __shfl(ig, (16 * c + n) & 63) : j;
      const bf16_t* row = dflt;
      ok = false;
      if (j < nm) {
        ok = sel >= 0 && sel < p.nb;
        if (ok) row = kv + (size_t)sel * HD;
      } else if (j < n_tot) {
        ok = true;
        row = loc + (size_t)(wbase + j - nm) * HD;
      }
      return row;
    };
    // groups of 4 chunks, four chunks in flight; refills are unconditional (past
    // the end they read the default row, masked off) so that no loaded register
    // is copied
    typename W::Frag fr[4];
    unsigned vm[4];
    const int nch = (n_tot + 15) / 16;
    const int ng = (nch + 3) / 4;
    const int ig0 = idx_group(0);
    int ig1 = idx_group(1);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bool ok;
      const bf16_t* row = row_of(c, ig0, ok);
      vm[c] = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
      W::load(fr[c], row);
    }
    for (int g = 0; g < ng; ++g) {
      const int ig2 = idx_group(g + 2);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (vm[c]) w.chunk(fr[c], vm[c], stage);
        bool ok;
        const bf16_t* row = row_of(4 * (g + 1) + c, ig1, ok);
        vm[c] = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
        W::load(fr[c], row);
      }
      ig1 = ig2;
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
