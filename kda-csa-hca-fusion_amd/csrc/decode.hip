// Decode-step kernels for the CSA / HCA caches (one new token per sequence).
//
// Restates CSADecodingCache.forward_step (/root/reference/ops_decoding_cache.py:783-1070)
// and HCADecodingCache.forward_step (:1268-1395) for long caches: a decode step
// is bound by reading the cache, so every kernel splits the cache across many
// workgroups instead of giving one workgroup to each sequence.
//
// idx_range_kernel   lightning-indexer logits of one range of <= RB cached
//   blocks of one sequence (ops_csa.py:503-536: relu(scale q_h . k_n / ||k_n||),
//   weighted head sum), then the range's top-k: a block-level 4 x 8-bit radix
//   select on order-preserving keys and an order-preserving compaction (ties
//   at the threshold taken in ascending block index). Keys are the cached rows
//   as stored (cache dtype) times a per-row fp32 1/||k|| (1 without
//   normalisation); q is split into bf16 hi + lo, so a bf16 key row gives the
//   logit to ~2^-16 relative error with two MFMAs.
//   With one range per sequence the result is sorted and final; otherwise the
//   selected (key, index) pairs are written in index order as candidates.
// idx_merge_kernel   the top-k of the candidates of all ranges of a sequence.
//   A global top-k lies in the union of the per-range top-ks under the same
//   tie rule, and the candidates are laid out range-major in index order, so
//   an order-preserving selection keeps the lowest-index rule. Output sorted by
//   (logit desc, index asc).
// attn_part_kernel   joint-softmax MQA over a slice of the attended rows of a
//   sequence (selected or all compressed blocks, then the ring window): per
//   head the running max M, sum L and the unnormalised o (MqaWave).
// attn_combine_kernel  merges the slices of a sequence and adds the sink:
//   o = sum_s o_s 2^(M_s-M) / (sum_s L_s 2^(M_s-M) + e^sink 2^-M), 0 when no
//   row is valid (the all-invalid rule of ops_decoding_cache.py:1044-1059).

#include <type_traits>

#include "attn_common.h"
#include "kch_csa.h"

namespace kch {

namespace {

constexpr int RB_MAX = 8192;  // blocks per indexer range

__device__ __forceinline__ uint32_t okey(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ void split8(const float* f, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16_t h = (bf16_t)f[i];
    hi[i] = h;
    lo[i] = (bf16_t)(f[i] - (float)h);
  }
}

// Exclusive prefix sum over the 256 threads of the block (scratch: 8 ints).
__device__ __forceinline__ int block_excl_scan(int v, int* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; ++w) off += scratch[w];
  __syncthreads();
  return x - v + off;
}

// Top-`topk` of `n` keys (order-preserving uint32, key(i)) held in LDS by a
// 256-thread block: returns the threshold key and sets *n_above (keys >
// threshold) and *n_tie_take (keys == threshold to take, lowest position first).
// Requires topk < n.
template <typename KeyF>
__device__ uint32_t block_radix_select(KeyF key, int n, int topk, uint32_t* hist, int* scratch,
                                       int* n_above, int* n_tie_take) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, pmask = 0;
  int need = topk, above_total = 0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += 256) {
      const uint32_t u = key(i);
      if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    // thread t: bin 255 - t (descending); cumulative count of larger bins
    const int c = (int)hist[255 - tid];
    const int cum = block_excl_scan(c, scratch);
    if (cum < need && cum + c >= need) {
      scratch[8] = 255 - tid;
      scratch[9] = cum;
    }
    __syncthreads();
    const int bin = scratch[8], above = scratch[9];
    __syncthreads();
    prefix |= (uint32_t)bin << shift;
    pmask |= 255u << shift;
    need -= above;
    above_total += above;
  }
  *n_above = above_total;
  *n_tie_take = need;
  return prefix;
}

// Order-preserving compaction of the selected positions (key > thr, or key ==
// thr among the first `tie_take` such positions; every position when
// take_all) into out[0 .. count): out[j] = val(i). Each thread scans one
// contiguous segment of the n positions. Returns the count.
template <typename KeyF, typename ValF>
__device__ int block_compact(KeyF key, ValF val, int n, uint32_t thr, int tie_take, bool take_all,
                             unsigned long long* out, int* scratch) {
  const int tid = threadIdx.x;
  const int seg = (n + 255) / 256;
  const int lo = min(n, tid * seg), hi = min(n, lo + seg);
  int eq = 0;
  if (!take_all)
    for (int i = lo; i < hi; ++i) eq += key(i) == thr;
  const int eq_before = block_excl_scan(eq, scratch);
  auto taken = [&](uint32_t u, int& e) {
    if (take_all) return true;
    if (u == thr) return (e++) < tie_take;
    return u > thr;
  };
  int cnt = 0, e = eq_before;
  for (int i = lo; i < hi; ++i) cnt += taken(key(i), e);
  int pos = block_excl_scan(cnt, scratch);
  e = eq_before;
  for (int i = lo; i < hi; ++i)
    if (taken(key(i), e)) out[pos++] = val(i);
  if (tid == 255) scratch[10] = pos;
  __syncthreads();
  const int total = scratch[10];
  __syncthreads();
  return total;
}

// Bitonic sort of s[0 .. cnt) descending, padded to a power of two with zeros.
__device__ void block_sort_desc(unsigned long long* s, int cnt) {
  const int tid = threadIdx.x;
  int pw = 1;
  while (pw < cnt) pw <<= 1;
  for (int i = cnt + tid; i < pw; i += 256) s[i] = 0ull;
  __syncthreads();
  for (int k = 2; k <= pw; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < pw / 2; i += 256) {
        const int a = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int c = a + j;
        const unsigned long long x = s[a], y = s[c];
        const bool desc = (a & k) == 0;
        if (desc ? (x < y) : (x > y)) {
          s[a] = y;
          s[c] = x;
        }
      }
      __syncthreads();
    }
  }
}

template <typename QT, typename KT, int CI>
__global__ __launch_bounds__(256) void idx_range_kernel(DecodeIdxParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int NS = CI / 32;
  uint32_t* keys = reinterpret_cast<uint32_t*>(smem);                          // [RB]
  uint32_t* hist = keys + p.rb;                                                 // [256]
  int* scratch = reinterpret_cast<int*>(hist + 256);                            // [16]
  unsigned long long* sel = reinterpret_cast<unsigned long long*>(scratch + 16);  // [ptop]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q4 = lane >> 4, n = lane & 15;
  const int b = blockIdx.x / p.nr, r = blockIdx.x - b * p.nr;
  const int r0 = r * p.rb;
  const int nr_blocks = min(p.rb, p.nb - r0);
  const int nIh = p.nIh;
  if (nr_blocks <= 0) {  // an empty trailing range: no candidates
    unsigned long long* out = p.cand + ((size_t)b * p.nr + r) * p.topk;
    for (int i = tid; i < p.topk; i += 256) out[i] = 0ull;
    return;
  }

  // ---- q fragments: column n = head (zero beyond nIh), split bf16 ----
  bf16x8 qhi[NS], qlo[NS];
  float wq = 0.f;
  {
    float f[NS][8];
    float ss = 0.f;
    const QT* qrow = static_cast<const QT*>(p.q_idx) + ((size_t)b * nIh + (n < nIh ? n : 0)) * CI;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      Load8<QT>::run(qrow + 32 * s + 8 * q4, f[s]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += f[s][i] * f[s][i];
    }
    const float inv = p.normalize_q ? l2_inv(colq_sum(ss)) : 1.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[s][i] = n < nIh ? f[s][i] * inv : 0.f;
      split8(f[s], qhi[s], qlo[s]);
    }
    if (n < nIh) wq = p.w_idx ? ld_f32(static_cast<const QT*>(p.w_idx) + (size_t)b * nIh + n) : 1.f;
  }

  // ---- logits of this range: wave w takes 16-block chunks w, w + 4, ... ----
  const KT* kbase = static_cast<const KT*>(p.keys) + (size_t)b * p.k_bstride;
  const float* ibase = p.inv_norm ? p.inv_norm + (size_t)b * p.n_bstride : nullptr;
  const int nchunk = (nr_blocks + 15) / 16;
  auto load_k = [&](int c, float (&kf)[NS][8]) {
    const int blk = r0 + min(16 * c + n, nr_blocks - 1);
    const KT* krow = kbase + (size_t)blk * CI;
#pragma unroll
    for (int s = 0; s < NS; ++s) Load8<KT>::run(krow + 32 * s + 8 * q4, kf[s]);
  };
  float kf[NS][8];
  if (wave < nchunk) load_k(wave, kf);
  for (int c = wave; c < nchunk; c += 4) {
    float cur[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) cur[s][i] = kf[s][i];
    if (c + 4 < nchunk) load_k(c + 4, kf);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      bf16x8 khi, klo;
      split8(cur[s], khi, klo);
      // D[block][head]: A = key rows, B = q columns
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, qhi[s], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, qlo[s], acc, 0, 0, 0);
      if constexpr (!std::is_same<KT, bf16_t>::value)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klo, qhi[s], acc, 0, 0, 0);
    }
    const int j0 = 16 * c + 4 * q4;  // range-local blocks j0 .. j0 + 3 of this lane
    float4 iv = make_float4(1.f, 1.f, 1.f, 1.f);
    if (ibase) {
      iv.x = ibase[r0 + min(j0, nr_blocks - 1)];
      iv.y = ibase[r0 + min(j0 + 1, nr_blocks - 1)];
      iv.z = ibase[r0 + min(j0 + 2, nr_blocks - 1)];
      iv.w = ibase[r0 + min(j0 + 3, nr_blocks - 1)];
    }
    const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = fmaxf(acc[e] * p.scale * ivs[e], 0.f) * wq;
      for (int d = 1; d < nIh; d <<= 1) v += __shfl_xor(v, d);
      if (n == 0 && j0 + e < nr_blocks) keys[j0 + e] = okey(v);
    }
  }
  __syncthreads();

  // ---- top-k of the range ----
  const int topk = p.topk;
  const bool take_all = nr_blocks <= topk;
  int above = 0, tie_take = 0;
  uint32_t thr = 0;
  auto key_at = [&](int i) { return keys[i]; };
  auto val_at = [&](int i) {
    return ((unsigned long long)keys[i] << 32) | (uint32_t)(~(uint32_t)(r0 + i));
  };
  if (!take_all) thr = block_radix_select(key_at, nr_blocks, topk, hist, scratch, &above, &tie_take);
  const int cnt = block_compact(key_at, val_at, nr_blocks, thr, tie_take, take_all, sel, scratch);
  if (p.nr == 1) {
    block_sort_desc(sel, cnt);
    int* out = p.idx_out + (size_t)b * topk;
    for (int i = tid; i < topk; i += 256) out[i] = i < cnt ? (int)(~(uint32_t)(sel[i] & 0xffffffffull)) : -1;
  } else {
    unsigned long long* out = p.cand + ((size_t)b * p.nr + r) * topk;
    for (int i = tid; i < topk; i += 256) out[i] = i < cnt ? sel[i] : 0ull;
  }
}

__global__ __launch_bounds__(256) void idx_merge_kernel(DecodeIdxParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int topk = p.topk, nr = p.nr, nc = nr * topk;
  unsigned long long* cand = reinterpret_cast<unsigned long long*>(smem);  // [nc]
  uint32_t* hist = reinterpret_cast<uint32_t*>(cand + nc);                 // [256]
  int* scratch = reinterpret_cast<int*>(hist + 256);                       // [16]
  int* roff = scratch + 16;                                                // [nr + 1]
  unsigned long long* sel = reinterpret_cast<unsigned long long*>(roff + ((nr + 2) & ~1));  // [ptop]
  const int tid = threadIdx.x, b = blockIdx.x;
  const unsigned long long* src = p.cand + (size_t)b * nc;
  // each range's list holds its selected pairs first, then zeros (no real key is
  // 0: every logit is >= 0, whose key is 2^31): count by binary search
  for (int r = tid; r < nr; r += 256) {
    const unsigned long long* lst = src + (size_t)r * topk;
    int lo = 0, hi = topk;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((lst[mid] >> 32) != 0ull) lo = mid + 1;
      else hi = mid;
    }
    roff[r + 1] = lo;
  }
  __syncthreads();
  if (tid == 0) {
    roff[0] = 0;
    for (int r = 0; r < nr; ++r) roff[r + 1] += roff[r];
  }
  __syncthreads();
  const int total = roff[nr];
  // compacted candidates: ranges ascending, index order within a range = index order
  for (int i = tid; i < nc; i += 256) {
    const int r = i / topk, j = i - r * topk;
    if (j < roff[r + 1] - roff[r]) cand[roff[r] + j] = src[i];
  }
  __syncthreads();
  auto key_at = [&](int i) { return (uint32_t)(cand[i] >> 32); };
  auto val_at = [&](int i) { return cand[i]; };
  int above = 0, tie_take = 0;
  uint32_t thr = 0;
  const bool take_all = total <= topk;
  if (!take_all) thr = block_radix_select(key_at, total, topk, hist, scratch, &above, &tie_take);
  const int cnt = block_compact(key_at, val_at, total, thr, tie_take, take_all, sel, scratch);
  block_sort_desc(sel, cnt);
  int* out = p.idx_out + (size_t)b * topk;
  for (int i = tid; i < topk; i += 256) out[i] = i < cnt ? (int)(~(uint32_t)(sel[i] & 0xffffffffull)) : -1;
}

template <int HD, typename QT>
__global__ __launch_bounds__(256) void attn_part_kernel(DecodeAttnParams p) {
  using W = MqaWave<HD>;
  __shared__ __attribute__((aligned(16))) bf16_t stage_all[4][16 * W::LDS_LD];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15;
  bf16_t* stage = stage_all[wv];
  const long long gs = (long long)blockIdx.x * 4 + wv;  // global split id
  if (gs >= (long long)p.B * p.nsplit) return;
  const int b = (int)(gs / p.nsplit), sp = (int)(gs - (long long)b * p.nsplit);
  const int nrows = p.na + p.ring_len;
  const int j0 = sp * p.rows_per_split, j1 = min(nrows, j0 + p.rows_per_split);

  const QT* qrow = static_cast<const QT*>(p.q) + ((size_t)b * p.nh + n) * HD;
  W w;
  w.template init<QT>(n < p.nh ? qrow : nullptr, p.normalize_q != 0, p.scale);
  const bf16_t* kv = p.kv + (size_t)b * p.kv_bstride;
  const bf16_t* ring = p.ring ? p.ring + (size_t)b * p.ring_bstride : nullptr;
  const int* idx = p.idx ? p.idx + (size_t)b * p.na : nullptr;
  // rows of padding lanes must still be readable: a cached block when there is
  // one, else the ring (a split only exists when one of the two holds rows)
  const bf16_t* dflt = p.na > 0 ? kv : ring;
  // chunk c covers rows j0 + 16c .. ; its row pointer and validity
  auto row_of = [&](int c, bool& ok) {
    const int j = j0 + 16 * c + n;
    ok = j < j1;
    const bf16_t* row = dflt;
    if (ok) {
      if (j < p.na) {
        const int blk = idx ? idx[j] : j;
        ok = blk >= 0 && blk < p.nb;
        if (ok) row = kv + (size_t)blk * HD;
      } else {
        row = ring + (size_t)(j - p.na) * HD;
      }
    }
    return row;
  };
  // software pipeline: the rows of chunk c + D are requested while chunk c is consumed
  constexpr int D = 4;
  typename W::Frag fr[D];
  unsigned vm[D];
  const int nch = (j1 - j0 + 15) / 16;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    bool ok;
    const bf16_t* row = row_of(d, ok);
    vm[d] = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
    if (d < nch) W::load(fr[d], row);
  }
  for (int c0 = 0; c0 < nch; c0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int c = c0 + d;
      if (c < nch) {
        if (vm[d]) w.chunk(fr[d], vm[d], stage);
        bool ok;
        const bf16_t* row = row_of(c + D, ok);
        vm[d] = (unsigned)__ballot(ok && lane < 16) & 0xffffu;
        if (c + D < nch) W::load(fr[d], row);
      }
    }
  }
  // partial state of head n: unnormalised o, M (log2 units), L
  if (n < p.nh) {
    float* po = p.part_o + ((size_t)gs * p.nh + n) * HD;
    const int q4 = 4 * (lane >> 4);
#pragma unroll
    for (int tt = 0; tt < W::NT; ++tt)
      *reinterpret_cast<float4*>(po + 16 * tt + q4) = make_float4(w.o[tt][0], w.o[tt][1], w.o[tt][2], w.o[tt][3]);
    if (lane < 16) *reinterpret_cast<float2*>(p.part_ml + ((size_t)gs * p.nh + n) * 2) = make_float2(w.M, w.L);
  }
}

template <typename OT>
__global__ __launch_bounds__(256) void attn_combine_kernel(DecodeAttnParams p) {
  // thread -> (head, 8 dims); a block covers 256 * 8 outputs of one sequence
  const int hd = p.hd, per_head = hd / 8;
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long total = (long long)p.B * p.nh * per_head;
  if (g >= total) return;
  const int d8 = (int)(g % per_head);
  const long long bh = g / per_head;
  const int h = (int)(bh % p.nh), b = (int)(bh / p.nh);
  const float2* ml = reinterpret_cast<const float2*>(p.part_ml) + (size_t)b * p.nsplit * p.nh + h;
  float M = -INFINITY;
  for (int s = 0; s < p.nsplit; ++s) M = fmaxf(M, ml[(size_t)s * p.nh].x);
  float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (M > -INFINITY) {
    for (int s = 0; s < p.nsplit; ++s) {
      const float2 v = ml[(size_t)s * p.nh];
      if (v.y <= 0.f) continue;
      const float a = fast_exp2(v.x - M);
      L += v.y * a;
      const float* po = p.part_o + (((size_t)b * p.nsplit + s) * p.nh + h) * hd + 8 * d8;
      const float4 x0 = *reinterpret_cast<const float4*>(po);
      const float4 x1 = *reinterpret_cast<const float4*>(po + 4);
      acc[0] += a * x0.x; acc[1] += a * x0.y; acc[2] += a * x0.z; acc[3] += a * x0.w;
      acc[4] += a * x1.x; acc[5] += a * x1.y; acc[6] += a * x1.z; acc[7] += a * x1.w;
    }
  }
  float f = 0.f;
  if (L > 0.f) {
    float denom = L;
    if (p.sink) denom += fast_exp2(p.sink[h] * kLog2eF - M);
    f = 1.f / denom;
  }
  OT* out = static_cast<OT*>(p.out) + ((size_t)b * p.nh + h) * hd + 8 * d8;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = from_f32<OT>(acc[i] * f);
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* p, long long n, uint32_t v) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

// Fills n 32-bit words (a kernel rather than a memset node, so that a captured
// graph replays it faithfully).
hipError_t fill_u32(void* p, long long n, uint32_t v, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     static_cast<uint32_t*>(p), n, v);
  return hipGetLastError();
}

int decode_merge_max() { return 16384; }

void decode_idx_plan(int nb, int topk, int* rb, int* nr) {
  // ranges of at most RB_MAX blocks; a single range when it fits
  const int r = (nb + RB_MAX - 1) / RB_MAX;
  *nr = r < 1 ? 1 : r;
  *rb = (nb + *nr - 1) / *nr;
  *rb = (*rb + 15) & ~15;
  (void)topk;
}

size_t decode_idx_lds(int rb, int topk) {
  int ptop = 1;
  while (ptop < topk) ptop <<= 1;
  return (size_t)rb * 4 + 256 * 4 + 16 * 4 + (size_t)ptop * 8;
}

size_t decode_merge_lds(int nr, int topk) {
  int ptop = 1;
  while (ptop < topk) ptop <<= 1;
  const size_t nc = (size_t)nr * topk;
  return nc * 8 + 256 * 4 + 16 * 4 + (size_t)((nr + 2) & ~1) * 4 + (size_t)ptop * 8;
}

hipError_t decode_idx_dispatch(const DecodeIdxParams& p, int qdtype, int kdtype, hipStream_t s) {
  const size_t lds = decode_idx_lds(p.rb, p.topk);
  const dim3 grid((unsigned)(p.B * p.nr)), block(256);
#define KCH_DIDX(QT, KT, CI) hipLaunchKernelGGL((idx_range_kernel<QT, KT, CI>), grid, block, lds, s, p)
#define KCH_DIDX_CI(QT, KT)             \
  if (p.cI == 64) KCH_DIDX(QT, KT, 64); \
  else if (p.cI == 128) KCH_DIDX(QT, KT, 128); \
  else KCH_DIDX(QT, KT, 32);
  if (qdtype == DT_F32) {
    if (kdtype == DT_BF16) { KCH_DIDX_CI(float, bf16_t) }
    else if (kdtype == DT_F16) { KCH_DIDX_CI(float, _Float16) }
    else { KCH_DIDX_CI(float, float) }
  } else if (qdtype == DT_BF16) {
    if (kdtype == DT_BF16) { KCH_DIDX_CI(bf16_t, bf16_t) }
    else if (kdtype == DT_F16) { KCH_DIDX_CI(bf16_t, _Float16) }
    else { KCH_DIDX_CI(bf16_t, float) }
  } else {
    if (kdtype == DT_BF16) { KCH_DIDX_CI(_Float16, bf16_t) }
    else if (kdtype == DT_F16) { KCH_DIDX_CI(_Float16, _Float16) }
    else { KCH_DIDX_CI(_Float16, float) }
  }
#undef KCH_DIDX_CI
#undef KCH_DIDX
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.nr == 1) return e;
  hipLaunchKernelGGL(idx_merge_kernel, dim3((unsigned)p.B), dim3(256), decode_merge_lds(p.nr, p.topk), s, p);
  return hipGetLastError();
}

hipError_t decode_attn_dispatch(const DecodeAttnParams& p, int qdtype, int odtype, hipStream_t s) {
  const long long nw = (long long)p.B * p.nsplit;
  const dim3 grid((unsigned)((nw + 3) / 4)), block(256);
  if (p.hd == 128) {
    if (qdtype == DT_F32) hipLaunchKernelGGL((attn_part_kernel<128, float>), grid, block, 0, s, p);
    else if (qdtype == DT_BF16) hipLaunchKernelGGL((attn_part_kernel<128, bf16_t>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((attn_part_kernel<128, _Float16>), grid, block, 0, s, p);
  } else {
    if (qdtype == DT_F32) hipLaunchKernelGGL((attn_part_kernel<64, float>), grid, block, 0, s, p);
    else if (qdtype == DT_BF16) hipLaunchKernelGGL((attn_part_kernel<64, bf16_t>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((attn_part_kernel<64, _Float16>), grid, block, 0, s, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long outs = (long long)p.B * p.nh * (p.hd / 8);
  const dim3 g2((unsigned)((outs + 255) / 256));
  if (odtype == DT_F32) hipLaunchKernelGGL((attn_combine_kernel<float>), g2, block, 0, s, p);
  else if (odtype == DT_BF16) hipLaunchKernelGGL((attn_combine_kernel<bf16_t>), g2, block, 0, s, p);
  else hipLaunchKernelGGL((attn_combine_kernel<_Float16>), g2, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace kch
