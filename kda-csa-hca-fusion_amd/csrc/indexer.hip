// Lightning indexer with top-k block selection for gfx950.
//
// Restates csa_lightning_indexer (/root/reference/ops_csa.py:330-573), forward:
//   logits[t, n] = sum_h w_idx[t, h] * relu(scale * <q_idx[t, h], k_idx[n]>)
//   masked to -inf unless n < (t + 1) // m (ops_csa.py:179-195), then the top
//   min(topk, n_blocks) blocks by descending logit, -1 for -inf and for padding
//   (ops_csa.py:550-554). normalize_qk L2-normalises q_idx (here) and k_idx
//   (by the caller) first (ops_csa.py:503-525).
// Tie rule on exactly-equal logits: ascending block index (the reference's
// torch.topk order is unspecified there).
//
// Mapping: one 4-wave workgroup per group of QPW = 16 / nIh consecutive
// queries; MFMA column n = (query n / nIh, head n % nIh). The waves split the
// logits by 16-block chunk, then take one query's selection each. The key
// rows come as fp32, or already split as the compression kernel writes them
// for csa_core (which spares every workgroup the conversion). The logits carry
// fp32-level error, as the reference's fp32 einsum does:
//   KM 0: fp32 rows, split here into three bf16 parts (x = hi + mid + lo on
//         both sides; the six cross products down to 2^-16, terms of 2^-24
//         dropped);
//   KM 1: rows of the three bf16 parts [hi | mid | lo], the same products;
//   KM 2: L2-normalised rows as the two fp16 parts of 256 x [hi | lo] (q split
//         the same way; hi*hi + hi*lo + lo*hi is 2^16 times the dot product to
//         about 2^-22 relative): three MFMAs per step instead of six; with
//         k_split 3 the same parts chunk-major (16-row chunks in the lanes'
//         load order), so that each load instruction reads 1 KB of contiguous
//         memory in whole cache lines instead of 64 bytes of each of 16 rows
//         (half of every line it touches, each line fetched twice): the logits
//         of configs[2] take half the time.
// Per query, the logits sit
// in LDS as 32-bit order keys. A row of up to 256 * RG visible blocks is
// selected by one wave in registers (the k-th largest key found bit by bit
// with ballot counts); a longer row by an 8-bit radix select in LDS. Either
// way the keys above the boundary key and, of the keys equal to it, the
// lowest block indices are taken (ascending index on ties), in index order;
// when asked, they are bitonic-sorted by (logit desc, index asc). The head
// count is a template parameter: with it known, the lane's (query, head)
// split and the head sum compile to shifts and two or four lane exchanges.

#include <type_traits>

#include "attn_common.h"
#include "kch_csa.h"

namespace kch {

namespace {

// Order-preserving map float -> uint32 (larger float, larger key); -0 maps to +0
// so that the two zeros tie as they do in a float comparison.
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_excl_scan(int v) { return wave_incl_scan(v) - v; }

typedef unsigned long long u64;

// Unique ordered value of a logit key and its block index (larger key first,
// then lower index).
__device__ __forceinline__ u64 kv64(uint32_t key, int index) {
  return ((u64)key << 32) | (uint32_t)(~(uint32_t)index);
}

__device__ __forceinline__ u64 shfl_xor64(u64 v, int d) {
  const int lo = __shfl_xor((int)(uint32_t)v, d), hi = __shfl_xor((int)(uint32_t)(v >> 32), d);
  return ((u64)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Lanes below this one with their bit set in m.
__device__ __forceinline__ int mbcnt64(unsigned long long m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  // (every lane's source lies in its own row for the patterns used here, so
  // no old value is needed: bound_ctrl)
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Sum over the NIH adjacent lanes (a query's heads) of a 16-lane row, with DPP
// exchanges instead of LDS permutes: quad_perm [1,0,3,2] and [2,3,0,1] pair
// lanes within a quad; once every lane of a quad holds the quad's sum,
// row_half_mirror (lane i <-> 7 - i of each 8) and row_mirror (i <-> 15 - i)
// bring in the neighbouring quad's and half row's. Each step adds two
// partials that every lane of the pair holds bit for bit, so all NIH lanes end
// with the same sum.
template <int NIH>
__device__ __forceinline__ float head_sum(float v) {
  if constexpr (NIH >= 2) v += dpp_mov<0xb1>(v);
  if constexpr (NIH >= 4) v += dpp_mov<0x4e>(v);
  if constexpr (NIH >= 8) v += dpp_mov<0x141>(v);
  if constexpr (NIH >= 16) v += dpp_mov<0x140>(v);
  return v;
}

// Groups of 256 blocks whose order keys one wave holds in registers (4 per
// lane and group): rows of up to 256 * RG visible blocks are selected there.
constexpr int RG = 8;

// Unsorted output: the selected indices go straight to global memory, so the
// launch needs no selection buffers in LDS.
__host__ __device__ inline bool indexer_lean(const IndexerParams& p) { return !p.sorted; }

// LDS of a launch with CT column tiles (CT * 16 / nIh queries, 4 * CT waves):
// logits (rows of whole 16-block chunks) and 16-byte sink words per lane,
// per-wave histograms when a row can exceed the
// register selection (nb > 256 RG), per-wave selection buffers unless lean.
__host__ __device__ inline size_t indexer_lds(int nb, int nIh, int topk, bool lean, int ct = 1) {
  int ptop = 1;
  while (ptop < topk) ptop <<= 1;
  const int nwv = 4 * ct;
  size_t z = (size_t)(ct * 16 / nIh) * ((nb + 15) & ~15) * 4 + (size_t)nwv * 256 * 4;
  if (nb > 256 * RG) z += (size_t)nwv * 256 * 4;
  if (!lean) z += (size_t)nwv * ptop * 8;
  return z;
}

// Top-k of one query's logits row lg[0 .. nv) (LDS, 16-byte aligned) by one
// wave: the order keys go to registers (lane l holds blocks 256 g + 4 l + e),
// the k-th largest key K is found bit by bit from the most significant bit
// that differs among them, each step counting the keys >= a candidate with
// ballots and scalar popcounts, and the keys above K plus the lowest-indexed
// keys equal to K (as many as still needed: the reference's order with ties
// by ascending index) are written in ascending block order: to sel as
// (key, ~index) values, or without sel as block indices to out[0 .. topk),
// -1 past the selected count. The search stops at the first candidate that
// exactly topk keys reach: those keys are the selection (no key equal to the
// k-th lies below the candidate, so no tie is split), typically after about
// log2(rows) bits instead of all of them. No LDS atomics, no LDS traffic but
// one read of the row.
template <typename IdxT>
__device__ __forceinline__ void select_in_registers(const float* lg, int nv, int topk, int lane,
                                                    u64* sel, IdxT* out) {
  uint32_t key[4 * RG];  // 0 = no block (every order key of a float is above 0)
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int b0 = 256 * g + 4 * lane;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (b0 < nv) v = *reinterpret_cast<const float4*>(lg + b0);
    key[4 * g + 0] = b0 + 0 < nv ? order_key(v.x) : 0u;
    key[4 * g + 1] = b0 + 1 < nv ? order_key(v.y) : 0u;
    key[4 * g + 2] = b0 + 2 < nv ? order_key(v.z) : 0u;
    key[4 * g + 3] = b0 + 3 < nv ? order_key(v.w) : 0u;
  }
  // groups of 256 blocks that hold a visible block (wave-uniform): the counts
  // and the output pass skip the groups past them, whose keys are all 0
  const int ng = (nv + 255) >> 8;
  uint32_t K = 0u;  // with nv <= topk every block is taken: keys > 0
  int need = 0;
  if (nv > topk) {
    uint32_t a = ~0u, o = 0u;
#pragma unroll
    for (int r = 0; r < 4 * RG; ++r) {
      if (key[r]) {
        a &= key[r];
        o |= key[r];
      }
    }
#pragma unroll
    for (int d = 32; d; d >>= 1) {
      a &= (uint32_t)__shfl_xor((int)a, d);
      o |= (uint32_t)__shfl_xor((int)o, d);
    }
    // (uniform values, held in scalar registers: the search loop is scalar)
    a = __builtin_amdgcn_readfirstlane(a);
    o = __builtin_amdgcn_readfirstlane(o);
    const uint32_t diff = a ^ o;
    const int hb = diff ? 31 - __clz((int)diff) : -1;  // highest bit that differs
    K = hb >= 31 ? 0u : (a & (~0u << (hb + 1)));      // the common leading bits
    // The bit search, compiled per count of groups holding visible blocks (no
    // per-group branch in the loop); each group's four ballots are formed
    // before they are counted, so that they take four scalar register pairs
    // instead of queueing on one.
    auto search = [&](auto ngc) {
      constexpr int NG = decltype(ngc)::value;
      for (int bit = hb; bit >= 0; --bit) {
        const uint32_t cand = K | (1u << bit);
        int c = 0;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          u64 bl[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) bl[e] = __builtin_amdgcn_ballot_w64(key[4 * g + e] >= cand);
          c += (__popcll(bl[0]) + __popcll(bl[1])) + (__popcll(bl[2]) + __popcll(bl[3]));
        }
        if (c == topk) {
          // exactly topk keys are >= cand: taking every key above cand - 1
          // (none equal to it is needed) selects them
          K = cand - 1u;
          break;
        }
        if (c > topk) K = cand;
      }
    };
    static_assert(RG == 8, "one search per group count");
    switch (ng) {
      case 1: search(std::integral_constant<int, 1>{}); break;
      case 2: search(std::integral_constant<int, 2>{}); break;
      case 3: search(std::integral_constant<int, 3>{}); break;
      case 4: search(std::integral_constant<int, 4>{}); break;
      case 5: search(std::integral_constant<int, 5>{}); break;
      case 6: search(std::integral_constant<int, 6>{}); break;
      case 7: search(std::integral_constant<int, 7>{}); break;
      default: search(std::integral_constant<int, 8>{}); break;
    }
    int gt = 0;
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      if (g < ng) {
#pragma unroll
        for (int e = 0; e < 4; ++e) gt += __popcll(__builtin_amdgcn_ballot_w64(key[4 * g + e] > K));
      }
    }
    need = topk - gt;  // keys equal to K still to take, lowest block index first
  }
  // The output pass in ascending block order; without keys equal to K still
  // needed (the usual case: the search stopped at an exact split, or every
  // visible block is taken) the equal-key ranks are not formed.
  int base_out = 0;
  auto emit = [&](auto tiesc) {
    constexpr bool TIES = decltype(tiesc)::value;
    int base_eq = 0;
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      if (g >= ng) break;
      int eq_incl = 0, eq_rank = 0;
      if constexpr (TIES) {
        int neq = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) neq += (key[4 * g + e] == K && key[4 * g + e]) ? 1 : 0;
        eq_incl = wave_incl_scan(neq);
        eq_rank = base_eq + eq_incl - neq;
      }
      bool take[4];
      int ntake = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k = key[4 * g + e];
        take[e] = k > K;
        if constexpr (TIES) {
          const bool eq = k == K && k;
          take[e] = take[e] || (eq && eq_rank < need);
          eq_rank += eq ? 1 : 0;
        }
        ntake += take[e] ? 1 : 0;
      }
      const int out_incl = wave_incl_scan(ntake);
      int at = base_out + out_incl - ntake;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (take[e]) {
          if (sel) sel[at] = kv64(key[4 * g + e], 256 * g + 4 * lane + e);
          else out[at] = (IdxT)(256 * g + 4 * lane + e);
          ++at;
        }
      }
      base_out += __builtin_amdgcn_readlane(out_incl, 63);
      if constexpr (TIES) base_eq += __builtin_amdgcn_readlane(eq_incl, 63);
    }
  };
  if (need > 0) emit(std::true_type{});
  else emit(std::false_type{});
  if (!sel)
    for (int i = base_out + lane; i < topk; i += 64) out[i] = (IdxT)-1;
}

}  // namespace

template <typename QT, int CI, int NIH, int KM, int CT>
__global__ __launch_bounds__(256 * CT, CT == 2 ? 4 : 1) void indexer_kernel(IndexerParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int NS = CI / 32;
  constexpr int nIh = NIH;
  constexpr int NWV = 4 * CT;         // waves per workgroup
  constexpr int QPT = 16 / NIH;       // queries per column tile
  constexpr int QPW = CT * QPT;       // queries per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int q4 = lane >> 4, n = lane & 15;
  const int groups_per_row = (p.T + QPW - 1) / QPW;
  const int b = blockIdx.x / groups_per_row;
  const int t0 = (blockIdx.x - b * groups_per_row) * QPW;
  const int nb = p.nb;
  const int topk = p.topk;

  // logits row stride: whole 16-block chunks, so that a chunk's four logits
  // per lane are one aligned 16-byte store within the row
  const int ldl = (nb + 15) & ~15;
  const size_t lg_bytes = (size_t)QPW * ldl * 4;
  int ptop = 1;
  while (ptop < topk) ptop <<= 1;
  // LDS: logits [QPW][ldl] | sink words [NWV][64][4] | (nb > 256 RG) histograms
  // [NWV][256] | (unless lean) selections [NWV][ptop]. Lean: unsorted output,
  // whose indices go straight to global memory.
  const bool lean = indexer_lean(p);
  const size_t hist_bytes = nb > 256 * RG ? (size_t)NWV * 256 * 4 : 0;
  float* logits = reinterpret_cast<float*>(smem);
  float* sink = reinterpret_cast<float*>(smem + lg_bytes) + 256 * wave + 4 * (threadIdx.x & 63);
  uint32_t* hist = reinterpret_cast<uint32_t*>(smem + lg_bytes + NWV * 256 * 4) + 256 * wave;
  u64* sel = reinterpret_cast<u64*>(smem + lg_bytes + NWV * 256 * 4 + hist_bytes) + (size_t)ptop * wave;

  auto nvis_of = [&](int t) {
    if (p.dense_visible) return nb;
    const int v = (p.q_pos0 + t + 1) / p.m;
    return v < nb ? v : nb;
  };

  // ---- this lane's query columns: tile ct, query jq = ct QPT + n / nIh, head n % nIh ----
  const int hh = n % nIh;
  int jq[CT], tq[CT];
  bool qok[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    jq[ct] = ct * QPT + n / nIh;
    tq[ct] = t0 + jq[ct];
    qok[ct] = tq[ct] < p.T;
  }
  // q parts: bf16 hi / mid / lo (KM 0, 1) or fp16 hi / lo of 256 q (KM 2)
  bf16x8 qhi[CT][NS], qmid[CT][NS], qlo[CT][NS];
  f16x8 qh16[CT][NS], ql16[CT][NS];
  float wq[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    float f[NS][8];
    float ss = 0.f;
    const QT* qrow = static_cast<const QT*>(p.q_idx) +
                     (((size_t)b * p.T + (qok[ct] ? tq[ct] : 0)) * nIh + hh) * CI;
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
      for (int i = 0; i < 8; ++i) f[s][i] = qok[ct] ? f[s][i] * inv : 0.f;
      if constexpr (KM == 2) split2_f16(f[s], qh16[ct][s], ql16[ct][s]);
      else split3_bf16(f[s], qhi[ct][s], qmid[ct][s], qlo[ct][s]);
    }
    wq[ct] = 0.f;
    if (qok[ct]) {
      const size_t wi = ((size_t)b * p.T + tq[ct]) * nIh + hh;
      wq[ct] = p.w_idx ? ld_f32(static_cast<const QT*>(p.w_idx) + wi) : 1.f;
    }
  }

  // ---- logits of all blocks visible to any query of the group ----
  int nv_max = 0;
  for (int j = 0; j < QPW; ++j)
    if (t0 + j < p.T) nv_max = max(nv_max, nvis_of(t0 + j));
  int nv_me[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) nv_me[ct] = qok[ct] ? nvis_of(tq[ct]) : 0;
  // key rows of chunk c (row 16c + n, clamped: past the end the last row is
  // re-read and masked); wave w takes chunks w, w + NWV, ..., D in flight;
  // refills are unconditional so that no loaded register is copied. A row is
  // CI fp32 (KM 0: 4 bytes per channel, split here), CI bf16 high, middle and
  // low parts (KM 1: 6 bytes per channel), or CI fp16 high and low parts
  // (KM 2: 4 bytes per channel).
  constexpr int D = CT == 1 ? 4 : 2;
  constexpr int ROW_BYTES = KM == 1 ? 6 * CI : 4 * CI;
  const int nch = (nv_max + 15) / 16;
  const int mine = nch > wave ? (nch - wave + NWV - 1) / NWV : 0;
  // batch stride: k_bstride (4-byte units, fp32 rows only) or nb whole rows
  const bool chunked = KM == 2 && p.k_split == 3;
  const long long kbs = (KM == 0 && p.k_bstride) ? p.k_bstride * 4
                        : chunked                ? (long long)((nb + 15) & ~15) * ROW_BYTES
                                                 : (long long)nb * ROW_BYTES;
  const char* kbase = reinterpret_cast<const char*>(p.k_idx) + (size_t)b * kbs;
  struct KFrag3 {
    bf16x8 hi[NS], mid[NS], lo[NS];
  };
  struct KFrag2 {
    f16x8 hi[NS], lo[NS];
  };
  using KFrag = std::conditional_t<KM == 2, KFrag2, KFrag3>;
  auto load = [&](int c, KFrag& kf) {
    const int r = min(16 * c + n, nb - 1);
    const char* krow = kbase + (size_t)r * ROW_BYTES;
    if constexpr (KM == 2) {
      if (chunked) {
        // chunk c (past the last: the last, masked) as 2 NS pieces of 1 KB
        const int cc = min(c, (nb - 1) >> 4);
        const _Float16* kc =
            reinterpret_cast<const _Float16*>(kbase + (size_t)cc * 16 * ROW_BYTES) + 8 * lane;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          kf.hi[s] = *reinterpret_cast<const f16x8*>(kc + 512 * s);
          kf.lo[s] = *reinterpret_cast<const f16x8*>(kc + 512 * (NS + s));
        }
        return;
      }
      const _Float16* kh = reinterpret_cast<const _Float16*>(krow);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kf.hi[s] = *reinterpret_cast<const f16x8*>(kh + 32 * s + 8 * q4);
        kf.lo[s] = *reinterpret_cast<const f16x8*>(kh + CI + 32 * s + 8 * q4);
      }
    } else if constexpr (KM == 1) {
      const bf16_t* kh = reinterpret_cast<const bf16_t*>(krow);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kf.hi[s] = *reinterpret_cast<const bf16x8*>(kh + 32 * s + 8 * q4);
        kf.mid[s] = *reinterpret_cast<const bf16x8*>(kh + CI + 32 * s + 8 * q4);
        kf.lo[s] = *reinterpret_cast<const bf16x8*>(kh + 2 * CI + 32 * s + 8 * q4);
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        float f[8];
        Load8<float>::run(reinterpret_cast<const float*>(krow) + 32 * s + 8 * q4, f);
        split3_bf16(f, kf.hi[s], kf.mid[s], kf.lo[s]);
      }
    }
  };
  // the products' scale (2^-16 undoes the fp16 parts' 256 on both sides)
  // folded into the head weight: relu(a s) w = relu(a) (s w) for s > 0
  const float lscale = KM == 2 ? p.scale * kSplit16Unscale : p.scale;
  const bool fold = lscale > 0.f;
  float wqs[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) wqs[ct] = fold ? wq[ct] * lscale : wq[ct];
  const float ascale = fold ? 1.f : lscale;
  auto consume = [&](int c, const KFrag& kf) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      // the smallest cross products first, so that each later (larger) term
      // is added to an accumulator of the smaller ones
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KM == 2) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf.hi[s], ql16[ct][s], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf.lo[s], qh16[ct][s], acc, 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf.hi[s], qh16[ct][s], acc, 0, 0, 0);
      } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf.mid[s], qmid[ct][s], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf.hi[s], qlo[ct][s], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf.lo[s], qhi[ct][s], acc, 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf.hi[s], qmid[ct][s], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf.mid[s], qhi[ct][s], acc, 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf.hi[s], qhi[ct][s], acc, 0, 0, 0);
      }
      // acc[e]: block 16c + 4*q4 + e, column n. The head-0 lane of a query
      // writes its four logits as one 16-byte store into the query's row
      // (whole chunks fit the padded row; blocks past the query's visible
      // count hold finite values that its selection never reads); the other
      // lanes, and every lane of a chunk past the last (uniform), write this
      // lane's sink words. No branch: one would cost the overlap of the
      // chunks loaded ahead.
      f32x4 v;
      if (fold) {  // (uniform) the scale is in the head weight
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = head_sum<NIH>(fmaxf(acc[e], 0.f) * wqs[ct]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = head_sum<NIH>(fmaxf(acc[e] * ascale, 0.f) * wqs[ct]);
      }
      float* dst = (hh == 0 && c < nch) ? logits + jq[ct] * ldl + 16 * c + 4 * q4 : sink;
      *reinterpret_cast<f32x4*>(dst) = v;
    }
  };
  KFrag kf[D];
  // (issued in order, each refill right after its consumer: the scheduler
  // would otherwise reorder them, and the wait before a chunk's use would then
  // also cover the chunks loaded after it)
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(wave + NWV * d, kf[d]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // chunks past this wave's last are consumed too: their blocks lie beyond
  // every query's visible count, so nothing is stored (a condition here would
  // cost the loads' overlap)
  for (int m0 = 0; m0 < mine; m0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(wave + NWV * (m0 + d), kf[d]);
      load(wave + NWV * (m0 + d + D), kf[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();

  // ---- per query: top-k (wave w takes queries w, w + NWV, ...) ----
  // Rows of up to 256 * RG visible blocks: select_in_registers. Longer rows:
  // an 8-bit radix select on the order keys below the leading bits common to
  // all of them, stopped as soon as the boundary digit holds exactly the keys
  // still needed, then one gather in index order. The selected (key, ~index)
  // values are sorted (descending) only when asked.
  constexpr int U = 8;  // LDS reads in flight per pass
  for (int j = wave; j < QPW; j += NWV) {
    const int t = t0 + j;
    if (t >= p.T) break;
    const int nv = nvis_of(t);
    const float* lg = logits + (size_t)j * ldl;
    const size_t orow = ((size_t)b * p.T + t) * topk;
    if (p.logits_out) {
      for (int i = lane; i < nb; i += 64)
        p.logits_out[((size_t)b * p.T + t) * nb + i] = i < nv ? lg[i] : -INFINITY;
    }
    // The radix select runs on the 32-bit order keys (written over the logits
    // in place by the first pass). It finds the boundary key K: every key
    // above K is taken, and of the keys equal to K the lowest indices, as
    // many as still needed -- the reference's order (descending logit, ties
    // by ascending index). A select stopped early (its boundary digit taken
    // whole) takes every key in or above the boundary bin.
    uint32_t* lk = reinterpret_cast<uint32_t*>(const_cast<float*>(lg));
    const int cnt = nv < topk ? nv : topk;
    if (nv <= 256 * RG) {
      if (lean) {
        if (p.idx64)
          select_in_registers(lg, nv, topk, lane, nullptr, static_cast<long long*>(p.idx_out) + orow);
        else
          select_in_registers(lg, nv, topk, lane, nullptr, static_cast<int*>(p.idx_out) + orow);
        continue;  // the indices are written
      }
      select_in_registers(lg, nv, topk, lane, sel, static_cast<int*>(nullptr));
    } else {
    uint32_t thr = 0u, mask = 0u;  // with mask = 0 every key is in the boundary bin
    int tie_take = 0x7fffffff;      // boundary-bin keys taken (in index order)
    if (nv > topk) {
      uint32_t a = ~0u, o = 0u;
      for (int i = lane; i < nv; i += 64) {
        const uint32_t k = order_key(lg[i]);
        lk[i] = k;
        a &= k;
        o |= k;
      }
#pragma unroll
      for (int d = 32; d; d >>= 1) {
        a &= (uint32_t)__shfl_xor((int)a, d);
        o |= (uint32_t)__shfl_xor((int)o, d);
      }
      wave_lds_sync();  // keys in place before the passes read them
      int lo_bit = (a ^ o) ? 32 - __clz((int)(a ^ o)) : 0;
      mask = lo_bit >= 32 ? 0u : (~0u << lo_bit);
      thr = a & mask;
      int need = topk;
      bool whole = false;  // the last pass took its boundary digit whole
      while (lo_bit > 0) {
        const int w = lo_bit < 8 ? lo_bit : 8;
        const int shift = lo_bit - w;
        const uint32_t dm = (1u << w) - 1u;
#pragma unroll
        for (int k = 0; k < 4; ++k) hist[lane + 64 * k] = 0u;
        // a wave's LDS operations complete in order: the clear precedes the adds
        for (int i0 = 0; i0 < nv; i0 += 64 * U) {
          uint32_t v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) v[u] = lk[min(i0 + 64 * u + lane, nv - 1)];
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (i0 + 64 * u + lane < nv && (v[u] & mask) == thr) atomicAdd(&hist[(v[u] >> shift) & dm], 1u);
        }
        wave_lds_sync();
        // digits in descending order: lane l holds dm - 4l .. dm - 4l - 3
        int c[4], tot = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int bin = (int)dm - 4 * lane - k;
          c[k] = bin >= 0 ? (int)hist[bin] : 0;
          tot += c[k];
        }
        int cum = wave_excl_scan(tot);
        int found_bin = -1, found_above = 0, found_cnt = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (found_bin < 0 && cum < need && cum + c[k] >= need) {
            found_bin = (int)dm - 4 * lane - k;
            found_above = cum;
            found_cnt = c[k];
          }
          cum += c[k];
        }
        const unsigned long long who = __ballot(found_bin >= 0);
        const int src = __ffsll((long long)who) - 1;
        const int bin = __shfl(found_bin, src);
        const int above = __shfl(found_above, src);
        const int bcnt = __shfl(found_cnt, src);
        wave_lds_sync();  // histogram reads done before the next pass clears it
        thr |= (uint32_t)bin << shift;
        mask |= dm << shift;
        need -= above;
        lo_bit = shift;
        if (bcnt == need) {  // the boundary digit's keys are all taken
          whole = true;
          break;
        }
      }
      if (!whole) tie_take = need;  // all 32 bits fixed: `need` of the keys equal to thr
    } else {
      for (int i = lane; i < nv; i += 64) lk[i] = order_key(lg[i]);
      wave_lds_sync();
    }
    // gather the cnt selected values (key, ~index) in index order; lean: the
    // indices straight to global memory, -1 past the selected count
    int at = 0, eqs = 0;
    for (int i0 = 0; i0 < nv; i0 += 64) {
      const int i = i0 + lane;
      const uint32_t k = i < nv ? lk[i] : 0u;
      const bool gt = i < nv && (k & mask) > thr;
      const bool eq = i < nv && (k & mask) == thr;
      const unsigned long long em = __ballot(eq);
      const bool tk = gt || (eq && eqs + mbcnt64(em) < tie_take);
      const unsigned long long tm = __ballot(tk);
      if (tk) {
        const int o = at + mbcnt64(tm);
        if (!lean) sel[o] = kv64(k, i);
        else if (p.idx64) static_cast<long long*>(p.idx_out)[orow + o] = i;
        else static_cast<int*>(p.idx_out)[orow + o] = i;
      }
      at += __popcll(tm);
      eqs += __popcll(em);
    }
    if (lean) {
      for (int i = at + lane; i < topk; i += 64) {
        if (p.idx64) static_cast<long long*>(p.idx_out)[orow + i] = -1;
        else static_cast<int*>(p.idx_out)[orow + i] = -1;
      }
      wave_lds_sync();  // this wave's reads of its row and histogram are done
      continue;
    }
    }
    wave_lds_sync();  // the selected values are in LDS
    if (p.sorted && cnt > 1) {
      // pad to a power of two with values that sort last, bitonic sort descending
      int pw = 1;
      while (pw < cnt) pw <<= 1;
      for (int i = cnt + lane; i < pw; i += 64) sel[i] = 0ull;
      wave_lds_sync();
      for (int k = 2; k <= pw; k <<= 1) {
        for (int jj = k >> 1; jj > 0; jj >>= 1) {
          for (int i = lane; i < pw / 2; i += 64) {
            const int lo = ((i & ~(jj - 1)) << 1) | (i & (jj - 1));
            const int hi = lo + jj;
            const u64 x = sel[lo], y = sel[hi];
            const bool desc = (lo & k) == 0;
            if (desc ? (x < y) : (x > y)) { sel[lo] = y; sel[hi] = x; }
          }
          wave_lds_sync();
        }
      }
    } else {
      wave_lds_sync();
    }
    // write indices (-1 beyond the selected count)
    for (int i = lane; i < topk; i += 64) {
      const int id = i < cnt ? (int)(~(uint32_t)(sel[i] & 0xffffffffull)) : -1;
      if (p.idx64) static_cast<long long*>(p.idx_out)[orow + i] = id;
      else static_cast<int*>(p.idx_out)[orow + i] = id;
    }
    wave_lds_sync();
  }
}

size_t indexer_lds_bytes(int nb, int nIh, int topk) { return indexer_lds(nb, nIh, topk, false); }

// Two column tiles (8 waves, twice the queries per key row read) when the
// logits of twice the queries leave room for two workgroups per CU; one
// otherwise, and for a single query per row (decode).
static int indexer_ct(const IndexerParams& p) {
  // (fp16-split keys of up to 64 channels: other row formats and widths need
  // more registers for a second tile than four waves per SIMD leave)
  return p.k_split >= 2 && p.cI <= 64 && p.T >= 16 &&
                 indexer_lds(p.nb, p.nIh, p.topk, indexer_lean(p), 2) <= 80 * 1024
             ? 2
             : 1;
}

hipError_t indexer_dispatch(const IndexerParams& p, int dtype, hipStream_t s) {
  const int CT = indexer_ct(p);
  const int QPW = CT * 16 / p.nIh;
  const size_t lds = indexer_lds(p.nb, p.nIh, p.topk, indexer_lean(p), CT);
  const unsigned groups = (unsigned)(p.B * ((p.T + QPW - 1) / QPW));
#define KCH_IDX_T(QT, CI, NIH, KS)                                                                   \
  do {                                                                                              \
    if (KS == 2 && CI <= 64 && CT == 2)                                                             \
      hipLaunchKernelGGL((indexer_kernel<QT, CI, NIH, KS, (KS == 2 && CI <= 64 ? 2 : 1)>), dim3(groups), \
                         dim3(512), lds, s, p);                                                     \
    else                                                                                            \
      hipLaunchKernelGGL((indexer_kernel<QT, CI, NIH, KS, 1>), dim3(groups), dim3(256), lds, s, p);  \
  } while (0)
#define KCH_IDX_NIH(QT, CI, NIH)                   \
  do {                                             \
    if (p.k_split >= 2) KCH_IDX_T(QT, CI, NIH, 2); \
    else if (p.k_split) KCH_IDX_T(QT, CI, NIH, 1); \
    else KCH_IDX_T(QT, CI, NIH, 0);                \
  } while (0)
#define KCH_IDX_LAUNCH(QT, CI)                \
  do {                                        \
    switch (p.nIh) {                          \
      case 1: KCH_IDX_NIH(QT, CI, 1); break;  \
      case 2: KCH_IDX_NIH(QT, CI, 2); break;  \
      case 4: KCH_IDX_NIH(QT, CI, 4); break;  \
      case 8: KCH_IDX_NIH(QT, CI, 8); break;  \
      default: KCH_IDX_NIH(QT, CI, 16); break; \
    }                                         \
  } while (0)
  if (dtype == DT_BF16) {
    if (p.cI == 64) KCH_IDX_LAUNCH(bf16_t, 64);
    else if (p.cI == 128) KCH_IDX_LAUNCH(bf16_t, 128);
    else KCH_IDX_LAUNCH(bf16_t, 32);
  } else if (dtype == DT_F32) {
    if (p.cI == 64) KCH_IDX_LAUNCH(float, 64);
    else if (p.cI == 128) KCH_IDX_LAUNCH(float, 128);
    else KCH_IDX_LAUNCH(float, 32);
  } else {
    if (p.cI == 64) KCH_IDX_LAUNCH(_Float16, 64);
    else if (p.cI == 128) KCH_IDX_LAUNCH(_Float16, 128);
    else KCH_IDX_LAUNCH(_Float16, 32);
  }
#undef KCH_IDX_LAUNCH
#undef KCH_IDX_NIH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Row-wise L2 normalisation (one wave per row, rows of up to 256 channels).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void l2norm_rows_kernel(const T* x, long long ldx, void* out,
                                                          int out_f32, int rows, int c, int normalize) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int ch = lane + 64 * u;
    v[u] = ch < c ? to_f32(x[(size_t)row * ldx + ch]) : 0.f;
    ss += v[u] * v[u];
  }
  const float inv = normalize ? l2_inv(wave_sum(ss)) : 1.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int ch = lane + 64 * u;
    if (ch >= c) continue;
    if (out_f32) static_cast<float*>(out)[(size_t)row * c + ch] = v[u] * inv;
    else static_cast<bf16_t*>(out)[(size_t)row * c + ch] = (bf16_t)(v[u] * inv);
  }
}

hipError_t l2norm_rows_dispatch(const void* x, long long ldx, void* out, int out_f32, int rows,
                                int c, int normalize, int dtype, hipStream_t s) {
  const dim3 grid((rows + 3) / 4), block(256);
  if (dtype == DT_F32)
    hipLaunchKernelGGL((l2norm_rows_kernel<float>), grid, block, 0, s, static_cast<const float*>(x), ldx,
                       out, out_f32, rows, c, normalize);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL((l2norm_rows_kernel<bf16_t>), grid, block, 0, s, static_cast<const bf16_t*>(x),
                       ldx, out, out_f32, rows, c, normalize);
  else
    hipLaunchKernelGGL((l2norm_rows_kernel<_Float16>), grid, block, 0, s,
                       static_cast<const _Float16*>(x), ldx, out, out_f32, rows, c, normalize);
  return hipGetLastError();
}

}  // namespace kch
