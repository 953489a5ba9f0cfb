// Decode-step kernels for the CSA / HCA caches (one new token per sequence).
//
// Restates CSADecodingCache.forward_step (/root/reference/ops_decoding_cache.py:783-1070)
// and HCADecodingCache.forward_step (:1268-1395) for long caches: a decode step
// is bound by reading the cache, so every kernel splits the cache across many
// workgroups instead of giving one workgroup to each sequence.
//
// idx_range_kernel   lightning-indexer logits of one range of <= RB_MAX cached
//   blocks of one sequence (ops_csa.py:503-536: relu(scale q_h . k_n / ||k_n||),
//   weighted head sum), then the range's top-k. Keys are the cached rows as
//   stored (cache dtype) times a per-row fp32 1/||k|| (1 without
//   normalisation); q is split into three bf16 parts hi + mid + lo, so a bf16
//   key row gives the logit to fp32-level error with three MFMAs (fp16 / fp32
//   rows are split the same way, six MFMAs). Each logit becomes a unique
//   64-bit value (order-preserving key, then the complement of the block
//   index), so "larger value" is exactly the reference's order with ties taken
//   in ascending block index, and a selection needs no tie bookkeeping.
//   Selection: each thread holds 32 values in registers; a threshold
//   estimated from 256 evenly spaced samples narrows an exact radix select
//   (reg_select) to the values at or above it (about 2 topk of them), all
//   values when the estimate misses. One range per sequence: sorted and final; otherwise the range's
//   top-k are candidates.
//   With keys_out the range only writes its logit keys there (score pass of
//   a score / select split).
// idx_select_kernel  the top-k of all logit keys of a sequence (at most
//   RB_MAX, held in LDS): radix select over the ordered 64-bit values, gather,
//   rank sort; output sorted, -1 padded.
// idx_merge_kernel   the top-k of the candidates of all ranges of a sequence
//   (a global top-k lies in the union of the per-range top-ks), by the same
//   estimate-gather-select over the candidates streamed from global memory;
//   output sorted by value (logit desc, index asc).
// attn_kernel   joint-softmax MQA over a group of the attended rows of a
//   sequence (selected or all compressed blocks, then the ring window): per
//   wave and head M, L and the unnormalised o (MqaWave), merged across the
//   workgroup; attn_combine_kernel merges the groups' partials and adds the
//   sink:
//   o = sum_s o_s 2^(M_s-M) / (sum_s L_s 2^(M_s-M) + e^sink 2^-M), 0 when no
//   row is valid (the all-invalid rule of ops_decoding_cache.py:1044-1059).

#include <type_traits>

#include "attn_common.h"
#include "kch_csa.h"

namespace kch {

namespace {

constexpr int RB_MAX = 8192;     // blocks per indexer range (keys held in LDS)
constexpr int WG_TARGET = 1024;  // indexer workgroups worth splitting a small batch for
constexpr int SV_CAP = 2048;     // key positions a range gathers at or above its estimate
constexpr int MV_CAP = 4096;     // candidates the merge gathers at or above its estimate

__device__ __forceinline__ uint32_t okey(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave index within the block, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Lanes below this one with their bit set in m.
__device__ __forceinline__ int mbcnt64(unsigned long long m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 32; d; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

// Exclusive prefix sum over the 256 threads of the block (scratch: 4 ints).
__device__ __forceinline__ int block_excl_scan(int v, int* scratch) {
  const int lane = threadIdx.x & 63, wave = wave_id();
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

typedef unsigned long long u64;

// Ordered value of a logit key and its block index: unique within a sequence,
// and larger for a larger logit, then for a lower index (the tie rule).
__device__ __forceinline__ u64 kv64(uint32_t key, int index) {
  return ((u64)key << 32) | (uint32_t)(~(uint32_t)index);
}
__device__ __forceinline__ int kv64_index(u64 v) { return (int)(~(uint32_t)(v & 0xffffffffull)); }

__device__ __forceinline__ u64 shfl_xor64(u64 v, int d) {
  const int lo = __shfl_xor((int)(uint32_t)v, d), hi = __shfl_xor((int)(uint32_t)(v >> 32), d);
  return ((u64)(uint32_t)hi << 32) | (uint32_t)lo;
}

// The topk largest of a set of unique values: exactly those with
// (v & mask) >= thr (mask: a run of leading ones).
struct Sel64 {
  u64 thr, mask;
};

// Radix select of the topk largest of n unique 64-bit values val(i), i < n,
// topk < n, by a 256-thread block. The leading bits common to all values are
// skipped (an AND / OR reduction); 8-bit digits are then resolved high to low
// and the search stops as soon as the boundary digit holds exactly the values
// still needed (at the latest when one value is left). hist: 256 words,
// scratch: 12 ints.
template <int SPLIT = 1, typename ValF>
__device__ Sel64 block_select64(ValF val, int n, int topk, uint32_t* hist, int* scratch) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  u64 a = ~0ull, o = 0ull;
  for (int i = tid; i < n; i += 256) {
    const u64 v = val(i);
    a &= v;
    o |= v;
  }
#pragma unroll
  for (int d = 32; d; d >>= 1) {
    a &= shfl_xor64(a, d);
    o |= shfl_xor64(o, d);
  }
  u64* s64 = reinterpret_cast<u64*>(scratch);  // 8 words = scratch[0 .. 15]
  if (lane == 0) {
    s64[wave] = a;
    s64[4 + wave] = o;
  }
  __syncthreads();
  a = s64[0] & s64[1] & s64[2] & s64[3];
  o = s64[4] | s64[5] | s64[6] | s64[7];
  __syncthreads();
  int lo_bit = 64 - __clzll((long long)(a ^ o));  // values differ (n >= 2): lo_bit >= 1
  u64 mask = lo_bit >= 64 ? 0ull : (~0ull << lo_bit);
  u64 thr = a & mask;
  int need = topk;
  while (lo_bit > 0) {
    const int w = lo_bit < 8 ? lo_bit : 8;
    const int shift = lo_bit - w;
    const uint32_t dm = (1u << w) - 1u;
#pragma unroll
    for (int w2 = 0; w2 < SPLIT; ++w2) hist[256 * w2 + tid] = 0u;
    __syncthreads();
    // SPLIT > 1: wave w counts into copy w % SPLIT (fewer colliding atomics)
    uint32_t* hw = hist + 256 * (wave % SPLIT);
    for (int i = tid; i < n; i += 256) {
      const u64 v = val(i);
      if ((v & mask) == thr) atomicAdd(&hw[(uint32_t)(v >> shift) & dm], 1u);
    }
    __syncthreads();
    // thread t: digit dm - t (descending); count of values in larger digits
    const int bin = (int)dm - tid;
    int c = 0;
    if (bin >= 0) {
#pragma unroll
      for (int w2 = 0; w2 < SPLIT; ++w2) c += (int)hist[256 * w2 + bin];
    }
    const int cum = block_excl_scan(c, scratch + 16);
    if (bin >= 0 && cum < need && cum + c >= need) {
      scratch[20] = bin;
      scratch[21] = cum;
      scratch[22] = c;
    }
    __syncthreads();
    const int sb = scratch[20], above = scratch[21], cnt = scratch[22];
    __syncthreads();
    thr |= (u64)sb << shift;
    mask |= (u64)dm << shift;
    need -= above;
    lo_bit = shift;
    if (cnt == need) break;  // the boundary digit's values are all taken
  }
  return Sel64{thr, mask};
}

// Calls put(slot, i, v) for every i < n with pred(v), v = val(i), slots 0,
// 1, ... in no particular order; slots past cap are skipped. *counter (LDS,
// zero on entry) ends as the number of such i. One LDS atomic per wave and 64
// values.
template <typename ValF, typename PredF, typename PutF>
__device__ void block_gather(ValF val, int n, PredF pred, PutF put, int cap, int* counter) {
  const int lane = threadIdx.x & 63;
  for (int base = wave_id() * 64; base < n; base += 256) {
    const int i = base + lane;
    u64 v = 0ull;
    bool t = false;
    if (i < n) {
      v = val(i);
      t = pred(v);
    }
    const u64 m = __ballot(t);
    if (m) {
      int at = 0;
      if (lane == 0) at = atomicAdd(counter, __popcll(m));
      at = __builtin_amdgcn_readlane(at, 0) + mbcnt64(m);
      if (t && at < cap) put(at, i, v);
    }
  }
}

// An estimate, from evenly spaced samples, of a value that at least topk of
// the n values reach: the sample ranked r among S = min(n, 256) samples, with
// r chosen three standard deviations past topk S / n. Returns false (no
// estimate) when the samples cannot bound the set below `cap` values or half
// of n. smp: 256 words of LDS, 16-byte aligned; scratch: 48 ints.
template <typename ValF>
__device__ bool sample_estimate(ValF val, int n, int topk, int cap, u64* smp, int* scratch, u64* est) {
  const int tid = threadIdx.x;
  const int S = n < 256 ? n : 256;
  const float ex = (float)topk * (float)S / (float)n;
  const int r = (int)ceilf(ex + 3.f * sqrtf(ex) + 2.f) - 1;
  const float keep = (float)(r + 1) * (float)n / (float)S * 1.25f;
  if (2 * (r + 1) > S || keep > (float)cap) return false;
  u64 v = 0ull;
  if (tid < S) v = val((int)(((long long)tid * n) / S));
  smp[tid] = v;  // zeros past S rank below every value
  __syncthreads();
  if (tid < S) {
    int rank = 0;
#pragma unroll 8
    for (int u = 0; u < S; u += 2) {
      const ulonglong2 pr = *reinterpret_cast<const ulonglong2*>(smp + u);
      rank += (pr.x > v) + (pr.y > v);
    }
    if (rank == r) *reinterpret_cast<u64*>(scratch + 40) = v;
  }
  __syncthreads();
  *est = *reinterpret_cast<const u64*>(scratch + 40);
  return true;
}

// Block-wide count, AND and OR (scratch: ints 0 .. 23, 8-byte aligned).
__device__ __forceinline__ void block_cnt_and_or(int& c, u64& a, u64& o, int* scratch) {
  const int lane = threadIdx.x & 63, wave = wave_id();
#pragma unroll
  for (int d = 32; d; d >>= 1) {
    c += __shfl_xor(c, d);
    a &= shfl_xor64(a, d);
    o |= shfl_xor64(o, d);
  }
  u64* s64 = reinterpret_cast<u64*>(scratch);
  if (lane == 0) {
    s64[wave] = a;
    s64[4 + wave] = o;
    scratch[16 + wave] = c;
  }
  __syncthreads();
  a = s64[0] & s64[1] & s64[2] & s64[3];
  o = s64[4] | s64[5] | s64[6] | s64[7];
  c = scratch[16] + scratch[17] + scratch[18] + scratch[19];
  __syncthreads();
}

// Radix select over values a thread holds: src.load(g) fetches them into
// registers g (once per pass, all reads issued together), src.get(g, k, ok)
// returns the k-th (k < R) and whether it takes part. The cnt > topk
// participating values have AND a and OR o. Returns thr / mask such that
// exactly topk of them have (v & mask) >= thr. 8-bit digits below the common
// prefix, high to low, histograms double-buffered so that a pass takes three
// barriers; stops once the boundary digit holds exactly the values still
// needed. hist: 512 words; scratch: ints 24 .. 31.
template <int R, typename Src>
__device__ Sel64 reg_select(const Src& src, int topk, u64 a, u64 o, uint32_t* hist, int* scratch) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  int lo_bit = 64 - __clzll((long long)(a ^ o));
  u64 mask = lo_bit >= 64 ? 0ull : (~0ull << lo_bit);
  u64 thr = a & mask;
  int need = topk, buf = 0;
  hist[tid] = 0u;
  hist[256 + tid] = 0u;
  __syncthreads();
  while (lo_bit > 0) {
    const int w = lo_bit < 8 ? lo_bit : 8;
    const int shift = lo_bit - w;
    const uint32_t dm = (1u << w) - 1u;
    uint32_t* h = hist + 256 * buf;
    typename Src::Regs g;
    src.load(g);
#pragma unroll
    for (int k = 0; k < R; ++k) {
      bool ok;
      const u64 v = src.get(g, k, ok);
      if (ok && (v & mask) == thr) atomicAdd(&h[(uint32_t)(v >> shift) & dm], 1u);
    }
    __syncthreads();
    hist[256 * (buf ^ 1) + tid] = 0u;  // the next pass's histogram
    // thread t: digit dm - t (descending); values in larger digits
    const int bin = (int)dm - tid;
    const int c = bin >= 0 ? (int)h[bin] : 0;
    int x = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d);
      if (lane >= d) x += y;
    }
    if (lane == 63) scratch[24 + wave] = x;
    __syncthreads();
    int cum = x - c;
    for (int w2 = 0; w2 < wave; ++w2) cum += scratch[24 + w2];
    if (bin >= 0 && cum < need && cum + c >= need) {
      scratch[28] = bin;
      scratch[29] = cum;
      scratch[30] = c;
    }
    __syncthreads();
    const int sb = scratch[28], above = scratch[29], cnt = scratch[30];
    thr |= (u64)sb << shift;
    mask |= (u64)dm << shift;
    need -= above;
    lo_bit = shift;
    buf ^= 1;
    if (cnt == need) break;  // the boundary digit's values are all taken
  }
  return Sel64{thr, mask};
}

// Block-wide count, AND and OR of the participating values of src.
template <int R, typename Src>
__device__ void reg_census(const Src& src, int& c, u64& a, u64& o, int* scratch) {
  typename Src::Regs g;
  src.load(g);
  c = 0;
  a = ~0ull;
  o = 0ull;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    bool ok;
    const u64 v = src.get(g, k, ok);
    c += ok;
    a &= ok ? v : ~0ull;
    o |= ok ? v : 0ull;
  }
  block_cnt_and_or(c, a, o, scratch);
}

// put(slot, v) for this thread's participating values with (v & mask) >= thr
// (all of them when take_all), slots 0, 1, ... in no particular order: one
// LDS atomic per wave. *counter (LDS) is zero on entry.
template <int R, typename Src, typename PutF>
__device__ void reg_gather(const Src& src, Sel64 sl, bool take_all, PutF put, int* counter) {
  const int lane = threadIdx.x & 63;
  typename Src::Regs g;
  src.load(g);
  int c = 0;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    bool ok;
    const u64 v = src.get(g, k, ok);
    c += ok && (take_all || (v & sl.mask) >= sl.thr);
  }
  int x = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  int base = 0;
  if (lane == 63 && x) base = atomicAdd(counter, x);
  int at = __builtin_amdgcn_readlane(base, 63) + x - c;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    bool ok;
    const u64 v = src.get(g, k, ok);
    if (ok && (take_all || (v & sl.mask) >= sl.thr)) put(at++, v);
  }
}

// Writes out(rank, v) for the cnt unique values s[0 .. cnt) (rank 0 = the
// largest), s 16-byte aligned with a zero at s[cnt] when cnt is odd; each
// thread ranks EPT values against all of them, two per LDS read.
template <int EPT, typename OutF>
__device__ void block_rank_sort(const u64* s, int cnt, OutF out) {
  const int tid = threadIdx.x;
  u64 v[EPT];
  int rk[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = tid + 256 * e;
    v[e] = i < cnt ? s[i] : ~0ull;
    rk[e] = 0;
  }
#pragma unroll 4
  for (int f = 0; f < cnt; f += 2) {
    const ulonglong2 pr = *reinterpret_cast<const ulonglong2*>(s + f);
#pragma unroll
    for (int e = 0; e < EPT; ++e) rk[e] += (pr.x > v[e]) + (pr.y > v[e]);
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e)
    if (tid + 256 * e < cnt) out(rk[e], v[e]);
}

// Bitonic sort of s[0 .. cnt) descending, padded to a power of two with zeros.
__device__ void block_sort_desc(u64* s, int cnt) {
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
        const u64 x = s[a], y = s[c];
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

// Bitonic sort, descending, of the cnt values s[0 .. cnt) padded with zeros to
// P = 256 EPT (zeros rank below every value); out(rank, v) for each value.
// Wave w holds positions 64 EPT w .. + 64 EPT - 1 in registers, lane l the EPT
// consecutive ones from 64 EPT w + EPT l: stages whose partner distance is
// below EPT compare within the lane, those below 64 EPT exchange by lane
// shuffles, and only the last stages of the two largest merges go through s
// (which holds P words).
template <int EPT, typename OutF>
__device__ void block_bitonic_desc(u64* s, int cnt, OutF out) {
  constexpr int P = 256 * EPT, WCH = 64 * EPT;
  constexpr int LOGP = EPT == 1 ? 8 : (EPT == 2 ? 9 : 10);
  static_assert((1 << LOGP) == P, "EPT in {1, 2, 4}");
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int base = wave * WCH + EPT * lane;
  u64 x[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) x[e] = base + e < cnt ? s[base + e] : 0ull;
  // constant trip counts: every stage unrolled, x indexed by constants
#pragma unroll
  for (int kk = 1; kk <= LOGP; ++kk) {
    const int k = 1 << kk;
#pragma unroll
    for (int jj = kk - 1; jj >= 0; --jj) {
      const int j = 1 << jj;
      // position p keeps the larger of the pair when it is the lower one of a
      // descending run or the upper one of an ascending run
      if (j >= WCH) {
        __syncthreads();  // every read of s by the previous stage is done
#pragma unroll
        for (int e = 0; e < EPT; ++e) s[base + e] = x[e];
        __syncthreads();
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const int p = base + e;
          const u64 y = s[p ^ j];
          const bool keep_max = ((p & j) == 0) == ((p & k) == 0);
          x[e] = keep_max ? (x[e] > y ? x[e] : y) : (x[e] < y ? x[e] : y);
        }
      } else if (j >= EPT) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const int p = base + e;
          const u64 y = shfl_xor64(x[e], j / EPT);
          const bool keep_max = ((p & j) == 0) == ((p & k) == 0);
          x[e] = keep_max ? (x[e] > y ? x[e] : y) : (x[e] < y ? x[e] : y);
        }
      } else {
        u64 nx[EPT];
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const int p = base + e;
          const u64 y = x[e ^ j];
          const bool keep_max = ((p & j) == 0) == ((p & k) == 0);
          nx[e] = keep_max ? (x[e] > y ? x[e] : y) : (x[e] < y ? x[e] : y);
        }
#pragma unroll
        for (int e = 0; e < EPT; ++e) x[e] = nx[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e)
    if (base + e < cnt) out(base + e, x[e]);
}

// Sorts the cnt selected values s[0 .. cnt) descending and writes their block
// indices to out[0 .. topk), -1 past cnt. s holds pow2_at_least(cnt + 1)
// words, 16-byte aligned. BITONIC: a bitonic network for 256 < cnt <= 1024
// (where s has room for its padding); kernels held to 128 VGPRs keep the rank
// count, whose registers they can afford.
template <bool BITONIC>
__device__ void write_sorted(u64* s, int cnt, int topk, int* out) {
  const int tid = threadIdx.x;
  for (int i = cnt + tid; i < topk; i += 256) out[i] = -1;
  auto put_idx = [&](int rank, u64 v) { out[rank] = kv64_index(v); };
  if constexpr (BITONIC) {
    if (cnt > 256 && cnt <= 512) {
      block_bitonic_desc<2>(s, cnt, put_idx);
      return;
    }
    if (cnt > 512 && cnt <= 1024) {
      block_bitonic_desc<4>(s, cnt, put_idx);
      return;
    }
  }
  if (cnt <= 2048) {
    if (tid == 0 && (cnt & 1)) s[cnt] = 0ull;
    __syncthreads();
    if (cnt <= 256) block_rank_sort<1>(s, cnt, put_idx);
    else if (cnt <= 512) block_rank_sort<2>(s, cnt, put_idx);
    else if (cnt <= 1024) block_rank_sort<4>(s, cnt, put_idx);
    else block_rank_sort<8>(s, cnt, put_idx);
  } else {
    block_sort_desc(s, cnt);
    for (int i = tid; i < cnt; i += 256) out[i] = kv64_index(s[i]);
  }
}

__host__ __device__ inline int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Eight key elements of one row as stored: bf16 rows feed the MFMA as they
// are; fp16 / fp32 rows are split into bf16 hi + mid + lo when consumed.
template <typename KT>
struct KeyFrag {
  bf16x8 v;
  __device__ __forceinline__ void load(const KT* p) { v = *reinterpret_cast<const bf16x8*>(p); }
};
template <>
struct KeyFrag<_Float16> {
  f16x8 v;
  __device__ __forceinline__ void load(const _Float16* p) { v = *reinterpret_cast<const f16x8*>(p); }
};
template <>
struct KeyFrag<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
};

// q's three parts (MFMA A operand)
struct QSplit {
  bf16x8 hi, mid, lo;
};

// acc += q . key, the smallest cross products first
template <typename KT>
__device__ __forceinline__ f32x4 key_mfma(const KeyFrag<KT>& k, const QSplit& q, f32x4 acc) {
  if constexpr (std::is_same<KT, bf16_t>::value) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.lo, k.v, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.mid, k.v, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.hi, k.v, acc, 0, 0, 0);
  } else {
    float f[8];
    if constexpr (std::is_same<KT, float>::value) {
      f[0] = k.a.x; f[1] = k.a.y; f[2] = k.a.z; f[3] = k.a.w;
      f[4] = k.b.x; f[5] = k.b.y; f[6] = k.b.z; f[7] = k.b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = (float)k.v[i];
    }
    bf16x8 khi, kmid, klo;
    split3_bf16(f, khi, kmid, klo);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.mid, kmid, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.lo, khi, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.hi, klo, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.mid, khi, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.hi, kmid, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q.hi, khi, acc, 0, 0, 0);
  }
  return acc;
}

// The logit keys of a range in LDS, as the values of thread t: positions
// 4 t + 1024 s + e (s < RB_MAX / 1024, e < 4); a value takes part when its
// position is in the range and it is at or above est.
struct RangeKeys {
  const uint32_t* keys;
  int n, r0;
  u64 est;
  struct Regs {
    uint4 q[RB_MAX / 1024];
  };
  __device__ __forceinline__ void load(Regs& g) const {
#pragma unroll
    for (int s = 0; s < RB_MAX / 1024; ++s)
      g.q[s] = *reinterpret_cast<const uint4*>(keys + 4 * threadIdx.x + 1024 * s);
  }
  __device__ __forceinline__ u64 get(const Regs& g, int k, bool& ok) const {
    const int pos = 4 * threadIdx.x + 1024 * (k >> 2) + (k & 3);
    const uint4 q = g.q[k >> 2];
    const uint32_t key = (k & 3) == 0 ? q.x : ((k & 3) == 1 ? q.y : ((k & 3) == 2 ? q.z : q.w));
    const u64 v = kv64(key, r0 + pos);
    ok = pos < n && v >= est;
    return v;
  }
};

// Gathered positions of a range's keys (sv[j], j < cnt), as the values of
// thread t: j = t + 256 k (k < SV_CAP / 256).
struct SvKeys {
  const uint32_t* keys;
  const unsigned short* sv;
  int cnt, r0;
  struct Regs {
    u64 v[SV_CAP / 256];
  };
  __device__ __forceinline__ void load(Regs& g) const {
#pragma unroll
    for (int k = 0; k < SV_CAP / 256; ++k) {
      const int j = threadIdx.x + 256 * k;
      const int pos = j < cnt ? sv[j] : 0;
      g.v[k] = kv64(keys[pos], r0 + pos);
    }
  }
  __device__ __forceinline__ u64 get(const Regs& g, int k, bool& ok) const {
    ok = (int)threadIdx.x + 256 * k < cnt;
    return g.v[k];
  }
};

// Survivor values held in registers, RM per thread (value k of thread t is
// survivor t + 256 k; those past cnt do not take part).
template <int RM>
struct RegVals {
  const u64* v;
  int cnt;
  struct Regs {};
  __device__ __forceinline__ void load(Regs&) const {}
  __device__ __forceinline__ u64 get(const Regs&, int k, bool& ok) const {
    ok = (int)threadIdx.x + 256 * k < cnt;
    return v[k];
  }
};

// LDS of the range kernel: keys [RB_MAX] | hist [512] | scratch [48] | counter [4] |
// sv [SV_CAP ushort], aliased by smp [256 u64] | sel [pow2(min(topk, rb) + 1) u64, one range only]
template <typename QT, typename KT, int CI, bool SCORE>
__global__ __launch_bounds__(256, 4) void idx_range_kernel(DecodeIdxParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int NS = CI / 32;
  // fragments in flight per wave: about 16 KB of key rows
  constexpr int VG = NS * 8 * (int)sizeof(KT) / 4;
  // (128-channel rows: the q parts take 48 registers, so one chunk fewer fits
  // in the 128 registers of four waves per SIMD)
  constexpr int VGQ = CI >= 128 ? 48 : 64;
  constexpr int D = VGQ / VG < 2 ? 2 : (VGQ / VG > 8 ? 8 : VGQ / VG);
  uint32_t* keys = reinterpret_cast<uint32_t*>(smem);       // [RB_MAX] (reads of whole 16-byte groups)
  uint32_t* hist = keys + RB_MAX;                            // [512]
  int* scratch = reinterpret_cast<int*>(hist + 512);         // [48]
  int* counter = scratch + 48;                               // [4]
  unsigned short* sv = reinterpret_cast<unsigned short*>(counter + 4);  // [SV_CAP]
  u64* smp = reinterpret_cast<u64*>(sv);                     // [256], before sv is gathered
  u64* sel = reinterpret_cast<u64*>(sv + SV_CAP);            // [ptop]

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int q4 = lane >> 4, n = lane & 15;
  const int b = blockIdx.x / p.nr, r = blockIdx.x - b * p.nr;
  const int r0 = r * p.rb;
  const int nb = p.n_seen ? min((p.n_seen[0] + 1) / p.m, p.cap) : p.nb;
  const int nr_blocks = min(p.rb, nb - r0);
  const int nIh = p.nIh;
  // a sequence's candidates: nr lists of topk (range r holds min(its blocks, topk))
  u64* cout = p.cand + ((size_t)b * p.nr + r) * p.topk;
  if (nr_blocks <= 0) {
    // only a device-driven step has empty ranges (those past its blocks); with
    // one range the selection is empty
    if (p.nr == 1)
      for (int i = tid; i < p.topk; i += 256) p.idx_out[(size_t)b * p.topk + i] = -1;
    return;
  }

  // ---- q fragments (MFMA A operand: row = index head n, zero beyond nIh), split bf16 ----
  QSplit qs[NS];
  float w4[4];  // weights of the heads 4 q4 + e this lane's accumulator rows hold
  {
    float f[NS][8];
    float ss = 0.f;
    const QT* qrow = static_cast<const QT*>(p.q_idx) + (size_t)b * (p.ld_qb ? p.ld_qb : (long long)nIh * CI) +
                     (size_t)(n < nIh ? n : 0) * CI;
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
      split3_bf16(f[s], qs[s].hi, qs[s].mid, qs[s].lo);
    }
    const QT* wrow = static_cast<const QT*>(p.w_idx) + (size_t)b * (p.ld_wb ? p.ld_wb : (long long)nIh);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int hh = 4 * q4 + e;
      w4[e] = hh < nIh ? (p.w_idx ? ld_f32(wrow + hh) : 1.f) : 0.f;
    }
  }

  // ---- logits: wave w takes 16-block chunks w, w + 4, ..., D of them in flight ----
  // D[head][block] = q_head . key_block: the head sum is then lane-local
  // (plus one or two cross-row adds when nIh > 4).
  const KT* kbase = static_cast<const KT*>(p.keys) + (size_t)b * p.k_bstride + (size_t)r0 * CI;
  // without inverse norms, a readable word (the first key) is loaded and replaced by 1
  const bool has_inv = p.inv_norm != nullptr;
  const float* ibase = has_inv ? p.inv_norm + (size_t)b * p.n_bstride + r0 : static_cast<const float*>(p.keys);
  const int istride = has_inv ? 1 : 0;
  const int nchunk = (nr_blocks + 15) / 16;
  const int mine = nchunk > wave ? (nchunk - wave + 3) / 4 : 0;
  KeyFrag<KT> kf[D][NS];
  float iv[D];
  // bf16 rows of 64 channels (128 bytes) load row-major: load A covers rows
  // 0..7 of the chunk, load B rows 8..15, lane (q, n) taking row n % 8, 16-byte
  // chunk q + 4 (n / 8) -- whole rows, contiguous 1 KB for consecutive blocks,
  // with nontemporal loads (read once). The fragments (lane (q, n): row n,
  // chunk q for k step 0, chunk 4 + q for step 1) are A / B and their
  // within-row rotation by 8 lanes: s0 = n < 8 ? A : rot8(B),
  // s1 = n < 8 ? rot8(A) : B.
  constexpr bool ROWMAJOR = std::is_same<KT, bf16_t>::value && CI == 64;
  auto load = [&](int m, KeyFrag<KT> (&f)[NS], float& ivv) {
    const int base = 16 * (wave + 4 * m);
    if constexpr (ROWMAJOR) {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const int c = q4 + 4 * (n >> 3);
      const int ja = min(base + (n & 7), nr_blocks - 1), jb = min(base + 8 + (n & 7), nr_blocks - 1);
      f[0].v = __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(
                                              reinterpret_cast<const u32x4*>(kbase + (size_t)ja * CI + 8 * c)));
      f[1].v = __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(
                                              reinterpret_cast<const u32x4*>(kbase + (size_t)jb * CI + 8 * c)));
    } else {
      const int jr = min(base + n, nr_blocks - 1);
      const KT* krow = kbase + (size_t)jr * CI + 8 * q4;
#pragma unroll
      for (int s = 0; s < NS; ++s) f[s].load(krow + 32 * s);
    }
    ivv = ibase[min(base + n, nr_blocks - 1) * istride];
  };
  auto rot8 = [](bf16x8 x) {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    i32x4 w = __builtin_bit_cast(i32x4, x);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __builtin_amdgcn_update_dpp(0, w[i], 0x128, 0xf, 0xf, false);  // row_ror:8
    return __builtin_bit_cast(bf16x8, w);
  };
  // consume slot d as chunk m, then (RELOAD) refill it with chunk m + D
  auto step = [&](int m, KeyFrag<KT> (&f)[NS], float& ivv, auto reload) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (ROWMAJOR) {
      KeyFrag<KT> g0, g1;
      const bf16x8 ra = rot8(f[0].v), rb = rot8(f[1].v);
      g0.v = n < 8 ? f[0].v : rb;
      g1.v = n < 8 ? ra : f[1].v;
      acc = key_mfma<KT>(g0, qs[0], acc);
      acc = key_mfma<KT>(g1, qs[1], acc);
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) acc = key_mfma<KT>(f[s], qs[s], acc);
    }
    const float sc = p.scale * (has_inv ? ivv : 1.f);
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) v += fmaxf(acc[e] * sc, 0.f) * w4[e];
    if constexpr (decltype(reload)::value) load(m + D, f, ivv);
    if (nIh > 4) v += __shfl_xor(v, 16);
    if (nIh > 8) v += __shfl_xor(v, 32);
    const int j = 16 * (wave + 4 * m) + n;
    if (q4 == 0 && j < nr_blocks) keys[j] = okey(v);
  };
#pragma unroll
  for (int d = 0; d < D; ++d) load(d, kf[d], iv[d]);
  // whole groups of D chunks without conditions (so that every wait for a slot
  // counts only the loads issued before it), then the remainder
  int m0 = 0;
  for (; m0 + D <= mine; m0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) step(m0 + d, kf[d], iv[d], std::true_type{});
  }
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (m0 + d < mine) step(m0 + d, kf[d], iv[d], std::false_type{});
  __syncthreads();
  if constexpr (SCORE) {
    // score pass only: the range's keys out, 16 bytes a thread
    uint32_t* kout = p.keys_out + (size_t)b * p.ko_bstride + r0;
    for (int i = 4 * tid; i < nr_blocks; i += 1024) {
      if (i + 4 <= nr_blocks) {
        *reinterpret_cast<uint4*>(kout + i) = *reinterpret_cast<const uint4*>(keys + i);
      } else {
        for (int e = i; e < nr_blocks; ++e) kout[e] = keys[e];
      }
    }
  } else {

  // ---- top-k of the range ----
  // Thread t owns the keys at positions 4 t + 1024 s + e (s < 8, e < 4),
  // re-read from LDS in every pass as eight unconditional 16-byte reads
  // (holding them would cost 64 VGPRs; words past the range are masked off); a
  // sampled estimate narrows the radix select to the values at or above it
  // (about 2 topk), all values when it misses.
  const int topk = p.topk;
  constexpr int RK = 4 * (RB_MAX / 1024);
  RangeKeys src{keys, nr_blocks, r0, 0ull};
  Sel64 sl{0ull, 0ull};
  bool all = nr_blocks <= topk, gathered = false;
  int c = 0;
  if (!all) {
    if (sample_estimate([&](int i) { return kv64(keys[i], r0 + i); }, nr_blocks, topk, SV_CAP, smp,
                        scratch, &src.est)) {
      // census of the values at or above the estimate, gathering their positions
      if (tid == 0) counter[2] = 0;
      __syncthreads();
      RangeKeys::Regs g;
      src.load(g);
      u64 a = ~0ull, o = 0ull;
      uint32_t okm = 0u;  // bit k: value k takes part
#pragma unroll
      for (int k = 0; k < RK; ++k) {
        bool ok;
        const u64 v = src.get(g, k, ok);
        okm |= (uint32_t)ok << k;
        a &= ok ? v : ~0ull;
        o |= ok ? v : 0ull;
      }
      c = __popc(okm);
      int x = c;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
      }
      int base = 0;
      if (lane == 63 && x) base = atomicAdd(counter + 2, x);
      int at = __builtin_amdgcn_readlane(base, 63) + x - c;
#pragma unroll
      for (int k = 0; k < RK; ++k) {
        if ((okm >> k) & 1u) {
          if (at < SV_CAP) sv[at] = (unsigned short)(4 * tid + 1024 * (k >> 2) + (k & 3));
          ++at;
        }
      }
      block_cnt_and_or(c, a, o, scratch);
      if (c >= topk && c <= SV_CAP) {
        gathered = true;
        all = c == topk;
        if (!all) sl = reg_select<SV_CAP / 256>(SvKeys{keys, sv, c, r0}, topk, a, o, hist, scratch);
      }
    }
    if (!gathered) {  // no estimate, or it missed: select among all
      src.est = 0ull;
      u64 a, o;
      reg_census<RK>(src, c, a, o, scratch);
      sl = reg_select<RK>(src, topk, a, o, hist, scratch);
    }
  }
  if (tid == 0) counter[0] = 0;
  __syncthreads();
  if (gathered) {
    const SvKeys gsrc{keys, sv, c, r0};
    if (p.nr == 1) {
      reg_gather<SV_CAP / 256>(gsrc, sl, all, [&](int at, u64 v) { sel[at] = v; }, counter);
      __syncthreads();
      write_sorted<false>(sel, topk, topk, p.idx_out + (size_t)b * topk);
    } else {
      reg_gather<SV_CAP / 256>(gsrc, sl, all, [&](int at, u64 v) { cout[at] = v; }, counter);
    }
    return;
  }
  if (tid == 0) counter[0] = 0;
  __syncthreads();
  if (p.nr == 1) {
    reg_gather<RK>(src, sl, all, [&](int at, u64 v) { sel[at] = v; }, counter);
    __syncthreads();
    write_sorted<false>(sel, min(nr_blocks, topk), topk, p.idx_out + (size_t)b * topk);
  } else {
    // candidates (any order) straight to global: min(nr_blocks, topk) of them
    reg_gather<RK>(src, sl, all, [&](int at, u64 v) { cout[at] = v; }, counter);
  }
  }
}

// LDS of the select kernel: keys [RB_MAX] | hist [1024] | scratch [48] | counter [4] |
// sel [pow2(topk + 1) u64]
__global__ __launch_bounds__(256) void idx_select_kernel(DecodeIdxParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  uint32_t* keys = reinterpret_cast<uint32_t*>(smem);     // [RB_MAX]
  uint32_t* hist = keys + RB_MAX;                          // [1024]
  int* scratch = reinterpret_cast<int*>(hist + 1024);      // [48]
  int* counter = scratch + 48;                             // [4]
  u64* sel = reinterpret_cast<u64*>(counter + 4);          // [pow2(topk + 1)]
  const int tid = threadIdx.x, b = blockIdx.x, topk = p.topk;
  const int nb = min(p.n_seen ? min((p.n_seen[0] + 1) / p.m, p.cap) : p.nb, RB_MAX);
  // the keys of the score pass (rows ko_bstride words apart, a multiple of 4)
  const uint32_t* src = p.keys_out + (size_t)b * p.ko_bstride;
  for (int i = 4 * tid; i < nb; i += 1024) {
    if (i + 4 <= nb) {
      *reinterpret_cast<uint4*>(keys + i) = *reinterpret_cast<const uint4*>(src + i);
    } else {
      for (int e = i; e < nb; ++e) keys[e] = src[e];
    }
  }
  if (tid == 0) counter[0] = 0;
  __syncthreads();
  int* out = p.idx_out + (size_t)b * topk;
  constexpr int RK = 4 * (RB_MAX / 1024);
  const RangeKeys rk{keys, nb, 0, 0ull};
  Sel64 sl{0ull, 0ull};
  const bool all = nb <= topk;
  if (!all) {
    sl = block_select64<4>([&](int i) { return kv64(keys[i], i); }, nb, topk, hist, scratch);
  }
  reg_gather<RK>(rk, sl, all, [&](int at, u64 v) { sel[at] = v; }, counter);
  __syncthreads();
  write_sorted<true>(sel, min(nb, topk), topk, out);
}

// Gather capacity of the merge: MV_CAP when an estimate can pay off, else
// just room for the samples.
__host__ __device__ inline int merge_cap(int topk) { return topk <= MV_CAP / 2 ? MV_CAP : 256; }

// LDS of the merge kernel: sv [merge_cap u64] | sel [pow2(topk + 1) u64] |
// hist [512] | scratch [48] | counter [4]
__global__ __launch_bounds__(256) void idx_merge_kernel(DecodeIdxParams p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int topk = p.topk, nr = p.nr;
  const int mcap = merge_cap(topk);
  u64* sv = reinterpret_cast<u64*>(smem);                   // [mcap]
  u64* sel = sv + mcap;                                      // [ptop]
  uint32_t* hist = reinterpret_cast<uint32_t*>(sel + pow2_at_least(topk + 1));  // [512]
  int* scratch = reinterpret_cast<int*>(hist + 512);         // [48]
  int* counter = scratch + 48;                               // [4]
  const int tid = threadIdx.x, b = blockIdx.x;
  const u64* src = p.cand + (size_t)b * nr * topk;
  // ranges holding blocks (all nr unless the step is device-driven)
  const int nb = p.n_seen ? min((p.n_seen[0] + 1) / p.m, p.cap) : p.nb;
  const int na = (nb + p.rb - 1) / p.rb;
  // candidate f of the sequence: ranges before the last hold c0 each
  const int c0 = min(p.rb, topk);
  const int cl = na > 0 ? min(nb - (na - 1) * p.rb, topk) : 0;
  const int N = na > 0 ? (na - 1) * c0 + cl : 0;
  // (when every range holds topk candidates they are contiguous)
  const bool contig = c0 == topk;
  auto gval = [&](int f) {
    if (contig) return src[f];
    const int r = min(f / c0, na - 1);
    return src[(size_t)r * topk + (f - r * c0)];
  };
  int cnt = N;
  if (N <= topk) {
    for (int f = tid; f < N; f += 256) sel[f] = gval(f);
    __syncthreads();
  } else {
    u64 est = 0ull;
    bool done = false;
    if (sample_estimate(gval, N, topk, mcap, sv, scratch, &est)) {
      // stream the candidates once: those at or above the estimate into sv
      if (tid == 0) counter[0] = 0;
      __syncthreads();
      constexpr int U = 32;  // loads in flight per thread
      const int lane = tid & 63;
      for (int base = wave_id() * 64 * U; base < N; base += 256 * U) {
        u64 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = gval(min(base + 64 * u + lane, N - 1));
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool t = base + 64 * u + lane < N && v[u] >= est;
          const u64 m = __ballot(t);
          if (m) {
            int at = 0;
            if (lane == 0) at = atomicAdd(counter, __popcll(m));
            at = __builtin_amdgcn_readlane(at, 0) + mbcnt64(m);
            if (t && at < mcap) sv[at] = v[u];
          }
        }
      }
      __syncthreads();
      const int total = counter[0];
      if (total >= topk && total <= mcap) {
        constexpr int RM = MV_CAP / 256;
        u64 rv[RM];
#pragma unroll
        for (int k = 0; k < RM; ++k) rv[k] = tid + 256 * k < total ? sv[tid + 256 * k] : 0ull;
        const RegVals<RM> src{rv, total};
        Sel64 sl{0ull, 0ull};
        if (total > topk) {
          int c;
          u64 a, o;
          reg_census<RM>(src, c, a, o, scratch);
          sl = reg_select<RM>(src, topk, a, o, hist, scratch);
        }
        if (tid == 0) counter[1] = 0;
        __syncthreads();
        reg_gather<RM>(src, sl, total == topk, [&](int at, u64 v) { sel[at] = v; }, counter + 1);
        done = true;
      }
    }
    if (!done) {
      const Sel64 sl = block_select64(gval, N, topk, hist, scratch);
      if (tid == 0) counter[1] = 0;
      __syncthreads();
      block_gather(gval, N, [&](u64 v) { return (v & sl.mask) >= sl.thr; },
                   [&](int at, int, u64 v) { sel[at] = v; }, topk, counter + 1);
    }
    __syncthreads();
    cnt = topk;
  }
  write_sorted<true>(sel, cnt, topk, p.idx_out + (size_t)b * topk);
}

// Merges the ngrp partials of (sequence b, head h), dims 8 d8 .. 8 d8 + 7,
// and adds the sink: one pass with a running reference point, the partial
// loads of four groups in flight.
template <int HD, typename OT>
__device__ __forceinline__ void combine_partials(const DecodeAttnParams& p, int b, int h, int d8) {
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  auto fold = [&](float2 ml, float4 x0, float4 x1) {
    if (!(ml.y > 0.f)) return;
    const float Mn = fmaxf(M, ml.x);
    const float a = fast_exp2(M - Mn), c = fast_exp2(ml.x - Mn);
    L = L * a + ml.y * c;
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * a + xs[i] * c;
    M = Mn;
  };
  const size_t s0 = (size_t)b * p.ngrp;
  auto ld = [&](int s, float2& ml, float4& x0, float4& x1) {
    const size_t sl = (s0 + s) * p.nh + h;
    ml = *reinterpret_cast<const float2*>(p.part_ml + sl * 2);
    const float* po = p.part_o + sl * HD + 8 * d8;
    x0 = *reinterpret_cast<const float4*>(po);
    x1 = *reinterpret_cast<const float4*>(po + 4);
  };
  int s = 0;
  for (; s + 4 <= p.ngrp; s += 4) {
    float2 ml[4];
    float4 x0[4], x1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ld(s + u, ml[u], x0[u], x1[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) fold(ml[u], x0[u], x1[u]);
  }
  for (; s < p.ngrp; ++s) {
    float2 ml;
    float4 x0, x1;
    ld(s, ml, x0, x1);
    fold(ml, x0, x1);
  }
  float f = 0.f;
  if (L > 0.f) {
    float denom = L;
    if (p.sink) denom += fast_exp2(p.sink[h] * kLog2eF - M);
    f = 1.f / denom;
  }
  OT* out = static_cast<OT*>(p.out) + ((size_t)b * p.nh + h) * HD + 8 * d8;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = from_f32<OT>(acc[i] * f);
}

// Decode attention over one group of rows of one sequence (a workgroup): the
// 4 waves take the group's 32-row steps in turn (wave w: steps w, w + 4,
// ...), two steps in flight per wave, merge their (M, L, o) in LDS, and
// either finish the sequence (one group) or leave a partial for
// attn_combine_kernel.
// DENSE (no index list: every cached block, then the ring) computes the row
// numbers of a step instead of loading them. That is not only fewer loads: the
// indexed form's index loads are issued behind the previous step's row loads,
// so waiting for them waits for those rows too; a kernel holding both forms
// gets that wait on the dense path as well (it sits where the paths join),
// which leaves one step in flight per wave instead of two.
template <int HD, typename QT, typename OT, bool DENSE>
__global__ __launch_bounds__(256, DENSE ? 3 : 2) void attn_kernel(DecodeAttnParams p) {
  using W = MqaWave<HD>;
  constexpr int STAGE = W::STAGE_ELEMS;                 // bf16 per wave
  constexpr int MERGE = 4 * 16 * HD + 4 * 16 * 2;       // floats: o and (M, L) per wave and head
  constexpr int LDS_BYTES = (4 * STAGE * 2 > MERGE * 4) ? 4 * STAGE * 2 : MERGE * 4;
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  const int tid = threadIdx.x, wv = wave_id(), lane = tid & 63, n = lane & 15;
  bf16_t* stage = reinterpret_cast<bf16_t*>(lds) + wv * STAGE;
  const int b = blockIdx.x / p.ngrp, g = blockIdx.x - b * p.ngrp;
  int nb = p.nb, na = p.na, ring_len = p.ring_len;
  if (p.n_seen) {
    const int t1 = p.n_seen[0] + 1;
    nb = min(t1 / p.m, p.cap);
    ring_len = min(t1, p.win);
    if (!p.idx) na = nb;
  }
  // the attended rows in 32-row steps: blocks j < na (padded to na_pad, a
  // multiple of 32, with masked rows), then the ring rows; a step holds only
  // one kind (row groups start at multiples of 64)
  const int na_pad = (na + 31) & ~31;
  const int nrows = na_pad + ring_len;
  const int jg0 = g * p.rows_per_group, jg1 = min(nrows, jg0 + p.rows_per_group);

  // The query's words are loaded first and converted only after the first
  // rows are requested: a wait for a load also waits for every load issued
  // before it, so the rows must not be issued ahead of the query.
  const QT* qrow = static_cast<const QT*>(p.q) + (size_t)b * (p.ld_qb ? p.ld_qb : (long long)p.nh * HD) +
                   (size_t)(n < p.nh ? n : 0) * HD;
  typedef uint32_t u32x4q __attribute__((ext_vector_type(4)));
  constexpr int QW = sizeof(QT) == 4 ? 2 : 1;  // 16-byte words per 8 query elements
  u32x4q qraw[W::NS][QW];
#pragma unroll
  for (int s = 0; s < W::NS; ++s)
#pragma unroll
    for (int h = 0; h < QW; ++h)
      qraw[s][h] = *reinterpret_cast<const u32x4q*>(qrow + 32 * s + 8 * (lane >> 4) + 4 * h);
  // Rows are read through buffer resources over this sequence's cached
  // blocks and ring rows with 32-bit byte offsets (an offset past a
  // resource's end reads zeros: a -1 slot, a block beyond nb, a padding row),
  // nontemporal (every row is read once). They are taken in the score layout
  // (MqaWave::chunk_sl): slot k of lane group q4 is row row_sl(k, q4) of the
  // step, the row whose scores the lane holds; its 8 block indices are
  // fetched a step ahead (16-byte loads when na is a multiple of 4).
  constexpr int ROWB = HD * 2;
  const int lane_off = 16 * (lane % W::TPR), q4 = lane >> 4;
  const int hmask = (W::TPR == 8 && ((lane >> 3) & 1)) ? -1 : 0;  // HD 64: slot i + 4
  const __amdgpu_buffer_rsrc_t rs_kv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t*>(p.kv + (size_t)b * p.kv_bstride), 0, nb * ROWB, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_ring = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t*>(p.ring ? p.ring + (size_t)b * p.ring_bstride : p.kv), 0,
      p.ring ? ring_len * ROWB : 0, 0x00020000);
  const bool has_idx = !DENSE && p.idx != nullptr && na > 0;
  const __amdgpu_buffer_rsrc_t rs_idx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int*>(has_idx ? p.idx + (size_t)b * p.na : nullptr), 0, has_idx ? na * 4 : 0,
      0x00020000);
  const bool idx16 = (na & 3) == 0;
  auto row_j = [&](int m) { return jg0 + 32 * (wv + 4 * m); };  // first row of step m
  struct Sel {
    int v[8];
  };
  auto load_sel = [&](int m, Sel& sl) {
    const int j0 = row_j(m);
    if constexpr (DENSE) {
      const int r0 = j0 < na_pad ? j0 : j0 - na_pad;
#pragma unroll
      for (int k = 0; k < 8; ++k) sl.v[k] = r0 + W::row_sl(k, q4);
    } else if (__builtin_amdgcn_readfirstlane(j0 < na_pad ? 1 : 0)) {
      if (p.idx) {
        if (idx16) {
          typedef int i32x4 __attribute__((ext_vector_type(4)));
          const i32x4 x = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, (j0 + 4 * q4) * 4, 0, 0));
          const i32x4 y = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, (j0 + 16 + 4 * q4) * 4, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sl.v[e] = x[e];
            sl.v[4 + e] = y[e];
          }
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k)
            sl.v[k] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_idx, (j0 + W::row_sl(k, q4)) * 4, 0, 0);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) sl.v[k] = j0 + W::row_sl(k, q4);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) sl.v[k] = j0 - na_pad + W::row_sl(k, q4);
    }
  };
  // the loads of step m; ok[k]: slot k is a row of this group. Returns
  // (uniform) 0 when no row of the step is, 2 when every row is (ok then
  // unset), else 1.
  auto load_rows = [&](int m, const Sel& sl, typename W::Rows& rr, bool (&ok)[8]) -> int {
    const int j0 = row_j(m);
    const int ms = __builtin_amdgcn_readfirstlane(j0 < na_pad ? 1 : 0);
    const __amdgpu_buffer_rsrc_t rs = ms ? rs_kv : rs_ring;
    // a step past the group (the loop loads two ahead) reads nothing from
    // memory: its offsets get bit 31 set, beyond every resource (< 2 GiB)
    const unsigned past = __builtin_amdgcn_readfirstlane(j0 >= jg1 ? 0x80000000u : 0u);
#pragma unroll
    for (int i = 0; i < W::NLI; ++i) {
      // (a select of values, not an indexed read: that would put sl in scratch memory)
      const int v = W::TPR == 8 ? sl.v[i] ^ ((sl.v[i] ^ sl.v[(i + 4) & 7]) & hmask) : sl.v[i];
      rr.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(((unsigned)v * ROWB + lane_off) | past),
                                                      0, 2 /* nontemporal */);
    }
    // a step wholly inside the group and its ring rows, or (dense) wholly
    // inside the cached blocks, is all valid
    if (j0 + 32 <= jg1 && (ms ? (DENSE && j0 + 32 <= min(na, nb)) : j0 - na_pad + 32 <= ring_len))
      return 2;
    bool any = false;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = j0 + W::row_sl(k, q4);
      const bool okb = (j < na) & ((unsigned)sl.v[k] < (unsigned)nb);
      const bool okr = j - na_pad < ring_len;
      ok[k] = (j < jg1) & (ms ? okb : okr);
      any |= ok[k];
    }
    return __ballot(any) != 0ull ? 1 : 0;
  };
  const TileOffsets<HD> to;
  const int nsg = (jg1 - jg0 + 31) / 32;                   // steps in the group
  const int mine = nsg > wv ? (nsg - wv + 3) / 4 : 0;      // this wave's
  // Two steps in flight (named registers: an indexed array of them ends up in
  // scratch memory). Indexed steps keep the indices of the two after them: a
  // step's indices are requested before the rows of the step ahead of it, so
  // waiting for them never waits for rows not yet consumed. Steps past this
  // wave's last are loaded (masked, any = false) rather than peeled.
  Sel s0, s1;
  typename W::Rows fr0, fr1;
  bool ok0[8], ok1[8];
  int any0, any1;
  if constexpr (DENSE) {
    load_sel(0, s0);
    any0 = load_rows(0, s0, fr0, ok0);
    load_sel(1, s0);
    any1 = load_rows(1, s0, fr1, ok1);
  } else {
    load_sel(0, s0);
    load_sel(1, s1);
    any0 = load_rows(0, s0, fr0, ok0);
    any1 = load_rows(1, s1, fr1, ok1);
    load_sel(2, s0);
    load_sel(3, s1);
  }
  W w;
  {
    float f[W::NS][8];
    const bool keep = n < p.nh;
#pragma unroll
    for (int s = 0; s < W::NS; ++s) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x;
        if constexpr (sizeof(QT) == 4) {
          x = __uint_as_float(qraw[s][i >> 2][i & 3]);
        } else {
          const uint32_t wd = qraw[s][0][i >> 1];
          const uint16_t hb = (uint16_t)((i & 1) ? (wd >> 16) : (wd & 0xffffu));
          if constexpr (std::is_same<QT, bf16_t>::value) x = __uint_as_float((uint32_t)hb << 16);
          else x = (float)__builtin_bit_cast(_Float16, hb);
        }
        f[s][i] = keep ? x : 0.f;
      }
    }
    w.setup(f, p.normalize_q != 0, p.scale);
  }
  for (int m0 = 0; m0 < mine; m0 += 2) {
    if constexpr (DENSE) {
      if (any0) w.chunk_sl(fr0, ok0, stage, to, any0 == 2);
      load_sel(m0 + 2, s0);
      any0 = load_rows(m0 + 2, s0, fr0, ok0);
      if (any1) w.chunk_sl(fr1, ok1, stage, to, any1 == 2);
      load_sel(m0 + 3, s0);
      any1 = load_rows(m0 + 3, s0, fr1, ok1);
    } else {
      if (any0) w.chunk_sl(fr0, ok0, stage, to, any0 == 2);
      any0 = load_rows(m0 + 2, s0, fr0, ok0);
      load_sel(m0 + 4, s0);
      if (any1) w.chunk_sl(fr1, ok1, stage, to, any1 == 2);
      any1 = load_rows(m0 + 3, s1, fr1, ok1);
      load_sel(m0 + 5, s1);
    }
  }
  w.finalize();

  // ---- merge the 4 waves: thread t -> head t / (HD / 8), dims 8 (t % (HD / 8)) ----
  __syncthreads();  // staging buffers are free
  float* mo = reinterpret_cast<float*>(lds);                // [4][16][HD]
  float* mml = mo + 4 * 16 * HD;                             // [4][16][2]
  {
    const int q4 = 4 * (lane >> 4);
#pragma unroll
    for (int t = 0; t < W::NT; ++t)
      *reinterpret_cast<float4*>(mo + (wv * 16 + n) * HD + 16 * t + q4) =
          make_float4(w.o[t][0], w.o[t][1], w.o[t][2], w.o[t][3]);
    if (lane < 16) *reinterpret_cast<float2*>(mml + (wv * 16 + n) * 2) = make_float2(w.M, w.L);
  }
  __syncthreads();
  constexpr int PH = HD / 8;  // threads per head
  const int h = tid / PH, d8 = tid - h * PH;
  const bool mine_out = h < p.nh;
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  auto fold = [&](float Ms, float Ls, const float* os) {
    if (!(Ls > 0.f)) return;
    const float Mn = fmaxf(M, Ms);
    const float a = fast_exp2(M - Mn), c = fast_exp2(Ms - Mn);  // M = -inf -> a = 0
    L = L * a + Ls * c;
    const float4 x0 = *reinterpret_cast<const float4*>(os), x1 = *reinterpret_cast<const float4*>(os + 4);
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = acc[i] * a + xs[i] * c;
    M = Mn;
  };
  if (mine_out) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float2 ml = *reinterpret_cast<const float2*>(mml + (s * 16 + h) * 2);
      fold(ml.x, ml.y, mo + (s * 16 + h) * HD + 8 * d8);
    }
  }
  auto finish = [&]() {
    float f = 0.f;
    if (L > 0.f) {
      float denom = L;
      if (p.sink) denom += fast_exp2(p.sink[h] * kLog2eF - M);
      f = 1.f / denom;
    }
    OT* out = static_cast<OT*>(p.out) + ((size_t)b * p.nh + h) * HD + 8 * d8;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = from_f32<OT>(acc[i] * f);
  };
  if (p.ngrp == 1) {
    if (mine_out) finish();
    return;
  }
  // ---- partial of this group, merged by attn_combine_kernel ----
  if (mine_out) {
    const size_t slot = ((size_t)b * p.ngrp + g) * p.nh + h;
    float* po = p.part_o + slot * HD + 8 * d8;
    *reinterpret_cast<float4*>(po) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4*>(po + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    if (d8 == 0) *reinterpret_cast<float2*>(p.part_ml + slot * 2) = make_float2(M, L);
  }
}

// Merges the ngrp partials of each (sequence, head): thread -> (sequence,
// head, 8 dims).
template <int HD, typename OT>
__global__ __launch_bounds__(256) void attn_combine_kernel(DecodeAttnParams p) {
  constexpr int PH = HD / 8;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)p.B * p.nh * PH) return;
  const int d8 = (int)(gid % PH);
  const long long bh = gid / PH;
  combine_partials<HD, OT>(p, (int)(bh / p.nh), (int)(bh % p.nh), d8);
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

int decode_range_max() { return RB_MAX; }

void decode_idx_plan(int B, int nb, int topk, int* rb, int* nr) {
  // ranges of at most RB_MAX blocks; a small batch is split further, down to
  // ranges of max(1024, 2 topk) blocks, for about WG_TARGET workgroups
  const int r_need = nb > 0 ? (nb + RB_MAX - 1) / RB_MAX : 1;
  const int rb_min = max(1024, 2 * topk);
  const int r_fine = (nb + rb_min - 1) / rb_min;
  const int r_par = (WG_TARGET + B - 1) / max(B, 1);
  const int r = max(1, max(r_need, min(r_par, r_fine)));
  int b = (nb + r - 1) / r;
  b = (b + 15) & ~15;
  *rb = b;
  *nr = b > 0 ? (nb + b - 1) / b : 1;  // every range holds at least one block
  if (*nr < 1) *nr = 1;
}

size_t decode_idx_lds(int rb, int topk, int nr) {
  const size_t base = (size_t)RB_MAX * 4 + 512 * 4 + 52 * 4 + (size_t)SV_CAP * 2;
  return base + (nr == 1 ? (size_t)pow2_at_least(min(topk, rb) + 1) * 8 : 0);
}

size_t decode_select_lds(int topk) {
  return (size_t)RB_MAX * 4 + 1024 * 4 + 52 * 4 + (size_t)pow2_at_least(topk + 1) * 8;
}

size_t decode_merge_lds(int topk) {
  return (size_t)merge_cap(topk) * 8 + (size_t)pow2_at_least(topk + 1) * 8 + 512 * 4 + 52 * 4;
}

bool decode_merge_fits(int topk) { return decode_merge_lds(topk) <= 160 * 1024; }

bool decode_idx_fits(int rb, int topk, int nr) { return decode_idx_lds(rb, topk, nr) <= 160 * 1024; }

hipError_t decode_idx_dispatch(const DecodeIdxParams& p, int qdtype, int kdtype, hipStream_t s) {
  const size_t lds = decode_idx_lds(p.rb, p.topk, p.nr);
  const dim3 grid((unsigned)(p.B * p.nr)), block(256);
#define KCH_DIDX(QT, KT, CI)                                                                   \
  if (p.keys_out) hipLaunchKernelGGL((idx_range_kernel<QT, KT, CI, true>), grid, block, lds, s, p); \
  else hipLaunchKernelGGL((idx_range_kernel<QT, KT, CI, false>), grid, block, lds, s, p)
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
  if (e != hipSuccess) return e;
  if (p.keys_out) {
    hipLaunchKernelGGL(idx_select_kernel, dim3((unsigned)p.B), dim3(256), decode_select_lds(p.topk), s, p);
    return hipGetLastError();
  }
  if (p.nr == 1) return e;
  hipLaunchKernelGGL(idx_merge_kernel, dim3((unsigned)p.B), dim3(256), decode_merge_lds(p.topk), s, p);
  return hipGetLastError();
}

hipError_t decode_attn_dispatch(const DecodeAttnParams& p, int qdtype, int odtype, hipStream_t s) {
  const dim3 grid((unsigned)((long long)p.B * p.ngrp)), block(256);
#define KCH_DATT_D(HD, QT, D)                                                                        \
  if (odtype == DT_F32) hipLaunchKernelGGL((attn_kernel<HD, QT, float, D>), grid, block, 0, s, p);    \
  else if (odtype == DT_BF16) hipLaunchKernelGGL((attn_kernel<HD, QT, bf16_t, D>), grid, block, 0, s, p); \
  else hipLaunchKernelGGL((attn_kernel<HD, QT, _Float16, D>), grid, block, 0, s, p);
#define KCH_DATT(HD, QT) \
  if (p.idx) { KCH_DATT_D(HD, QT, false) } else { KCH_DATT_D(HD, QT, true) }
  if (p.hd == 128) {
    if (qdtype == DT_F32) { KCH_DATT(128, float) }
    else if (qdtype == DT_BF16) { KCH_DATT(128, bf16_t) }
    else { KCH_DATT(128, _Float16) }
  } else {
    if (qdtype == DT_F32) { KCH_DATT(64, float) }
    else if (qdtype == DT_BF16) { KCH_DATT(64, bf16_t) }
    else { KCH_DATT(64, _Float16) }
  }
#undef KCH_DATT
#undef KCH_DATT_D
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ngrp == 1) return e;
  const long long outs = (long long)p.B * p.nh * (p.hd / 8);
  const dim3 g2((unsigned)((outs + 255) / 256));
#define KCH_DCMB(HD)                                                                           \
  if (odtype == DT_F32) hipLaunchKernelGGL((attn_combine_kernel<HD, float>), g2, block, 0, s, p); \
  else if (odtype == DT_BF16) hipLaunchKernelGGL((attn_combine_kernel<HD, bf16_t>), g2, block, 0, s, p); \
  else hipLaunchKernelGGL((attn_combine_kernel<HD, _Float16>), g2, block, 0, s, p);
  if (p.hd == 128) { KCH_DCMB(128) } else { KCH_DCMB(64) }
#undef KCH_DCMB
  return hipGetLastError();
}

}  // namespace kch
