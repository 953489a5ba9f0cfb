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
//   compress_lanes_kernel (short blocks, aligned rows) and compress_rows_kernel
//   (long blocks) compute the same outputs with 16-byte row accesses.
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

// One channel of a compressed key row: bf16 (key_f32 0), fp32 (1), the
// three bf16 parts x = hi + mid + lo of the fp32 value (2), stored as three
// part rows [hi(c) | mid(c) | lo(c)], or (3, L2-normalised rows only) the two
// fp16 parts of 256 x, [hi(c) | lo(c)] -- the splits the indexer's MFMA
// products use. Format 4 holds the parts of format 3 chunk-major: the rows of
// each 16-row chunk (the last one padded) in the order the indexer's lanes
// load them, so that each of its loads reads 1 KB of contiguous memory:
// piece j = part * c / 32 + ch / 32 of the chunk is 64 lanes of 8 channels,
// lane (row % 16) + 16 * ((ch % 32) / 8), element ch % 8.
__device__ __forceinline__ size_t chunked_key_offset(size_t orow, int nb, int c, int part, int ch) {
  // batch row and block (B * nb < 2^31: the caller's row count)
  const unsigned bi = (unsigned)orow / (unsigned)nb, r = (unsigned)orow - bi * (unsigned)nb;
  const size_t chunk = (size_t)bi * (unsigned)((nb + 15) >> 4) + (r >> 4);
  const int piece = part * (c >> 5) + (ch >> 5);
  const int lane = (int)(r & 15) + 16 * ((ch & 31) >> 3);
  return chunk * 32 * (size_t)c + (size_t)piece * 512 + (size_t)lane * 8 + (ch & 7);
}

__device__ __forceinline__ void store_key(const CompressParams& p, size_t orow, int c, int ch,
                                          float x) {
  if (p.key_f32 == 1) {
    static_cast<float*>(p.out_key)[orow * c + ch] = x;
  } else if (p.key_f32 == 2) {
    const bf16_t hi = (bf16_t)x;
    const float r = x - (float)hi;
    const bf16_t mid = (bf16_t)r;
    bf16_t* row = static_cast<bf16_t*>(p.out_key) + orow * 3 * c;
    row[ch] = hi;
    row[c + ch] = mid;
    row[2 * c + ch] = (bf16_t)(r - (float)mid);
  } else if (p.key_f32 == 3) {
    const float xs = x * kSplit16Scale;
    const _Float16 hi = (_Float16)xs;
    _Float16* row = static_cast<_Float16*>(p.out_key) + orow * 2 * c;
    row[ch] = hi;
    row[c + ch] = (_Float16)(xs - (float)hi);
  } else if (p.key_f32 == 4) {
    const float xs = x * kSplit16Scale;
    const _Float16 hi = (_Float16)xs;
    const int nb = p.T / p.m;
    _Float16* base = static_cast<_Float16*>(p.out_key);
    base[chunked_key_offset(orow, nb, c, 0, ch)] = hi;
    base[chunked_key_offset(orow, nb, c, 1, ch)] = (_Float16)(xs - (float)hi);
  } else {
    static_cast<bf16_t*>(p.out_key)[orow * c + ch] = (bf16_t)x;
  }
}

namespace {


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
    // pass 1: max of the logits; pass 2: exp-weighted sums (torch.softmax
    // order; the exponentials of the hardware's exp2, within 2 ulp)
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
      const float e = exp_hw(to_f32(Za[(ta + j) * p.ldZa + ch]) + p.Ba[j * c + ch] - mx);
      den += e;
      num += e * to_f32(Ca[(ta + j) * p.ldCa + ch]);
    }
    if (prev)
      for (int j = 0; j < m; ++j) {
        const float e = exp_hw(to_f32(Zb[(tb + j) * p.ldZb + ch]) + p.Bb[j * c + ch] - mx);
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
      store_key(p, orow, c, lane + 64 * u, acc[u] * inv);
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

// Eight consecutive channels ch0 .. ch0 + 7 of a compressed key row in
// every format of store_key (ch0 a multiple of 8): one or two whole stores
// per part instead of eight scalar ones.
__device__ __forceinline__ void store_key8(const CompressParams& p, size_t orow, int c, int ch0,
                                           const float (&x)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  if (p.key_f32 == 1) {
    float* d = static_cast<float*>(p.out_key) + orow * c + ch0;
    *reinterpret_cast<float4*>(d) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(d + 4) = make_float4(x[4], x[5], x[6], x[7]);
  } else if (p.key_f32 == 2) {
    float hi[8], mid[8], lo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bf16_t h = (bf16_t)x[i];
      const float r = x[i] - (float)h;
      const bf16_t md = (bf16_t)r;
      hi[i] = (float)h;
      mid[i] = (float)md;
      lo[i] = r - (float)md;
    }
    bf16_t* row = static_cast<bf16_t*>(p.out_key) + orow * 3 * c;
    *reinterpret_cast<bf16x8*>(row + ch0) = to_bf16x8(hi);
    *reinterpret_cast<bf16x8*>(row + c + ch0) = to_bf16x8(mid);
    *reinterpret_cast<bf16x8*>(row + 2 * c + ch0) = to_bf16x8(lo);
  } else if (p.key_f32 == 3 || p.key_f32 == 4) {
    h8 hi, lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float xs = x[i] * kSplit16Scale;
      hi[i] = (_Float16)xs;
      lo[i] = (_Float16)(xs - (float)hi[i]);
    }
    _Float16* base = static_cast<_Float16*>(p.out_key);
    if (p.key_f32 == 3) {
      *reinterpret_cast<h8*>(base + orow * 2 * c + ch0) = hi;
      *reinterpret_cast<h8*>(base + orow * 2 * c + c + ch0) = lo;
    } else {
      const int nb = p.T / p.m;
      *reinterpret_cast<h8*>(base + chunked_key_offset(orow, nb, c, 0, ch0)) = hi;
      *reinterpret_cast<h8*>(base + chunked_key_offset(orow, nb, c, 1, ch0)) = lo;
    }
  } else {
    *reinterpret_cast<bf16x8*>(static_cast<bf16_t*>(p.out_key) + orow * c + ch0) = to_bf16x8(x);
  }
}

// Lane-parallel compression for short blocks (m, or 2m when overlapped,
// below 16 rows; c in {32,64,128}, 16-byte aligned rows): LPR = C / 8 lanes
// per compressed block, each owning 8 channels with 16-byte loads and stores,
// 64 / LPR blocks per wave. Per channel the same two passes as
// compress_kernel, in the same order (max over the a-branch logits then the
// b-branch ones; sums likewise), so the block values are those of
// compress_kernel bit for bit; the row norms reduce over the block's LPR lanes.
// MR > 0 (two-byte inputs, m <= MR): the block's rows are all loaded before
// the passes, which then run from registers.
template <typename InT, bool OVERLAP, int C, int MR>
__global__ __launch_bounds__(256) void compress_lanes_kernel(CompressParams p) {
  constexpr int LPR = C / 8;
  constexpr int BPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int nb = p.T / p.m;
  const long long blocks = (long long)p.B * nb;
  const long long gblk = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * BPW + lane / LPR;
  const bool active = gblk < blocks;
  const long long gb = active ? gblk : blocks - 1;  // (inactive lanes compute a copy, store nothing)
  const int b = (int)(gb / nb), blk = (int)(gb - (long long)b * nb);
  const int m = p.m;
  const int ch0 = 8 * (lane % LPR);
  const InT* Ca = static_cast<const InT*>(p.Ca);
  const InT* Za = static_cast<const InT*>(p.Za);
  const InT* Cb = static_cast<const InT*>(p.Cb);
  const InT* Zb = static_cast<const InT*>(p.Zb);
  const size_t ta = (size_t)b * p.T + (size_t)blk * m;
  const bool prev = OVERLAP && blk > 0;
  const size_t tb = ta - m;
  float mx[8], z[8], bp[8], cv[8], den[8], num[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mx[i] = -INFINITY;
    den[i] = num[i] = 0.f;
  }
  if constexpr (MR > 0) {
    // every Z and C row of the block loaded at once (16 bytes each, one
    // round trip), then both passes from registers
    static_assert(sizeof(InT) == 2, "register rows hold 8 two-byte values");
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 zr[2][MR], cr[2][MR];
    const size_t tbs = prev ? tb : ta;  // (a readable row when there is no b-branch)
#pragma unroll
    for (int j = 0; j < MR; ++j) {
      if (j < m) {
        zr[0][j] = *reinterpret_cast<const u32x4*>(Za + (ta + j) * p.ldZa + ch0);
        cr[0][j] = *reinterpret_cast<const u32x4*>(Ca + (ta + j) * p.ldCa + ch0);
        if (OVERLAP) {
          zr[1][j] = *reinterpret_cast<const u32x4*>(Zb + (tbs + j) * p.ldZb + ch0);
          cr[1][j] = *reinterpret_cast<const u32x4*>(Cb + (tbs + j) * p.ldCb + ch0);
        }
      }
    }
    auto unpack = [](const u32x4& r, float* f) { Load8<InT>::run(reinterpret_cast<const InT*>(&r), f); };
#pragma unroll
    for (int br = 0; br < (OVERLAP ? 2 : 1); ++br) {
      if (br == 1 && !prev) break;
      const float* Bp = br ? p.Bb : p.Ba;
#pragma unroll
      for (int j = 0; j < MR; ++j) {
        if (j < m) {
          unpack(zr[br][j], z);
          Load8<float>::run(Bp + j * C + ch0, bp);
#pragma unroll
          for (int i = 0; i < 8; ++i) mx[i] = fmaxf(mx[i], z[i] + bp[i]);
        }
      }
    }
#pragma unroll
    for (int br = 0; br < (OVERLAP ? 2 : 1); ++br) {
      if (br == 1 && !prev) break;
      const float* Bp = br ? p.Bb : p.Ba;
#pragma unroll
      for (int j = 0; j < MR; ++j) {
        if (j < m) {
          unpack(zr[br][j], z);
          unpack(cr[br][j], cv);
          Load8<float>::run(Bp + j * C + ch0, bp);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float e = exp_hw(z[i] + bp[i] - mx[i]);
            den[i] += e;
            num[i] += e * cv[i];
          }
        }
      }
    }
  } else {
    for (int j = 0; j < m; ++j) {
      Load8<InT>::run(Za + (ta + j) * p.ldZa + ch0, z);
      Load8<float>::run(p.Ba + j * C + ch0, bp);
#pragma unroll
      for (int i = 0; i < 8; ++i) mx[i] = fmaxf(mx[i], z[i] + bp[i]);
    }
    if (prev)
      for (int j = 0; j < m; ++j) {
        Load8<InT>::run(Zb + (tb + j) * p.ldZb + ch0, z);
        Load8<float>::run(p.Bb + j * C + ch0, bp);
#pragma unroll
        for (int i = 0; i < 8; ++i) mx[i] = fmaxf(mx[i], z[i] + bp[i]);
      }
    for (int j = 0; j < m; ++j) {
      Load8<InT>::run(Za + (ta + j) * p.ldZa + ch0, z);
      Load8<float>::run(p.Ba + j * C + ch0, bp);
      Load8<InT>::run(Ca + (ta + j) * p.ldCa + ch0, cv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = exp_hw(z[i] + bp[i] - mx[i]);
        den[i] += e;
        num[i] += e * cv[i];
      }
    }
    if (prev)
      for (int j = 0; j < m; ++j) {
        Load8<InT>::run(Zb + (tb + j) * p.ldZb + ch0, z);
        Load8<float>::run(p.Bb + j * C + ch0, bp);
        Load8<InT>::run(Cb + (tb + j) * p.ldCb + ch0, cv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float e = exp_hw(z[i] + bp[i] - mx[i]);
          den[i] += e;
          num[i] += e * cv[i];
        }
      }
  }
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = num[i] / den[i];
  // sum of squares over the block's LPR lanes (aligned lane groups)
  auto group_sum = [&](float v) {
#pragma unroll
    for (int d = 1; d < LPR; d <<= 1) v += __shfl_xor(v, d);
    return v;
  };
  const size_t orow = (size_t)b * nb + blk;
  if (p.out_raw && active) {
    float* d = p.out_raw + orow * C + ch0;
    *reinterpret_cast<float4*>(d) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4*>(d + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  if (p.out_key) {
    float inv = 1.f;
    if (p.normalize) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += acc[i] * acc[i];
      inv = l2_inv(group_sum(ss));
    }
    float kx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) kx[i] = acc[i] * inv;
    if (active) store_key8(p, orow, C, ch0, kx);
  }
  if (p.local) {
    // window keys of the block's m source tokens (from the a-branch values)
    for (int j = 0; j < m; ++j) {
      const size_t t = ta + j;
      Load8<InT>::run(Ca + t * p.ldCa + ch0, cv);
      float inv = 1.f;
      if (p.normalize) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += cv[i] * cv[i];
        inv = l2_inv(group_sum(ss));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) cv[i] *= inv;
      if (active) *reinterpret_cast<bf16x8*>(p.local + t * C + ch0) = to_bf16x8(cv);
    }
  }
}

// Row-parallel compression for long blocks (m or 2m >= 16 rows, c in {64,128},
// 16-byte aligned rows). A workgroup (4 waves) takes one compressed block:
// lane l of wave w owns channels 8 (l % LPR) .. + 7 of the row slot
// w * RPW + l / LPR; the slots take the block's rows round-robin, four rows
// in flight per slot. Each slot keeps, per channel, an online softmax of its
// rows (running max, sum of exp, exp-weighted sum of C); the slots are then
// merged (lane shuffles, then LDS across the waves) into the same weighted
// mean as the two-pass form of compress_kernel. The per-token window keys are
// written from the slot that reads the token's a-branch row.
template <typename InT, bool OVERLAP, int C>
__global__ __launch_bounds__(256) void compress_rows_kernel(CompressParams p) {
  constexpr int LPR = C / 8;           // lanes per row
  constexpr int RPW = 64 / LPR;        // row slots per wave
  constexpr int NSLOT = 4 * RPW;
  constexpr int U = 4;                 // rows in flight per slot
  __shared__ float part[4][3][C];
  __shared__ float red[4];
  const int nb = p.T / p.m;
  const int b = blockIdx.x / nb, blk = blockIdx.x - b * nb;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int slot = wv * RPW + lane / LPR, ch0 = 8 * (lane % LPR);
  const int m = p.m;
  const int nrows = (OVERLAP && blk > 0) ? 2 * m : m;
  const InT* Ca = static_cast<const InT*>(p.Ca);
  const InT* Za = static_cast<const InT*>(p.Za);
  const InT* Cb = static_cast<const InT*>(p.Cb);
  const InT* Zb = static_cast<const InT*>(p.Zb);
  const long long ta = (long long)b * p.T + (long long)blk * m;  // token of a-branch row 0

  float mx[8], den[8], num[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    mx[i] = -INFINITY;
    den[i] = 0.f;
    num[i] = 0.f;
  }
  for (int r0 = slot; r0 < nrows; r0 += U * NSLOT) {
    float z[U][8], v[U][8];
    bool bsel[U];
    long long tok[U];
    // loads of U rows (past the end: row r0 again, not used)
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int rr = r0 + k * NSLOT;
      const int r = rr < nrows ? rr : r0;
      const bool bb = OVERLAP && r >= m;
      const int j = bb ? r - m : r;
      bsel[k] = bb;
      tok[k] = bb ? ta - m + j : ta + j;
      const InT* zp = bb ? Zb + tok[k] * p.ldZb : Za + tok[k] * p.ldZa;
      const InT* cp = bb ? Cb + tok[k] * p.ldCb : Ca + tok[k] * p.ldCa;
      const float* bp = (bb ? p.Bb : p.Ba) + (size_t)j * C + ch0;
      Load8<InT>::run(zp + ch0, z[k]);
      Load8<InT>::run(cp + ch0, v[k]);
      const float4 b0 = *reinterpret_cast<const float4*>(bp);
      const float4 b1 = *reinterpret_cast<const float4*>(bp + 4);
      z[k][0] += b0.x; z[k][1] += b0.y; z[k][2] += b0.z; z[k][3] += b0.w;
      z[k][4] += b1.x; z[k][5] += b1.y; z[k][6] += b1.z; z[k][7] += b1.w;
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      if (r0 + k * NSLOT >= nrows) continue;  // same for the whole slot
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // online softmax step: one exp per element (the hardware exp2)
        const float d = z[k][i] - mx[i];
        const bool up = d > 0.f;
        const float e = exp_hw(up ? -d : d);  // mx = -inf: d = +inf, e = 0
        den[i] = up ? fmaf(den[i], e, 1.f) : den[i] + e;
        num[i] = up ? fmaf(num[i], e, v[k][i]) : fmaf(e, v[k][i], num[i]);
        mx[i] = up ? z[k][i] : mx[i];
      }
      if (p.local && !bsel[k]) {
        // window key of this token: L2norm over the row's LPR lanes
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += v[k][i] * v[k][i];
#pragma unroll
        for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o);
        const float inv = p.normalize ? l2_inv(ss) : 1.f;
        float f[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = v[k][i] * inv;
        *reinterpret_cast<bf16x8*>(p.local + tok[k] * C + ch0) = to_bf16x8(f);
      }
    }
  }
  // merge the slots of the wave (lanes LPR, 2 LPR, .. apart), then the waves
#pragma unroll
  for (int o = LPR; o < 64; o <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float m2 = __shfl_xor(mx[i], o), d2 = __shfl_xor(den[i], o), n2 = __shfl_xor(num[i], o);
      const float mm = fmaxf(mx[i], m2);
      if (mm != -INFINITY) {
        const float e1 = exp_hw(mx[i] - mm), e2 = exp_hw(m2 - mm);
        den[i] = den[i] * e1 + d2 * e2;
        num[i] = num[i] * e1 + n2 * e2;
        mx[i] = mm;
      }
    }
  }
  if (lane < LPR) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      part[wv][0][ch0 + i] = mx[i];
      part[wv][1][ch0 + i] = den[i];
      part[wv][2][ch0 + i] = num[i];
    }
  }
  __syncthreads();
  const int ch = threadIdx.x;
  float acc = 0.f;
  if (ch < C) {
    float M = part[0][0][ch];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, part[w][0][ch]);
    float dd = 0.f, nn = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = part[w][0][ch];
      if (mw != -INFINITY) {
        const float e = exp_hw(mw - M);
        dd += part[w][1][ch] * e;
        nn += part[w][2][ch] * e;
      }
    }
    acc = nn / dd;
  }
  const size_t orow = (size_t)b * nb + blk;
  if (ch < C && p.out_raw) p.out_raw[orow * C + ch] = acc;
  if (p.out_key) {
    float inv = 1.f;
    if (p.normalize) {
      const float s = wave_sum(acc * acc);  // channels >= C contribute 0
      if (lane == 0) red[wv] = s;
      __syncthreads();
      inv = l2_inv(red[0] + red[1] + red[2] + red[3]);
    }
    if (ch < C) store_key(p, orow, C, ch, acc * inv);
  }
}

// The row-parallel kernel applies: 16-byte aligned 8-channel groups everywhere.
static bool compress_rows_ok(const CompressParams& p, int dtype) {
  const int rows = p.m * (p.overlap ? 2 : 1);
  if (rows < 16 || (p.c != 64 && p.c != 128)) return false;
  const long long es = dtype == DT_F32 ? 4 : 2;
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; };
  auto ld_ok = [&](long long ld) { return (ld * es) % 16 == 0; };
  bool ok = al(p.Ca) && al(p.Za) && al(p.Ba) && al(p.local) && ld_ok(p.ldCa) && ld_ok(p.ldZa);
  if (p.overlap) ok = ok && al(p.Cb) && al(p.Zb) && al(p.Bb) && ld_ok(p.ldCb) && ld_ok(p.ldZb);
  return ok;
}

template <bool OVERLAP, int C>
static void launch_compress_rows(const CompressParams& p, int dtype, hipStream_t stream) {
  const dim3 grid(p.B * (p.T / p.m)), block(256);
  if (dtype == DT_F32) hipLaunchKernelGGL((compress_rows_kernel<float, OVERLAP, C>), grid, block, 0, stream, p);
  else if (dtype == DT_BF16) hipLaunchKernelGGL((compress_rows_kernel<bf16_t, OVERLAP, C>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((compress_rows_kernel<_Float16, OVERLAP, C>), grid, block, 0, stream, p);
}

// The lane-parallel form: short blocks, c in {32,64,128}, 16-byte aligned rows
// (Ba / Bb rows of c fp32 are then 16-byte aligned too).
static bool compress_lanes_ok(const CompressParams& p, int dtype) {
  const int rows = p.m * (p.overlap ? 2 : 1);
  if (rows >= 16 || (p.c != 32 && p.c != 64 && p.c != 128)) return false;
  const long long es = dtype == DT_F32 ? 4 : 2;
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; };
  auto ld_ok = [&](long long ld) { return (ld * es) % 16 == 0; };
  bool ok = al(p.Ca) && al(p.Za) && al(p.Ba) && al(p.local) && al(p.out_raw) && al(p.out_key) &&
            ld_ok(p.ldCa) && ld_ok(p.ldZa);
  if (p.overlap) ok = ok && al(p.Cb) && al(p.Zb) && al(p.Bb) && ld_ok(p.ldCb) && ld_ok(p.ldZb);
  return ok;
}

template <bool OVERLAP, int C>
static void launch_compress_lanes(const CompressParams& p, int dtype, hipStream_t stream) {
  constexpr int BPW = 64 / (C / 8);
  const long long blocks = (long long)p.B * (p.T / p.m);
  const long long waves = (blocks + BPW - 1) / BPW;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  const bool regs = p.m <= 4;
  if (dtype == DT_F32)
    hipLaunchKernelGGL((compress_lanes_kernel<float, OVERLAP, C, 0>), grid, block, 0, stream, p);
  else if (dtype == DT_BF16) {
    if (regs) hipLaunchKernelGGL((compress_lanes_kernel<bf16_t, OVERLAP, C, 4>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((compress_lanes_kernel<bf16_t, OVERLAP, C, 0>), grid, block, 0, stream, p);
  } else {
    if (regs) hipLaunchKernelGGL((compress_lanes_kernel<_Float16, OVERLAP, C, 4>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((compress_lanes_kernel<_Float16, OVERLAP, C, 0>), grid, block, 0, stream, p);
  }
}

hipError_t compress_dispatch(const CompressParams& p, int dtype, hipStream_t stream) {
  if (p.B * (p.T / p.m) > 0 && compress_lanes_ok(p, dtype)) {
    if (p.overlap) {
      if (p.c == 128) launch_compress_lanes<true, 128>(p, dtype, stream);
      else if (p.c == 64) launch_compress_lanes<true, 64>(p, dtype, stream);
      else launch_compress_lanes<true, 32>(p, dtype, stream);
    } else {
      if (p.c == 128) launch_compress_lanes<false, 128>(p, dtype, stream);
      else if (p.c == 64) launch_compress_lanes<false, 64>(p, dtype, stream);
      else launch_compress_lanes<false, 32>(p, dtype, stream);
    }
    return hipGetLastError();
  }
  if (p.B * (p.T / p.m) > 0 && compress_rows_ok(p, dtype)) {
    if (p.overlap) {
      if (p.c == 128) launch_compress_rows<true, 128>(p, dtype, stream);
      else launch_compress_rows<true, 64>(p, dtype, stream);
    } else {
      if (p.c == 128) launch_compress_rows<false, 128>(p, dtype, stream);
      else launch_compress_rows<false, 64>(p, dtype, stream);
    }
    return hipGetLastError();
  }
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

// Selected indices a wave keeps in LDS (IDXL): the whole top-k of its query.
constexpr int kIdxLds = 512;

template <int HD, typename QT, typename OT, bool SPARSE, bool IDXL = false>
__global__ __launch_bounds__(256, 3) void attn_prefill_kernel(AttnParams p) {
  using W = MqaWave<HD>;
  static_assert(!IDXL || SPARSE, "LDS indices are the selected blocks'");
  __shared__ __attribute__((aligned(16))) bf16_t stage_all[4][W::STAGE_ELEMS];
  __shared__ __attribute__((aligned(16))) int idx_all[IDXL ? 4 * kIdxLds : 4];
  static_assert(16 * HD * sizeof(OT) <= sizeof(stage_all[0]), "output rows fit in the stage");
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  bf16_t* stage = stage_all[wv];
  const int T = p.T;
  // query index: consecutive queries of one batch row per workgroup
  const long long qi = (long long)blockIdx.x * 4 + wv;
  if (qi >= (long long)p.B * T) return;
  const int b = (int)(qi / T), t = (int)(qi - (long long)b * T);

  // The query's words are requested first and converted once the first rows
  // are in flight: their latency overlaps the index and row requests (a wait
  // for a load also waits for the loads issued before it, so the query goes
  // first). A padding head (n >= nh) reads head 0 and is zeroed.
  const QT* qrow = static_cast<const QT*>(p.q) + ((size_t)qi * p.nh + (n < p.nh ? n : 0)) * HD;
  typedef uint32_t u32x4q __attribute__((ext_vector_type(4)));
  constexpr int QWD = sizeof(QT) == 4 ? 2 : 1;  // 16-byte words per 8 query elements
  u32x4q qraw[W::NS][QWD];
#pragma unroll
  for (int s = 0; s < W::NS; ++s)
#pragma unroll
    for (int h = 0; h < QWD; ++h)
      qraw[s][h] = *reinterpret_cast<const u32x4q*>(qrow + 32 * s + 8 * (lane >> 4) + 4 * h);
  W w;
  auto setup_q = [&]() {
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
  };

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
  const int nm = p.nb > 0 ? n_main : 0;
  // the compressed rows are padded to whole 32-row steps (padding rows are
  // masked), so that every step is wholly compressed or wholly window rows
  const int nm_pad = (nm + 31) & ~31;
  const int n_tot = nm_pad + n_win;
  if (nm + n_win > 0) {
    // Rows are read through two buffer resources, the compressed rows of this
    // batch row and its window rows, with 32-bit byte offsets: an offset past
    // a resource's end (a -1 slot, a block index out of range, a padding row)
    // reads zeros, so a row address is one multiply-add and no row needs a
    // readable default.
    constexpr int ROWB = HD * 2;  // bytes per row
    const __amdgpu_buffer_rsrc_t rs_kv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(kv), 0, p.nb > 0 ? p.nb * ROWB : 0, 0x00020000);
    const int nloc = n_win > 0 ? (p.local_count >= 0 ? p.local_count : T) : 0;
    const __amdgpu_buffer_rsrc_t rs_loc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(loc ? loc : kv), 0, nloc * ROWB, 0x00020000);
    const int lane_off = 16 * (lane % W::TPR);
    const int q4 = lane >> 4;
    const int hmask = (W::TPR == 8 && ((lane >> 3) & 1)) ? -1 : 0;
    // Rows are taken in the score layout (MqaWave::chunk_sl): this lane's slot
    // k of a 32-row step is row row_sl(k, q4), whose score it holds. The row
    // indices of a step (selected block, causal block or window position) are
    // fetched two steps ahead of the row loads that use them: the selected
    // ones through a buffer resource over this query's topk entries (16-byte
    // loads when nm is a multiple of 4, so that no load straddles its end;
    // reads past it give 0, and such rows are masked by j < nm).
    const bool has_idx = SPARSE && nm > 0;
    const __amdgpu_buffer_rsrc_t rs_idx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int*>(has_idx ? p.idx + (size_t)qi * p.topk : nullptr), 0, has_idx ? nm * 4 : 0,
        0x00020000);
    const bool idx16 = (nm & 3) == 0;
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    // IDXL (nm <= kIdxLds): the query's indices go to the wave's LDS once, 8
    // per lane, and each step reads its own from there. The row gathers are
    // then the loop's only memory loads, so every wait before a row's use
    // counts exactly the loads issued after it (an index load in a branch of
    // the loop made the waits there drain every load in flight).
    int* const idx_lds = idx_all + (IDXL ? wv * kIdxLds : 0);
    if constexpr (IDXL) {
      if (has_idx) {
        i32x4 a, c;
        if (idx16) {
          a = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, 32 * lane, 0, 0));
          c = __builtin_bit_cast(i32x4,
                                 __builtin_amdgcn_raw_buffer_load_b128(rs_idx, 32 * lane + 16, 0, 0));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[e] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_idx, 32 * lane + 4 * e, 0, 0);
            c[e] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_idx, 32 * lane + 16 + 4 * e, 0, 0);
          }
        }
        *reinterpret_cast<i32x4*>(idx_lds + 8 * lane) = a;
        *reinterpret_cast<i32x4*>(idx_lds + 8 * lane + 4) = c;
        wave_lds_sync();
      }
    }
    struct Sel {
      int v[8];
    };
    auto load_sel = [&](int st, Sel& sl) {
      const int j0 = 32 * st;
      if (__builtin_amdgcn_readfirstlane(j0 < nm_pad ? 1 : 0)) {
        if constexpr (IDXL) {
          const i32x4 a = *reinterpret_cast<const i32x4*>(idx_lds + j0 + 4 * q4);
          const i32x4 c = *reinterpret_cast<const i32x4*>(idx_lds + j0 + 16 + 4 * q4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sl.v[e] = a[e];
            sl.v[4 + e] = c[e];
          }
        } else if (SPARSE) {
          if (idx16) {
            const i32x4 a = __builtin_bit_cast(
                i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, (j0 + 4 * q4) * 4, 0, 0));
            const i32x4 c = __builtin_bit_cast(
                i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_idx, (j0 + 16 + 4 * q4) * 4, 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              sl.v[e] = a[e];
              sl.v[4 + e] = c[e];
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
        for (int k = 0; k < 8; ++k) sl.v[k] = wbase + (j0 - nm_pad) + W::row_sl(k, q4);
      }
    };
    // the row loads of step st from its indices; ok[k]: slot k is a row of
    // this query. Returns (uniform) 0 when no row of the step is, 2 when every
    // row is (ok then unset), else 1.
    auto load_rows = [&](int st, const Sel& sl, typename W::Rows& rr, bool (&ok)[8]) -> int {
      const int j0 = 32 * st;
      const int ms = __builtin_amdgcn_readfirstlane(j0 < nm_pad ? 1 : 0);
      const __amdgpu_buffer_rsrc_t rs = ms ? rs_kv : rs_loc;
      // a step past the query's rows (the loop loads two ahead) reads nothing
      // from memory: its offsets get bit 31 set, beyond every resource (< 2 GiB)
      const unsigned past = __builtin_amdgcn_readfirstlane(j0 >= n_tot ? 0x80000000u : 0u);
#pragma unroll
      for (int i = 0; i < W::NLI; ++i) {
        // HD 64: the upper 8 lanes of a group take slot i + 4 (a select of
        // values, not an indexed read: that would put sl in scratch memory)
        const int v = W::TPR == 8 ? sl.v[i] ^ ((sl.v[i] ^ sl.v[(i + 4) & 7]) & hmask) : sl.v[i];
        rr.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(((unsigned)v * ROWB + lane_off) | past), 0, 0);
      }
      // a step wholly inside the window rows is all valid; one wholly inside
      // the selected slots needs only each slot's -1 / range test
      if (!ms && j0 - nm_pad + 32 <= n_win) return 2;
      bool any = false;
      if (ms && j0 + 32 <= nm) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          ok[k] = (unsigned)sl.v[k] < (unsigned)p.nb;
          any |= ok[k];
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int j = j0 + W::row_sl(k, q4);
          const bool okm = (j < nm) & ((unsigned)sl.v[k] < (unsigned)p.nb);
          const bool okw = j - nm_pad < n_win;
          ok[k] = ms ? okm : okw;
          any |= ok[k];
        }
      }
      return __ballot(any) != 0ull ? 1 : 0;
    };
    // two steps of rows in flight and the indices of the two after them
    // (named registers: an indexed array of them ends up in scratch memory)
    const TileOffsets<HD> to;
    const int nst = (n_tot + 31) / 32;
    const int ng = (nst + 1) / 2;
    Sel s0, s1;
    typename W::Rows fr0, fr1;
    bool ok0[8], ok1[8];
    load_sel(0, s0);
    load_sel(1, s1);
    int any0 = load_rows(0, s0, fr0, ok0);
    int any1 = load_rows(1, s1, fr1, ok1);
    load_sel(2, s0);
    load_sel(3, s1);
    setup_q();
    for (int g = 0; g < ng; ++g) {
      if (any0) w.chunk_sl(fr0, ok0, stage, to, any0 == 2);
      any0 = load_rows(2 * g + 2, s0, fr0, ok0);
      load_sel(2 * g + 4, s0);
      if (any1) w.chunk_sl(fr1, ok1, stage, to, any1 == 2);
      any1 = load_rows(2 * g + 3, s1, fr1, ok1);
      load_sel(2 * g + 5, s1);
    }
  } else {
    setup_q();
  }
  w.finalize();
  const float f = w.finish(p.sink != nullptr, (p.sink && n < p.nh) ? p.sink[n] : 0.f);
  wave_lds_sync();  // the last step's V^T reads are done before the stage is reused
  store_rows<HD, OT>(w.o, f, static_cast<OT*>(p.out) + (size_t)qi * p.nh * HD, p.nh, stage);
}

// ---------------------------------------------------------------------------
// Dense joint-softmax MQA over query tiles (the naive_hca core with window
// positions [t-win+1, t]). A workgroup takes QG = 4 * QW consecutive queries
// of one sequence. Their key rows -- the union of the causally visible
// compressed blocks, then the union of the window positions -- are streamed
// through LDS 64 rows at a time and shared by the four waves; each wave owns
// QW queries and masks, per query, the rows outside that query's own set, so
// every query attends to exactly the rows of the per-query kernel above.
//
// LDS tile: rows of HD bf16; 16-byte chunk c of row r is stored at chunk
// c ^ tile_swz(r % 16). The swizzle keeps the three access patterns free of
// bank conflicts: the tile loads (a row's chunks by consecutive lanes), the
// key-fragment reads (chunk 4s + lane / 16 of row lane % 16) and the
// transposing V^T reads (32 lanes read two adjacent chunks of 8 rows).
// ---------------------------------------------------------------------------
constexpr int kTileGroup = 16;  // consecutive query tiles kept on one XCD

template <int HD, int QW, int NWV, int MINB, typename QT, typename OT>
__global__ __launch_bounds__(64 * NWV, MINB) void attn_dense_tile_kernel(AttnParams p, int ntile) {
  using W = MqaWave<HD>;
  constexpr int NTH = 64 * NWV;         // threads per workgroup
  constexpr int QG = NWV * QW;          // queries per workgroup
  constexpr int KC = 128;               // key rows per LDS tile
  constexpr int TPR = HD / 8;           // 16-byte chunks per row
  constexpr int RSTEP = NTH / TPR;      // rows per load pass of the workgroup
  constexpr int NLD = KC / RSTEP;       // loads per thread per tile
  static_assert(NLD == 1 || NLD == 2 || NLD == 4, "tile loads per thread");
  static_assert(RSTEP % 16 == 0, "load rows keep their swizzle");
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) bf16_t tile[2][KC * HD];

  // Workgroup i runs on XCD i % 8. Groups of kTileGroup consecutive tiles
  // (which share window rows) stay on one XCD, hence one L2, and the groups
  // are dealt to the XCDs round-robin, so that every XCD gets the same mix of
  // short (early) and long (late) queries.
  const int xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3);
  const int tix = ((slot / kTileGroup) * 8 + xcd) * kTileGroup + slot % kTileGroup;
  if (tix >= ntile) return;
  const int T = p.T;
  const int tps = (T + QG - 1) / QG;
  const int b = tix / tps;
  const int t0 = (tix - b * tps) * QG;
  const int tl = min(t0 + QG, T) - 1;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int tid = threadIdx.x;
  const int lane = tid & 63, q4 = lane >> 4, n = lane & 15;

  auto nvis = [&](int t) { return max(0, min(p.nb, (p.pos0 + t + 1) / p.m)); };
  const bf16_t* kv = p.kv_comp + (size_t)b * (p.kv_bstride ? p.kv_bstride : (long long)p.nb * HD);
  const int nc = p.nb > 0 ? nvis(tl) : 0;
  const bf16_t* loc = nullptr;
  int wlo = 0, nw = 0;
  if (p.win > 0 && p.kv_local) {
    loc = p.kv_local + (size_t)b * (p.local_bstride ? p.local_bstride : (long long)T * HD);
    wlo = max(t0 - p.win + 1, 0);
    nw = tl - wlo + 1;
  }
  const int R = nc + nw;

  // Tile loads: thread tid takes 16-byte chunk tid % TPR of rows
  // tid / TPR + RSTEP i. Row j of the union is row j of kvb below nc, else
  // row j of lcb (window position wlo + j - nc); past R, row R - 1 again
  // (loaded, never read).
  const int lrow = tid / TPR, lch = tid % TPR;
  const int soff = lrow * HD + 8 * (lch ^ tile_swz<HD>(lrow & 15));
  const bf16_t* kvb = kv + 8 * lch;
  const bf16_t* lcb = loc ? loc + (long long)(wlo - nc) * HD + 8 * lch : kvb;
  auto src_of = [&](int j) -> const bf16_t* {
    const int jj = min(j, R - 1);
    return (jj < nc ? kvb : lcb) + (size_t)(unsigned)jj * HD;
  };
  // named registers (an indexed array of them ends up in scratch memory)
  uint4 pf0, pf1, pf2, pf3;
  auto issue = [&](int c) {
    pf0 = *reinterpret_cast<const uint4*>(src_of(c * KC + lrow));
    if constexpr (NLD >= 2) pf1 = *reinterpret_cast<const uint4*>(src_of(c * KC + lrow + RSTEP));
    if constexpr (NLD == 4) {
      pf2 = *reinterpret_cast<const uint4*>(src_of(c * KC + lrow + 2 * RSTEP));
      pf3 = *reinterpret_cast<const uint4*>(src_of(c * KC + lrow + 3 * RSTEP));
    }
  };
  // the first tile's rows are in flight while the queries load
  if (R > 0) issue(0);

  // This wave's queries and, per query, its rows: [0, a) and [lo, hi].
  W w[QW];
  int a_[QW], lo_[QW], hi_[QW];
#pragma unroll
  for (int u = 0; u < QW; ++u) {
    const int t = t0 + QW * wv + u;
    const bool live = t < T;
    const QT* qrow = static_cast<const QT*>(p.q) +
                     (((size_t)b * T + (live ? t : tl)) * p.nh + min(n, p.nh - 1)) * HD;
    w[u].template init_always<QT>(qrow, live && n < p.nh, p.normalize_q != 0, p.scale);
    a_[u] = live && p.nb > 0 ? nvis(t) : 0;
    lo_[u] = 1;
    hi_[u] = 0;
    if (live && nw > 0) {
      lo_[u] = nc + max(t - p.win + 1, 0) - wlo;
      hi_[u] = nc + t - wlo;
    }
  }

  if (R > 0) {
    const TileOffsets<HD> to;
    // 32 rows of the tile (LDS row base `rows`, key index j0 of row 0)
    auto rows32 = [&](const bf16_t* rows, int j0) {
      f32x4 sa[QW], sb[QW];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        bf16x8 kf[W::NS];
#pragma unroll
        for (int s2 = 0; s2 < W::NS; ++s2)
          kf[s2] = *reinterpret_cast<const bf16x8*>(rows + 16 * HD * h + to.key(s2));
#pragma unroll
        for (int u = 0; u < QW; ++u) {
          if (h == 0) sa[u] = w[u].scores(kf);
          else sb[u] = w[u].scores(kf);
        }
      }
      bf16x8 pb[QW];
#pragma unroll
      for (int u = 0; u < QW; ++u) {
        float sc[8] = {sa[u][0], sa[u][1], sa[u][2], sa[u][3], sb[u][0], sb[u][1], sb[u][2], sb[u][3]};
        const bool full = (j0 + 32 <= a_[u]) || (j0 >= lo_[u] && j0 + 31 <= hi_[u]);
        if (!full) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int j = j0 + 4 * q4 + (e < 4 ? e : 12 + e);
            const bool ok = (j < a_[u]) | ((j >= lo_[u]) & (j <= hi_[u]));
            sc[e] = ok ? sc[e] : -INFINITY;
          }
        }
        pb[u] = w[u].softmax32(sc);
      }
      // each V^T fragment serves every query of the wave
#pragma unroll
      for (int t = 0; t < W::NT; ++t) {
        const bf16x8 va = W::vt_frag(rows, to, t);
#pragma unroll
        for (int u = 0; u < QW; ++u)
          w[u].o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[u], w[u].o[t], 0, 0, 0);
      }
    };

    const int nct = (R + KC - 1) / KC;
    auto store = [&](bf16_t* dst) {
      *reinterpret_cast<uint4*>(dst + soff) = pf0;
      if constexpr (NLD >= 2) *reinterpret_cast<uint4*>(dst + soff + RSTEP * HD) = pf1;
      if constexpr (NLD == 4) {
        *reinterpret_cast<uint4*>(dst + soff + 2 * RSTEP * HD) = pf2;
        *reinterpret_cast<uint4*>(dst + soff + 3 * RSTEP * HD) = pf3;
      }
    };
    // one tile: the next tile's rows are in flight while this one is consumed
    auto step = [&](int c, const bf16_t* cur, bf16_t* nxt) {
      issue(c + 1);
      const int nsc = min(KC / 32, (R - c * KC + 31) / 32);
#pragma unroll
      for (int sc = 0; sc < KC / 32; ++sc)
        if (sc < nsc) rows32(cur + 32 * sc * HD, c * KC + 32 * sc);
      store(nxt);
      __syncthreads();
    };
    store(tile[0]);
    __syncthreads();
    // two tiles per iteration, so that each LDS buffer address is static
    for (int c = 0; c < nct; c += 2) {
      step(c, tile[0], tile[1]);
      if (c + 1 < nct) step(c + 1, tile[1], tile[0]);
    }
  }

  // Output rows through LDS (whole-row stores): each wave stages its block in
  // its own slice of the tile buffers, which every wave is done reading (the
  // tile loop ends with a barrier; without rows it never ran).
  static_assert(NWV * 16 * HD * sizeof(OT) <= sizeof(tile), "staging fits in the tile buffers");
#pragma unroll
  for (int u = 0; u < QW; ++u) {
    const int t = t0 + QW * wv + u;
    w[u].finalize();
    const float f = w[u].finish(p.sink != nullptr, (p.sink && n < p.nh) ? p.sink[n] : 0.f);
    if (u > 0) wave_lds_sync();  // the previous query's staged rows are read
    if (t < T)
      store_rows<HD, OT>(w[u].o, f, static_cast<OT*>(p.out) + ((size_t)b * T + t) * p.nh * HD, p.nh,
                         reinterpret_cast<char*>(&tile[0][0]) + wv * 16 * HD * sizeof(OT));
  }
}

// Query-tile shape: QW queries per wave, NWV waves per workgroup, at least
// MINB workgroups per CU.
constexpr int kTileQW = 1, kTileWaves = 8, kTileMinBlocks = 2;

template <int HD>
static hipError_t launch_dense_tile(const AttnParams& p, int qdtype, int odtype, hipStream_t s) {
  constexpr int QW = kTileQW, NWV = kTileWaves, MINB = kTileMinBlocks, QG = NWV * QW;
  const long long ntile = (long long)p.B * ((p.T + QG - 1) / QG);
  const long long ngroup = (ntile + kTileGroup - 1) / kTileGroup;
  const dim3 grid((unsigned)(((ngroup + 7) / 8) * 8 * kTileGroup)), block(64 * NWV);
#define KCH_TILE_LAUNCH(QT, OT) \
  hipLaunchKernelGGL((attn_dense_tile_kernel<HD, QW, NWV, MINB, QT, OT>), grid, block, 0, s, p, (int)ntile)
  if (qdtype == DT_BF16) {
    if (odtype == DT_F32) KCH_TILE_LAUNCH(bf16_t, float);
    else KCH_TILE_LAUNCH(bf16_t, bf16_t);
  } else if (qdtype == DT_F32) {
    if (odtype == DT_F32) KCH_TILE_LAUNCH(float, float);
    else KCH_TILE_LAUNCH(float, bf16_t);
  } else {
    if (odtype == DT_F32) KCH_TILE_LAUNCH(_Float16, float);
    else KCH_TILE_LAUNCH(_Float16, _Float16);
  }
#undef KCH_TILE_LAUNCH
  return hipGetLastError();
}

template <int HD, bool SPARSE>
static hipError_t launch_attn(const AttnParams& p, int qdtype, int odtype, hipStream_t s) {
  const long long nq = (long long)p.B * p.T;
  const dim3 grid((unsigned)((nq + 3) / 4)), block(256);
  const bool idxl = SPARSE && p.topk <= kIdxLds;
#define KCH_ATTN_LAUNCH(QT, OT)                                                                 \
  do {                                                                                          \
    if (idxl) hipLaunchKernelGGL((attn_prefill_kernel<HD, QT, OT, SPARSE, SPARSE>), grid, block, 0, s, p); \
    else hipLaunchKernelGGL((attn_prefill_kernel<HD, QT, OT, SPARSE, false>), grid, block, 0, s, p); \
  } while (0)
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
  // dense with a window of positions: query tiles sharing the key rows
  if (!sparse && p.local_count < 0)
    return p.hd == 128 ? launch_dense_tile<128>(p, qdtype, odtype, s)
                       : launch_dense_tile<64>(p, qdtype, odtype, s);
  if (p.hd == 128) return sparse ? launch_attn<128, true>(p, qdtype, odtype, s)
                                 : launch_attn<128, false>(p, qdtype, odtype, s);
  return sparse ? launch_attn<64, true>(p, qdtype, odtype, s)
                : launch_attn<64, false>(p, qdtype, odtype, s);
}

}  // namespace kch
