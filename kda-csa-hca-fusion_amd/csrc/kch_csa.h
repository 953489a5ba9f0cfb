// Internal launch interface of the CSA / HCA kernels (csa_hca.hip, indexer.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "kch_device.h"

namespace kch {

// KV compression. Rows of C*/Z* are `ld*` elements apart ([B, T] rows of c
// channels each); B_pos / Ba / Bb are fp32 [m, c].
struct CompressParams {
  const void* Ca; const void* Za; const void* Cb; const void* Zb;
  long long ldCa, ldZa, ldCb, ldZb;
  const float* Ba; const float* Bb;
  float* out_raw;   // [B, nb, c] fp32 or null
  void* out_key;    // [B, nb, c] bf16 (key_f32 0) / fp32 (1), [B, nb, 3, c] split bf16 (2),
                    // [B, nb, 2, c] split fp16 (3), the same chunk-major in whole 16-row
                    // chunks (4), or null
  bf16_t* local;    // [B, T, c] bf16 window keys (from Ca) or null
  int B, T, m, c;
  int overlap, normalize, key_f32;
};
hipError_t compress_dispatch(const CompressParams& p, int dtype, hipStream_t stream);

// Joint-softmax MQA (prefill: one query per token of [B, T]).
struct AttnParams {
  const void* q;            // [B, T, nh, hd] (raw; normalised in-kernel if normalize_q)
  const bf16_t* kv_comp;    // [B, nb, hd] key/value rows
  const int* idx;           // [B, T, topk] selected rows (sparse) or null
  const bf16_t* kv_local;   // [B, T, hd] window rows or null
  const float* sink;        // [nh] or null
  void* out;                // [B, T, nh, hd]
  int B, T, nb, nh, hd, topk, m, win, normalize_q;
  float scale;
  long long kv_bstride;     // elements between batches of kv_comp (0: nb * hd)
  long long local_bstride;  // elements between batches of kv_local (0: T * hd)
  int local_count;          // < 0: window of positions [t-win+1, t]; >= 0: the first
                            // local_count rows of kv_local are the window (ring buffer)
  int pos0;                 // position of query 0 (causal block rule of the dense mode)
};
hipError_t attn_dispatch(const AttnParams& p, bool sparse, int qdtype, int odtype, hipStream_t s);

// Lightning indexer + top-k.
struct IndexerParams {
  const void* q_idx;     // [B, T, nIh, cI]
  const void* k_idx;     // [B, nb, cI] fp32, or (k_split 1) [B, nb, 3, cI] bf16 high / middle /
                         // low parts of each row, or (k_split 2, L2-normalised rows and
                         // normalize_q) [B, nb, 2, cI] fp16 high / low parts of 256 x, or
                         // (k_split 3) the same parts chunk-major, [B, ceil(nb / 16)] chunks
                         // of 16 rows in the lanes' load order (compression key format 4);
                         // already L2-normalised when normalize
  const void* w_idx;     // [B, T, nIh] or null (= ones)
  void* idx_out;         // [B, T, topk] int32 or int64
  float* logits_out;     // optional [B, T, nb] fp32 (diagnostics / tests) or null
  int B, T, nb, nIh, cI, topk, m;
  int q_pos0;            // position of query 0 (decode: the cache's token index)
  int normalize_q, idx64, dense_visible;  // dense_visible: every block visible
  int sorted;            // 1: indices by descending logit; 0: the same set in ascending index
  float scale;
  long long k_bstride;   // 4-byte units between batches of fp32 k_idx (0: nb * cI; split rows: nb rows)
  int k_split;           // 0: fp32 rows; 1: bf16 three-part rows; 2: fp16 two-part rows;
                         // 3: fp16 two-part chunks
};
hipError_t indexer_dispatch(const IndexerParams& p, int dtype, hipStream_t s);
size_t indexer_lds_bytes(int nb, int nIh, int topk);  // dynamic LDS of the indexer kernel

// Decode-step indexer (decode.hip): one query per sequence over every cached block.
struct DecodeIdxParams {
  const void* q_idx;       // [B, nIh, cI] (normalised in-kernel when normalize_q)
  const void* w_idx;       // [B, nIh] or null (= ones), q_idx's dtype
  const void* keys;        // [B, *, cI] cached key rows (bf16 or fp32), batch stride k_bstride
  const float* inv_norm;   // [B, *] 1 / ||key row||, batch stride n_bstride; null = 1
  long long k_bstride, n_bstride;
  unsigned long long* cand;  // [B, nr, topk] per-range candidates (nr > 1)
  int* idx_out;            // [B, topk] selected blocks, sorted, -1 padded
  int B, nb, nIh, cI, topk;
  int rb, nr;              // range size and count (decode_idx_plan)
  int normalize_q;
  float scale;
  long long ld_qb = 0, ld_wb = 0;  // elements between batches of q_idx / w_idx (0: nIh cI, nIh)
  // device-driven step: nb = (*n_seen + 1) / m, at most cap (nr ranges cover cap)
  const int* n_seen = nullptr;
  int m = 1, cap = 0;
  // score / select split (nb <= decode_range_max()): the ranges only write
  // their logit keys to keys_out [B, ko_bstride], then one workgroup per
  // sequence selects from all of them
  uint32_t* keys_out = nullptr;
  long long ko_bstride = 0;
};
void decode_idx_plan(int B, int nb, int topk, int* rb, int* nr);
int decode_range_max();  // most blocks one indexer range holds
size_t decode_select_lds(int topk);
bool decode_merge_fits(int topk);  // the merge kernel's LDS holds its buffers for topk
hipError_t fill_u32(void* p, long long n, uint32_t v, hipStream_t s);
size_t decode_idx_lds(int rb, int topk, int nr);
bool decode_idx_fits(int rb, int topk, int nr);  // the range kernel's LDS fits one CU's 160 KB
size_t decode_merge_lds(int topk);
hipError_t decode_idx_dispatch(const DecodeIdxParams& p, int qdtype, int kdtype, hipStream_t s);

// Decode-step joint-softmax MQA, split over the attended rows (decode.hip).
// Rows of sequence b: j < na -> compressed block idx[b][j] (or j without idx;
// -1 = unused), then the ring_len rows of the ring. Group g (a workgroup)
// covers rows [g * rows_per_group, ...); with several groups per sequence
// each leaves M, L and the unnormalised o per head for the combine kernel.
struct DecodeAttnParams {
  const void* q;           // [B, nh, hd]
  const bf16_t* kv;        // [B, *, hd] key/value rows, batch stride kv_bstride
  const int* idx;          // [B, na] or null (dense)
  const bf16_t* ring;      // [B, *, hd] window rows, batch stride ring_bstride
  const float* sink;       // [nh] or null
  void* out;               // [B, nh, hd]
  float* part_o;           // [B, ngrp, nh, hd]  partials of the row groups (ngrp > 1)
  float* part_ml;          // [B, ngrp, nh, 2]
  long long kv_bstride, ring_bstride;
  int B, nb, nh, hd, na, ring_len, ngrp, rows_per_group, normalize_q;
  float scale;
  long long ld_qb = 0;  // elements between batches of q (0: nh hd)
  // device-driven step: t1 = *n_seen + 1 tokens cached, nb = min(t1 / m, cap),
  // ring_len = min(t1, win), and without idx na = nb (dense)
  const int* n_seen = nullptr;
  int m = 1, win = 0, cap = 0;
};
hipError_t decode_attn_dispatch(const DecodeAttnParams& p, int qdtype, int odtype, hipStream_t s);

// Row-wise L2 normalisation: out[r] = x[r] / max(||x[r]||, 1e-12) (or a copy).
hipError_t l2norm_rows_dispatch(const void* x, long long ldx, void* out, int out_f32, int rows,
                                int c, int normalize, int dtype, hipStream_t s);

}  // namespace kch
