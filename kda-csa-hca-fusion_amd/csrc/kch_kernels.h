// Internal launch interface between the C-ABI layer (abi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace kch {

// Contiguous row-major tensors; element types follow the dtype enum of the ABI.
//   q, k : [B, T, H, K]      v, o : [B, T, HV, V]
//   g    : [B, T, HV, K]     beta : [B, T, HV]
//   s0, s_out : [B, HV, K, V] fp32 (either may be null)
struct KdaParams {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* s0;
  void* o;
  float* s_out;
  int B, T, H, HV, K, V;
  float scale;
  float g_clamp_min;  // -inf disables the clamp
  // the fp64 recurrence (kda_recurrent_f64_dispatch): scale and clamp in fp64;
  // s0 and s_out then point to fp64 states
  double scale64 = 0.0;
  double g_clamp_min64 = 0.0;
};

// Gradients of the KDA recurrence (kda_backward.hip). States (s0, ds_final,
// ds0) are fp32, or fp64 for fp64 inputs; gradients are in the input dtype.
struct KdaBwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const void* s0;        // initial state or null
  const void* d_o;       // dL/do [B,T,HV,V]
  const void* ds_final;  // dL/dS_T [B,HV,K,V] or null
  void* dq;
  void* dk;
  void* dv;
  void* dg;
  void* dbeta;
  void* ds0;             // dL/dS0 or null
  void* ck = nullptr;    // workspace regions, set by kda_bwd_dispatch
  void* part = nullptr;
  int B, T, H, HV, K, V;
  double scale, g_clamp_min;  // -inf disables the clamp
};
size_t kda_bwd_ws_bytes(int B, int T, int HV, int K, int V, bool f64);
// K in {16, 32, 64, 128, 256}; dtype DT_F32 / DT_BF16 / DT_F16 / DT_F64; ws
// 256-byte aligned, kda_bwd_ws_bytes bytes
hipError_t kda_bwd_dispatch(KdaBwdParams p, int dtype, void* ws, hipStream_t stream);
// Sums the per-value-head partial records at p.part ([B,T,HV,(3K+1)] per
// slice of `cols` columns of V) into dq, dk, dg (clamp mask), dbeta.
hipError_t kda_bwd_reduce_launch(const KdaBwdParams& p, int cols, int dtype, hipStream_t stream);
// Chunked backward of naive_chunk_kda (kda_chunk_bwd.hip): bf16/fp16/fp32
// inputs, K and V in {64, 128}, chunks of 64; ws 256-byte aligned,
// kda_chunk_bwd_ws_bytes bytes.
bool kda_chunk_bwd_supported(int K, int V, int dtype);
size_t kda_chunk_bwd_ws_bytes(int B, int T, int H, int HV, int K, int V);
hipError_t kda_chunk_bwd_dispatch(KdaBwdParams p, int dtype, void* ws, hipStream_t stream);

// Gradients of the HCA attention (hca_backward.hip), fp32 tensors, c in
// {64, 128}, nh <= 256 / (c / 8), T a multiple of m2.
struct HcaBwdParams {
  const void* q;        // [B,T,nh,c] queries as given (not normalised), in qdt
  const void* dout;     // [B,T,nh,c], in qdt
  const float* kc;      // [B,nb,c] L2-normalised compressed rows
  const float* raw;     // [B,nb,c] compressed rows
  const float* kl;      // [B,T,c] L2-normalised window rows (win > 0)
  const float* lsrc;    // [B,T,c] rows the window keys normalise (win > 0)
  const float* C;       // [B,T,c] compression inputs
  const float* Z;
  const float* Bpos;    // [m2,c]
  const float* sink;    // [nh] or null
  void* dq;             // [B,T,nh,c], in qdt
  float* dC;            // [B,T,c]
  float* dZ;            // [B,T,c]
  float* dBp;           // [B,nb,m2,c] per-block terms of dB_pos
  float* dlocal;        // [B,T,c] gradient of the window rows' source, or null: added to dC
  float* sink_part;     // [B,T,nh] p_sink * D per query and head, or null
  int normalize = 1;    // 0: queries and keys are used as given (no L2 norms)
  int qdt = 0;          // storage of q, dout, dq: 0 fp32, 1 bf16, 2 fp16 (the SIMT path: fp32)
  // CSA: the selected blocks (idx [B,T,topk], -1 = unused) instead of every
  // causal block, its bitmap sel [B,T,ceil(nb/32)], the overlapped
  // compression's second branch, and the per-slot gradient of the selected
  // rows against themselves (slot_grad [B,T,topk], for the STE surrogate)
  const int* idx = nullptr;
  const uint32_t* sel = nullptr;
  int topk = 0;
  int sparse = 0;  // CSA: only the selected blocks (none when topk = 0)
  const float* Cb = nullptr;
  const float* Zb = nullptr;
  const float* Bb = nullptr;
  float* dCb = nullptr;
  float* dZb = nullptr;
  float* dBbp = nullptr;
  float* slot_grad = nullptr;
  // CSA, full-softmax STE: the sum over the selected slots of each selected
  // row's gradient, gsum [B,T,c] (written, the heads of this call summed)
  float* gsum = nullptr;
  float* lse = nullptr;  // workspace regions, set by hca_bwd_dispatch
  float* dval = nullptr;
  float* rq = nullptr;
  float* part_b = nullptr;
  float* part_w = nullptr;
  // MFMA path (attn_bwd_mfma.hip): the two-part bf16 splits of qn and dout
  // ([B,T,16,c], heads padded to 16) and of the compressed and window rows;
  // mfma_parts: part_b holds [B, nchunk, nb, c] per-chunk partials of the
  // compressed rows (chunk ci = queries [ci part_qc, (ci+1) part_qc), written
  // for the chunks a row's queries reach), part_w the window rows' [B, T, c]
  bf16_t* qs_hi = nullptr;
  bf16_t* qs_lo = nullptr;
  bf16_t* ds_hi = nullptr;
  bf16_t* ds_lo = nullptr;
  bf16_t* kc_hi = nullptr;
  bf16_t* kc_lo = nullptr;
  bf16_t* kl_hi = nullptr;
  bf16_t* kl_lo = nullptr;
  int mfma_parts = 0;
  int part_qc = 0;
  int B, T, nh, c, m2, nb, win;
  float scale;
};
// MFMA attention backward (normalised queries and keys, c in {64, 128}, nh <= 16)
bool attn_bwd_mfma_supported(const HcaBwdParams& p);
size_t attn_bwd_mfma_ws_bytes(int B, int T, int c, int m2, int win, int topk);
hipError_t attn_bwd_mfma_dispatch(HcaBwdParams p, void* ws, hipStream_t s);
size_t hca_bwd_ws_bytes(int B, int T, int nh, int c, int m2, int win, int topk);

// The STE surrogate's backward for the indexer (hca_backward.hip): fp32,
// cI in {64, 128}, nIh in {1, 2, 4, 8}, nIh * cI <= 512.
struct SteBwdParams {
  const float* qi;    // [B,T,nIh,cI] indexer queries as given
  const float* w;     // [B,T,nIh] head weights
  const float* kc;    // [B,nb,cI] compressed indexer keys (L2-normalised when normalize)
  const float* dsel;  // [B,T,nb] the slot gradients at the selected blocks, 0 elsewhere
  float* dqi;         // [B,T,nIh,cI]
  float* dw;          // [B,T,nIh]
  float* part = nullptr;  // workspace regions, set by ste_bwd_dispatch
  float* lse = nullptr;
  float* dval = nullptr;
  float* rq = nullptr;
  int B, T, nb, m, nIh, cI, normalize;
  float scale;
};
size_t ste_bwd_ws_bytes(int B, int T, int nIh, int cI, int m);
// bp: the key compression's inputs and outputs for the block kernel
hipError_t ste_bwd_dispatch(SteBwdParams p, HcaBwdParams bp, void* ws, hipStream_t stream);
hipError_t hca_bwd_dispatch(HcaBwdParams p, void* ws, hipStream_t stream);

hipError_t kda_chunk_dispatch(const KdaParams& p, int dtype, hipStream_t stream);
// fp64 inputs, state and arithmetic (kda_recurrent.hip)
hipError_t kda_recurrent_f64_dispatch(const KdaParams& p, hipStream_t stream);
// bf16 / fp16 inputs, K in {64, 128}, V a multiple of 64 (kda_chunk_lp.hip)
hipError_t kda_chunk_lp_dispatch(const KdaParams& p, int dtype, hipStream_t stream);
hipError_t kda_recurrent_dispatch(const KdaParams& p, int dtype, hipStream_t stream);
// Two-kernel chunk path (kda_split.hip): bf16 / fp16, K in {64,128}, V in {64,128};
// ws is 256-byte aligned and holds kda_split_ws_bytes bytes.
bool kda_split_supported(int K, int V, int dtype);
size_t kda_split_ws_bytes(int B, int T, int HV, int K, int V);
hipError_t kda_split_dispatch(const KdaParams& p, void* ws, int dtype, hipStream_t stream);

// Causal depthwise convolution, kernel 3 (kda_frontend.hip).
//   x, out : [B, T, d]   lookback : [B, 2, d] or null (zeros)
//   weight : [d, 3]      bias : [d] or null            (all of the dtype)
struct ShortConvParams {
  const void* x;
  const void* lookback;
  const void* weight;
  const void* bias;
  void* out;
  int B, T, d;
};
hipError_t short_conv_dispatch(const ShortConvParams& p, int dtype, hipStream_t stream);

// KDA activations (kda_frontend.hip). Row r = b*T + t of `proj` holds
// [q (H*K) | k (H*K) | v (HV*V) | beta logits (HV) | ...], ld_proj elements
// apart; row r of `gl` holds the HV*K gate pre-activations, ld_gl apart.
// Outputs are contiguous: q, k [B,T,H,K]; v [B,T,HV,V]; g [B,T,HV,K]; beta [B,T,HV].
struct KdaGatesParams {
  const void* proj;
  long long ld_proj;
  const void* gl;
  long long ld_gl;
  void* q;
  void* k;
  void* v;
  void* g;
  void* beta;
  int B, T, H, HV, K, V;
  float decay_scale;
};
hipError_t kda_gates_dispatch(const KdaGatesParams& p, int dtype, hipStream_t stream);

// Backward of the activations (frontend_backward.hip): dproj receives the
// q | k | v | beta columns (the caller zeroes the rest), dgl the gate's.
struct KdaGatesBwdParams {
  const void* proj;
  long long ld_proj;
  const void* gl;
  long long ld_gl;
  const void* dq;
  const void* dk;
  const void* dv;
  const void* dg;
  const void* dbeta;
  void* dproj;   // ld_proj apart, as proj
  void* dgl;     // ld_gl apart, as gl
  int B, T, H, HV, K, V;
  float decay_scale;
};
hipError_t kda_gates_bwd_dispatch(const KdaGatesBwdParams& p, int dtype, hipStream_t stream);

// Backward of the short convolution: dx [B,T,d]; dw [d,3] and db [d] fp32,
// accumulated (zeroed by the caller).
struct ShortConvBwdParams {
  const void* x;
  const void* lookback;
  const void* weight;
  const void* dy;
  void* dx;
  float* dw;
  float* db;
  void* dlookback;  // [B, 2, d] or null: gradient of the lookback rows x[-2], x[-1]
  int B, T, d;
};
hipError_t short_conv_bwd_dispatch(const ShortConvBwdParams& p, int dtype, hipStream_t stream);

// Backward of the fp32 LayerNorm: dx [rows,d]; dw, db [d] fp32, accumulated.
struct LayerNormBwdParams {
  const void* x;
  const void* w;
  const void* dy;
  void* dx;
  float* dw;
  float* db;
  long long rows;
  int d;
  float eps;
};
hipError_t layer_norm_bwd_dispatch(const LayerNormBwdParams& p, int dtype, int wdtype, hipStream_t stream);

// fp32 LayerNorm of rows of d elements (kda_frontend.hip).
struct LayerNormParams {
  const void* x;
  const void* w;
  const void* b;  // may be null
  void* out;
  int rows, d;
  float eps;
};
hipError_t layer_norm_dispatch(const LayerNormParams& p, int dtype, int wdtype, hipStream_t stream);

// y[M, N] = x[M, K] w[N, K]^T for M <= 16 rows (linear_rows.hip), optionally
//   x <- LayerNorm(x) first (ln_w non-null: the rows are normalised into LDS,
//        M * K <= kLinearLnMax),
//   y <- res + y (res non-null; y rounded to the dtype before the add, as a
//        separate residual add would see it),
//   and (*counter)++ by one thread (counter non-null).
// With the norm, conv_w non-null makes x the KDA layer's front for one token
// (KDAHybridLayer.forward_functional, ops_fused.py:480-551): h = LN(x) rounded
// to the dtype, then x <- bias + w0 look[0] + w1 look[1] + w2 h, the causal
// depthwise convolution over [lookback ; h]; tile 0 writes h to h_out (the
// lookback's next row), the lookback itself is only read.
constexpr int kLinearLnMax = 32768;
struct LinearRowsParams {
  const void* x = nullptr;
  const void* w = nullptr;
  void* y = nullptr;
  long long ldx = 0, ldw = 0, ldy = 0;  // row strides in elements
  int M = 0, N = 0, K = 0;
  const void* ln_w = nullptr;  // [K] of ln_wdtype
  const void* ln_b = nullptr;  // [K] of ln_wdtype or null
  float ln_eps = 0.f;
  int ln_wdtype = 0;
  const void* res = nullptr;   // [M, N], row stride ldr, of the dtype (may be y itself)
  long long ldr = 0;
  int* counter = nullptr;
  const void* conv_w = nullptr;  // [K, 3] of the dtype (with ln_w)
  const void* conv_b = nullptr;  // [K] of the dtype or null
  const void* look = nullptr;    // [M, 2, K] of the dtype
  void* h_out = nullptr;         // [M, K] of the dtype
};
hipError_t linear_rows_dispatch(const LinearRowsParams& p, int dtype, hipStream_t stream);

// Y[M, N] = X[M, K] W[N, K]^T for many rows and K in {32, 64, 128, 256}
// (rows_up.hip): the low-rank query up-projection of a prefill. x, w, y of
// one dtype, row strides ldx, ldw, ldy.
struct RowsProjParams {
  const void* x;
  const void* w;
  void* y;
  long long ldx, ldw, ldy;
  long long M;
  int N, K;
};
hipError_t rows_up_dispatch(const RowsProjParams& p, int dtype, hipStream_t stream);

// ---- device-driven decode step (decode_step.hip) ----
// n_seen: tokens the caches held before this step (device int); the step's
// token is number n_seen of its sequence.

// LayerNorm of x rows -> causal depthwise conv over [lookback ; h] ->
// lookback <- [lookback[1] ; h]. x [B, d] (row stride ldx); lookback [B, 2, d];
// conv_w [d, 3]; conv_b [d] or null; out [B, d]; all of dtype except ln_w /
// ln_b (wdtype). d a multiple of 8, at most 4096.
struct KdaFrontParams {
  const void* x;
  long long ldx;
  const void* ln_w;
  const void* ln_b;
  float eps;
  void* lookback;
  const void* conv_w;
  const void* conv_b;
  void* out;
  int B, d;
};
hipError_t kda_front_dispatch(const KdaFrontParams& p, int dtype, int wdtype, hipStream_t s);

// One token's KDA activations and recurrent update. proj [B, ld_proj] rows:
// q (H*K) | k (H*K) | v (HV*V) | beta logits (HV) | g_down (K); g_up [HV*K, K];
// state [B, HV, K, V] fp32 updated in place; o [B, HV*V]. K in {16, 32, 64,
// 128, 256}, V a multiple of 32.
struct KdaStepParams {
  const void* proj;
  long long ld_proj;
  const void* g_up;
  float* state;
  void* o;
  int B, H, HV, K, V;
  float scale, decay_scale, g_clamp_min;
  // non-null: the conv lookback [B, 2, d] advances, look <- [look[1] ; h_in]
  // (h_in [B, d]: the token's LayerNorm rows), each workgroup a slice of d
  void* look = nullptr;
  const void* h_in = nullptr;
  int d = 0;
};
hipError_t kda_step_dispatch(const KdaStepParams& p, int dtype, hipStream_t s);

// One token appended to a CSA (csa = 1) or HCA cache. proj [B, ld_proj] rows
// start with [Ca | Cb | Za | Zb | K_idx | Z_idx] (CSA: widths c x 4, cI x 2) or
// [C | Z] (HCA); acc [B, m, W] holds the rows of the block being filled
// (W = 4c + 2cI or 2c); prev [B, m, 2c] the [Cb | Zb] rows of the last
// completed CSA block. Written: ring row n_seen % win (L2-normalised when
// normalize), accumulator slot n_seen % m, and on a block's last token block
// n_seen / m of c_rows (dtype), c_keys (bf16, normalised when normalize),
// k_rows (dtype) and k_inv (fp32 1 / max(||row||, 1e-12)), then prev.
struct CacheStepParams {
  const void* proj;
  long long ld_proj;
  void* acc;
  void* prev;
  const float* Ba;   // [m, c] a-branch (HCA: B_pos)
  const float* Bb;   // [m, c] b-branch (CSA)
  const float* Bk;   // [m, cI] indexer keys (CSA)
  void* ring;        // [B, win, c] or null
  void* c_rows;      // [B, cap, c]
  void* c_keys;      // [B, cap, c] bf16
  void* k_rows;      // [B, cap, cI] (CSA)
  float* k_inv;      // [B, cap] (CSA)
  const int* n_seen;
  int B, c, cI, m, win, cap, normalize, csa;
};
hipError_t cache_step_dispatch(const CacheStepParams& p, int dtype, hipStream_t s);
// The append and a row projection (no norm, residual or counter; bf16 / fp16)
// in one launch (decode_step.hip).
hipError_t cache_step_rows_dispatch(const CacheStepParams& cp, const LinearRowsParams& lp, int dtype,
                                   hipStream_t s);


// Generic CSA / HCA forward (csa_hca_generic.hip): T = float or double
// (f64), any head dims, indexer heads and indexer mask.
struct GenCompressParams {
  const void* Ca;
  const void* Cb;  // null: single branch
  const void* Za;
  const void* Zb;
  const void* Ba;
  const void* Bb;
  void* out;       // [B, T/m, c]
  int B, T, m, c, overlapped;
};
struct GenIndexerParams {
  const void* q;     // [B,T,nIh,cI]
  const void* k;     // [B,nb,cI] (normalised by the caller when normalize_qk)
  const void* w;     // [B,T,nIh] or null (every head weighs 1)
  const void* mask;  // uint8, element (b, t, n) at b*mask_bstride + t*mask_tstride + n, or null
  long long mask_bstride, mask_tstride;
  void* logits;      // [B,T,nb] or null
  void* idx;         // int64 [B,T,topk]
  int B, T, nb, nIh, cI, topk, normalize_q, sortN;
  int causal_m;      // mask null: block n visible when n < (t+1)/causal_m (0: every block)
  double scale;
};
struct GenAttnParams {
  const void* q;      // [B,T,nh,c]
  const void* kv;     // [B,nb,c] key/value rows (normalised when the keys are)
  const void* idx;    // int64 [B,T,topk] (CSA) or null (HCA: every block b < (t+1)/m)
  const void* local;  // [B,T,c] window rows (win > 0)
  const void* sink;   // [nh] or null
  void* out;          // [B,T,nh,c]
  void* ws;           // [B,T,nh,K] scores and weights, K = (topk or nb) + win
  int B, T, nb, nh, c, topk, win, m, normalize_q, hca;
  double scale;
};
int gen_sort_n(int nb);
size_t gen_indexer_smem(int nIh, int cI, int nb, bool f64);
size_t gen_attn_smem(int nh, int c, int K, bool f64);
hipError_t gen_compress_launch(const GenCompressParams& p, bool f64, hipStream_t s);
hipError_t gen_l2norm_launch(const void* x, void* y, long long rows, int c, int normalize, bool f64,
                             hipStream_t s);
hipError_t gen_indexer_launch(GenIndexerParams p, bool f64, hipStream_t s);
hipError_t gen_attn_launch(const GenAttnParams& p, bool f64, hipStream_t s);

}  // namespace kch
