/*
 * kch.h -- C ABI of the MI355X (gfx950) hybrid-attention forward path.
 *
 * One shared library (libkch.so) implements the forward hot path of the
 * reference repository 183600/kda-csa-hca-fusion with hand-written HIP
 * kernels. Every entry point here replaces one reference operator (cited as
 * file:line into that repository); the Python host package `kch` mirrors the
 * reference's call signatures on top of these functions.
 *
 * Conventions shared by all entry points
 *   - Pointers are device pointers to contiguous row-major tensors.
 *   - `dtype` names the storage type of the floating-point activations:
 *       0 = fp32, 1 = bf16, 2 = fp16.  Internal compute is fp32
 *       (matching the reference's compute dtype, ops_kda.py:125-127).
 *   - `stream` is a hipStream_t (cast to void*); work is enqueued
 *     asynchronously on it and nothing is allocated or freed.
 *   - Return value 0 = success; otherwise a KCH_ERR_* code, with a message
 *     available from kch_last_error() (per calling thread).
 *   - With KCH_SYNC set to a value other than "0" in the environment (read
 *     once, at the first call), every entry point waits for the device after
 *     its launches and returns an error raised while its kernels ran as its
 *     own KCH_ERR_HIP, naming itself. A debugging mode: the wait serialises
 *     the streams and must not be used under graph capture.
 */
#ifndef KCH_H
#define KCH_H

#ifdef __cplusplus
extern "C" {
#endif

#define KCH_ABI_VERSION 19

#define KCH_OK 0
#define KCH_ERR_INVALID 1     /* bad pointer / shape / argument */
#define KCH_ERR_UNSUPPORTED 2 /* shape or dtype outside the kernels' coverage */
#define KCH_ERR_HIP 3         /* HIP runtime error at launch */

#define KCH_DT_F32 0
#define KCH_DT_BF16 1
#define KCH_DT_F16 2

int kch_abi_version(void);
const char* kch_last_error(void);

/*
 * Chunkwise-parallel KDA forward (WY/UT transform, fp32 state).
 * Replaces naive_chunk_kda (ops_kda.py:464-494) and the use_chunk=True branch
 * of kda_forward (ops_kda_backend.py:237-244).
 *   q, k  [B,T,H,K]   v, o  [B,T,HV,V]   g [B,T,HV,K]   beta [B,T,HV]  (dtype)
 *   s0    [B,HV,K,V] fp32 initial state, or NULL for zeros
 *   s_out [B,HV,K,V] fp32 final state, or NULL
 *   g_clamp_min: lower clamp of g; -INFINITY disables it (ops_kda.py:392-393)
 * Coverage: K in {64,128}; V a multiple of 64; HV a multiple of H.
 * The result does not depend on a chunk size (the kernel's internal chunk is
 * 64 tokens for bf16/fp16 and 32 for fp32).
 */
int kch_kda_chunk_fwd(const void* q, const void* k, const void* v, const void* g,
                      const void* beta, const float* s0, void* o, float* s_out,
                      int B, int T, int H, int HV, int K, int V, float scale,
                      float g_clamp_min, int dtype, void* stream);

/*
 * Workspace bytes kch_kda_chunk_fwd_ws needs for these sizes, or 0 when the
 * sizes run without one (fp32 inputs, V = 192, 256, ...).
 */
size_t kch_kda_chunk_ws_bytes(int B, int T, int H, int HV, int K, int V, int dtype);

/*
 * kch_kda_chunk_fwd with a caller-provided device workspace (256-byte aligned,
 * at least kch_kda_chunk_ws_bytes bytes; ignored when that is 0). Replaces the
 * same reference function. For bf16 / fp16 inputs with K, V in {64, 128} the
 * state-independent part of every chunk runs fully parallel and writes its
 * operands to the workspace; a second kernel carries the state through the
 * chunks. Same arguments, coverage and results as kch_kda_chunk_fwd.
 */
int kch_kda_chunk_fwd_ws(const void* q, const void* k, const void* v, const void* g,
                         const void* beta, const float* s0, void* o, float* s_out,
                         int B, int T, int H, int HV, int K, int V, float scale,
                         float g_clamp_min, int dtype, void* ws, size_t ws_bytes,
                         void* stream);

/*
 * Per-token KDA recurrence (decode steps and short sequences).
 * Replaces naive_recurrent_kda (ops_kda.py:175-267) and the use_chunk=False
 * branch of kda_forward (ops_kda_backend.py:245-251). Same tensor layout as
 * kch_kda_chunk_fwd. Coverage: K in {16,32,64,128,256}; any V.
 */
int kch_kda_recurrent_fwd(const void* q, const void* k, const void* v, const void* g,
                          const void* beta, const float* s0, void* o, float* s_out,
                          int B, int T, int H, int HV, int K, int V, float scale,
                          float g_clamp_min, int dtype, void* stream);

/*
 * The same recurrence for float64 inputs: fp64 arithmetic and fp64 states
 * (s0, s_out [B, HV, K, V]), scale and gate clamp in fp64, as the reference
 * computes fp64 inputs (ops_kda.py:125-127, 175-267). naive_chunk_kda on
 * fp64 inputs is the same function (ops_kda.py:464-494) and runs here too.
 * Coverage: K in {16,32,64,128,256}; any V.
 */
int kch_kda_recurrent_fwd_f64(const double* q, const double* k, const double* v, const double* g,
                              const double* beta, const double* s0, double* o, double* s_out,
                              int B, int T, int H, int HV, int K, int V, double scale,
                              double g_clamp_min, void* stream);

/*
 * Gradients of the KDA recurrence: the backward of naive_recurrent_kda
 * (ops_kda.py:175-267), which the reference obtains from autograd and tests in
 * run_correctness.py:765-833 (finite differences) and :1032-1092 (chunk
 * gradients == recurrent gradients; naive_chunk_kda, ops_kda.py:464-494, is
 * the same function and has these gradients too).
 * Inputs: the forward's q, k [B,T,H,K], v [B,T,HV,V], g [B,T,HV,K],
 * beta [B,T,HV] (dtype KCH_DT_F32 / BF16 / F16, or KCH_DT_F64 = 3), s0
 * [B,HV,K,V] or NULL, d_o = dL/do [B,T,HV,V] (input dtype), ds_final =
 * dL/dS_T [B,HV,K,V] or NULL. States are fp32, fp64 for fp64 inputs.
 * Outputs: dq, dk, dv, dg, dbeta in the input dtype, laid out as their
 * inputs; ds0 = dL/dS0 or NULL. dg is zero where g < g_clamp_min (the clamp's
 * gradient). Arithmetic in fp32 (fp64 for fp64). ws: 256-byte aligned, at
 * least kch_kda_recurrent_bwd_ws_bytes bytes. Coverage: K in
 * {16,32,64,128,256}, any V, T >= 1.
 */
#define KCH_DT_F64 3
size_t kch_kda_recurrent_bwd_ws_bytes(int B, int T, int HV, int K, int V, int dtype);
int kch_kda_recurrent_bwd(const void* q, const void* k, const void* v, const void* g,
                          const void* beta, const void* s0, const void* d_o,
                          const void* ds_final, void* dq, void* dk, void* dv, void* dg,
                          void* dbeta, void* ds0, int B, int T, int H, int HV, int K, int V,
                          double scale, double g_clamp_min, int dtype, void* ws,
                          size_t ws_bytes, void* stream);

/*
 * Gradients of naive_chunk_kda (ops_kda.py:340-536, differentiated by the
 * reference's autograd through the chunk form, including its clamp(max=50) of
 * the in-chunk decay exponents) computed in the chunk form: four kernels
 * (per-chunk prepare, forward state pass, reverse state pass, per-chunk
 * gradients) on split-bf16 MFMA products in fp32. Same arguments and layouts
 * as kch_kda_recurrent_bwd; chunks of 64 tokens. Coverage: dtype KCH_DT_F32 /
 * BF16 / F16, K and V in {64, 128}, T >= 1 (other shapes and fp64 take
 * kch_kda_recurrent_bwd). Tensors 16-byte aligned; ws 256-byte aligned, at
 * least kch_kda_chunk_bwd_ws_bytes bytes.
 */
size_t kch_kda_chunk_bwd_ws_bytes(int B, int T, int H, int HV, int K, int V, int dtype);
int kch_kda_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                      const void* s0, const void* d_o, const void* ds_final, void* dq, void* dk,
                      void* dv, void* dg, void* dbeta, void* ds0, int B, int T, int H, int HV, int K,
                      int V, double scale, double g_clamp_min, int dtype, void* ws, size_t ws_bytes,
                      void* stream);


/*
 * Generic CSA / HCA forward: the inputs the MFMA kernels above do not take.
 * float64 (dtype KCH_DT_F64; the reference computes in fp64 for fp64 inputs,
 * ops_csa.py:229,263,510,922 and ops_hca.py:138) or float32 (KCH_DT_F32) for
 * head dims c or c_I above 128, more than 16 indexer heads, or an indexer
 * mask other than the standard block-causal one. Every sum in the dtype;
 * contiguous tensors.
 *
 * kch_gen_compress: csa_compress_kv (ops_csa.py:198-234; Cb = Zb = Bb = NULL)
 *   or csa_compress_kv_overlapped (ops_csa.py:237-305): Ca, Za (Cb, Zb)
 *   [B,T,c], Ba (Bb) [m,c] -> out [B,T/m,c].
 * kch_gen_l2norm: F.normalize(x, dim=-1) (eps 1e-12) of rows [rows,c] (a copy
 *   when normalize = 0).
 * kch_gen_indexer: csa_lightning_indexer (ops_csa.py:330-573): q [B,T,nIh,cI],
 *   k [B,nb,cI] (already L2-normalised when normalize_qk), w [B,T,nIh] or
 *   NULL, mask (uint8, element (b,t,n) at b*mask_bstride + t*mask_tstride + n;
 *   NULL: block n visible when n < (t+1)/causal_m, every block when causal_m
 *   is 0), logits [B,T,nb] or NULL, idx int64
 *   [B,T,topk]: descending logit, ties by ascending block index, -1 for
 *   infinite logits and past min(topk, nb). The sort runs in LDS: nb and
 *   nIh*cI are bounded by 64 KiB of it (KCH_ERR_UNSUPPORTED beyond).
 * kch_gen_attn: the joint softmax attention of naive_csa (idx given: the
 *   selected rows, row maximum clamped at 0 with a sink, ops_csa.py:1100-1155)
 *   or naive_hca (idx NULL, hca = 1: every block b < (t+1)/m, plain row
 *   maximum, ops_hca.py:166-186), plus the causal window of win rows of local
 *   [B,T,c] and the sink [nh] or NULL: q [B,T,nh,c] (L2-normalised inside
 *   when normalize_q), kv [B,nb,c] -> out [B,T,nh,c]. ws: at least
 *   kch_gen_attn_ws_bytes bytes (sparse = idx != NULL).
 */
int kch_gen_compress(const void* Ca, const void* Cb, const void* Za, const void* Zb, const void* Ba,
                     const void* Bb, void* out, int B, int T, int m, int c, int dtype, void* stream);
int kch_gen_l2norm(const void* x, void* y, long long rows, int c, int normalize, int dtype,
                   void* stream);
int kch_gen_indexer(const void* q, const void* k, const void* w, const void* mask,
                    long long mask_bstride, long long mask_tstride, void* logits, long long* idx,
                    int B, int T, int nb, int nIh, int cI, int topk, int causal_m, double scale,
                    int normalize_q, int dtype, void* stream);
size_t kch_gen_attn_ws_bytes(int B, int T, int nh, int nb, int topk, int win, int sparse, int dtype);
int kch_gen_attn(const void* q, const void* kv, const long long* idx, const void* local,
                 const void* sink, void* out, int B, int T, int nb, int nh, int c, int topk, int win,
                 int m, double scale, int normalize_q, int hca, int dtype, void* ws, size_t ws_bytes,
                 void* stream);

/*
 * Gradients of the HCA attention: the backward of hca_core (ops_hca.py:132-194,
 * which the reference differentiates with autograd; the gradient check of the
 * hybrid stack, run_correctness.py:2710-2830, runs through it). q, d_out and
 * dq [B,T,nh,c] are stored in qdt (KCH_DT_F32 / BF16 / F16; bf16 and fp16
 * need nh <= 16, the MFMA kernels' limit: the caller runs more heads as
 * groups), the queries as given (the kernel normalises them); the other
 * tensors are fp32: kc / raw
 * [B,T/m2,c] (the L2-normalised and the raw compressed rows of C, Z, B_pos,
 * from kch_compress), kl / lsrc [B,T,c] (the normalised window rows and the
 * rows they normalise; NULL when win = 0), C, Z [B,T,c], B_pos [m2,c], sink
 * [nh] or NULL. Outputs: dq [B,T,nh,c]; dC, dZ [B,T,c]; dBp [B,T/m2,m2,c]
 * (summed over the first two axes it is dB_pos); dlocal [B,T,c] (the window
 * rows' source gradient) or NULL to add it into dC; sink_part [B,T,nh]
 * (p_sink * D; dsink = -its sum over B and T) or NULL. Coverage: c in {64,
 * 128}, nh <= 16 (c = 128) or 32 (c = 64), T a multiple of m2, T >= 1. ws:
 * 256-byte aligned, kch_hca_attn_bwd_ws_bytes bytes.
 */
size_t kch_hca_attn_bwd_ws_bytes(int B, int T, int nh, int c, int m2, int win);
int kch_hca_attn_bwd(const void* q, const void* d_out, const float* kc, const float* raw,
                     const float* kl, const float* lsrc, const float* C, const float* Z,
                     const float* B_pos, const float* sink, void* dq, float* dC, float* dZ,
                     float* dBp, float* dlocal, float* sink_part, int B, int T, int nh, int c,
                     int m2, int win, float scale, int qdt, void* ws, size_t ws_bytes, void* stream);

/*
 * Gradients of the CSA attention: the backward of the sparse attention of
 * csa_core / naive_csa (ops_csa.py:869-1155, differentiated by autograd in the
 * reference; run_correctness.py:1312-1473, 2710-2830) with the selection held
 * fixed. Tensors as for kch_hca_attn_bwd, plus: idx [B,T,topk] int32 (the
 * selection, -1 = unused slot), the overlapped compression's inputs Ca, Cb,
 * Za, Zb [B,T,c], Ba, Bb [m,c] (kc / raw from kch_compress_overlapped; kl,
 * lsrc the window rows of Ca), normalize = 0 for normalize_qk=False (queries
 * and keys used as given; q, d_out, dq then fp32). Outputs: dq; dCa, dCb, dZa, dZb [B,T,c] (dCb, dZb
 * must be zeroed by the caller: the last block's second-branch rows receive
 * nothing); dBap, dBbp [B,T/m,m,c]; sink_part as for HCA; slot_grad
 * [B,T,topk] (zeroed by the caller): the gradient of each selected row dotted
 * with that row, which the STE surrogate (ops_csa.py:1033-1099) turns into
 * the indexer's gradient; gsum [B,T,c] or NULL: the sum over the selected
 * slots of the selected rows' gradients (written), which the full-softmax
 * surrogate's dense term (ops_csa.py:1050-1071) consumes. The window rows'
 * gradient is added into dCa.
 */
size_t kch_csa_attn_bwd_ws_bytes(int B, int T, int nh, int c, int m, int win, int topk);
int kch_csa_attn_bwd(const void* q, const void* d_out, const float* kc, const float* raw,
                     const float* kl, const float* lsrc, const int* idx, const float* Ca,
                     const float* Cb, const float* Za, const float* Zb, const float* Ba,
                     const float* Bb, const float* sink, void* dq, float* dCa, float* dCb,
                     float* dZa, float* dZb, float* dBap, float* dBbp, float* sink_part,
                     float* slot_grad, float* gsum, int B, int T, int nh, int c, int m, int topk,
                     int win, float scale, int normalize, int qdt, void* ws, size_t ws_bytes,
                     void* stream);

/*
 * The STE surrogate's backward for the CSA indexer (ops_csa.py:1033-1099,
 * ste_mode='topk_columns'; the soft weights of ops_csa.py:545-572 over the
 * logits of ops_csa.py:503-536): given dsel [B,T,nb] (each selected slot's
 * value from kch_csa_attn_bwd's slot_grad, scattered to its block, 0
 * elsewhere), the indexer queries q_idx [B,T,nIh,cI], head weights w_idx
 * [B,T,nIh], the compressed indexer keys kc / raw [B,nb,cI] (kch_compress of
 * K_idx, Z_idx, B_idx; kc normalised when normalize), writes dq_idx, dw_idx,
 * dK_idx, dZ_idx and the per-block dB_idx terms dBp [B,nb,m,cI]. fp32; cI in
 * {64, 128}, nIh in {1, 2, 4, 8}, nIh * cI <= 512.
 */
size_t kch_csa_ste_bwd_ws_bytes(int B, int T, int nIh, int cI, int m);
int kch_csa_ste_bwd(const float* q_idx, const float* w_idx, const float* kc, const float* raw,
                    const float* K_idx, const float* Z_idx, const float* B_idx, const float* dsel,
                    float* dq_idx, float* dw_idx, float* dK_idx, float* dZ_idx, float* dBp, int B,
                    int T, int m, int nIh, int cI, float scale, int normalize, void* ws,
                    size_t ws_bytes, void* stream);

/*
 * Backward of the KDA layer's front end and of the stack's LayerNorm (the
 * autograd backward of ops_fused.py:480-581 and :42-60, exercised by the
 * hybrid gradient test run_correctness.py:2710-2830).
 * kch_kda_gates_bwd: given the forward's proj / gl rows (as kch_kda_gates)
 *   and dq, dk [B,T,H,K], dv [B,T,HV,V], dg [B,T,HV,K], dbeta [B,T,HV],
 *   writes the q | k | v | beta columns of dproj (ld_proj apart; the caller
 *   zeroes the others) and dgl (ld_gl apart). K <= 256.
 * kch_short_conv_bwd: dx [B,T,d] of the causal 3-tap depthwise conv, and adds
 *   the taps' and the bias's gradients into fp32 dw [d,3] and db [d] (db may
 *   be NULL). dlookback [B,2,d] (dtype, or NULL): the gradient of the two
 *   lookback rows, for callers that keep the lookback attached to the
 *   previous chunk's graph (ops_fused.py:480-527 with detach_lookback=False).
 * kch_layer_norm_bwd: dx of the fp32 LayerNorm over the last dim (d <= 4096),
 *   and adds dw, db (fp32 [d]). dtype / wdtype: the input's and the weight's.
 */
int kch_kda_gates_bwd(const void* proj, long long ld_proj, const void* gl, long long ld_gl,
                      const void* dq, const void* dk, const void* dv, const void* dg,
                      const void* dbeta, void* dproj, void* dgl, int B, int T, int H, int HV, int K,
                      int V, float decay_scale, int dtype, void* stream);
int kch_short_conv_bwd(const void* x, const void* lookback, const void* weight, const void* dy,
                       void* dx, float* dw, float* db, void* dlookback, int B, int T, int d,
                       int dtype, void* stream);
int kch_layer_norm_bwd(const void* x, const void* w, const void* dy, void* dx, float* dw, float* db,
                       long long rows, int d, float eps, int dtype, int wdtype, void* stream);

/*
 * Single-branch softmax-gated KV compression, [B,T,c] -> [B,T/m,c].
 * Replaces csa_compress_kv (ops_csa.py:198-234); used for the CSA indexer keys
 * (ops_csa.py:874) and for HCA (ops_hca.py:134).
 *   C, Z   rows of c values, ld* elements apart (dtype); B_pos [m,c] fp32
 *   out_raw  [B,T/m,c] fp32 block values, or NULL
 *   out_key  [B,T/m,c] key rows, L2-normalised when `normalize`: bf16
 *            (key_f32 = 0), fp32 (1), split (2): [B,T/m,3,c] bf16, each
 *            row's high, middle then low parts of its fp32 value
 *            (x = hi + mid + lo, the operands of kch_csa_indexer_topk with
 *            key_split = 1), or (3, normalize only) [B,T/m,2,c] fp16, the
 *            high then low parts of 256 x (key_split = 2), or (4, normalize
 *            only, c a multiple of 32) those parts chunk-major
 *            (key_split = 3): per batch row ceil(T/m/16) chunks of 16 rows,
 *            each 2c/32 pieces of 64 lanes x 8 fp16, where channel ch of row r,
 *            part p (0 high, 1 low) is piece p c/32 + ch/32, lane r % 16 +
 *            16 ((ch % 32) / 8), element ch % 8 (the last chunk's rows past
 *            T/m are not written); or NULL
 *   local    [B,T,c] bf16 per-token window keys L2norm(C) (raw C when not
 *            `normalize`), or NULL
 * T must be a multiple of m (callers right-pad as ops_csa.py:772-777 does).
 */
int kch_compress(const void* C, long long ldC, const void* Z, long long ldZ, const float* B_pos,
                 float* out_raw, void* out_key, int key_f32, int normalize, void* local, int B,
                 int T, int m, int c, int dtype, void* stream);

/*
 * Two-branch overlapped compression: block i mixes Ca_i with Cb_{i-1}
 * (block 0: the b-branch has -inf logits and zero values).
 * Replaces csa_compress_kv_overlapped (ops_csa.py:237-305). Outputs as in
 * kch_compress; `local` is built from Ca (the CSA window keys,
 * ops_csa.py:1108-1116).
 */
int kch_compress_overlapped(const void* Ca, long long ldCa, const void* Cb, long long ldCb,
                            const void* Za, long long ldZa, const void* Zb, long long ldZb,
                            const float* Ba, const float* Bb, float* out_raw, void* out_key,
                            int key_f32, int normalize, void* local, int B, int T, int m, int c,
                            int dtype, void* stream);

/*
 * Lightning indexer + top-k. Replaces csa_lightning_indexer
 * (ops_csa.py:330-573) in its forward (hard top-k) form.
 *   q_idx [B,T,nIh,cI] (dtype), k_idx [B,nb,cI] fp32, or with key_split = 1
 *   [B,nb,3,cI] bf16 high / middle / low parts of each row (kch_compress
 *   key_f32 = 2), or with key_split = 2 (normalize_q only) [B,nb,2,cI] fp16
 *   high / low parts of 256 x (key_f32 = 3), or with key_split = 3
 *   (normalize_q only) those parts chunk-major (key_f32 = 4: each of the
 *   indexer's loads reads 1 KB of contiguous memory); the logits carry
 *   fp32-level error (three-part bf16 or two-part fp16 products);
 *   already L2-normalised when normalize_q. w_idx [B,T,nIh] (dtype) or NULL
 *   (= all ones)
 *   idx_out [B,T,topk] int64 (idx64) or int32: the top-k blocks by descending
 *   logit, ties by ascending index (sorted), or the same set in ascending
 *   block index (sorted = 0); -1 for masked blocks and padding
 *   logits_out [B,T,nb] fp32 (masked = -inf) or NULL
 * Block n is visible to query t when n < (pos0 + t + 1) / m, or always when
 * dense_visible (decode). nIh in {1,2,4,8,16}; cI in {32,64,128}.
 */
int kch_csa_indexer_topk(const void* q_idx, const void* k_idx, const void* w_idx, void* idx_out,
                         int idx64, float* logits_out, int B, int T, int nb, int nIh, int cI,
                         int topk, int m, int pos0, int dense_visible, int normalize_q, float scale,
                         int sorted, int key_split, int dtype, void* stream);

/*
 * CSA core attention over the selected compressed blocks plus the sliding
 * window, one joint softmax with an optional sink. Replaces the attention part
 * of naive_csa (ops_csa.py:959-1155).
 *   q [B,T,nh,hd] (qdtype; L2-normalised in-kernel when normalize_q)
 *   kv_comp [B,nb,hd] bf16 key/value rows, idx [B,T,topk] int32 (-1 = unused)
 *   kv_local [B,T,hd] bf16 window rows or NULL; sink [nh] fp32 or NULL
 *   out [B,T,nh,hd] (odtype)
 * nh <= 16; hd in {64,128}.
 */
int kch_csa_sparse_attn(const void* q, const void* kv_comp, const int* idx, const void* kv_local,
                        const float* sink, void* out, int B, int T, int nb, int nh, int hd,
                        int topk, int win, float scale, int normalize_q, int qdtype, int odtype,
                        void* stream);

/*
 * HCA core attention: dense MQA over the compressed blocks b < (t+1)/m plus
 * the window, one joint softmax with an optional sink. Replaces the attention
 * part of naive_hca (ops_hca.py:136-194). Arguments as kch_csa_sparse_attn.
 */
int kch_hca_attn(const void* q, const void* kv_comp, const void* kv_local, const float* sink,
                 void* out, int B, int T, int nb, int nh, int hd, int m, int win, float scale,
                 int normalize_q, int qdtype, int odtype, void* stream);

/*
 * Row-wise L2 normalisation x / max(||x||, 1e-12) (F.normalize, as used at
 * ops_csa.py:523-525,1110-1112 and ops_hca.py:135,154), or a plain copy when
 * !normalize. x rows are ldx elements apart; out is [rows,c] fp32 or bf16.
 */
int kch_l2norm_rows(const void* x, long long ldx, void* out, int out_f32, int rows, int c,
                    int normalize, int dtype, void* stream);

/*
 * One CSA decode step for the last appended token of each sequence:
 * lightning indexer over every cached block (all are complete, hence visible),
 * top-k, then one joint softmax over the selected blocks, the ring-buffer
 * window and the sink. Replaces CSADecodingCache.forward_step
 * (ops_decoding_cache.py:783-1070).
 *   q [B,nh,hd] (normalised in-kernel when normalize_q), q_idx [B,nIh,cI]
 *   (normalised in-kernel when normalize_qidx), w_idx [B,nIh] or NULL (qdtype)
 *   kv_comp [B,*,hd] bf16 key/value rows (batch stride kv_bstride elements)
 *   k_idx [B,*,cI] fp32 indexer keys (already L2-normalised when normalize_qidx)
 *   ring [B,*,hd] bf16: the first ring_len rows are the window (any order)
 *   idx_ws [B,topk] int32 workspace; out [B,nh,hd] (odtype)
 */
int kch_csa_decode_step(const void* q, const void* q_idx, const void* w_idx, const void* kv_comp,
                        long long kv_bstride, const float* k_idx, long long k_bstride,
                        const void* ring, long long ring_bstride, int ring_len, const float* sink,
                        void* out, int* idx_ws, int B, int nb, int nh, int hd, int nIh, int cI,
                        int topk, float scale, float idx_scale, int normalize_q,
                        int normalize_qidx, int qdtype, int odtype, void* stream);

/*
 * One HCA decode step: dense MQA over every cached compressed block plus the
 * ring-buffer window and the sink. Replaces HCADecodingCache.forward_step
 * (ops_decoding_cache.py:1268-1395). Arguments as kch_csa_decode_step.
 */
int kch_hca_decode_step(const void* q, const void* kv_comp, long long kv_bstride, const void* ring,
                        long long ring_bstride, int ring_len, const float* sink, void* out, int B,
                        int nb, int nh, int hd, float scale, int normalize_q, int qdtype, int odtype,
                        void* stream);

/*
 * Workspace bytes of one kch_csa_decode (sparse = 1) or kch_hca_decode
 * (sparse = 0) step for these sizes.
 */
size_t kch_decode_ws_bytes(int B, int nb, int nh, int hd, int topk, int ring_len, int sparse);

/*
 * One CSA decode step, split across the cache (CSADecodingCache.forward_step,
 * ops_decoding_cache.py:783-1070): lightning indexer + top-k over every cached
 * block (all are complete, hence visible), then one joint softmax over the
 * selected blocks, the ring window and the sink.
 *   q [B,nh,hd], q_idx [B,nIh,cI], w_idx [B,nIh] or NULL (qdtype); q_idx is
 *     L2-normalised in-kernel when normalize_qidx, q when normalize_q
 *   kv_comp [B,*,hd] bf16 attention rows (batch stride kv_bstride elements)
 *   k_rows [B,*,cI] indexer key rows as cached (kdtype), k_inv [B,*] fp32
 *     1/max(||row||, 1e-12) or NULL for 1 (batch strides k_bstride, kinv_bstride)
 *   ring [B,*,hd] bf16: the first ring_len rows are the window (any order)
 *   out [B,nh,hd] (odtype); idx_out [B,topk] int32 selected blocks or NULL
 *   ws: kch_decode_ws_bytes(B, nb, nh, hd, topk, ring_len, 1) bytes, 256-aligned
 * Ties at the top-k threshold are taken in ascending block index. Coverage as
 * kch_csa_decode_step; nb <= 16384 * 8192 / topk cached blocks.
 */
int kch_csa_decode(const void* q, const void* q_idx, const void* w_idx, const void* kv_comp,
                   long long kv_bstride, const void* k_rows, long long k_bstride,
                   const float* k_inv, long long kinv_bstride, const void* ring,
                   long long ring_bstride, int ring_len, const float* sink, void* out,
                   int* idx_out, int B, int nb, int nh, int hd, int nIh, int cI, int topk,
                   float scale, float idx_scale, int normalize_q, int normalize_qidx,
                   int qdtype, int kdtype, int odtype, void* ws, size_t ws_bytes, void* stream);

/*
 * One HCA decode step, split across the cache (HCADecodingCache.forward_step,
 * ops_decoding_cache.py:1268-1395): dense MQA over every cached compressed
 * block, the ring window and the sink. Arguments as kch_csa_decode; ws holds
 * kch_decode_ws_bytes(B, nb, nh, hd, 0, ring_len, 0) bytes.
 */
int kch_hca_decode(const void* q, const void* kv_comp, long long kv_bstride, const void* ring,
                   long long ring_bstride, int ring_len, const float* sink, void* out, int B,
                   int nb, int nh, int hd, float scale, int normalize_q, int qdtype, int odtype,
                   void* ws, size_t ws_bytes, void* stream);

/*
 * kch_csa_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). It has no counterpart in the reference.
 * The workspace kch_csa_decode takes lives instead in a file-scope device
 * array of KCH_NOALLOC_SCRATCH_BYTES (16 MiB), one copy per GPU, held from the
 * library's load until the process ends; its device address is looked up on
 * the first call on each device. Arguments, coverage and results are those of
 * kch_csa_decode. A call whose workspace (kch_decode_ws_bytes) exceeds
 * KCH_NOALLOC_SCRATCH_BYTES returns KCH_ERR_UNSUPPORTED. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race and must be serialised by the caller.
 */
#define KCH_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int kch_csa_decode_noalloc(const void* q, const void* q_idx, const void* w_idx,
                           const void* kv_comp, long long kv_bstride, const void* k_rows,
                           long long k_bstride, const float* k_inv, long long kinv_bstride,
                           const void* ring, long long ring_bstride, int ring_len,
                           const float* sink, void* out, int* idx_out, int B, int nb, int nh,
                           int hd, int nIh, int cI, int topk, float scale, float idx_scale,
                           int normalize_q, int normalize_qidx, int qdtype, int kdtype,
                           int odtype, void* stream);

/*
 * Causal depthwise convolution with kernel 3 of the KDA layer
 * (KDAHybridLayer.forward_functional, ops_fused.py:480-527: nn.Conv1d with
 * groups=d over [lookback ; x], or over [0 ; 0 ; x] without a lookback):
 *   out[b,t,c] = bias[c] + w[c,0] x[b,t-2,c] + w[c,1] x[b,t-1,c] + w[c,2] x[b,t,c]
 *   x, out [B,T,d]; lookback [B,2,d] or NULL (zeros) supplies x[b,-2], x[b,-1];
 *   weight [d,3] (the Conv1d weight [d,1,3]); bias [d] or NULL. All of dtype.
 * For d % 8 == 0, x / out / lookback must be 16-byte aligned.
 */
int kch_short_conv(const void* x, const void* lookback, const void* weight, const void* bias,
                   void* out, int B, int T, int d, int dtype, void* stream);

/*
 * KDA layer activations (ops_fused.py:559-581): from the projection rows
 *   proj[r] = [q (H*K) | k (H*K) | v (HV*V) | beta logits (HV) | ...] (ld_proj apart)
 *   gl[r]   = g_up(g_down(x_conv)) (HV*K, ld_gl apart),  r = b*T + t,
 * writes q, k = L2norm(silu(.)) per head [B,T,H,K]; v = silu(.) [B,T,HV,V];
 * g = -softplus(gl) * decay_scale [B,T,HV,K]; beta = sigmoid(.) [B,T,HV].
 * K <= 256.
 */
int kch_kda_gates(const void* proj, long long ld_proj, const void* gl, long long ld_gl, void* q,
                  void* k, void* v, void* g, void* beta, int B, int T, int H, int HV, int K, int V,
                  float decay_scale, int dtype, void* stream);

/*
 * LayerNorm computed in fp32 and returned in the input dtype (_Fp32LayerNorm,
 * ops_fused.py:42-60: F.layer_norm(x.float(), w.float(), b.float()).to(dtype)):
 *   out[r] = (x[r] - mean) / sqrt(var + eps) * w + b   (mean, biased var over d)
 * x, out [rows, d] contiguous, of dtype; w, b [d] of wdtype (b may be NULL).
 */
int kch_layer_norm(const void* x, const void* w, const void* b, void* out, int rows, int d,
                   float eps, int dtype, int wdtype, void* stream);

/*
 * Linear map of up to 16 rows, torch.nn.functional.linear without bias as the
 * layer projections of a decode step call it (ops_fused.py:571-581,609,713,739;
 * run_decoding.py:334-336,522,598,783,815):
 *   y[m, n] = sum_k x[m, k] * w[n, k]   (fp32 accumulation, result in dtype)
 * x [M, K] (row stride ldx), w [N, K] (row stride ldw), y [M, N] (row stride
 * ldy), all of dtype (1 bf16, 2 fp16). 1 <= M <= 16; K a multiple of 32; x and
 * w 16-byte aligned with ldx, ldw multiples of 8.
 */
int kch_linear_rows(const void* x, long long ldx, const void* w, long long ldw, void* y,
                    long long ldy, int M, int N, int K, int dtype, void* stream);

/*
 * The low-rank query up-projection of a prefill, torch.nn.functional.linear
 * without bias for many rows and a short K: q = W_UQ cQ of naive_hca
 * (ops_hca.py:140) and naive_csa's q / q_idx (ops_csa.py:923 and 877):
 *   y[m, n] = sum_k x[m, k] * w[n, k]   (fp32 accumulation, result in dtype)
 * x [M, K], w [N, K], y [M, N] with row strides ldx, ldw, ldy, all of dtype
 * (bf16 or fp16). K in {32, 64, 128, 256}; x and w 16-byte aligned with row
 * strides multiples of 8; when N % 8 == 0, y 16-byte aligned with ldy a
 * multiple of 8.
 */
int kch_linear_up(const void* x, long long ldx, const void* w, long long ldw, void* y,
                  long long ldy, long long M, int N, int K, int dtype, void* stream);

/* ---- Device-driven decode step ----------------------------------------
 * The entry points below make up one single-token decode step of
 * HybridDecoding (run_decoding.py:601-851) in which every count that changes
 * from step to step is derived on the GPU from n_seen, a device int holding
 * the number of tokens the caches held before the step: the step's launches
 * are then identical on every step and one captured graph replays it. The
 * caller keeps the caches' buffers at fixed addresses with room for `cap`
 * compressed blocks, and increments n_seen once at the end of each step
 * (kch_linear_rows_fused's counter, on the step's last launch).
 */

/*
 * kch_linear_rows with the pieces of a decode sub-layer around it
 * (HybridKCHAttention.forward, ops_fused.py:879-955: x + layer(norm(x))):
 *   ln_w != NULL: x rows are first replaced by LayerNorm(x) (_Fp32LayerNorm,
 *     ops_fused.py:42-60; fp32, rounded to dtype), ln_w / ln_b [K] of
 *     ln_wdtype (ln_b may be NULL), K <= 4096, M * K <= 32768;
 *   res != NULL: y = res + y, y rounded to dtype before the add (res [M, N],
 *     row stride ldr, of dtype; may be y itself);
 *   counter != NULL: *counter += 1 (one thread, after nothing else reads it).
 */
int kch_linear_rows_fused(const void* x, long long ldx, const void* w, long long ldw, void* y,
                          long long ldy, int M, int N, int K, const void* ln_w, const void* ln_b,
                          float ln_eps, int ln_wdtype, const void* res, long long ldr, int* counter,
                          int dtype, void* stream);

/*
 * The front of a KDA sub-layer for one token (KDAHybridLayer.forward_functional,
 * ops_fused.py:480-551, after the norm of HybridKCHAttention.forward): h =
 * LayerNorm(x) (as kch_layer_norm), out = causal depthwise conv3 over
 * [lookback ; h] (as kch_short_conv), then lookback <- [lookback[1] ; h] in
 * place. x [B, d] (row stride ldx), lookback [B, 2, d], conv_w [d, 3], conv_b
 * [d] or NULL, out [B, d] of dtype; ln_w, ln_b [d] of wdtype. d a multiple of
 * 8, at most 4096; operands 16-byte aligned.
 */
int kch_kda_decode_front(const void* x, long long ldx, const void* ln_w, const void* ln_b,
                         float eps, void* lookback, const void* conv_w, const void* conv_b,
                         void* out, int B, int d, int dtype, int wdtype, void* stream);

/*
 * The rest of a KDA sub-layer for one token, in one launch: the activations of
 * ops_fused.py:571-581 (as kch_kda_gates, with the g_up product inside) and the
 * recurrent update of naive_recurrent_kda (ops_kda.py:175-267, as
 * kch_kda_recurrent_fwd with T = 1). proj [B, ld_proj] rows hold q (H*K) |
 * k (H*K) | v (HV*V) | beta logits (HV) | g_down (K); g_up [HV*K, K] of dtype
 * (16-byte aligned); state [B, HV, K, V] fp32, updated in place; o [B, HV*V].
 * K in {16, 32, 64, 128, 256}, V a multiple of 32.
 */
int kch_kda_decode_step(const void* proj, long long ld_proj, const void* g_up, float* state,
                        void* o, int B, int H, int HV, int K, int V, float scale,
                        float decay_scale, float g_clamp_min, int dtype, void* stream);

/*
 * CSADecodingCache.append_step for one token (ops_decoding_cache.py:631-782).
 * proj [B, ld_proj] rows start with [Ca | Cb | Za | Zb | K_idx | Z_idx] (widths
 * c, c, c, c, cI, cI, dtype); acc [B, m, 4c + 2cI] the rows of the block being
 * filled; prev [B, m, 2c] the [Cb | Zb] rows of the last completed block; Ba,
 * Bb [m, c], B_idx [m, cI] fp32. Writes ring row (n_seen % win) of ring [B, win,
 * c] (the token's Ca, L2-normalised when normalize), accumulator slot n_seen %
 * m, and when the token completes block n_seen / m (< cap): its overlapped
 * compressed row into c_rows [B, cap, c] (dtype) and c_keys [B, cap, c] (bf16,
 * L2-normalised when normalize), its indexer key row into k_rows [B, cap, cI]
 * (dtype) with k_inv [B, cap] = 1 / max(||row||, 1e-12), and its [Cb | Zb] rows
 * into prev. c + cI <= 256.
 */
int kch_csa_cache_append(const void* proj, long long ld_proj, void* acc, void* prev,
                         const float* Ba, const float* Bb, const float* B_idx, void* ring,
                         void* c_rows, void* c_keys, void* k_rows, float* k_inv,
                         const int* n_seen, int B, int c, int cI, int m, int win, int cap,
                         int normalize, int dtype, void* stream);

/*
 * HCADecodingCache.append_step for one token (ops_decoding_cache.py:1200-1267):
 * proj rows start with [C | Z] (c each); acc [B, m2, 2c]; B_pos [m2, c] fp32;
 * ring, c_rows, c_keys as kch_csa_cache_append. c <= 256.
 */
int kch_hca_cache_append(const void* proj, long long ld_proj, void* acc, const float* B_pos,
                         void* ring, void* c_rows, void* c_keys, const int* n_seen, int B, int c,
                         int m2, int win, int cap, int normalize, int dtype, void* stream);

/*
 * The front of a KDA sub-layer and its input projection for one token, in one
 * launch: h = LayerNorm(x) (as kch_kda_decode_front: _Fp32LayerNorm rounded to
 * the dtype), then the causal depthwise convolution over [lookback ; h]
 * (KDAHybridLayer.forward_functional, ops_fused.py:480-551), then
 * y = conv W^T (the fused input projection, ops_fused.py:571-581), d = K.
 * The lookback [B, 2, d] is only read; h [B, d] is written to h_out, and
 * kch_kda_decode_step_shift of the same step advances the lookback from it.
 * bf16 / fp16, B <= 16, d a multiple of 32 (at most 4096, B d <= 32768),
 * operands 16-byte aligned; ln_w / ln_b of wdtype.
 */
int kch_kda_front_rows(const void* x, long long ldx, const void* ln_w, const void* ln_b,
                       float eps, int wdtype, const void* lookback, const void* conv_w,
                       const void* conv_b, void* h_out, const void* w, long long ldw, void* y,
                       long long ldy, int B, int N, int d, int dtype, void* stream);

/*
 * kch_kda_decode_step that also advances the conv lookback:
 * lookback [B, 2, d] <- [lookback[1] ; h] with h [B, d] from
 * kch_kda_front_rows (ops_fused.py:480-527, the lookback carried to the next
 * token), the channels split over the step's workgroups.
 */
int kch_kda_decode_step_shift(const void* proj, long long ld_proj, const void* g_up, float* state,
                              void* o, int B, int H, int HV, int K, int V, float scale,
                              float decay_scale, float g_clamp_min, void* lookback,
                              const void* h, int d, int dtype, void* stream);

/*
 * kch_csa_cache_append / kch_hca_cache_append and a row projection of the same
 * decode step, y[b, :] = x[b, :] W^T for the B rows (W [N, K], row strides
 * ldx, ldw, ldy in elements; kch_linear_rows_fused without norm, residual or
 * counter), in one launch: both read only the step's projection row, so their
 * workgroups run side by side. It serves the decode step's query
 * up-projection (the q of CSADecodingCache.forward_step /
 * HCADecodingCache.forward_step, ops_decoding_cache.py:783-1070, 1268-1395,
 * from W_UQ, ops_csa.py:876-878,923 and ops_hca.py:136-141) beside the append
 * (ops_decoding_cache.py:631-782, 1200-1267). Results are those of the two
 * separate calls. bf16 / fp16 only, B <= 16, K a multiple of 32, x and W rows
 * 16-byte aligned.
 */
int kch_csa_cache_append_rows(const void* proj, long long ld_proj, void* acc, void* prev,
                              const float* Ba, const float* Bb, const float* B_idx, void* ring,
                              void* c_rows, void* c_keys, void* k_rows, float* k_inv,
                              const int* n_seen, int B, int c, int cI, int m, int win, int cap,
                              int normalize, const void* x, long long ldx, const void* w,
                              long long ldw, void* y, long long ldy, int N, int K, int dtype,
                              void* stream);
int kch_hca_cache_append_rows(const void* proj, long long ld_proj, void* acc, const float* B_pos,
                              void* ring, void* c_rows, void* c_keys, const int* n_seen, int B,
                              int c, int m2, int win, int cap, int normalize, const void* x,
                              long long ldx, const void* w, long long ldw, void* y, long long ldy,
                              int N, int K, int dtype, void* stream);

/*
 * Workspace bytes of kch_csa_decode_dyn (sparse = 1) / kch_hca_decode_dyn for
 * caches of up to cap blocks and a window of win rows.
 */
size_t kch_decode_dyn_ws_bytes(int B, int cap, int nh, int hd, int topk, int win, int sparse);

/*
 * kch_csa_decode with the block count and window length taken from the device
 * counter: nb = min((*n_seen + 1) / m, cap), ring_len = min(*n_seen + 1, win)
 * (CSADecodingCache.forward_step, ops_decoding_cache.py:783-1070, after
 * kch_csa_cache_append of the same step). q, q_idx, w_idx rows are ld_q,
 * ld_qidx, ld_w elements apart per sequence; ring [B, win, hd] with batch
 * stride ring_bstride; idx_out [B, topk] receives the selection; ws holds
 * kch_decode_dyn_ws_bytes(B, cap, nh, hd, topk, win, 1) bytes, 256-byte
 * aligned. topk >= 1.
 */
int kch_csa_decode_dyn(const void* q, long long ld_q, const void* q_idx, long long ld_qidx,
                       const void* w_idx, long long ld_w, const void* kv_comp,
                       long long kv_bstride, const void* k_rows, long long k_bstride,
                       const float* k_inv, long long kinv_bstride, const void* ring,
                       long long ring_bstride, const int* n_seen, int m, int win, int cap,
                       const float* sink, void* out, int* idx_out, int B, int nh, int hd, int nIh,
                       int cI, int topk, float scale, float idx_scale, int normalize_q,
                       int normalize_qidx, int qdtype, int kdtype, int odtype, void* ws,
                       size_t ws_bytes, void* stream);

/*
 * kch_hca_decode with nb = min((*n_seen + 1) / m2, cap) and ring_len =
 * min(*n_seen + 1, win) from the device counter (HCADecodingCache.forward_step,
 * ops_decoding_cache.py:1268-1395); ws holds kch_decode_dyn_ws_bytes(B, cap,
 * nh, hd, 0, win, 0) bytes.
 */
int kch_hca_decode_dyn(const void* q, long long ld_q, const void* kv_comp, long long kv_bstride,
                       const void* ring, long long ring_bstride, const int* n_seen, int m2,
                       int win, int cap, const float* sink, void* out, int B, int nh, int hd,
                       float scale, int normalize_q, int qdtype, int odtype, void* ws,
                       size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KCH_H */
