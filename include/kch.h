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
 */
#ifndef KCH_H
#define KCH_H

#ifdef __cplusplus
extern "C" {
#endif

#define KCH_ABI_VERSION 1

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
 * Per-token KDA recurrence (decode steps and short sequences).
 * Replaces naive_recurrent_kda (ops_kda.py:175-267) and the use_chunk=False
 * branch of kda_forward (ops_kda_backend.py:245-251). Same tensor layout as
 * kch_kda_chunk_fwd. Coverage: K in {16,32,64,128,256}; any V.
 */
int kch_kda_recurrent_fwd(const void* q, const void* k, const void* v, const void* g,
                          const void* beta, const float* s0, void* o, float* s_out,
                          int B, int T, int H, int HV, int K, int V, float scale,
                          float g_clamp_min, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KCH_H */
