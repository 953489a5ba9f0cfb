// C-ABI entry points: argument validation, dispatch, error reporting.
// Declarations and the reference operator each one replaces: include/kch.h.

#include <cmath>
#include <cstdint>
#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <string>

#include "../../include/kch.h"
#include "kch_csa.h"
#include "kch_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

// KCH_SYNC (environment, read once): wait for the device after each entry
// point's launches, so that an execution error is reported by the entry point
// that caused it rather than by a later call.
bool sync_mode() {
  static const bool on = [] {
    const char* e = getenv("KCH_SYNC");
    return e && *e && !(e[0] == '0' && e[1] == 0);
  }();
  return on;
}

int hip_status(const char* fn, hipError_t e) {
  if (e == hipSuccess && sync_mode()) e = hipDeviceSynchronize();
  if (e != hipSuccess) return fail(KCH_ERR_HIP, "%s: HIP error %s", fn, hipGetErrorString(e));
  return KCH_OK;
}

bool dtype_ok(int d) { return d == KCH_DT_F32 || d == KCH_DT_BF16 || d == KCH_DT_F16; }

int check_kda_common(const char* fn, const void* q, const void* k, const void* v, const void* g,
                     const void* beta, void* o, int B, int T, int H, int HV, int K, int V,
                     int dtype) {
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || T < 0 || H < 1 || HV < 1 || K < 1 || V < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d H=%d HV=%d K=%d V=%d", fn, B, T, H, HV,
                K, V);
  if (HV % H) return fail(KCH_ERR_INVALID, "%s: HV=%d must be divisible by H=%d", fn, HV, H);
  return KCH_OK;
}

int check_kda_pointers(const char* fn, const void* q, const void* k, const void* v, const void* g,
                       const void* beta, void* o, int B, int T) {
  if (B * T > 0 && (!q || !k || !v || !g || !beta || !o))
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  return KCH_OK;
}

kch::KdaParams make_kda(const void* q, const void* k, const void* v, const void* g,
                        const void* beta, const float* s0, void* o, float* s_out, int B, int T,
                        int H, int HV, int K, int V, float scale, float g_clamp_min) {
  kch::KdaParams p;
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta;
  p.s0 = s0; p.o = o; p.s_out = s_out;
  p.B = B; p.T = T; p.H = H; p.HV = HV; p.K = K; p.V = V;
  p.scale = scale; p.g_clamp_min = g_clamp_min;
  return p;
}

}  // namespace

extern "C" {

int kch_abi_version(void) { return KCH_ABI_VERSION; }

const char* kch_last_error(void) { return g_last_error.c_str(); }

// Shared checks and the empty-input case of the chunk entry points; returns
// KCH_OK with *done set when nothing remains to launch.
static int chunk_prologue(const char* fn, const void* q, const void* k, const void* v,
                          const void* g, const void* beta, const float* s0, void* o,
                          float* s_out, int B, int T, int H, int HV, int K, int V,
                          float g_clamp_min, int dtype, void* stream, bool* done) {
  *done = false;
  int rc = check_kda_common(fn, q, k, v, g, beta, o, B, T, H, HV, K, V, dtype);
  if (rc) return rc;
  if (K != 64 && K != 128)
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not supported (64 or 128)", fn, K);
  if (V % 64) return fail(KCH_ERR_UNSUPPORTED, "%s: V=%d must be a multiple of 64", fn, V);
  if (std::isnan(g_clamp_min)) return fail(KCH_ERR_INVALID, "%s: g_clamp_min is NaN", fn);
  rc = check_kda_pointers(fn, q, k, v, g, beta, o, B, T);
  if (rc) return rc;
  if (B == 0 || T == 0) {
    // nothing to compute; the state passes through unchanged
    *done = true;
    if (s_out && B > 0) {
      // zeros by the fill kernel, not a memset node (graph-capture safe)
      const size_t n = (size_t)B * HV * K * V * sizeof(float);
      hipError_t e = s0 ? hipMemcpyAsync(s_out, s0, n, hipMemcpyDeviceToDevice, (hipStream_t)stream)
                        : kch::fill_u32(s_out, (long long)(n / 4), 0u, (hipStream_t)stream);
      return hip_status(fn, e);
    }
    return KCH_OK;
  }
  if ((long long)T * HV * (K > V ? K : V) >= (1LL << 31) || (long long)T * H * K >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: T * heads * head_dim must stay below 2^31", fn);
  if (dtype != KCH_DT_F32) {
    const uintptr_t any = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)g | (uintptr_t)o;
    if (any & 15)
      return fail(KCH_ERR_INVALID, "%s: q, k, v, g and o must be 16-byte aligned", fn);
  }
  return KCH_OK;
}

int kch_kda_chunk_fwd(const void* q, const void* k, const void* v, const void* g,
                      const void* beta, const float* s0, void* o, float* s_out, int B, int T,
                      int H, int HV, int K, int V, float scale, float g_clamp_min, int dtype,
                      void* stream) {
  const char* fn = "kch_kda_chunk_fwd";
  bool done;
  int rc = chunk_prologue(fn, q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, g_clamp_min,
                          dtype, stream, &done);
  if (rc || done) return rc;
  kch::KdaParams p = make_kda(q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, scale, g_clamp_min);
  return hip_status(fn, kch::kda_chunk_dispatch(p, dtype, (hipStream_t)stream));
}

size_t kch_kda_chunk_ws_bytes(int B, int T, int H, int HV, int K, int V, int dtype) {
  if (B <= 0 || T <= 0 || H < 1 || HV < 1 || HV % H || !kch::kda_split_supported(K, V, dtype))
    return 0;
  return kch::kda_split_ws_bytes(B, T, HV, K, V);
}

int kch_kda_chunk_fwd_ws(const void* q, const void* k, const void* v, const void* g,
                         const void* beta, const float* s0, void* o, float* s_out, int B, int T,
                         int H, int HV, int K, int V, float scale, float g_clamp_min, int dtype,
                         void* ws, size_t ws_bytes, void* stream) {
  const char* fn = "kch_kda_chunk_fwd_ws";
  bool done;
  int rc = chunk_prologue(fn, q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, g_clamp_min,
                          dtype, stream, &done);
  if (rc || done) return rc;
  kch::KdaParams p = make_kda(q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, scale, g_clamp_min);
  const size_t need = kch_kda_chunk_ws_bytes(B, T, H, HV, K, V, dtype);
  if (need == 0) return hip_status(fn, kch::kda_chunk_dispatch(p, dtype, (hipStream_t)stream));
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  return hip_status(fn, kch::kda_split_dispatch(p, ws, dtype, (hipStream_t)stream));
}

int kch_kda_recurrent_fwd(const void* q, const void* k, const void* v, const void* g,
                          const void* beta, const float* s0, void* o, float* s_out, int B, int T,
                          int H, int HV, int K, int V, float scale, float g_clamp_min, int dtype,
                          void* stream) {
  const char* fn = "kch_kda_recurrent_fwd";
  int rc = check_kda_common(fn, q, k, v, g, beta, o, B, T, H, HV, K, V, dtype);
  if (rc) return rc;
  if (K != 16 && K != 32 && K != 64 && K != 128 && K != 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not supported (16/32/64/128/256)", fn, K);
  if (std::isnan(g_clamp_min)) return fail(KCH_ERR_INVALID, "%s: g_clamp_min is NaN", fn);
  rc = check_kda_pointers(fn, q, k, v, g, beta, o, B, T);
  if (rc) return rc;
  if (B == 0) return KCH_OK;
  if (T == 0) {
    if (s_out) {
      // zeros by the fill kernel, not a memset node (graph-capture safe)
      const size_t n = (size_t)B * HV * K * V * sizeof(float);
      hipError_t e = s0 ? hipMemcpyAsync(s_out, s0, n, hipMemcpyDeviceToDevice, (hipStream_t)stream)
                        : kch::fill_u32(s_out, (long long)(n / 4), 0u, (hipStream_t)stream);
      return hip_status(fn, e);
    }
    return KCH_OK;
  }
  kch::KdaParams p = make_kda(q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, scale, g_clamp_min);
  return hip_status(fn, kch::kda_recurrent_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_kda_recurrent_fwd_f64(const double* q, const double* k, const double* v, const double* g,
                              const double* beta, const double* s0, double* o, double* s_out, int B,
                              int T, int H, int HV, int K, int V, double scale, double g_clamp_min,
                              void* stream) {
  const char* fn = "kch_kda_recurrent_fwd_f64";
  int rc = check_kda_common(fn, q, k, v, g, beta, o, B, T, H, HV, K, V, KCH_DT_F32);
  if (rc) return rc;
  if (K != 16 && K != 32 && K != 64 && K != 128 && K != 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not supported (16/32/64/128/256)", fn, K);
  if (std::isnan(g_clamp_min) || std::isnan(scale))
    return fail(KCH_ERR_INVALID, "%s: g_clamp_min or scale is NaN", fn);
  rc = check_kda_pointers(fn, q, k, v, g, beta, o, B, T);
  if (rc) return rc;
  if ((long long)T * HV * (K > V ? K : V) >= (1LL << 31) || (long long)T * H * K >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: T * heads * head_dim must stay below 2^31", fn);
  if (B == 0) return KCH_OK;
  if (T == 0) {
    if (s_out) {
      // zeros by the fill kernel, not a memset node (graph-capture safe)
      const size_t n = (size_t)B * HV * K * V * sizeof(double);
      hipError_t e = s0 ? hipMemcpyAsync(s_out, s0, n, hipMemcpyDeviceToDevice, (hipStream_t)stream)
                        : kch::fill_u32(s_out, (long long)(n / 4), 0u, (hipStream_t)stream);
      return hip_status(fn, e);
    }
    return KCH_OK;
  }
  kch::KdaParams p = make_kda(q, k, v, g, beta, reinterpret_cast<const float*>(s0), o,
                              reinterpret_cast<float*>(s_out), B, T, H, HV, K, V, (float)scale,
                              (float)g_clamp_min);
  p.scale64 = scale;
  p.g_clamp_min64 = g_clamp_min;
  return hip_status(fn, kch::kda_recurrent_f64_dispatch(p, (hipStream_t)stream));
}

size_t kch_kda_recurrent_bwd_ws_bytes(int B, int T, int HV, int K, int V, int dtype) {
  if (B <= 0 || T <= 0 || HV < 1 || V < 1 || (K != 16 && K != 32 && K != 64 && K != 128 && K != 256))
    return 0;
  if (!dtype_ok(dtype) && dtype != KCH_DT_F64) return 0;
  return kch::kda_bwd_ws_bytes(B, T, HV, K, V, dtype == KCH_DT_F64);
}

int kch_kda_recurrent_bwd(const void* q, const void* k, const void* v, const void* g,
                          const void* beta, const void* s0, const void* d_o,
                          const void* ds_final, void* dq, void* dk, void* dv, void* dg,
                          void* dbeta, void* ds0, int B, int T, int H, int HV, int K, int V,
                          double scale, double g_clamp_min, int dtype, void* ws,
                          size_t ws_bytes, void* stream) {
  const char* fn = "kch_kda_recurrent_bwd";
  if (!dtype_ok(dtype) && dtype != KCH_DT_F64)
    return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || T < 1 || H < 1 || HV < 1 || K < 1 || V < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d H=%d HV=%d K=%d V=%d (T >= 1)", fn, B, T,
                H, HV, K, V);
  if (HV % H) return fail(KCH_ERR_INVALID, "%s: HV=%d must be divisible by H=%d", fn, HV, H);
  if (K != 16 && K != 32 && K != 64 && K != 128 && K != 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not supported (16/32/64/128/256)", fn, K);
  if (std::isnan(g_clamp_min) || std::isnan(scale))
    return fail(KCH_ERR_INVALID, "%s: g_clamp_min or scale is NaN", fn);
  if ((long long)T * HV * (K > V ? K : V) >= (1LL << 31) || (long long)T * H * K >= (1LL << 31) ||
      (long long)B * T * HV * ((V + 31) / 32) * (3 * K + 1) >= (1LL << 40))
    return fail(KCH_ERR_UNSUPPORTED, "%s: T * heads * head_dim must stay below 2^31", fn);
  if (B == 0) return KCH_OK;
  if (!q || !k || !v || !g || !beta || !d_o || !dq || !dk || !dv || !dg || !dbeta)
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  const size_t need = kch_kda_recurrent_bwd_ws_bytes(B, T, HV, K, V, dtype);
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  kch::KdaBwdParams p;
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta; p.s0 = s0;
  p.d_o = d_o; p.ds_final = ds_final;
  p.dq = dq; p.dk = dk; p.dv = dv; p.dg = dg; p.dbeta = dbeta; p.ds0 = ds0;
  p.B = B; p.T = T; p.H = H; p.HV = HV; p.K = K; p.V = V;
  p.scale = scale;
  p.g_clamp_min = g_clamp_min;
  return hip_status(fn, kch::kda_bwd_dispatch(p, dtype, ws, (hipStream_t)stream));
}

size_t kch_kda_chunk_bwd_ws_bytes(int B, int T, int H, int HV, int K, int V, int dtype) {
  if (B <= 0 || T <= 0 || H < 1 || HV < 1 || HV % H || !dtype_ok(dtype)) return 0;
  if (!kch::kda_chunk_bwd_supported(K, V, dtype)) return 0;
  return kch::kda_chunk_bwd_ws_bytes(B, T, H, HV, K, V);
}

int kch_kda_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                      const void* s0, const void* d_o, const void* ds_final, void* dq, void* dk,
                      void* dv, void* dg, void* dbeta, void* ds0, int B, int T, int H, int HV, int K,
                      int V, double scale, double g_clamp_min, int dtype, void* ws, size_t ws_bytes,
                      void* stream) {
  const char* fn = "kch_kda_chunk_bwd";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d not supported (fp32/bf16/fp16)", fn, dtype);
  if (B < 0 || T < 1 || H < 1 || HV < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d H=%d HV=%d (T >= 1)", fn, B, T, H, HV);
  if (HV % H) return fail(KCH_ERR_INVALID, "%s: HV=%d must be divisible by H=%d", fn, HV, H);
  if (!kch::kda_chunk_bwd_supported(K, V, dtype))
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d V=%d not supported (64 or 128 each)", fn, K, V);
  if (std::isnan(g_clamp_min) || std::isnan(scale))
    return fail(KCH_ERR_INVALID, "%s: g_clamp_min or scale is NaN", fn);
  if ((long long)B * T * HV * (3 * K + 1) >= (1LL << 40) || (long long)T * HV * K >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: tensors too large", fn);
  if (B == 0) return KCH_OK;
  if (!q || !k || !v || !g || !beta || !d_o || !dq || !dk || !dv || !dg || !dbeta)
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  const void* ptrs[] = {q, k, v, g, beta, s0, d_o, ds_final, dq, dk, dv, dg, dbeta, ds0};
  for (const void* ptr : ptrs)
    if ((uintptr_t)ptr & 15) return fail(KCH_ERR_INVALID, "%s: tensors must be 16-byte aligned", fn);
  const size_t need = kch_kda_chunk_bwd_ws_bytes(B, T, H, HV, K, V, dtype);
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  kch::KdaBwdParams p;
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta; p.s0 = s0;
  p.d_o = d_o; p.ds_final = ds_final;
  p.dq = dq; p.dk = dk; p.dv = dv; p.dg = dg; p.dbeta = dbeta; p.ds0 = ds0;
  p.B = B; p.T = T; p.H = H; p.HV = HV; p.K = K; p.V = V;
  p.scale = scale;
  p.g_clamp_min = g_clamp_min;
  return hip_status(fn, kch::kda_chunk_bwd_dispatch(p, dtype, ws, (hipStream_t)stream));
}

static bool gen_dtype_ok(int d) { return d == KCH_DT_F32 || d == KCH_DT_F64; }
static const size_t kGenSmemMax = 65536;

int kch_gen_compress(const void* Ca, const void* Cb, const void* Za, const void* Zb, const void* Ba,
                     const void* Bb, void* out, int B, int T, int m, int c, int dtype, void* stream) {
  const char* fn = "kch_gen_compress";
  if (!gen_dtype_ok(dtype)) return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (fp32 or fp64)", fn, dtype);
  if (B < 0 || T < 0 || m < 1 || c < 1 || T % m)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d m=%d c=%d (T a multiple of m)", fn, B, T, m, c);
  const bool two = Cb || Zb || Bb;
  if (two && !(Cb && Zb && Bb)) return fail(KCH_ERR_INVALID, "%s: Cb, Zb, Bb go together", fn);
  if ((long long)B * T * c >= (1LL << 40)) return fail(KCH_ERR_UNSUPPORTED, "%s: tensors too large", fn);
  if (B == 0 || T == 0) return KCH_OK;
  if (!Ca || !Za || !Ba || !out) return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  kch::GenCompressParams p;
  p.Ca = Ca; p.Cb = Cb; p.Za = Za; p.Zb = Zb; p.Ba = Ba; p.Bb = Bb; p.out = out;
  p.B = B; p.T = T; p.m = m; p.c = c; p.overlapped = two ? 1 : 0;
  return hip_status(fn, kch::gen_compress_launch(p, dtype == KCH_DT_F64, (hipStream_t)stream));
}

int kch_gen_l2norm(const void* x, void* y, long long rows, int c, int normalize, int dtype,
                   void* stream) {
  const char* fn = "kch_gen_l2norm";
  if (!gen_dtype_ok(dtype)) return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (fp32 or fp64)", fn, dtype);
  if (rows < 0 || c < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes rows=%lld c=%d", fn, rows, c);
  if (rows == 0) return KCH_OK;
  if (!x || !y) return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(fn, kch::gen_l2norm_launch(x, y, rows, c, normalize, dtype == KCH_DT_F64,
                                               (hipStream_t)stream));
}

int kch_gen_indexer(const void* q, const void* k, const void* w, const void* mask,
                    long long mask_bstride, long long mask_tstride, void* logits, long long* idx,
                    int B, int T, int nb, int nIh, int cI, int topk, int causal_m, double scale,
                    int normalize_q, int dtype, void* stream) {
  const char* fn = "kch_gen_indexer";
  if (!gen_dtype_ok(dtype)) return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (fp32 or fp64)", fn, dtype);
  if (B < 0 || T < 0 || nb < 0 || nIh < 1 || cI < 1 || topk < 0 || causal_m < 0)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d nb=%d nIh=%d cI=%d topk=%d m=%d", fn, B, T,
                nb, nIh, cI, topk, causal_m);
  if (std::isnan(scale)) return fail(KCH_ERR_INVALID, "%s: scale is NaN", fn);
  if (nb > (1 << 20)) return fail(KCH_ERR_UNSUPPORTED, "%s: nb=%d too large", fn, nb);
  const size_t smem = kch::gen_indexer_smem(nIh, cI, nb, dtype == KCH_DT_F64);
  if (smem > kGenSmemMax)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nIh*cI=%d and n_blocks=%d need %zu bytes of LDS (max %zu)",
                fn, nIh * cI, nb, smem, kGenSmemMax);
  if (B == 0 || T == 0 || (topk == 0 && !logits)) return KCH_OK;
  if (!q || (!k && nb) || (!idx && topk)) return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  kch::GenIndexerParams p;
  p.q = q; p.k = k; p.w = w; p.mask = mask; p.mask_bstride = mask_bstride;
  p.mask_tstride = mask_tstride; p.logits = logits; p.idx = idx;
  p.B = B; p.T = T; p.nb = nb; p.nIh = nIh; p.cI = cI; p.topk = topk;
  p.normalize_q = normalize_q; p.sortN = 0; p.causal_m = causal_m; p.scale = scale;
  return hip_status(fn, kch::gen_indexer_launch(p, dtype == KCH_DT_F64, (hipStream_t)stream));
}

size_t kch_gen_attn_ws_bytes(int B, int T, int nh, int nb, int topk, int win, int sparse, int dtype) {
  if (B < 0 || T < 0 || nh < 1 || nb < 0 || topk < 0 || win < 0 || !gen_dtype_ok(dtype)) return 0;
  const size_t K = (size_t)(sparse ? topk : nb) + win;
  return (size_t)B * T * nh * K * (dtype == KCH_DT_F64 ? 8 : 4) + 256;
}

int kch_gen_attn(const void* q, const void* kv, const long long* idx, const void* local,
                 const void* sink, void* out, int B, int T, int nb, int nh, int c, int topk, int win,
                 int m, double scale, int normalize_q, int hca, int dtype, void* ws, size_t ws_bytes,
                 void* stream) {
  const char* fn = "kch_gen_attn";
  if (!gen_dtype_ok(dtype)) return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (fp32 or fp64)", fn, dtype);
  if (B < 0 || T < 0 || nb < 0 || nh < 1 || c < 1 || topk < 0 || win < 0 || m < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d nb=%d nh=%d c=%d topk=%d win=%d m=%d", fn,
                B, T, nb, nh, c, topk, win, m);
  if (std::isnan(scale)) return fail(KCH_ERR_INVALID, "%s: scale is NaN", fn);
  const int K = (idx ? topk : nb) + win;
  const size_t smem = kch::gen_attn_smem(nh, c, K, dtype == KCH_DT_F64);
  if (smem > kGenSmemMax)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nh*c=%d with %d candidates needs %zu bytes of LDS (max %zu)",
                fn, nh * c, K, smem, kGenSmemMax);
  if (B == 0 || T == 0) return KCH_OK;
  if (!q || !out || (!kv && nb) || (win > 0 && !local))
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  const size_t need = kch_gen_attn_ws_bytes(B, T, nh, nb, topk, win, idx != nullptr, dtype);
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  kch::GenAttnParams p;
  p.q = q; p.kv = kv; p.idx = idx; p.local = local; p.sink = sink; p.out = out; p.ws = ws;
  p.B = B; p.T = T; p.nb = nb; p.nh = nh; p.c = c; p.topk = topk; p.win = win; p.m = m;
  p.normalize_q = normalize_q; p.hca = hca; p.scale = scale;
  return hip_status(fn, kch::gen_attn_launch(p, dtype == KCH_DT_F64, (hipStream_t)stream));
}

size_t kch_hca_attn_bwd_ws_bytes(int B, int T, int nh, int c, int m2, int win) {
  if (B <= 0 || T <= 0 || nh < 1 || (c != 64 && c != 128) || m2 < 1 || T % m2 || win < 0) return 0;
  return kch::hca_bwd_ws_bytes(B, T, nh, c, m2, win, 0);
}

int kch_hca_attn_bwd(const void* q, const void* d_out, const float* kc, const float* raw,
                     const float* kl, const float* lsrc, const float* C, const float* Z,
                     const float* B_pos, const float* sink, void* dq, float* dC, float* dZ,
                     float* dBp, float* dlocal, float* sink_part, int B, int T, int nh, int c,
                     int m2, int win, float scale, int qdt, void* ws, size_t ws_bytes, void* stream) {
  const char* fn = "kch_hca_attn_bwd";
  if (qdt < 0 || qdt > 2) return fail(KCH_ERR_INVALID, "%s: dtype %d (0 fp32, 1 bf16, 2 fp16)", fn, qdt);
  if (qdt != 0 && nh > 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: bf16 / fp16 q and d_out take at most 16 heads a call (nh=%d)",
                fn, nh);
  if (B < 0 || T < 1 || nh < 1 || m2 < 1 || win < 0)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d nh=%d m2=%d win=%d (T >= 1)", fn, B, T, nh,
                m2, win);
  if (T % m2) return fail(KCH_ERR_INVALID, "%s: T=%d must be a multiple of m2=%d", fn, T, m2);
  if (c != 64 && c != 128) return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d not supported (64 or 128)", fn, c);
  if ((long long)T * c * 4 >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: T=%d rows of a batch row exceed 2 GiB (32-bit row offsets)", fn, T);
  if (nh * (c / 8) > 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nh=%d heads of %d exceed one workgroup", fn, nh, c);
  if (std::isnan(scale)) return fail(KCH_ERR_INVALID, "%s: scale is NaN", fn);
  if ((long long)B * T * nh * c >= (1LL << 40))
    return fail(KCH_ERR_UNSUPPORTED, "%s: tensors too large", fn);
  if (B == 0) return KCH_OK;
  if (!q || !d_out || !kc || !raw || !C || !Z || !B_pos || !dq || !dC || !dZ || !dBp)
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  if (win > 0 && (!kl || !lsrc)) return fail(KCH_ERR_INVALID, "%s: window rows required (win > 0)", fn);
  const size_t need = kch_hca_attn_bwd_ws_bytes(B, T, nh, c, m2, win);
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  for (const void* ptr : {(const void*)q, (const void*)d_out, (const void*)kc, (const void*)kl,
                          (const void*)dq})
    if ((uintptr_t)ptr & 15) return fail(KCH_ERR_INVALID, "%s: q, d_out, kc, kl, dq must be 16-byte aligned", fn);
  kch::HcaBwdParams p;
  p.q = q; p.dout = d_out; p.kc = kc; p.raw = raw; p.kl = kl; p.lsrc = lsrc;
  p.C = C; p.Z = Z; p.Bpos = B_pos; p.sink = sink;
  p.dq = dq; p.dC = dC; p.dZ = dZ; p.dBp = dBp; p.dlocal = dlocal; p.sink_part = sink_part;
  p.qdt = qdt;
  p.B = B; p.T = T; p.nh = nh; p.c = c; p.m2 = m2; p.nb = T / m2; p.win = win;
  p.scale = scale;
  return hip_status(fn, kch::hca_bwd_dispatch(p, ws, (hipStream_t)stream));
}

size_t kch_csa_attn_bwd_ws_bytes(int B, int T, int nh, int c, int m, int win, int topk) {
  if (B <= 0 || T <= 0 || nh < 1 || (c != 64 && c != 128) || m < 1 || T % m || win < 0 || topk < 0)
    return 0;
  return kch::hca_bwd_ws_bytes(B, T, nh, c, m, win, topk);
}

int kch_csa_attn_bwd(const void* q, const void* d_out, const float* kc, const float* raw,
                     const float* kl, const float* lsrc, const int* idx, const float* Ca,
                     const float* Cb, const float* Za, const float* Zb, const float* Ba,
                     const float* Bb, const float* sink, void* dq, float* dCa, float* dCb,
                     float* dZa, float* dZb, float* dBap, float* dBbp, float* sink_part,
                     float* slot_grad, float* gsum, int B, int T, int nh, int c, int m, int topk,
                     int win, float scale, int normalize, int qdt, void* ws, size_t ws_bytes,
                     void* stream) {
  const char* fn = "kch_csa_attn_bwd";
  if (qdt < 0 || qdt > 2) return fail(KCH_ERR_INVALID, "%s: dtype %d (0 fp32, 1 bf16, 2 fp16)", fn, qdt);
  if (qdt != 0 && (nh > 16 || !normalize))
    return fail(KCH_ERR_UNSUPPORTED,
                "%s: bf16 / fp16 q and d_out need normalize=1 and at most 16 heads a call (nh=%d)", fn,
                nh);
  if (B < 0 || T < 1 || nh < 1 || m < 1 || win < 0 || topk < 0)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d nh=%d m=%d win=%d topk=%d (T >= 1)", fn, B,
                T, nh, m, win, topk);
  if (T % m) return fail(KCH_ERR_INVALID, "%s: T=%d must be a multiple of m=%d", fn, T, m);
  if (c != 64 && c != 128) return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d not supported (64 or 128)", fn, c);
  if ((long long)T * c * 4 >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: T=%d rows of a batch row exceed 2 GiB (32-bit row offsets)", fn, T);
  if (nh * (c / 8) > 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nh=%d heads of %d exceed one workgroup", fn, nh, c);
  if (std::isnan(scale)) return fail(KCH_ERR_INVALID, "%s: scale is NaN", fn);
  if ((long long)B * T * nh * c >= (1LL << 40) || (long long)B * T * topk >= (1LL << 40))
    return fail(KCH_ERR_UNSUPPORTED, "%s: tensors too large", fn);
  if (B == 0) return KCH_OK;
  if (!q || !d_out || !kc || !raw || !Ca || !Cb || !Za || !Zb || !Ba || !Bb || !dq || !dCa || !dCb ||
      !dZa || !dZb || !dBap || !dBbp || (topk > 0 && !idx))
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  if (win > 0 && (!kl || !lsrc)) return fail(KCH_ERR_INVALID, "%s: window rows required (win > 0)", fn);
  const size_t need = kch_csa_attn_bwd_ws_bytes(B, T, nh, c, m, win, topk);
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  for (const void* ptr : {(const void*)q, (const void*)d_out, (const void*)kc, (const void*)kl,
                          (const void*)dq})
    if ((uintptr_t)ptr & 15) return fail(KCH_ERR_INVALID, "%s: q, d_out, kc, kl, dq must be 16-byte aligned", fn);
  kch::HcaBwdParams p;
  p.q = q; p.dout = d_out; p.kc = kc; p.raw = raw; p.kl = kl; p.lsrc = lsrc;
  p.C = Ca; p.Z = Za; p.Bpos = Ba; p.sink = sink;
  p.Cb = Cb; p.Zb = Zb; p.Bb = Bb;
  p.dq = dq; p.dC = dCa; p.dZ = dZa; p.dBp = dBap; p.dlocal = nullptr; p.sink_part = sink_part;
  p.dCb = dCb; p.dZb = dZb; p.dBbp = dBbp;
  p.idx = topk > 0 ? idx : nullptr;
  p.topk = topk;
  p.sparse = 1;
  p.slot_grad = topk > 0 ? slot_grad : nullptr;
  p.gsum = gsum;
  p.normalize = normalize ? 1 : 0;
  p.qdt = qdt;
  p.B = B; p.T = T; p.nh = nh; p.c = c; p.m2 = m; p.nb = T / m; p.win = win;
  p.scale = scale;
  return hip_status(fn, kch::hca_bwd_dispatch(p, ws, (hipStream_t)stream));
}

size_t kch_csa_ste_bwd_ws_bytes(int B, int T, int nIh, int cI, int m) {
  if (B <= 0 || T <= 0 || m < 1 || T % m || (cI != 64 && cI != 128) || nIh < 1 || nIh * cI > 512)
    return 0;
  return kch::ste_bwd_ws_bytes(B, T, nIh, cI, m);
}

int kch_csa_ste_bwd(const float* q_idx, const float* w_idx, const float* kc, const float* raw,
                    const float* K_idx, const float* Z_idx, const float* B_idx, const float* dsel,
                    float* dq_idx, float* dw_idx, float* dK_idx, float* dZ_idx, float* dBp, int B,
                    int T, int m, int nIh, int cI, float scale, int normalize, void* ws,
                    size_t ws_bytes, void* stream) {
  const char* fn = "kch_csa_ste_bwd";
  if (B < 0 || T < 1 || m < 1 || nIh < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d m=%d nIh=%d (T >= 1)", fn, B, T, m, nIh);
  if (T % m) return fail(KCH_ERR_INVALID, "%s: T=%d must be a multiple of m=%d", fn, T, m);
  if ((cI != 64 && cI != 128) || (nIh != 1 && nIh != 2 && nIh != 4 && nIh != 8) || nIh * cI > 512)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nIh=%d, cI=%d not supported (cI 64 / 128, nIh * cI <= 512)",
                fn, nIh, cI);
  if (std::isnan(scale)) return fail(KCH_ERR_INVALID, "%s: scale is NaN", fn);
  if ((long long)B * T * (T / m) >= (1LL << 40)) return fail(KCH_ERR_UNSUPPORTED, "%s: too large", fn);
  if (B == 0) return KCH_OK;
  if (!q_idx || !w_idx || !kc || !raw || !K_idx || !Z_idx || !B_idx || !dsel || !dq_idx || !dw_idx ||
      !dK_idx || !dZ_idx || !dBp)
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  const size_t need = kch_csa_ste_bwd_ws_bytes(B, T, nIh, cI, m);
  if (!ws || ws_bytes < need)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required, got %zu", fn, need,
                ws ? ws_bytes : (size_t)0);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  kch::SteBwdParams p;
  p.qi = q_idx; p.w = w_idx; p.kc = kc; p.dsel = dsel; p.dqi = dq_idx; p.dw = dw_idx;
  p.B = B; p.T = T; p.nb = T / m; p.m = m; p.nIh = nIh; p.cI = cI; p.normalize = normalize ? 1 : 0;
  p.scale = scale;
  kch::HcaBwdParams bp;
  bp.q = nullptr; bp.dout = nullptr; bp.kc = kc; bp.raw = raw; bp.kl = nullptr; bp.lsrc = nullptr;
  bp.C = K_idx; bp.Z = Z_idx; bp.Bpos = B_idx; bp.sink = nullptr;
  bp.dq = nullptr; bp.dC = dK_idx; bp.dZ = dZ_idx; bp.dBp = dBp; bp.dlocal = nullptr;
  bp.sink_part = nullptr;
  bp.normalize = p.normalize;
  bp.B = B; bp.T = T; bp.nh = 1; bp.c = cI; bp.m2 = m; bp.nb = T / m; bp.win = 0; bp.scale = scale;
  return hip_status(fn, kch::ste_bwd_dispatch(p, bp, ws, (hipStream_t)stream));
}

int kch_kda_gates_bwd(const void* proj, long long ld_proj, const void* gl, long long ld_gl,
                      const void* dq, const void* dk, const void* dv, const void* dg,
                      const void* dbeta, void* dproj, void* dgl, int B, int T, int H, int HV, int K,
                      int V, float decay_scale, int dtype, void* stream) {
  const char* fn = "kch_kda_gates_bwd";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || T < 0 || H < 1 || HV < 1 || K < 1 || V < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (K > 256) return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d > 256 not supported", fn, K);
  if (ld_proj < 2LL * H * K + (long long)HV * V + HV || ld_gl < (long long)HV * K)
    return fail(KCH_ERR_INVALID, "%s: row strides too small", fn);
  if ((long long)B * T == 0) return KCH_OK;
  if (!proj || !gl || !dq || !dk || !dv || !dg || !dbeta || !dproj || !dgl)
    return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  kch::KdaGatesBwdParams p;
  p.proj = proj; p.ld_proj = ld_proj; p.gl = gl; p.ld_gl = ld_gl;
  p.dq = dq; p.dk = dk; p.dv = dv; p.dg = dg; p.dbeta = dbeta; p.dproj = dproj; p.dgl = dgl;
  p.B = B; p.T = T; p.H = H; p.HV = HV; p.K = K; p.V = V;
  p.decay_scale = decay_scale;
  return hip_status(fn, kch::kda_gates_bwd_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_short_conv_bwd(const void* x, const void* lookback, const void* weight, const void* dy,
                       void* dx, float* dw, float* db, void* dlookback, int B, int T, int d,
                       int dtype, void* stream) {
  const char* fn = "kch_short_conv_bwd";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || T < 0 || d < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d d=%d", fn, B, T, d);
  if ((long long)B * T == 0) return KCH_OK;
  if (!x || !weight || !dy || !dx || !dw) return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  kch::ShortConvBwdParams p;
  p.x = x; p.lookback = lookback; p.weight = weight; p.dy = dy; p.dx = dx; p.dw = dw; p.db = db;
  p.dlookback = dlookback;
  p.B = B; p.T = T; p.d = d;
  return hip_status(fn, kch::short_conv_bwd_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_layer_norm_bwd(const void* x, const void* w, const void* dy, void* dx, float* dw, float* db,
                       long long rows, int d, float eps, int dtype, int wdtype, void* stream) {
  const char* fn = "kch_layer_norm_bwd";
  if (!dtype_ok(dtype) || !dtype_ok(wdtype))
    return fail(KCH_ERR_INVALID, "%s: unknown dtype %d / %d", fn, dtype, wdtype);
  if (rows < 0 || d < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes rows=%lld d=%d", fn, rows, d);
  if (d > 4096) return fail(KCH_ERR_UNSUPPORTED, "%s: d=%d > 4096 not supported", fn, d);
  if (rows == 0) return KCH_OK;
  if (!x || !w || !dy || !dx || !dw) return fail(KCH_ERR_INVALID, "%s: null tensor pointer", fn);
  kch::LayerNormBwdParams p;
  p.x = x; p.w = w; p.dy = dy; p.dx = dx; p.dw = dw; p.db = db; p.rows = rows; p.d = d; p.eps = eps;
  return hip_status(fn, kch::layer_norm_bwd_dispatch(p, dtype, wdtype, (hipStream_t)stream));
}

// key row formats of kch_compress: 0 bf16, 1 fp32, 2 bf16 three-part, 3 fp16
// two-part (normalised rows), 4 the parts of 3 chunk-major (c a multiple of 32)
static int check_key_format(const char* fn, int key_f32, int normalize, int c) {
  if (key_f32 < 0 || key_f32 > 4) return fail(KCH_ERR_INVALID, "%s: key format %d", fn, key_f32);
  if (key_f32 >= 3 && !normalize)
    return fail(KCH_ERR_INVALID, "%s: fp16 split keys (key_f32=%d) need normalize", fn, key_f32);
  if (key_f32 == 4 && c % 32)
    return fail(KCH_ERR_UNSUPPORTED, "%s: chunk-major keys need c %% 32 == 0 (c=%d)", fn, c);
  return KCH_OK;
}

int kch_compress(const void* C, long long ldC, const void* Z, long long ldZ, const float* B_pos,
                 float* out_raw, void* out_key, int key_f32, int normalize, void* local, int B,
                 int T, int m, int c, int dtype, void* stream) {
  const char* fn = "kch_compress";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (m < 1) return fail(KCH_ERR_INVALID, "%s: compression factor m=%d must be >= 1", fn, m);
  if (B < 0 || T < 0 || c < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d c=%d", fn, B, T, c);
  if (T % m) return fail(KCH_ERR_INVALID, "%s: T=%d must be divisible by m=%d", fn, T, m);
  if (c > 128) return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d > 128 not supported", fn, c);
  if (int rc = check_key_format(fn, key_f32, normalize, c)) return rc;
  if (B * T == 0) return KCH_OK;
  if (!C || !Z || !B_pos) return fail(KCH_ERR_INVALID, "%s: null input pointer", fn);
  if (ldC < c || ldZ < c) return fail(KCH_ERR_INVALID, "%s: row strides must be >= c", fn);
  kch::CompressParams p{C, Z, nullptr, nullptr, ldC, ldZ, 0, 0, B_pos, nullptr, out_raw, out_key,
                        (kch::bf16_t*)local, B, T, m, c, 0, normalize, key_f32};
  return hip_status(fn, kch::compress_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_compress_overlapped(const void* Ca, long long ldCa, const void* Cb, long long ldCb,
                            const void* Za, long long ldZa, const void* Zb, long long ldZb,
                            const float* Ba, const float* Bb, float* out_raw, void* out_key,
                            int key_f32, int normalize, void* local, int B, int T, int m, int c,
                            int dtype, void* stream) {
  const char* fn = "kch_compress_overlapped";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (m < 1) return fail(KCH_ERR_INVALID, "%s: compression factor m=%d must be >= 1", fn, m);
  if (B < 0 || T < 0 || c < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d c=%d", fn, B, T, c);
  if (T % m) return fail(KCH_ERR_INVALID, "%s: T=%d must be divisible by m=%d", fn, T, m);
  if (c > 128) return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d > 128 not supported", fn, c);
  if (int rc = check_key_format(fn, key_f32, normalize, c)) return rc;
  if (B * T == 0) return KCH_OK;
  if (!Ca || !Cb || !Za || !Zb || !Ba || !Bb) return fail(KCH_ERR_INVALID, "%s: null input pointer", fn);
  if (ldCa < c || ldCb < c || ldZa < c || ldZb < c)
    return fail(KCH_ERR_INVALID, "%s: row strides must be >= c", fn);
  kch::CompressParams p{Ca, Za, Cb, Zb, ldCa, ldZa, ldCb, ldZb, Ba, Bb, out_raw, out_key,
                        (kch::bf16_t*)local, B, T, m, c, 1, normalize, key_f32};
  return hip_status(fn, kch::compress_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_csa_indexer_topk(const void* q_idx, const void* k_idx, const void* w_idx, void* idx_out,
                         int idx64, float* logits_out, int B, int T, int nb, int nIh, int cI,
                         int topk, int m, int pos0, int dense_visible, int normalize_q, float scale,
                         int sorted, int key_split, int dtype, void* stream) {
  const char* fn = "kch_csa_indexer_topk";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (topk < 0) return fail(KCH_ERR_INVALID, "%s: topk=%d must be >= 0", fn, topk);
  if (B < 0 || T < 0 || nb < 0 || m < 1 || pos0 < 0)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d nb=%d m=%d", fn, B, T, nb, m);
  if (nIh != 1 && nIh != 2 && nIh != 4 && nIh != 8 && nIh != 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nIh=%d not in {1,2,4,8,16}", fn, nIh);
  if (cI != 32 && cI != 64 && cI != 128)
    return fail(KCH_ERR_UNSUPPORTED, "%s: cI=%d not in {32,64,128}", fn, cI);
  if (key_split < 0 || key_split > 3) return fail(KCH_ERR_INVALID, "%s: key_split=%d", fn, key_split);
  if (key_split >= 2 && !normalize_q)
    return fail(KCH_ERR_INVALID, "%s: fp16 split keys (key_split=%d) need normalize_q", fn, key_split);
  if (B * T == 0 || topk == 0) return KCH_OK;
  if (!q_idx || !idx_out || (nb > 0 && !k_idx)) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  const long long lds = (long long)kch::indexer_lds_bytes(nb, nIh, topk);
  if (lds > 160 * 1024)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nb=%d with nIh=%d and topk=%d exceeds the LDS budget", fn,
                nb, nIh, topk);
  if (nb == 0) {
    // no block at all: every slot is -1 (a fill kernel: graph-capture safe)
    const long long words = (long long)B * T * topk * (idx64 ? 2 : 1);
    return hip_status(fn, kch::fill_u32(idx_out, words, 0xffffffffu, (hipStream_t)stream));
  }
  kch::IndexerParams p{q_idx, k_idx, w_idx, idx_out, logits_out, B, T, nb, nIh, cI, topk, m,
                       pos0, normalize_q, idx64, dense_visible, sorted ? 1 : 0, scale, 0,
                       key_split};
  return hip_status(fn, kch::indexer_dispatch(p, dtype, (hipStream_t)stream));
}

static int check_attn(const char* fn, int B, int T, int nb, int nh, int hd, int qdtype, int odtype) {
  if (!dtype_ok(qdtype) || !dtype_ok(odtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype", fn);
  if (B < 0 || T < 0 || nb < 0) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (nh < 1 || nh > 16) return fail(KCH_ERR_UNSUPPORTED, "%s: nh=%d not in [1, 16]", fn, nh);
  if (hd != 64 && hd != 128) return fail(KCH_ERR_UNSUPPORTED, "%s: head dim %d not in {64,128}", fn, hd);
  if (odtype != KCH_DT_F32 && odtype != qdtype)
    return fail(KCH_ERR_UNSUPPORTED, "%s: output dtype must be fp32 or the query dtype", fn);
  if ((long long)(T > nb ? T : nb) * hd * 2 >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: a batch row's key rows exceed 2 GiB (32-bit row offsets)", fn);
  return KCH_OK;
}

int kch_csa_sparse_attn(const void* q, const void* kv_comp, const int* idx, const void* kv_local,
                        const float* sink, void* out, int B, int T, int nb, int nh, int hd,
                        int topk, int win, float scale, int normalize_q, int qdtype, int odtype,
                        void* stream) {
  const char* fn = "kch_csa_sparse_attn";
  int rc = check_attn(fn, B, T, nb, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (topk < 0 || win < 0) return fail(KCH_ERR_INVALID, "%s: topk / window must be >= 0", fn);
  if (B * T == 0) return KCH_OK;
  if (!q || !out || (topk > 0 && (!idx || !kv_comp)) || (win > 0 && !kv_local))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::AttnParams p{q, (const kch::bf16_t*)kv_comp, idx, (const kch::bf16_t*)kv_local, sink, out,
                    B, T, nb, nh, hd, topk, 1, win, normalize_q, scale, 0, 0, -1, 0};
  return hip_status(fn, kch::attn_dispatch(p, true, qdtype, odtype, (hipStream_t)stream));
}

int kch_hca_attn(const void* q, const void* kv_comp, const void* kv_local, const float* sink,
                 void* out, int B, int T, int nb, int nh, int hd, int m, int win, float scale,
                 int normalize_q, int qdtype, int odtype, void* stream) {
  const char* fn = "kch_hca_attn";
  int rc = check_attn(fn, B, T, nb, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (m < 1 || win < 0) return fail(KCH_ERR_INVALID, "%s: m must be >= 1 and window >= 0", fn);
  if (B * T == 0) return KCH_OK;
  if (!q || !out || (nb > 0 && !kv_comp) || (win > 0 && !kv_local))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::AttnParams p{q, (const kch::bf16_t*)kv_comp, nullptr, (const kch::bf16_t*)kv_local, sink,
                    out, B, T, nb, nh, hd, 0, m, win, normalize_q, scale, 0, 0, -1, 0};
  return hip_status(fn, kch::attn_dispatch(p, false, qdtype, odtype, (hipStream_t)stream));
}

int kch_l2norm_rows(const void* x, long long ldx, void* out, int out_f32, int rows, int c,
                    int normalize, int dtype, void* stream) {
  const char* fn = "kch_l2norm_rows";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (rows < 0 || c < 1 || c > 256 || ldx < c) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (rows == 0) return KCH_OK;
  if (!x || !out) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  return hip_status(fn, kch::l2norm_rows_dispatch(x, ldx, out, out_f32, rows, c, normalize, dtype,
                                                  (hipStream_t)stream));
}

int kch_csa_decode_step(const void* q, const void* q_idx, const void* w_idx, const void* kv_comp,
                        long long kv_bstride, const float* k_idx, long long k_bstride,
                        const void* ring, long long ring_bstride, int ring_len, const float* sink,
                        void* out, int* idx_ws, int B, int nb, int nh, int hd, int nIh, int cI,
                        int topk, float scale, float idx_scale, int normalize_q,
                        int normalize_qidx, int qdtype, int odtype, void* stream) {
  const char* fn = "kch_csa_decode_step";
  int rc = check_attn(fn, B, 1, nb, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (topk < 0 || ring_len < 0) return fail(KCH_ERR_INVALID, "%s: topk / ring_len must be >= 0", fn);
  if (nIh != 1 && nIh != 2 && nIh != 4 && nIh != 8 && nIh != 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nIh=%d not in {1,2,4,8,16}", fn, nIh);
  if (cI != 32 && cI != 64 && cI != 128)
    return fail(KCH_ERR_UNSUPPORTED, "%s: cI=%d not in {32,64,128}", fn, cI);
  if (B == 0) return KCH_OK;
  if (!q || !out || (ring_len > 0 && !ring)) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  const int use_sel = (topk > 0 && nb > 0);
  if (use_sel) {
    if (!q_idx || !k_idx || !kv_comp || !idx_ws) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
    const long long lds = (long long)kch::indexer_lds_bytes(nb, nIh, topk);
    if (lds > 160 * 1024)
      return fail(KCH_ERR_UNSUPPORTED, "%s: %d cached blocks exceed the indexer LDS budget", fn, nb);
    kch::IndexerParams ip{q_idx, k_idx, w_idx, idx_ws, nullptr, B, 1, nb, nIh, cI, topk, 1,
                          0, normalize_qidx, 0, 1, 1, idx_scale, k_bstride, 0};
    rc = hip_status(fn, kch::indexer_dispatch(ip, qdtype, s));
    if (rc) return rc;
  }
  kch::AttnParams p{q, (const kch::bf16_t*)kv_comp, idx_ws, (const kch::bf16_t*)ring, sink, out,
                    B, 1, nb, nh, hd, use_sel ? topk : 0, 1, 0, 0, scale, kv_bstride,
                    ring_bstride, ring_len, 0};
  return hip_status(fn, kch::attn_dispatch(p, true, qdtype, odtype, s));
}

int kch_hca_decode_step(const void* q, const void* kv_comp, long long kv_bstride, const void* ring,
                        long long ring_bstride, int ring_len, const float* sink, void* out, int B,
                        int nb, int nh, int hd, float scale, int normalize_q, int qdtype, int odtype,
                        void* stream) {
  const char* fn = "kch_hca_decode_step";
  int rc = check_attn(fn, B, 1, nb, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (ring_len < 0) return fail(KCH_ERR_INVALID, "%s: ring_len must be >= 0", fn);
  if (B == 0) return KCH_OK;
  if (!q || !out || (nb > 0 && !kv_comp) || (ring_len > 0 && !ring))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  // every cached block is complete, hence visible: nvis = min(nb, (pos0 + 1) / 1)
  kch::AttnParams p{q, (const kch::bf16_t*)kv_comp, nullptr, (const kch::bf16_t*)ring, sink, out,
                    B, 1, nb, nh, hd, 0, 1, 0, 0, scale, kv_bstride, ring_bstride, ring_len, nb};
  return hip_status(fn, kch::attn_dispatch(p, false, qdtype, odtype, (hipStream_t)stream));
}

int kch_short_conv(const void* x, const void* lookback, const void* weight, const void* bias,
                   void* out, int B, int T, int d, int dtype, void* stream) {
  const char* fn = "kch_short_conv";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || T < 0 || d < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d T=%d d=%d", fn, B, T, d);
  if ((long long)B * T * d >= (1LL << 40)) return fail(KCH_ERR_INVALID, "%s: tensor too large", fn);
  if ((long long)B * T == 0) return KCH_OK;
  if (!x || !weight || !out) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (d % 8 == 0) {
    const uintptr_t a = (uintptr_t)x | (uintptr_t)out | (uintptr_t)lookback;
    if (a % 16) return fail(KCH_ERR_INVALID, "%s: x / out / lookback must be 16-byte aligned", fn);
  }
  kch::ShortConvParams p{x, lookback, weight, bias, out, B, T, d};
  return hip_status(fn, kch::short_conv_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_kda_gates(const void* proj, long long ld_proj, const void* gl, long long ld_gl, void* q,
                  void* k, void* v, void* g, void* beta, int B, int T, int H, int HV, int K, int V,
                  float decay_scale, int dtype, void* stream) {
  const char* fn = "kch_kda_gates";
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || T < 0 || H < 1 || HV < 1 || K < 1 || V < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (K > 256) return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d > 256 not supported", fn, K);
  if (ld_proj < 2LL * H * K + (long long)HV * V + HV || ld_gl < (long long)HV * K)
    return fail(KCH_ERR_INVALID, "%s: row strides too small", fn);
  if ((long long)B * T >= (1LL << 31)) return fail(KCH_ERR_INVALID, "%s: too many rows", fn);
  if ((long long)B * T == 0) return KCH_OK;
  if (!proj || !gl || !q || !k || !v || !g || !beta)
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::KdaGatesParams p{proj, ld_proj, gl, ld_gl, q, k, v, g, beta, B, T, H, HV, K, V,
                        decay_scale};
  return hip_status(fn, kch::kda_gates_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_layer_norm(const void* x, const void* w, const void* b, void* out, int rows, int d,
                   float eps, int dtype, int wdtype, void* stream) {
  const char* fn = "kch_layer_norm";
  if (!dtype_ok(dtype) || !dtype_ok(wdtype))
    return fail(KCH_ERR_INVALID, "%s: unknown dtype %d / %d", fn, dtype, wdtype);
  if (rows < 0 || d < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (rows == 0) return KCH_OK;
  if (!x || !w || !out) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::LayerNormParams p{x, w, b, out, rows, d, eps};
  return hip_status(fn, kch::layer_norm_dispatch(p, dtype, wdtype, (hipStream_t)stream));
}

int kch_linear_rows(const void* x, long long ldx, const void* w, long long ldw, void* y,
                    long long ldy, int M, int N, int K, int dtype, void* stream) {
  const char* fn = "kch_linear_rows";
  if (dtype != KCH_DT_BF16 && dtype != KCH_DT_F16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (bf16 or fp16 only)", fn, dtype);
  if (M < 0 || N < 0 || K < 0) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (M == 0 || N == 0) return KCH_OK;
  if (M > 16) return fail(KCH_ERR_UNSUPPORTED, "%s: M=%d > 16 rows", fn, M);
  if (K < 32 || K % 32) return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not a multiple of 32", fn, K);
  if (!x || !w || !y) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (ldx < K || ldw < K || ldy < N)
    return fail(KCH_ERR_INVALID, "%s: row strides (%lld, %lld, %lld) below the row lengths", fn,
                ldx, ldw, ldy);
  if ((ldx | ldw) % 8 || (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: x and w rows must be 16-byte aligned", fn);
  kch::LinearRowsParams p{x, w, y, ldx, ldw, ldy, M, N, K};
  return hip_status(fn, kch::linear_rows_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_linear_rows_fused(const void* x, long long ldx, const void* w, long long ldw, void* y,
                          long long ldy, int M, int N, int K, const void* ln_w, const void* ln_b,
                          float ln_eps, int ln_wdtype, const void* res, long long ldr, int* counter,
                          int dtype, void* stream) {
  const char* fn = "kch_linear_rows_fused";
  if (dtype != KCH_DT_BF16 && dtype != KCH_DT_F16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (bf16 or fp16 only)", fn, dtype);
  if (M < 0 || N < 0 || K < 0) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (M == 0 || N == 0) {
    if (counter) return fail(KCH_ERR_INVALID, "%s: a counter needs a launch (M, N >= 1)", fn);
    return KCH_OK;
  }
  if (M > 16) return fail(KCH_ERR_UNSUPPORTED, "%s: M=%d > 16 rows", fn, M);
  if (K < 32 || K % 32) return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not a multiple of 32", fn, K);
  if (!x || !w || !y) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (ldx < K || ldw < K || ldy < N || (res && ldr < N))
    return fail(KCH_ERR_INVALID, "%s: row strides below the row lengths", fn);
  if ((ldx | ldw) % 8 || (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: x and w rows must be 16-byte aligned", fn);
  kch::LinearRowsParams p{x, w, y, ldx, ldw, ldy, M, N, K};
  if (ln_w) {
    if (!dtype_ok(ln_wdtype)) return fail(KCH_ERR_INVALID, "%s: unknown norm dtype %d", fn, ln_wdtype);
    if (K > 4096 || (long long)M * K > kch::kLinearLnMax)
      return fail(KCH_ERR_UNSUPPORTED, "%s: a normalised input holds at most 4096 columns and %d "
                  "elements (M=%d, K=%d)", fn, kch::kLinearLnMax, M, K);
    if ((reinterpret_cast<uintptr_t>(ln_w) | reinterpret_cast<uintptr_t>(ln_b)) % 16)
      return fail(KCH_ERR_UNSUPPORTED, "%s: norm parameters must be 16-byte aligned", fn);
    if (std::isnan(ln_eps) || ln_eps < 0.f) return fail(KCH_ERR_INVALID, "%s: bad eps", fn);
    p.ln_w = ln_w;
    p.ln_b = ln_b;
    p.ln_eps = ln_eps;
    p.ln_wdtype = ln_wdtype;
  } else if (ln_b) {
    return fail(KCH_ERR_INVALID, "%s: a norm bias without a norm weight", fn);
  }
  p.res = res;
  p.ldr = ldr;
  p.counter = counter;
  return hip_status(fn, kch::linear_rows_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_linear_up(const void* x, long long ldx, const void* w, long long ldw, void* y,
                  long long ldy, long long M, int N, int K, int dtype, void* stream) {
  const char* fn = "kch_linear_up";
  if (dtype != KCH_DT_BF16 && dtype != KCH_DT_F16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (bf16 or fp16 only)", fn, dtype);
  if (M < 0 || N < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes M=%lld N=%d", fn, M, N);
  if (K != 32 && K != 64 && K != 128 && K != 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not in {32, 64, 128, 256}", fn, K);
  if ((M + 63) / 64 >= (1LL << 31)) return fail(KCH_ERR_INVALID, "%s: too many rows", fn);
  if (M == 0) return KCH_OK;
  if (!x || !w || !y) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (ldx < K || ldw < K || ldy < N)
    return fail(KCH_ERR_INVALID, "%s: row strides below the row lengths", fn);
  if ((ldx | ldw) % 8 || (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: x and w rows must be 16-byte aligned", fn);
  if (N % 8 == 0 && (ldy % 8 || reinterpret_cast<uintptr_t>(y) % 16))
    return fail(KCH_ERR_UNSUPPORTED, "%s: y rows must be 16-byte aligned", fn);
  kch::RowsProjParams p{x, w, y, ldx, ldw, ldy, M, N, K};
  return hip_status(fn, kch::rows_up_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_kda_decode_front(const void* x, long long ldx, const void* ln_w, const void* ln_b,
                         float eps, void* lookback, const void* conv_w, const void* conv_b,
                         void* out, int B, int d, int dtype, int wdtype, void* stream) {
  const char* fn = "kch_kda_decode_front";
  if (!dtype_ok(dtype) || !dtype_ok(wdtype))
    return fail(KCH_ERR_INVALID, "%s: unknown dtype %d / %d", fn, dtype, wdtype);
  if (B < 0 || d < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d d=%d", fn, B, d);
  if (d % 8 || d > 4096) return fail(KCH_ERR_UNSUPPORTED, "%s: d=%d (a multiple of 8, at most 4096)", fn, d);
  if (ldx < d) return fail(KCH_ERR_INVALID, "%s: row stride %lld below d=%d", fn, ldx, d);
  if (B == 0) return KCH_OK;
  if (!x || !ln_w || !lookback || !conv_w || !out) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  const uintptr_t a = (uintptr_t)x | (uintptr_t)ln_w | (uintptr_t)ln_b | (uintptr_t)lookback |
                      (uintptr_t)conv_w | (uintptr_t)conv_b | (uintptr_t)out;
  if (a % 16 || ldx % 8) return fail(KCH_ERR_INVALID, "%s: operands must be 16-byte aligned", fn);
  if (std::isnan(eps) || eps < 0.f) return fail(KCH_ERR_INVALID, "%s: bad eps", fn);
  kch::KdaFrontParams p{x, ldx, ln_w, ln_b, eps, lookback, conv_w, conv_b, out, B, d};
  return hip_status(fn, kch::kda_front_dispatch(p, dtype, wdtype, (hipStream_t)stream));
}

}  // extern "C"

// kch_kda_decode_step, and with lookback non-null the conv lookback's advance.
static int kda_decode_step(const char* fn, const void* proj, long long ld_proj, const void* g_up,
                           float* state, void* o, int B, int H, int HV, int K, int V, float scale,
                           float decay_scale, float g_clamp_min, void* lookback, const void* h,
                           int d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || H < 1 || HV < 1 || V < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (HV % H) return fail(KCH_ERR_INVALID, "%s: HV=%d must be divisible by H=%d", fn, HV, H);
  if (K != 16 && K != 32 && K != 64 && K != 128 && K != 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: K=%d not in {16, 32, 64, 128, 256}", fn, K);
  if (V % 32) return fail(KCH_ERR_UNSUPPORTED, "%s: V=%d must be a multiple of 32", fn, V);
  if (ld_proj < 2LL * H * K + (long long)HV * V + HV + K)
    return fail(KCH_ERR_INVALID, "%s: row stride %lld too small", fn, ld_proj);
  if ((long long)B * HV * (V / 32) >= (1LL << 31)) return fail(KCH_ERR_INVALID, "%s: too large", fn);
  if (std::isnan(g_clamp_min)) return fail(KCH_ERR_INVALID, "%s: g_clamp_min is NaN", fn);
  if (B == 0) return KCH_OK;
  if (!proj || !g_up || !state || !o) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if ((uintptr_t)g_up % 16) return fail(KCH_ERR_INVALID, "%s: g_up must be 16-byte aligned", fn);
  kch::KdaStepParams p{proj, ld_proj, g_up, state, o, B, H, HV, K, V, scale, decay_scale,
                       g_clamp_min};
  p.look = lookback;
  p.h_in = h;
  p.d = d;
  return hip_status(fn, kch::kda_step_dispatch(p, dtype, (hipStream_t)stream));
}

extern "C" {

int kch_kda_decode_step(const void* proj, long long ld_proj, const void* g_up, float* state,
                        void* o, int B, int H, int HV, int K, int V, float scale,
                        float decay_scale, float g_clamp_min, int dtype, void* stream) {
  return kda_decode_step("kch_kda_decode_step", proj, ld_proj, g_up, state, o, B, H, HV, K, V,
                         scale, decay_scale, g_clamp_min, nullptr, nullptr, 0, dtype, stream);
}

int kch_kda_front_rows(const void* x, long long ldx, const void* ln_w, const void* ln_b,
                       float eps, int wdtype, const void* lookback, const void* conv_w,
                       const void* conv_b, void* h_out, const void* w, long long ldw, void* y,
                       long long ldy, int B, int N, int d, int dtype, void* stream) {
  const char* fn = "kch_kda_front_rows";
  if (dtype != KCH_DT_BF16 && dtype != KCH_DT_F16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (bf16 or fp16 only)", fn, dtype);
  if (!dtype_ok(wdtype)) return fail(KCH_ERR_INVALID, "%s: unknown norm dtype %d", fn, wdtype);
  if (B < 0 || N < 0 || d < 1) return fail(KCH_ERR_INVALID, "%s: bad sizes", fn);
  if (B == 0 || N == 0) return KCH_OK;
  if (B > 16) return fail(KCH_ERR_UNSUPPORTED, "%s: B=%d > 16 rows", fn, B);
  if (d < 32 || d % 32 || d > 4096 || (long long)B * d > kch::kLinearLnMax)
    return fail(KCH_ERR_UNSUPPORTED, "%s: d=%d (a multiple of 32, at most 4096; B d at most %d)",
                fn, d, kch::kLinearLnMax);
  if (!x || !ln_w || !lookback || !conv_w || !h_out || !w || !y)
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (ldx < d || ldw < d || ldy < N)
    return fail(KCH_ERR_INVALID, "%s: row strides below the row lengths", fn);
  const uintptr_t a = (uintptr_t)x | (uintptr_t)ln_w | (uintptr_t)ln_b | (uintptr_t)lookback |
                      (uintptr_t)conv_w | (uintptr_t)conv_b | (uintptr_t)h_out | (uintptr_t)w;
  if (a % 16 || (ldx | ldw) % 8) return fail(KCH_ERR_UNSUPPORTED, "%s: operands must be 16-byte aligned", fn);
  if (std::isnan(eps) || eps < 0.f) return fail(KCH_ERR_INVALID, "%s: bad eps", fn);
  kch::LinearRowsParams p{x, w, y, ldx, ldw, ldy, B, N, d};
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.ln_eps = eps;
  p.ln_wdtype = wdtype;
  p.conv_w = conv_w;
  p.conv_b = conv_b;
  p.look = lookback;
  p.h_out = h_out;
  return hip_status(fn, kch::linear_rows_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_kda_decode_step_shift(const void* proj, long long ld_proj, const void* g_up, float* state,
                              void* o, int B, int H, int HV, int K, int V, float scale,
                              float decay_scale, float g_clamp_min, void* lookback,
                              const void* h, int d, int dtype, void* stream) {
  const char* fn = "kch_kda_decode_step_shift";
  if (d < 1) return fail(KCH_ERR_INVALID, "%s: d=%d", fn, d);
  if (B > 0 && (!lookback || !h)) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  int rc = kda_decode_step(fn, proj, ld_proj, g_up, state, o, B, H, HV, K, V, scale, decay_scale,
                           g_clamp_min, lookback, h, d, dtype, stream);
  return rc;
}

// Shared checks of the cache append entry points.
static int check_cache_append(const char* fn, const void* proj, long long ld_proj, long long width,
                              const void* acc, const void* c_rows, const void* c_keys,
                              const int* n_seen, int B, int c, int m, int win, const void* ring,
                              int cap, int dtype) {
  if (!dtype_ok(dtype)) return fail(KCH_ERR_INVALID, "%s: unknown dtype %d", fn, dtype);
  if (B < 0 || c < 1 || m < 1 || win < 0 || cap < 1)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d c=%d m=%d win=%d cap=%d", fn, B, c, m, win, cap);
  if (ld_proj < width) return fail(KCH_ERR_INVALID, "%s: row stride %lld below %lld", fn, ld_proj, width);
  if (!proj || !acc || !c_rows || !c_keys || !n_seen || (win > 0 && !ring))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  return KCH_OK;
}

int kch_csa_cache_append(const void* proj, long long ld_proj, void* acc, void* prev,
                         const float* Ba, const float* Bb, const float* B_idx, void* ring,
                         void* c_rows, void* c_keys, void* k_rows, float* k_inv,
                         const int* n_seen, int B, int c, int cI, int m, int win, int cap,
                         int normalize, int dtype, void* stream) {
  const char* fn = "kch_csa_cache_append";
  if (c < 1 || cI < 1 || c > 256 || c + cI > 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d, cI=%d (c + cI at most 256)", fn, c, cI);
  int rc = check_cache_append(fn, proj, ld_proj, 4LL * c + 2LL * cI, acc, c_rows, c_keys, n_seen,
                              B, c, m, win, ring, cap, dtype);
  if (rc) return rc;
  if (B == 0) return KCH_OK;
  if (!prev || !Ba || !Bb || !B_idx || !k_rows || !k_inv)
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::CacheStepParams p{proj, ld_proj, acc, prev, Ba, Bb, B_idx, win > 0 ? ring : nullptr,
                         c_rows, c_keys, k_rows, k_inv, n_seen, B, c, cI, m, win, cap,
                         normalize != 0, 1};
  return hip_status(fn, kch::cache_step_dispatch(p, dtype, (hipStream_t)stream));
}

int kch_hca_cache_append(const void* proj, long long ld_proj, void* acc, const float* B_pos,
                         void* ring, void* c_rows, void* c_keys, const int* n_seen, int B, int c,
                         int m2, int win, int cap, int normalize, int dtype, void* stream) {
  const char* fn = "kch_hca_cache_append";
  if (c < 1 || c > 256) return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d > 256", fn, c);
  int rc = check_cache_append(fn, proj, ld_proj, 2LL * c, acc, c_rows, c_keys, n_seen, B, c, m2,
                              win, ring, cap, dtype);
  if (rc) return rc;
  if (B == 0) return KCH_OK;
  if (!B_pos) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::CacheStepParams p{proj, ld_proj, acc, nullptr, B_pos, nullptr, nullptr,
                         win > 0 ? ring : nullptr, c_rows, c_keys, nullptr, nullptr, n_seen, B, c,
                         0, m2, win, cap, normalize != 0, 0};
  return hip_status(fn, kch::cache_step_dispatch(p, dtype, (hipStream_t)stream));
}

// A row projection y = x W^T launched beside a cache append: bf16 / fp16, M
// rows (M <= 16), K a multiple of 32, 16-byte aligned x and w rows.
static int rows_beside(const char* fn, const void* x, long long ldx, const void* w, long long ldw,
                       void* y, long long ldy, int M, int N, int K, int dtype,
                       kch::LinearRowsParams* out) {
  if (dtype != KCH_DT_BF16 && dtype != KCH_DT_F16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: dtype %d (bf16 or fp16 only)", fn, dtype);
  if (M > 16) return fail(KCH_ERR_UNSUPPORTED, "%s: B=%d > 16 rows", fn, M);
  if (N < 1 || K < 32 || K % 32)
    return fail(KCH_ERR_UNSUPPORTED, "%s: N=%d, K=%d (K a multiple of 32)", fn, N, K);
  if (!x || !w || !y) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (ldx < K || ldw < K || ldy < N)
    return fail(KCH_ERR_INVALID, "%s: row strides below the row lengths", fn);
  if ((ldx | ldw) % 8 || (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: x and w rows must be 16-byte aligned", fn);
  *out = kch::LinearRowsParams{x, w, y, ldx, ldw, ldy, M, N, K};
  return KCH_OK;
}

int kch_csa_cache_append_rows(const void* proj, long long ld_proj, void* acc, void* prev,
                              const float* Ba, const float* Bb, const float* B_idx, void* ring,
                              void* c_rows, void* c_keys, void* k_rows, float* k_inv,
                              const int* n_seen, int B, int c, int cI, int m, int win, int cap,
                              int normalize, const void* x, long long ldx, const void* w,
                              long long ldw, void* y, long long ldy, int N, int K, int dtype,
                              void* stream) {
  const char* fn = "kch_csa_cache_append_rows";
  if (c < 1 || cI < 1 || c > 256 || c + cI > 256)
    return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d, cI=%d (c + cI at most 256)", fn, c, cI);
  int rc = check_cache_append(fn, proj, ld_proj, 4LL * c + 2LL * cI, acc, c_rows, c_keys, n_seen,
                              B, c, m, win, ring, cap, dtype);
  if (rc) return rc;
  if (B == 0) return KCH_OK;
  if (!prev || !Ba || !Bb || !B_idx || !k_rows || !k_inv)
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::LinearRowsParams lp;
  if ((rc = rows_beside(fn, x, ldx, w, ldw, y, ldy, B, N, K, dtype, &lp))) return rc;
  kch::CacheStepParams p{proj, ld_proj, acc, prev, Ba, Bb, B_idx, win > 0 ? ring : nullptr,
                         c_rows, c_keys, k_rows, k_inv, n_seen, B, c, cI, m, win, cap,
                         normalize != 0, 1};
  return hip_status(fn, kch::cache_step_rows_dispatch(p, lp, dtype, (hipStream_t)stream));
}

int kch_hca_cache_append_rows(const void* proj, long long ld_proj, void* acc, const float* B_pos,
                              void* ring, void* c_rows, void* c_keys, const int* n_seen, int B,
                              int c, int m2, int win, int cap, int normalize, const void* x,
                              long long ldx, const void* w, long long ldw, void* y, long long ldy,
                              int N, int K, int dtype, void* stream) {
  const char* fn = "kch_hca_cache_append_rows";
  if (c < 1 || c > 256) return fail(KCH_ERR_UNSUPPORTED, "%s: c=%d > 256", fn, c);
  int rc = check_cache_append(fn, proj, ld_proj, 2LL * c, acc, c_rows, c_keys, n_seen, B, c, m2,
                              win, ring, cap, dtype);
  if (rc) return rc;
  if (B == 0) return KCH_OK;
  if (!B_pos) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  kch::LinearRowsParams lp;
  if ((rc = rows_beside(fn, x, ldx, w, ldw, y, ldy, B, N, K, dtype, &lp))) return rc;
  kch::CacheStepParams p{proj, ld_proj, acc, nullptr, B_pos, nullptr, nullptr,
                         win > 0 ? ring : nullptr, c_rows, c_keys, nullptr, nullptr, n_seen, B, c,
                         0, m2, win, cap, normalize != 0, 0};
  return hip_status(fn, kch::cache_step_rows_dispatch(p, lp, dtype, (hipStream_t)stream));
}

}  // extern "C"

namespace {

// Workspace plan of a decode step (kch_csa_decode / kch_hca_decode).
struct DecodePlan {
  int rb = 0, nr = 0;             // indexer ranges (sparse with blocks and topk > 0)
  bool split = false;             // score / select split: off_keys holds [B, ko] keys
  long long ko = 0;
  size_t off_keys = 0;
  int na = 0, ngrp = 0, grows = 0;  // attended rows before the ring, row groups, rows per group
  size_t off_cand = 0, off_idx = 0, off_po = 0, off_pml = 0, bytes = 0;
};

size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

DecodePlan decode_plan(int B, int nb, int nh, int hd, int topk, int ring_len, bool sparse,
                       bool one_range = false) {
  DecodePlan pl;
  const bool sel = sparse && nb > 0 && topk > 0;
  if (sel) kch::decode_idx_plan(B, nb, topk, &pl.rb, &pl.nr);
  if (sel && one_range && nb <= kch::decode_range_max() &&
      kch::decode_select_lds(topk) <= 160 * 1024) {
    // a device-driven step's capacity: ranges of 256 blocks write their logit
    // keys, one workgroup per sequence selects from all of them (no merge)
    pl.split = true;
    pl.rb = 256;
    pl.nr = (nb + 255) / 256;
    pl.ko = (nb + 3) & ~3;
  }
  pl.na = sparse ? (sel ? topk : 0) : nb;
  // the attention takes the attended blocks in whole 32-row steps (padded)
  const long long rows = (long long)((pl.na + 31) & ~31) + ring_len;
  // row groups (one workgroup each): about 768 over the batch (three resident
  // per CU: one round), at least 128 rows, at most 64 per sequence, a
  // multiple of 64 rows
  long long grows = ((long long)B * rows + 767) / 768;
  grows = grows < 128 ? 128 : grows;
  grows = grows < (rows + 63) / 64 ? (rows + 63) / 64 : grows;
  grows = (grows + 63) & ~63LL;
  // a short step (at most 24 steps of 32 rows per sequence, a batch the
  // minimum group size would spread over one round) takes one group per
  // sequence: a merge launch costs more than the group's extra steps
  if (rows <= 768 && (long long)B * rows <= 768LL * 128) grows = (rows + 63) & ~63LL;
  pl.grows = (int)grows;
  pl.ngrp = rows > 0 ? (int)((rows + grows - 1) / grows) : 0;
  size_t off = 0;
  pl.off_keys = off;
  if (pl.split) off += a256((size_t)B * pl.ko * 4);
  pl.off_cand = off;
  if (sel && pl.nr > 1 && !pl.split) off += a256((size_t)B * pl.nr * topk * 8);
  pl.off_idx = off;
  if (sel) off += a256((size_t)B * topk * 4);
  pl.off_po = off;
  if (pl.ngrp > 1) off += a256((size_t)B * pl.ngrp * nh * hd * 4);
  pl.off_pml = off;
  if (pl.ngrp > 1) off += a256((size_t)B * pl.ngrp * nh * 2 * 4);
  pl.bytes = off;
  return pl;
}

// Per-step counts of a device-driven decode step (decode_step.hip).
struct DynStep {
  const int* n_seen = nullptr;
  int m = 1, win = 0, cap = 0;
  long long ld_qb = 0;
};

int run_decode_attn(const char* fn, const DecodePlan& pl, const void* q, const void* kv_comp,
                    long long kv_bstride, const int* idx, const void* ring, long long ring_bstride,
                    int ring_len, const float* sink, void* out, int B, int nb, int nh, int hd,
                    float scale, int normalize_q, int qdtype, int odtype, char* ws,
                    hipStream_t s, const DynStep& dyn = DynStep()) {
  if ((long long)nb * hd * 2 >= (1LL << 31) || (long long)ring_len * hd * 2 >= (1LL << 31))
    return fail(KCH_ERR_UNSUPPORTED, "%s: a sequence's cached rows exceed 2 GiB (32-bit row offsets)", fn);
  kch::DecodeAttnParams a;
  a.n_seen = dyn.n_seen;
  a.m = dyn.m;
  a.win = dyn.win;
  a.cap = dyn.cap;
  a.ld_qb = dyn.ld_qb;
  a.q = q;
  a.kv = (const kch::bf16_t*)kv_comp;
  a.idx = idx;
  a.ring = (const kch::bf16_t*)ring;
  a.sink = sink;
  a.out = out;
  a.part_o = (float*)(ws + pl.off_po);
  a.part_ml = (float*)(ws + pl.off_pml);
  a.kv_bstride = kv_bstride;
  a.ring_bstride = ring_bstride;
  a.B = B; a.nb = nb; a.nh = nh; a.hd = hd; a.na = pl.na; a.ring_len = ring_len;
  a.ngrp = pl.ngrp; a.rows_per_group = pl.grows; a.normalize_q = normalize_q;
  a.scale = scale;
  if (pl.ngrp == 0) {
    // nothing to attend to: the output is zero (hd is even, so 16-bit outputs fill whole words)
    const long long elems = (long long)B * nh * hd;
    const long long words = odtype == KCH_DT_F32 ? elems : elems / 2;
    return hip_status(fn, kch::fill_u32(out, words, 0u, s));
  }
  return hip_status(fn, kch::decode_attn_dispatch(a, qdtype, odtype, s));
}

}  // namespace

extern "C" {

size_t kch_decode_ws_bytes(int B, int nb, int nh, int hd, int topk, int ring_len, int sparse) {
  if (B <= 0 || nb < 0 || nh < 1 || hd < 1 || topk < 0 || ring_len < 0) return 0;
  return decode_plan(B, nb, nh, hd, topk, ring_len, sparse != 0).bytes;
}

int kch_csa_decode(const void* q, const void* q_idx, const void* w_idx, const void* kv_comp,
                   long long kv_bstride, const void* k_rows, long long k_bstride,
                   const float* k_inv, long long kinv_bstride, const void* ring,
                   long long ring_bstride, int ring_len, const float* sink, void* out,
                   int* idx_out, int B, int nb, int nh, int hd, int nIh, int cI, int topk,
                   float scale, float idx_scale, int normalize_q, int normalize_qidx,
                   int qdtype, int kdtype, int odtype, void* ws, size_t ws_bytes, void* stream) {
  const char* fn = "kch_csa_decode";
  int rc = check_attn(fn, B, 1, nb, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (!dtype_ok(kdtype)) return fail(KCH_ERR_INVALID, "%s: unknown key dtype %d", fn, kdtype);
  if (topk < 0 || ring_len < 0) return fail(KCH_ERR_INVALID, "%s: topk / ring_len must be >= 0", fn);
  if (nIh != 1 && nIh != 2 && nIh != 4 && nIh != 8 && nIh != 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nIh=%d not in {1,2,4,8,16}", fn, nIh);
  if (cI != 32 && cI != 64 && cI != 128)
    return fail(KCH_ERR_UNSUPPORTED, "%s: cI=%d not in {32,64,128}", fn, cI);
  if (B == 0) return KCH_OK;
  const DecodePlan pl = decode_plan(B, nb, nh, hd, topk, ring_len, true);
  if (!ws || ws_bytes < pl.bytes)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required", fn, pl.bytes);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  if (!q || !out || (ring_len > 0 && !ring)) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  int* idx = nullptr;
  if (pl.nr > 0) {
    if (!q_idx || !k_rows || !kv_comp) return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
    if (pl.nr > 1 && !kch::decode_merge_fits(topk))
      return fail(KCH_ERR_UNSUPPORTED, "%s: %d cached blocks with topk=%d exceed the merge capacity",
                  fn, nb, topk);
    if (!kch::decode_idx_fits(pl.rb, topk, pl.nr))
      return fail(KCH_ERR_UNSUPPORTED,
                  "%s: %d cached blocks with topk=%d exceed the indexer's LDS (%zu bytes > 160 KB)",
                  fn, nb, topk, kch::decode_idx_lds(pl.rb, topk, pl.nr));
    idx = idx_out ? idx_out : (int*)(w + pl.off_idx);
    kch::DecodeIdxParams ip;
    ip.q_idx = q_idx; ip.w_idx = w_idx; ip.keys = k_rows; ip.inv_norm = k_inv;
    ip.k_bstride = k_bstride; ip.n_bstride = kinv_bstride;
    ip.cand = (unsigned long long*)(w + pl.off_cand);
    ip.idx_out = idx;
    ip.B = B; ip.nb = nb; ip.nIh = nIh; ip.cI = cI; ip.topk = topk; ip.rb = pl.rb; ip.nr = pl.nr;
    ip.normalize_q = normalize_qidx; ip.scale = idx_scale;
    rc = hip_status(fn, kch::decode_idx_dispatch(ip, qdtype, kdtype, s));
    if (rc) return rc;
  } else if (idx_out && topk > 0) {
    rc = hip_status(fn, kch::fill_u32(idx_out, (long long)B * topk, 0xffffffffu, s));  // all -1
    if (rc) return rc;
  }
  return run_decode_attn(fn, pl, q, kv_comp, kv_bstride, idx, ring, ring_bstride, ring_len, sink,
                         out, B, nb, nh, hd, scale, normalize_q, qdtype, odtype, w, s);
}

int kch_hca_decode(const void* q, const void* kv_comp, long long kv_bstride, const void* ring,
                   long long ring_bstride, int ring_len, const float* sink, void* out, int B,
                   int nb, int nh, int hd, float scale, int normalize_q, int qdtype, int odtype,
                   void* ws, size_t ws_bytes, void* stream) {
  const char* fn = "kch_hca_decode";
  int rc = check_attn(fn, B, 1, nb, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (ring_len < 0) return fail(KCH_ERR_INVALID, "%s: ring_len must be >= 0", fn);
  if (B == 0) return KCH_OK;
  const DecodePlan pl = decode_plan(B, nb, nh, hd, 0, ring_len, false);
  if (!ws || ws_bytes < pl.bytes)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required", fn, pl.bytes);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  if (!q || !out || (nb > 0 && !kv_comp) || (ring_len > 0 && !ring))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  return run_decode_attn(fn, pl, q, kv_comp, kv_bstride, nullptr, ring, ring_bstride, ring_len,
                         sink, out, B, nb, nh, hd, scale, normalize_q, qdtype, odtype, (char*)ws,
                         (hipStream_t)stream);
}

size_t kch_decode_dyn_ws_bytes(int B, int cap, int nh, int hd, int topk, int win, int sparse) {
  if (B <= 0 || cap < 1 || nh < 1 || hd < 1 || topk < 0 || win < 0) return 0;
  return decode_plan(B, cap, nh, hd, topk, win, sparse != 0, true).bytes;
}

int kch_csa_decode_dyn(const void* q, long long ld_q, const void* q_idx, long long ld_qidx,
                       const void* w_idx, long long ld_w, const void* kv_comp,
                       long long kv_bstride, const void* k_rows, long long k_bstride,
                       const float* k_inv, long long kinv_bstride, const void* ring,
                       long long ring_bstride, const int* n_seen, int m, int win, int cap,
                       const float* sink, void* out, int* idx_out, int B, int nh, int hd, int nIh,
                       int cI, int topk, float scale, float idx_scale, int normalize_q,
                       int normalize_qidx, int qdtype, int kdtype, int odtype, void* ws,
                       size_t ws_bytes, void* stream) {
  const char* fn = "kch_csa_decode_dyn";
  int rc = check_attn(fn, B, 1, cap, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (!dtype_ok(kdtype)) return fail(KCH_ERR_INVALID, "%s: unknown key dtype %d", fn, kdtype);
  if (m < 1 || win < 0 || cap < 1) return fail(KCH_ERR_INVALID, "%s: bad m / win / cap", fn);
  if (topk < 1) return fail(KCH_ERR_UNSUPPORTED, "%s: topk=%d (at least 1)", fn, topk);
  if (nIh != 1 && nIh != 2 && nIh != 4 && nIh != 8 && nIh != 16)
    return fail(KCH_ERR_UNSUPPORTED, "%s: nIh=%d not in {1,2,4,8,16}", fn, nIh);
  if (cI != 32 && cI != 64 && cI != 128)
    return fail(KCH_ERR_UNSUPPORTED, "%s: cI=%d not in {32,64,128}", fn, cI);
  if (ld_q < (long long)nh * hd || ld_qidx < (long long)nIh * cI || (w_idx && ld_w < nIh))
    return fail(KCH_ERR_INVALID, "%s: query row strides too small", fn);
  if (B == 0) return KCH_OK;
  const DecodePlan pl = decode_plan(B, cap, nh, hd, topk, win, true, true);
  if (!ws || ws_bytes < pl.bytes)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required", fn, pl.bytes);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  if (!q || !q_idx || !kv_comp || !k_rows || !out || !idx_out || !n_seen || (win > 0 && !ring))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  if (pl.nr > 1 && !pl.split && !kch::decode_merge_fits(topk))
    return fail(KCH_ERR_UNSUPPORTED, "%s: cap=%d blocks with topk=%d exceed the merge capacity", fn,
                cap, topk);
  if (!kch::decode_idx_fits(pl.rb, topk, pl.nr))
    return fail(KCH_ERR_UNSUPPORTED, "%s: cap=%d blocks with topk=%d exceed the indexer's LDS", fn,
                cap, topk);
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)ws;
  kch::DecodeIdxParams ip;
  ip.q_idx = q_idx; ip.w_idx = w_idx; ip.keys = k_rows; ip.inv_norm = k_inv;
  ip.k_bstride = k_bstride; ip.n_bstride = kinv_bstride;
  ip.cand = (unsigned long long*)(w + pl.off_cand);
  ip.idx_out = idx_out;
  ip.B = B; ip.nb = cap; ip.nIh = nIh; ip.cI = cI; ip.topk = topk; ip.rb = pl.rb; ip.nr = pl.nr;
  ip.normalize_q = normalize_qidx; ip.scale = idx_scale;
  ip.ld_qb = ld_qidx; ip.ld_wb = ld_w;
  ip.n_seen = n_seen; ip.m = m; ip.cap = cap;
  if (pl.split) {
    ip.keys_out = (uint32_t*)(w + pl.off_keys);
    ip.ko_bstride = pl.ko;
  }
  rc = hip_status(fn, kch::decode_idx_dispatch(ip, qdtype, kdtype, s));
  if (rc) return rc;
  DynStep dyn;
  dyn.n_seen = n_seen; dyn.m = m; dyn.win = win; dyn.cap = cap; dyn.ld_qb = ld_q;
  return run_decode_attn(fn, pl, q, kv_comp, kv_bstride, idx_out, win > 0 ? ring : nullptr,
                         ring_bstride, win, sink, out, B, cap, nh, hd, scale, normalize_q, qdtype,
                         odtype, w, s, dyn);
}

int kch_hca_decode_dyn(const void* q, long long ld_q, const void* kv_comp, long long kv_bstride,
                       const void* ring, long long ring_bstride, const int* n_seen, int m2,
                       int win, int cap, const float* sink, void* out, int B, int nh, int hd,
                       float scale, int normalize_q, int qdtype, int odtype, void* ws,
                       size_t ws_bytes, void* stream) {
  const char* fn = "kch_hca_decode_dyn";
  int rc = check_attn(fn, B, 1, cap, nh, hd, qdtype, odtype);
  if (rc) return rc;
  if (m2 < 1 || win < 0 || cap < 1) return fail(KCH_ERR_INVALID, "%s: bad m2 / win / cap", fn);
  if (ld_q < (long long)nh * hd) return fail(KCH_ERR_INVALID, "%s: query row stride too small", fn);
  if (B == 0) return KCH_OK;
  const DecodePlan pl = decode_plan(B, cap, nh, hd, 0, win, false, true);
  if (!ws || ws_bytes < pl.bytes)
    return fail(KCH_ERR_INVALID, "%s: workspace of %zu bytes required", fn, pl.bytes);
  if ((uintptr_t)ws & 255) return fail(KCH_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  if (!q || !kv_comp || !out || !n_seen || (win > 0 && !ring))
    return fail(KCH_ERR_INVALID, "%s: null pointer", fn);
  DynStep dyn;
  dyn.n_seen = n_seen; dyn.m = m2; dyn.win = win; dyn.cap = cap; dyn.ld_qb = ld_q;
  return run_decode_attn(fn, pl, q, kv_comp, kv_bstride, nullptr, win > 0 ? ring : nullptr,
                         ring_bstride, win, sink, out, B, cap, nh, hd, scale, normalize_q, qdtype,
                         odtype, (char*)ws, (hipStream_t)stream, dyn);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free CSA decode step. The workspace of kch_csa_decode lives in a
// file-scope device array, one copy per GPU, so the call needs no allocation
// from its caller or from this library.

namespace {

static __device__ __align__(256) unsigned char scratch[KCH_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of the copy of `scratch` on the stream's GPU. In host code
// the array's name is only a handle: its address comes from
// hipGetSymbolAddress, called once per device with that device current.
int scratch_address(const char* fn, hipStream_t s, void** out) {
  int dev = -1;
  hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(fn, e);
  if (dev < 0 || dev >= kMaxDevices)
    return fail(KCH_ERR_UNSUPPORTED, "%s: device %d beyond the %d this library tracks", fn, dev,
                kMaxDevices);
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = -1;
      e = hipGetDevice(&cur);
      if (e != hipSuccess) return hip_status(fn, e);
      if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_status(fn, e);
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      const hipError_t back = cur != dev ? hipSetDevice(cur) : hipSuccess;
      if (e != hipSuccess || !p)
        return fail(KCH_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                    hipGetErrorString(e));
      if (back != hipSuccess) return hip_status(fn, back);
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return KCH_OK;
}

}  // namespace

extern "C" {

int kch_csa_decode_noalloc(const void* q, const void* q_idx, const void* w_idx,
                           const void* kv_comp, long long kv_bstride, const void* k_rows,
                           long long k_bstride, const float* k_inv, long long kinv_bstride,
                           const void* ring, long long ring_bstride, int ring_len,
                           const float* sink, void* out, int* idx_out, int B, int nb, int nh,
                           int hd, int nIh, int cI, int topk, float scale, float idx_scale,
                           int normalize_q, int normalize_qidx, int qdtype, int kdtype,
                           int odtype, void* stream) {
  const char* fn = "kch_csa_decode_noalloc";
  if (B < 0 || nb < 0 || nh < 1 || hd < 1 || topk < 0 || ring_len < 0)
    return fail(KCH_ERR_INVALID, "%s: bad sizes B=%d nb=%d nh=%d hd=%d topk=%d ring_len=%d", fn,
                B, nb, nh, hd, topk, ring_len);
  if (B == 0) return KCH_OK;
  const size_t need = decode_plan(B, nb, nh, hd, topk, ring_len, true).bytes;
  if (need > (size_t)KCH_NOALLOC_SCRATCH_BYTES)
    return fail(KCH_ERR_UNSUPPORTED,
                "%s: B=%d nb=%d topk=%d ring_len=%d needs %zu bytes of scratch, more than the "
                "%d this entry point holds; call kch_csa_decode with a workspace",
                fn, B, nb, topk, ring_len, need, (int)KCH_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(fn, (hipStream_t)stream, &ws);
  if (rc) return rc;
  return kch_csa_decode(q, q_idx, w_idx, kv_comp, kv_bstride, k_rows, k_bstride, k_inv,
                        kinv_bstride, ring, ring_bstride, ring_len, sink, out, idx_out, B, nb, nh,
                        hd, nIh, cI, topk, scale, idx_scale, normalize_q, normalize_qidx, qdtype,
                        kdtype, odtype, ws, (size_t)KCH_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
