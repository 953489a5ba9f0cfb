// C-ABI entry points: argument validation, dispatch, error reporting.
// Declarations and the reference operator each one replaces: include/kch.h.

#include <cmath>
#include <cstdint>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/kch.h"
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

int hip_status(const char* fn, hipError_t e) {
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

int kch_kda_chunk_fwd(const void* q, const void* k, const void* v, const void* g,
                      const void* beta, const float* s0, void* o, float* s_out, int B, int T,
                      int H, int HV, int K, int V, float scale, float g_clamp_min, int dtype,
                      void* stream) {
  const char* fn = "kch_kda_chunk_fwd";
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
    if (s_out && B > 0) {
      const size_t n = (size_t)B * HV * K * V * sizeof(float);
      hipError_t e = s0 ? hipMemcpyAsync(s_out, s0, n, hipMemcpyDeviceToDevice, (hipStream_t)stream)
                        : hipMemsetAsync(s_out, 0, n, (hipStream_t)stream);
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
  kch::KdaParams p = make_kda(q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, scale, g_clamp_min);
  return hip_status(fn, kch::kda_chunk_dispatch(p, dtype, (hipStream_t)stream));
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
      const size_t n = (size_t)B * HV * K * V * sizeof(float);
      hipError_t e = s0 ? hipMemcpyAsync(s_out, s0, n, hipMemcpyDeviceToDevice, (hipStream_t)stream)
                        : hipMemsetAsync(s_out, 0, n, (hipStream_t)stream);
      return hip_status(fn, e);
    }
    return KCH_OK;
  }
  kch::KdaParams p = make_kda(q, k, v, g, beta, s0, o, s_out, B, T, H, HV, K, V, scale, g_clamp_min);
  return hip_status(fn, kch::kda_recurrent_dispatch(p, dtype, (hipStream_t)stream));
}

}  // extern "C"
