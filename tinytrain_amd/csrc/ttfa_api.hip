// C ABI of libttfa.so: argument validation and dispatch (declarations in include/ttfa.h).
//
// Validation runs before any HIP call, so every argument error is reported without a
// GPU (and without touching the HIP runtime).  Launch failures come back as the
// positive hipError_t of hipGetLastError().
#include <math.h>
#include <stdint.h>

#include <atomic>

#include "ttfa.h"
#include "fa_kernels.h"

// Delta rows of ttfa_bwd_static: a file-scope device array, one copy per GPU the library
// runs on, held until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address): it passes the
// per-device address hipGetSymbolAddress returns (static_scratch_ptr below).
static __device__ __align__(256) float scratch[TTFA_BWD_STATIC_MAX_ROWS];

namespace {

int check_common(int B, int Hq, int Hkv, int T, int D, int dtype, float scale) {
  if (dtype != TTFA_BF16 && dtype != TTFA_F32) return TTFA_E_DTYPE;
  if (D != 64 && D != 128) return TTFA_E_HEAD_DIM;
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return TTFA_E_GROUP;
  if (B < 1 || T < 1) return TTFA_E_SEQ;
  // Per-head byte extents must fit the 32-bit buffer descriptors used by the kernels,
  // and total element counts must fit int64 with margin.
  const int64_t esz = dtype == TTFA_BF16 ? 2 : 4;
  if ((int64_t)T * D * esz > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  if ((int64_t)B * Hq > (int64_t)0x7fffffff / 4) return TTFA_E_SEQ;
  if ((int64_t)B * Hq * ((T + 127) / 128) > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  // fp32 grids: one workgroup per 16-row block of every query and KV head.
  if (dtype == TTFA_F32 && (int64_t)B * (Hq + Hkv) * ((T + 15) / 16) > (int64_t)0x7fffffff)
    return TTFA_E_SEQ;
  if (!(scale > 0.f) || !isfinite(scale)) return TTFA_E_SCALE;
  return TTFA_OK;
}

// Packed variable-length sequences: bf16 only; n_seq, total, max_seqlen >= 1; per-
// sequence byte extents within the 32-bit buffer descriptors; grids within int range.
int check_varlen(int n_seq, int total, int max_seqlen, int Hq, int Hkv, int D, int dtype,
                 float scale) {
  if (dtype != TTFA_BF16) return TTFA_E_DTYPE;
  if (D != 64 && D != 128) return TTFA_E_HEAD_DIM;
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return TTFA_E_GROUP;
  if (n_seq < 1 || total < 1 || max_seqlen < 1) return TTFA_E_SEQ;
  if ((int64_t)max_seqlen * D * 2 > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  if ((int64_t)((max_seqlen + 127) / 128) * n_seq * Hq > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  if ((int64_t)Hq * total > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  if (!(scale > 0.f) || !isfinite(scale)) return TTFA_E_SCALE;
  return TTFA_OK;
}

// KV-cache decode: bf16; G * Tq query columns fit one 32-wide MFMA tile; cache byte
// extents within the 32-bit buffer descriptors.
int check_decode(int B, int Hq, int Hkv, int Tq, int Lmax, int D, int dtype, float scale) {
  if (dtype != TTFA_BF16) return TTFA_E_DTYPE;
  if (D != 64 && D != 128) return TTFA_E_HEAD_DIM;
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return TTFA_E_GROUP;
  if (B < 1 || Tq < 1 || Lmax < 1) return TTFA_E_SEQ;
  if ((int64_t)(Hq / Hkv) * Tq > 32) return TTFA_E_QROWS;
  if ((int64_t)Lmax * D * 2 > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  if ((int64_t)B * Hq * Tq > (int64_t)0x7fffffff / 4) return TTFA_E_SEQ;
  if (!(scale > 0.f) || !isfinite(scale)) return TTFA_E_SCALE;
  return TTFA_OK;
}

// Device address of `scratch` on the current device, resolved once per device (the first
// ttfa_bwd_static call on it) and cached; *out stays null on failure.
hipError_t static_scratch_ptr(float **out) {
  static std::atomic<uintptr_t> addr[64];  // by device ordinal, 0 = not resolved yet
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  uintptr_t a = addr[dev].load(std::memory_order_acquire);
  if (a == 0) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    a = reinterpret_cast<uintptr_t>(ptr);
    addr[dev].store(a, std::memory_order_release);
  }
  *out = reinterpret_cast<float *>(a);
  return hipSuccess;
}

int check_ptrs(const void *const *ptrs, int n) {
  for (int i = 0; i < n; ++i)
    if (ptrs[i] == nullptr) return TTFA_E_NULL;
  for (int i = 0; i < n; ++i)
    if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15u) return TTFA_E_ALIGN;
  return TTFA_OK;
}

}  // namespace

extern "C" {

int ttfa_abi_version(void) { return TTFA_ABI_VERSION; }

int ttfa_d128_wide(int B, int Hq, int T, int *fwd_wide, int *dq_wide) {
  if (!fwd_wide || !dq_wide) return TTFA_E_NULL;
  if (B < 1 || Hq < 1 || T < 1) return TTFA_E_SEQ;
  *fwd_wide = ttfa::fwd128_uses_wide(B, Hq, T) ? 1 : 0;
  *dq_wide = ttfa::dq128_uses_wide(B, Hq, T) ? 1 : 0;
  return TTFA_OK;
}

const char *ttfa_strerror(int code) {
  switch (code) {
    case TTFA_OK: return "success";
    case TTFA_E_NULL: return "ttfa: a required pointer is NULL";
    case TTFA_E_HEAD_DIM: return "ttfa: head dim D must be 64 or 128";
    case TTFA_E_GROUP: return "ttfa: Hq must be a positive multiple of Hkv";
    case TTFA_E_SEQ: return "ttfa: B and T must be >= 1 and sizes must fit the kernels' index range";
    case TTFA_E_ALIGN: return "ttfa: every pointer must be 16-byte aligned";
    case TTFA_E_DTYPE: return "ttfa: dtype must be TTFA_BF16 or TTFA_F32";
    case TTFA_E_SCALE: return "ttfa: scale must be finite and > 0";
    case TTFA_E_EPS: return "ttfa: eps must be in [0, 1)";
    case TTFA_E_QROWS: return "ttfa: decode needs (Hq / Hkv) * Tq <= 32 query rows per KV head";
    case TTFA_E_SCRATCH:
      return "ttfa: ttfa_bwd_static needs B * Hq * T <= TTFA_BWD_STATIC_MAX_ROWS (1048576)";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "ttfa: unknown status code";
}

int ttfa_fwd(const void *q, const void *k, const void *v, void *o, float *lse, int B, int Hq,
             int Hkv, int T, int D, int dtype, float scale, void *hip_stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k, v, o, lse};
  if ((rc = check_ptrs(ptrs, 5))) return rc;
  hipStream_t s = static_cast<hipStream_t>(hip_stream);
  hipError_t e = dtype == TTFA_BF16
                     ? ttfa::launch_fwd_bf16(q, k, v, o, lse, B, Hq, Hkv, T, D, scale, s)
                     : ttfa::launch_fwd_f32(q, k, v, o, lse, B, Hq, Hkv, T, D, scale, s);
  return static_cast<int>(e);
}

int ttfa_bwd_dq(const void *q, const void *k, const void *v, const void *o, const void *dout,
                const float *lse, float *delta_ws, void *dq, int B, int Hq, int Hkv, int T,
                int D, int dtype, float scale, void *hip_stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k, v, o, dout, lse, delta_ws, dq};
  if ((rc = check_ptrs(ptrs, 8))) return rc;
  hipStream_t s = static_cast<hipStream_t>(hip_stream);
  hipError_t e =
      dtype == TTFA_BF16
          ? ttfa::launch_bwd_dq_bf16(q, k, v, o, dout, lse, delta_ws, dq, B, Hq, Hkv, T, D, scale, s)
          : ttfa::launch_bwd_dq_f32(q, k, v, o, dout, lse, delta_ws, dq, B, Hq, Hkv, T, D, scale, s);
  return static_cast<int>(e);
}

int ttfa_bwd_dkdv(const void *q, const void *k, const void *v, const void *dout,
                  const float *lse, const float *delta_ws, void *dk, void *dv, int B, int Hq,
                  int Hkv, int T, int D, int dtype, float scale, void *hip_stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k, v, dout, lse, delta_ws, dk, dv};
  if ((rc = check_ptrs(ptrs, 8))) return rc;
  hipStream_t s = static_cast<hipStream_t>(hip_stream);
  hipError_t e =
      dtype == TTFA_BF16
          ? ttfa::launch_bwd_dkdv_bf16(q, k, v, dout, lse, delta_ws, dk, dv, B, Hq, Hkv, T, D, scale, s)
          : ttfa::launch_bwd_dkdv_f32(q, k, v, dout, lse, delta_ws, dk, dv, B, Hq, Hkv, T, D, scale, s);
  return static_cast<int>(e);
}

int ttfa_varlen_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                    const int *cu_seqlens, int n_seq, int total, int max_seqlen, int Hq, int Hkv,
                    int D, int dtype, float scale, void *hip_stream) {
  int rc = check_varlen(n_seq, total, max_seqlen, Hq, Hkv, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k, v, o, lse};
  if ((rc = check_ptrs(ptrs, 5))) return rc;
  if (cu_seqlens == nullptr) return TTFA_E_NULL;
  if (reinterpret_cast<uintptr_t>(cu_seqlens) & 3u) return TTFA_E_ALIGN;
  return static_cast<int>(ttfa::launch_fwd_varlen_bf16(q, k, v, o, lse, cu_seqlens, n_seq, total,
                                                       max_seqlen, Hq, Hkv, D, scale,
                                                       static_cast<hipStream_t>(hip_stream)));
}

int ttfa_varlen_bwd(const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, float *delta_ws, void *dq, void *dk,
                    void *dv, const int *cu_seqlens, int n_seq, int total, int max_seqlen,
                    int Hq, int Hkv, int D, int dtype, float scale, void *hip_stream) {
  int rc = check_varlen(n_seq, total, max_seqlen, Hq, Hkv, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k, v, o, dout, lse, delta_ws, dq, dk, dv};
  if ((rc = check_ptrs(ptrs, 10))) return rc;
  if (cu_seqlens == nullptr) return TTFA_E_NULL;
  if (reinterpret_cast<uintptr_t>(cu_seqlens) & 3u) return TTFA_E_ALIGN;
  return static_cast<int>(ttfa::launch_bwd_varlen_bf16(
      q, k, v, o, dout, lse, delta_ws, dq, dk, dv, cu_seqlens, n_seq, total, max_seqlen, Hq, Hkv,
      D, scale, static_cast<hipStream_t>(hip_stream)));
}

long long ttfa_decode_workspace_bytes(int B, int Hq, int Hkv, int Tq, int max_seqlen, int D) {
  if (check_decode(B, Hq, Hkv, Tq, max_seqlen, D, TTFA_BF16, 1.f)) return -1;
  const ttfa::DecodeSplit sp = ttfa::decode_split(B, Hkv, max_seqlen);
  return (long long)B * Hq * Tq * sp.n_splits * (D + 2) * (long long)sizeof(float);
}

int ttfa_decode_fwd(const void *q, const void *k_cache, const void *v_cache,
                    const int *cache_seqlens, void *o, float *lse, float *workspace, int B,
                    int Hq, int Hkv, int Tq, int max_seqlen, int D, int dtype, float scale,
                    void *hip_stream) {
  int rc = check_decode(B, Hq, Hkv, Tq, max_seqlen, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k_cache, v_cache, o, lse, workspace};
  if ((rc = check_ptrs(ptrs, 6))) return rc;
  if (cache_seqlens == nullptr) return TTFA_E_NULL;
  if (reinterpret_cast<uintptr_t>(cache_seqlens) & 3u) return TTFA_E_ALIGN;
  return static_cast<int>(ttfa::launch_decode_bf16(q, k_cache, v_cache, cache_seqlens, o, lse,
                                                   workspace, B, Hq, Hkv, Tq, max_seqlen, D,
                                                   scale, static_cast<hipStream_t>(hip_stream)));
}

int ttfa_bwd(const void *q, const void *k, const void *v, const void *o, const void *dout,
             const float *lse, float *delta_ws, void *dq, void *dk, void *dv, int B, int Hq,
             int Hkv, int T, int D, int dtype, float scale, void *hip_stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, scale);
  if (rc) return rc;
  const void *ptrs[] = {q, k, v, o, dout, lse, delta_ws, dq, dk, dv};
  if ((rc = check_ptrs(ptrs, 10))) return rc;
  if (dtype == TTFA_F32)
    return static_cast<int>(ttfa::launch_bwd_f32(q, k, v, o, dout, lse, delta_ws, dq, dk, dv, B,
                                                 Hq, Hkv, T, D, scale,
                                                 static_cast<hipStream_t>(hip_stream)));
  rc = ttfa_bwd_dq(q, k, v, o, dout, lse, delta_ws, dq, B, Hq, Hkv, T, D, dtype, scale, hip_stream);
  if (rc) return rc;
  return ttfa_bwd_dkdv(q, k, v, dout, lse, delta_ws, dk, dv, B, Hq, Hkv, T, D, dtype, scale,
                       hip_stream);
}

int ttfa_bwd_static(const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, void *dq, void *dk, void *dv, int B,
                    int Hq, int Hkv, int T, int D, int dtype, float scale, void *hip_stream) {
  int rc = check_common(B, Hq, Hkv, T, D, dtype, scale);
  if (rc) return rc;
  if ((int64_t)B * Hq * T > TTFA_BWD_STATIC_MAX_ROWS) return TTFA_E_SCRATCH;
  const void *ptrs[] = {q, k, v, o, dout, lse, dq, dk, dv};
  if ((rc = check_ptrs(ptrs, 9))) return rc;
  float *delta = nullptr;
  hipError_t e = static_scratch_ptr(&delta);
  if (e != hipSuccess) return static_cast<int>(e);
  // Every call writes all B * Hq * T rows of Delta (dQ pass) before the dK/dV pass reads
  // them, so nothing left by an earlier call is ever read and nothing needs clearing.
  return ttfa_bwd(q, k, v, o, dout, lse, delta, dq, dk, dv, B, Hq, Hkv, T, D, dtype, scale,
                  hip_stream);
}

}  // extern "C"
