// Declarations shared by the backward translation units: the dK/dV pass's per-head view,
// the kernel templates (fa_bwd.hip defines the dQ kernels; the dK/dV kernels, batched and
// packed variable-length, exist only as the D = 64 and D = 128 specializations in
// fa_bwd_dkdv64.hip and fa_bwd_dkdv128.hip, hand-scheduled stage streams), the staged-tile
// helpers of those passes and the dynamic-LDS opt-in.
#pragma once

#include <atomic>

#include "fa_common.h"

namespace ttfa {

// One KV head's rows (k, v, dk, dv: T rows of D) for one sequence, and the G query heads
// that read it: query head g's q / dout rows at q + g * head_stride (elements), its lse /
// delta values at lse + g * row_stride.
struct DkvHead {
  const bf16 *k, *v;
  bf16 *dk, *dv;
  const bf16 *q, *dout;
  const float *lse, *delta;
  int64_t head_stride, row_stride;
  int G, T;
};

// LDS byte address of a pointer into the workgroup's shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const TTFA_LDS void *)p;
}

template <int D>
__global__ void fa_bwd_dq_bf16_kernel(const bf16 *__restrict__ Q, const bf16 *__restrict__ K,
                                      const bf16 *__restrict__ V, const bf16 *__restrict__ O,
                                      const bf16 *__restrict__ dO, const float *__restrict__ LSE,
                                      float *__restrict__ Delta, bf16 *__restrict__ dQ, int B,
                                      int Hq, int Hkv, int T, float scale_log2, float scale);
// D = 128 dQ pass over 256-row tiles, 64 rows per wave (fa_bwd_dq128.hip): for launches
// whose 256-row pairs fill the resident workgroup slots and whose T exceeds 1792.
__global__ void fa_bwd_dq_wide_bf16_kernel(const bf16 *__restrict__ Q, const bf16 *__restrict__ K,
                                           const bf16 *__restrict__ V, const bf16 *__restrict__ O,
                                           const bf16 *__restrict__ dO,
                                           const float *__restrict__ LSE, float *__restrict__ Delta,
                                           bf16 *__restrict__ dQ, int B, int Hq, int Hkv, int T,
                                           float scale_log2, float scale, int paired);
template <int D>
__global__ void fa_bwd_dkdv_bf16_kernel(const bf16 *__restrict__ Q, const bf16 *__restrict__ K,
                                        const bf16 *__restrict__ V, const bf16 *__restrict__ dO,
                                        const float *__restrict__ LSE,
                                        const float *__restrict__ Delta, bf16 *__restrict__ dK,
                                        bf16 *__restrict__ dV, int B, int Hq, int Hkv, int T,
                                        float scale_log2, float scale, int paired);
template <int D>
__global__ void fa_bwd_dkdv_varlen_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ LSE, const float *__restrict__ Delta,
    bf16 *__restrict__ dK, bf16 *__restrict__ dV, const int *__restrict__ cu_seqlens, int n_seq,
    int total, int max_seqlen, int Hq, int Hkv, float scale_log2, float scale);
template <>
__global__ void fa_bwd_dkdv_bf16_kernel<64>(const bf16 *__restrict__ Q, const bf16 *__restrict__ K,
                                            const bf16 *__restrict__ V, const bf16 *__restrict__ dO,
                                            const float *__restrict__ LSE,
                                            const float *__restrict__ Delta, bf16 *__restrict__ dK,
                                            bf16 *__restrict__ dV, int B, int Hq, int Hkv, int T,
                                            float scale_log2, float scale, int paired);
template <>
__global__ void fa_bwd_dkdv_bf16_kernel<128>(const bf16 *__restrict__ Q, const bf16 *__restrict__ K,
                                             const bf16 *__restrict__ V, const bf16 *__restrict__ dO,
                                             const float *__restrict__ LSE,
                                             const float *__restrict__ Delta, bf16 *__restrict__ dK,
                                             bf16 *__restrict__ dV, int B, int Hq, int Hkv, int T,
                                             float scale_log2, float scale, int paired);
template <>
__global__ void fa_bwd_dkdv_varlen_bf16_kernel<64>(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ LSE, const float *__restrict__ Delta,
    bf16 *__restrict__ dK, bf16 *__restrict__ dV, const int *__restrict__ cu_seqlens, int n_seq,
    int total, int max_seqlen, int Hq, int Hkv, float scale_log2, float scale);
template <>
__global__ void fa_bwd_dkdv_varlen_bf16_kernel<128>(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ LSE, const float *__restrict__ Delta,
    bf16 *__restrict__ dK, bf16 *__restrict__ dV, const int *__restrict__ cu_seqlens, int n_seq,
    int total, int max_seqlen, int Hq, int Hkv, float scale_log2, float scale);
// LDS bytes of the dK/dV passes (batched and packed varlen): two 128-row stages of Q and dO
// tiles plus their -LSE/scale and -Delta rows.
constexpr int kDkv64LdsBytes = 2 * (2 * 128 * 64 * 2 + 2 * 128 * 4);
constexpr int kDkv128LdsBytes = 2 * (2 * 128 * 128 * 2 + 2 * 128 * 4);
// D = 128 dQ pass: two 128-key stages of K and V tiles (workgroups of 256 query rows).
constexpr int kDq128LdsBytes = 2 * 2 * 128 * 128 * 2;

// Raises KERN's dynamic-LDS limit (needed above 64 KiB) once per device: later launches,
// including launches under stream capture, make no attribute call.
template <auto KERN>
static hipError_t allow_lds(size_t bytes) {
  static std::atomic<uint64_t> done{0};  // bit d: set on device d
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? uint64_t{1} << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(reinterpret_cast<const void *>(KERN),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_release);
  return e;
}

}  // namespace ttfa
