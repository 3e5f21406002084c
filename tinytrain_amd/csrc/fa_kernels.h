// Host-side launchers of the attention kernels (one per kernel family and dtype).
// Arguments are validated by the C ABI layer (ttfa_api.hip) before these run.
#pragma once

#include <hip/hip_runtime.h>

namespace ttfa {

hipError_t launch_fwd_bf16(const void *q, const void *k, const void *v, void *o, float *lse,
                           int B, int Hq, int Hkv, int T, int D, float scale, hipStream_t stream);

// Which bf16 D = 128 kernels a shape runs: the 256-row forward / dQ pass (64 rows per wave)
// or the 128-row ones.  A fixed rule on the shape alone (never on the device's occupancy),
// so a shape's output bits are the same on every device: the wide kernels differ from the
// 128-row ones by rounding.
constexpr int kWideSlots = 256;  // one 256-row workgroup per CU on the 256 CUs of an MI355X
bool fwd128_uses_wide(int B, int Hq, int T);
bool dq128_uses_wide(int B, int Hq, int T);
hipError_t launch_bwd_dq_bf16(const void *q, const void *k, const void *v, const void *o,
                              const void *dout, const float *lse, float *delta, void *dq,
                              int B, int Hq, int Hkv, int T, int D, float scale,
                              hipStream_t stream);
hipError_t launch_bwd_dkdv_bf16(const void *q, const void *k, const void *v, const void *dout,
                                const float *lse, const float *delta, void *dk, void *dv,
                                int B, int Hq, int Hkv, int T, int D, float scale,
                                hipStream_t stream);

// Packed variable-length sequences, bf16: q/o [Hq, total, D], k/v [Hkv, total, D],
// lse/delta [Hq, total]; cu_seqlens [n_seq + 1] int32 on the device.
hipError_t launch_fwd_varlen_bf16(const void *q, const void *k, const void *v, void *o,
                                  float *lse, const int *cu_seqlens, int n_seq, int total,
                                  int max_seqlen, int Hq, int Hkv, int D, float scale,
                                  hipStream_t stream);
hipError_t launch_bwd_varlen_bf16(const void *q, const void *k, const void *v, const void *o,
                                  const void *dout, const float *lse, float *delta, void *dq,
                                  void *dk, void *dv, const int *cu_seqlens, int n_seq,
                                  int total, int max_seqlen, int Hq, int Hkv, int D, float scale,
                                  hipStream_t stream);

// KV-cache decode: q/o [B, Hq, Tq, D], caches [B, Hkv, Lmax, D], lse [B, Hq, Tq],
// cache_seqlens [B] int32 on the device; workspace of decode_workspace_floats() floats.
struct DecodeSplit {
  int wkeys;     // keys per wave (a multiple of 32)
  int n_chunks;  // workgroups per (batch, KV head)
  int n_splits;  // partials per query row (4 per workgroup)
};
DecodeSplit decode_split(int B, int Hkv, int Lmax);
hipError_t launch_decode_bf16(const void *q, const void *k_cache, const void *v_cache,
                              const int *cache_seqlens, void *o, float *lse, float *workspace,
                              int B, int Hq, int Hkv, int Tq, int Lmax, int D, float scale,
                              hipStream_t stream);

hipError_t launch_fwd_f32(const void *q, const void *k, const void *v, void *o, float *lse,
                          int B, int Hq, int Hkv, int T, int D, float scale, hipStream_t stream);
hipError_t launch_bwd_dq_f32(const void *q, const void *k, const void *v, const void *o,
                             const void *dout, const float *lse, float *delta, void *dq,
                             int B, int Hq, int Hkv, int T, int D, float scale,
                             hipStream_t stream);
hipError_t launch_bwd_dkdv_f32(const void *q, const void *k, const void *v, const void *dout,
                               const float *lse, const float *delta, void *dk, void *dv,
                               int B, int Hq, int Hkv, int T, int D, float scale,
                               hipStream_t stream);
// Both fp32 backward passes as one launch (same results, bitwise, as dq then dkdv).
hipError_t launch_bwd_f32(const void *q, const void *k, const void *v, const void *o,
                          const void *dout, const float *lse, float *delta, void *dq, void *dk,
                          void *dv, int B, int Hq, int Hkv, int T, int D, float scale,
                          hipStream_t stream);

}  // namespace ttfa
