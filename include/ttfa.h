/*
 * ttfa.h -- C ABI of the MI355X (gfx950) causal GQA FlashAttention library
 * (libttfa.so, built from tinytrain_amd/csrc).
 *
 * The library replaces the launch layer of the reference's attention kernels
 * (XinqiWan412/tinytrain, kernels/flash_attn.py).  Every entry point takes plain
 * device pointers, sizes and a hipStream_t passed as void*; no torch types appear
 * in the signatures.  The caller owns all memory.  The library allocates nothing,
 * never synchronises the stream, keeps no state between calls and may be called
 * from several host threads at once; the one exception is ttfa_bwd_static, whose
 * Delta rows live in a static device array shared by its calls on a GPU.
 *
 * Layout contract (kernels/flash_attn.py:220-232, 246-258):
 *   q, o, dout, dq : [B, Hq,  T, D] contiguous, element type `dtype`
 *   k, v, dk, dv   : [B, Hkv, T, D] contiguous, element type `dtype`
 *   lse            : [B, Hq,  T]    contiguous fp32, natural-log logsumexp of the
 *                    scaled scores, lse = m + ln(l) (kernels/flash_attn.py:67)
 *   delta_ws       : [B, Hq,  T]    fp32 workspace, rowsum(O * dO)
 *                    (kernels/flash_attn.py:70-90, 255)
 * Causal mask always on; query head h reads KV head h / (Hq / Hkv)
 * (kernels/flash_attn.py:24, 227); the caller passes scale = 1/sqrt(D)
 * (kernels/flash_attn.py:237, 257).
 *
 * Supported: dtype TTFA_BF16 or TTFA_F32, D in {64, 128}, T >= 1, Hq % Hkv == 0,
 * all pointers non-null and 16-byte aligned.
 *
 * Return value: 0 on success; a negative TTFA_E* code when validation fails
 * (checked before any HIP call, so argument errors are testable without a GPU);
 * a positive hipError_t when a launch fails.  ttfa_strerror() names both kinds.
 */
#ifndef TTFA_H
#define TTFA_H

#ifdef __cplusplus
extern "C" {
#endif

#define TTFA_ABI_VERSION 6

enum ttfa_dtype { TTFA_BF16 = 0, TTFA_F32 = 1 };

enum ttfa_status {
  TTFA_OK = 0,
  TTFA_E_NULL = -1,        /* a required pointer is NULL                         */
  TTFA_E_HEAD_DIM = -2,    /* D is not 64 or 128                                 */
  TTFA_E_GROUP = -3,       /* Hq % Hkv != 0, or Hq < 1, Hkv < 1                  */
  TTFA_E_SEQ = -4,         /* T < 1, B < 1, or element counts overflow int64     */
  TTFA_E_ALIGN = -5,       /* a pointer is not 16-byte aligned                   */
  TTFA_E_DTYPE = -6,       /* dtype is not a ttfa_dtype                          */
  TTFA_E_SCALE = -7,       /* scale is not finite and positive                   */
  TTFA_E_EPS = -8,         /* eps is not in [0, 1)                               */
  TTFA_E_QROWS = -9,       /* decode: (Hq / Hkv) * Tq > 32                       */
  TTFA_E_SCRATCH = -10,    /* ttfa_bwd_static: B * Hq * T > TTFA_BWD_STATIC_MAX_ROWS */
};

/* Library ABI version (TTFA_ABI_VERSION of the build). No reference counterpart. */
int ttfa_abi_version(void);

/* Static description of a status code (negative: validation, positive: hipError_t).
 * No reference counterpart. */
const char *ttfa_strerror(int code);

/*
 * Which bf16 D = 128 kernels ttfa_fwd / ttfa_bwd run for a shape: *fwd_wide and
 * *dq_wide are set to 1 when the forward / the dQ pass use the 256-row kernels (64
 * query rows per wave), 0 when they use the 128-row ones.  The two differ by
 * rounding, and the choice is a rule on (B, Hq, T) alone, so a shape gives the same
 * bits on every device.  Makes no HIP call.  TTFA_E_SEQ for B, Hq or T < 1,
 * TTFA_E_NULL for a NULL output.  An introspection query for tests and profiling; no
 * reference counterpart.
 */
int ttfa_d128_wide(int B, int Hq, int T, int *fwd_wide, int *dq_wide);

/*
 * Forward: o = softmax(q k^T * scale, causal) v and lse, for every (b, hq).
 * Replaces _forward + fwd_kernel, kernels/flash_attn.py:220-243 and :12-67.
 */
int ttfa_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
             int B, int Hq, int Hkv, int T, int D, int dtype, float scale,
             void *hip_stream);

/*
 * Backward: dq, dk, dv from q, k, v, o, dout and the forward's lse.  Writes
 * delta_ws = rowsum(o * dout) first (it is recomputed on every call, never read
 * from a previous one).  dk/dv are reduced over the Hq/Hkv query heads of each KV
 * head inside one workgroup, without atomics, so results are bitwise reproducible.
 * Replaces _backward + bwd_preprocess + bwd_dkdv_kernel + bwd_dq_kernel,
 * kernels/flash_attn.py:246-277, :70-90, :93-159, :162-217.
 */
int ttfa_bwd(const void *q, const void *k, const void *v, const void *o,
             const void *dout, const float *lse, float *delta_ws, void *dq,
             void *dk, void *dv, int B, int Hq, int Hkv, int T, int D, int dtype,
             float scale, void *hip_stream);

/*
 * ttfa_bwd without the delta_ws argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Delta (rowsum(o * dout), B * Hq * T fp32 values) goes
 * to a library-owned static device array of TTFA_BWD_STATIC_MAX_ROWS floats (4 MiB), one
 * copy per GPU, held until the process ends; the call allocates nothing and frees nothing.
 * Same kernels, arguments and results (bitwise) as ttfa_bwd.
 *   - B * Hq * T > TTFA_BWD_STATIC_MAX_ROWS returns TTFA_E_SCRATCH (before any HIP call).
 *   - The first call on a device resolves the array's address there (hipGetSymbolAddress,
 *     cached per device); make that first call outside stream capture.
 *   - Every call writes all the Delta rows it reads, so no state carries over between
 *     calls, but calls that overlap in time on one GPU (several streams or host threads)
 *     share the array and race: serialise them.
 */
#define TTFA_BWD_STATIC_MAX_ROWS (1 << 20)

int ttfa_bwd_static(const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, void *dq, void *dk, void *dv,
                    int B, int Hq, int Hkv, int T, int D, int dtype, float scale,
                    void *hip_stream);

/*
 * The two launches ttfa_bwd is made of, exported separately so a caller (or a
 * profiler) can run or time each pass on its own.  ttfa_bwd == ttfa_bwd_dq then
 * ttfa_bwd_dkdv on the same stream, bitwise.  (For fp32, ttfa_bwd runs both passes as
 * one launch whose dK/dV workgroups form Delta themselves, with the same results.)
 *
 * ttfa_bwd_dq: writes delta_ws = rowsum(o * dout) and dq.
 *   Replaces bwd_preprocess + bwd_dq_kernel (kernels/flash_attn.py:70-90, :162-217)
 *   and their launches (:260-261, :271-275).
 * ttfa_bwd_dkdv: reads delta_ws (as written by ttfa_bwd_dq for the same o, dout)
 *   and writes dk, dv.
 *   Replaces bwd_dkdv_kernel (kernels/flash_attn.py:93-159) and its launch (:264-268).
 */
int ttfa_bwd_dq(const void *q, const void *k, const void *v, const void *o,
                const void *dout, const float *lse, float *delta_ws, void *dq,
                int B, int Hq, int Hkv, int T, int D, int dtype, float scale,
                void *hip_stream);

int ttfa_bwd_dkdv(const void *q, const void *k, const void *v, const void *dout,
                  const float *lse, const float *delta_ws, void *dk, void *dv,
                  int B, int Hq, int Hkv, int T, int D, int dtype, float scale,
                  void *hip_stream);

/*
 * Packed variable-length (cu_seqlens) causal attention, bf16 only.  Every sequence s
 * occupies rows cu_seqlens[s] .. cu_seqlens[s+1]-1 of each head and attends causally
 * within itself only (a block-diagonal causal mask).  No reference kernel has this; it is
 * the varlen item of the reference's roadmap (README.md:158) on the same kernels as
 * ttfa_fwd / ttfa_bwd.
 *
 *   q, o, dout, dq : [Hq,  total, D] bf16 contiguous (head-major, tokens packed)
 *   k, v, dk, dv   : [Hkv, total, D] bf16 contiguous
 *   lse, delta_ws  : [Hq,  total]    fp32
 *   cu_seqlens     : [n_seq + 1] int32 in device memory, 4-byte aligned, non-decreasing,
 *                    cu_seqlens[0] = 0, cu_seqlens[n_seq] = total, every length
 *                    <= max_seqlen.  A sequence with bounds outside 0..total or
 *                    decreasing is skipped (its rows are not written).  A sequence
 *                    longer than max_seqlen is processed as its first max_seqlen tokens,
 *                    the same way in the forward and in both backward passes: o, lse,
 *                    dq, dk and dv of those rows are exact (a causal row depends only on
 *                    earlier keys) and its rows from position max_seqlen on are not
 *                    written.
 * Validation as above, plus TTFA_E_DTYPE for anything but TTFA_BF16 and TTFA_E_SEQ
 * for n_seq, total or max_seqlen < 1.  Results for each sequence are bitwise those of
 * ttfa_fwd / ttfa_bwd on that sequence alone (B = 1, T = its length).
 */
int ttfa_varlen_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
                    const int *cu_seqlens, int n_seq, int total, int max_seqlen, int Hq, int Hkv,
                    int D, int dtype, float scale, void *hip_stream);

int ttfa_varlen_bwd(const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, float *delta_ws, void *dq, void *dk,
                    void *dv, const int *cu_seqlens, int n_seq, int total, int max_seqlen,
                    int Hq, int Hkv, int D, int dtype, float scale, void *hip_stream);

/*
 * KV-cache decode attention, bf16 only: Tq new query rows per (batch, query head)
 * against the first cache_seqlens[b] keys of a [B, Hkv, max_seqlen, D] cache.  Query
 * row i of batch b sits at position cache_seqlens[b] - Tq + i and sees cache keys
 * 0 .. cache_seqlens[b] - Tq + i (the new tokens' K/V are already in the cache): the
 * last Tq rows of the reference's causal attention (model.py:94-98).  No reference
 * kernel exists (generate.py:7-20 recomputes the prefix; README.md:158 plans a KV
 * cache).
 *
 *   q, o              : [B, Hq, Tq, D] bf16 contiguous
 *   k_cache, v_cache  : [B, Hkv, max_seqlen, D] bf16 contiguous
 *   cache_seqlens     : [B] int32 in device memory, 4-byte aligned; values are clamped
 *                       to 0 .. max_seqlen; a row that sees no key gets O = 0, LSE = -inf
 *   lse               : [B, Hq, Tq] fp32 out (natural log)
 *   workspace         : ttfa_decode_workspace_bytes(...) bytes, 16-byte aligned (fp32
 *                       per-split partials; overwritten)
 * Supported: D in {64, 128}, Hq % Hkv == 0, (Hq / Hkv) * Tq <= 32 (TTFA_E_QROWS),
 * B, Tq, max_seqlen >= 1.  Two launches on hip_stream (split pass, merge pass).
 */
long long ttfa_decode_workspace_bytes(int B, int Hq, int Hkv, int Tq, int max_seqlen, int D);

int ttfa_decode_fwd(const void *q, const void *k_cache, const void *v_cache,
                    const int *cache_seqlens, void *o, float *lse, float *workspace, int B,
                    int Hq, int Hkv, int Tq, int max_seqlen, int D, int dtype, float scale,
                    void *hip_stream);

/*
 * Fused attention prologue (bf16 only): q/k RMSNorm + rotate-half RoPE + the layout
 * change from the projections' [B, T, H, D] to the attention's [B, H, T, D].
 * Replaces model.py:83-93 of the reference (q_norm / k_norm, RMSNorm :24-35, the
 * transposes, apply_rope :48-56 with cos/sin rounded to bf16, and the .contiguous()
 * copies before the attention call); no kernel of the reference does this.
 *
 *   q_raw            : [B, T, Hq,  D] bf16 contiguous (q_proj output viewed per head)
 *   k_raw, v_raw     : [B, T, Hkv, D] bf16 contiguous
 *   q_norm_w, k_norm_w : [D] fp32 RMSNorm weights
 *   cos, sin         : [T, D] bf16, rows 0..T-1 of the RoPE tables (the reference's
 *                      fp32 tables rounded to bf16, as apply_rope does)
 *   q                : [B, Hq,  T, D] bf16 out;  k, v : [B, Hkv, T, D] bf16 out
 *   rstd_q, rstd_k   : [B, T, Hq] / [B, T, Hkv] fp32 out, 1/sqrt(mean(x^2)+eps) per
 *                      row (saved for the backward)
 * Supported: D in {64, 128}, B, T >= 1, Hq % Hkv == 0, eps in [0, 1), every pointer
 * non-null and 16-byte aligned.  Same status codes as above.
 */
int ttfa_qk_prologue_fwd(const void *q_raw, const void *k_raw, const void *v_raw,
                         const float *q_norm_w, const float *k_norm_w, const void *cos,
                         const void *sin, void *q, void *k, void *v, float *rstd_q,
                         float *rstd_k, int B, int T, int Hq, int Hkv, int D, float eps,
                         void *hip_stream);

/*
 * Bytes of fp32 workspace ttfa_qk_prologue_bwd needs for the given shape (per-
 * workgroup partial sums of the norm-weight gradients), or -1 for an invalid shape.
 */
long long ttfa_qk_prologue_workspace_bytes(int B, int T, int Hq, int Hkv, int D);

/*
 * Backward of ttfa_qk_prologue_fwd: dq [B, Hq, T, D], dk/dv [B, Hkv, T, D] (gradients
 * of its outputs) -> dq_raw, dk_raw, dv_raw in the input layouts, and the fp32 [D]
 * gradients of the two norm weights (overwritten, not accumulated).  Reads q_raw,
 * k_raw and the rstd rows the forward wrote.  The weight gradients are summed in a
 * fixed order (no atomics): results are bitwise reproducible.  Two launches on
 * hip_stream.
 */
int ttfa_qk_prologue_bwd(const void *dq, const void *dk, const void *dv, const void *q_raw,
                         const void *k_raw, const float *q_norm_w, const float *k_norm_w,
                         const void *cos, const void *sin, const float *rstd_q,
                         const float *rstd_k, void *dq_raw, void *dk_raw, void *dv_raw,
                         float *dq_norm_w, float *dk_norm_w, float *workspace, int B, int T,
                         int Hq, int Hkv, int D, void *hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* TTFA_H */
