// Causal GQA FlashAttention backward, bf16 in / fp32 accumulate, gfx950.
//
// Two passes, both recomputing P from the forward's LSE (kernels/flash_attn.py:143-145,
// :208-209) instead of storing it:
//
//  1. dQ pass (reference: bwd_preprocess :70-90 fused with bwd_dq_kernel :162-217).
//     A row tile = 128 query rows of one (batch, head), 4 waves x 32 rows.  A workgroup
//     takes one row tile, longest first (single_item), so the row body is inlined once
//     (three workgroups per CU fit without spills at D = 64).  Key tiles run from the row
//     tile's diagonal down to key 0.  (Long sequences at D = 128 take the 256-row pass of
//     fa_bwd_dq128.hip.)
//     The prologue computes Delta = rowsum(O * dO) for the tile's own rows from the
//     same registers that hold dO, and writes it to the workspace
//     for pass 2 (so there is no separate preprocess launch and dO is read once here).
//     Per key tile from LDS (64 keys for D=64, 32 for D=128), one 32-key block at a time:
//     S^T = K Q^T and
//     dP^T - Delta = V dO^T - Delta (the dP accumulator starts at -Delta, a per-lane
//     constant, so dS costs one multiply), P^T = exp2(S^T*scale*log2e - LSE*log2e),
//     dS^T = P^T (dP^T - Delta), dQ^T += K^T dS^T with K^T read by ds_read_b64_tr_b16.
//     Every lane owns one query row, so LSE and Delta are per-lane scalars.
//
//  2. dK/dV pass (reference: bwd_dkdv_kernel :93-159): fa_bwd_dkdv64.hip and
//     fa_bwd_dkdv128.hip, whose per-stage work is a generated instruction stream; this
//     file holds their launchers.  A key tile = 128 keys of one (batch, kv head), 4 waves
//     x 32 keys, walking the G query heads of its group and their 128-row Q/dO stages from
//     the diagonal to the end; dK and dV accumulate in registers across the whole group,
//     so the group reduction needs no atomics and the result is bitwise deterministic
//     (reference loop :125-152).
//
// Both passes fill their LDS tiles with buffer_load ... lds (global -> LDS, 16 bytes per
// lane, no staging VGPRs), the next tile's loads in flight while the current tile is
// computed.  Tiles entirely above the diagonal are skipped; only tiles crossing the
// diagonal or the ragged end of T run the masked body.
#include "fa_bwd.h"
#include "fa_common.h"
#include "fa_kernels.h"

namespace ttfa {

namespace {

// The K/V tiles of the dQ pass use layout 1 (conflict-free row reads).
constexpr int kDqLayout = 1;

template <int D>
struct DqTile {
  static constexpr int BM = 128;                 // query rows per workgroup
  static constexpr int BN = D == 64 ? 64 : 32;   // keys per LDS tile
  static constexpr int KB = BN / 32;             // 32-key blocks per tile
  static constexpr int KK = D / 16, DB = D / 32, CH = D / 8;
  static constexpr int LOADS = BN * CH / 256;    // 16-byte loads per thread per K (or V) tile
  // [stage][K|V] bf16; at D = 64 then the row tile's dO (its Q shares stage 1 in the
  // prologue), so both arrive as coalesced direct-to-LDS loads (dq_rows)
  static constexpr int LDS_BYTES = 2 * 2 * BN * D * 2 + (D == 64 ? BM * D * 2 : 0);
};

// One key tile of the dQ pass for one wave, one 32-key block at a time.
template <int D, bool MASK>
__device__ __forceinline__ void dq_tile(const bf16 *Kt, const bf16 *Vt, const bf16x8 (&qf)[D / 16],
                                        const bf16x8 (&dof)[D / 16], const f32x16 &ndelta,
                                        f32x16 (&dqacc)[D / 32], float lse_t, float scale_log2,
                                        int k0, int qrow, int T, int lane) {
  using P = DqTile<D>;
  const int lq = lane & 31, lg = lane >> 5;
#pragma unroll
  for (int kb = 0; kb < P::KB; ++kb) {
    // Inside T, a 32-key block after every row of the wave contributes nothing
    // (wave-uniform: the wave's rows start at qrow - lq).
    if (MASK && k0 + P::BN <= T && k0 + 32 * kb > qrow - lq + 31) continue;
    f32x16 s, dp;
    {
      bf16x8 kf[P::KK], vf[P::KK];
#pragma unroll
      for (int kk = 0; kk < P::KK; ++kk) {
        kf[kk] = lds_read_row8<D, kDqLayout>(Kt, kb * 32 + lq, 2 * kk + lg);
        vf[kk] = lds_read_row8<D, kDqLayout>(Vt, kb * 32 + lq, 2 * kk + lg);
      }
      s = mfma32(kf[0], qf[0], f32x16{});
      dp = mfma32(vf[0], dof[0], ndelta);
#pragma unroll
      for (int kk = 1; kk < P::KK; ++kk) {
        s = mfma32(kf[kk], qf[kk], s);
        dp = mfma32(vf[kk], dof[kk], dp);
      }
    }
    if (MASK) {
      const int kbase = k0 + 32 * kb;
      if (k0 + P::BN <= T) {
        const int rel = kbase - (qrow - lq), dl = lq - 4 * lg;
        if (rel > 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) s[r] = -INFINITY;
        } else if (rel == 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) > dl) s[r] = -INFINITY;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kbase + 8 * (r >> 2) + 4 * lg + (r & 3);
          if (key > qrow || key >= T) s[r] = -INFINITY;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r)  // dS^T = P^T (dP^T - Delta); -inf scores give P = 0
      s[r] = exp2f_fast(__builtin_fmaf(s[r], scale_log2, -lse_t)) * dp[r];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const bf16x8 dsb = pack8(s, 8 * m);
      bf16x8 kt[P::DB];
#pragma unroll
      for (int db = 0; db < P::DB; ++db) kt[db] = lds_read_trT<D, kDqLayout>(Kt, 32 * kb + 16 * m, 32 * db, lane);
#pragma unroll
      for (int db = 0; db < P::DB; ++db) dqacc[db] = mfma32(kt[db], dsb, dqacc[db]);
    }
  }
}

}  // namespace

// ---------------------------------------------------------------- pass 1: Delta + dQ
// One query head's rows (q, o, dout, dq: T rows of D; lse, delta: T values) and its KV
// head's rows (k, v) for one sequence.
struct DqHead {
  const bf16 *q, *k, *v, *o, *dout;
  const float *lse;
  float *delta;
  bf16 *dq;
  int T;
};

// Delta and dQ for the 128 query rows of row tile qt of one head.  Ends with a
// workgroup barrier, so the caller may reuse the LDS ring right away.
template <int D>
__device__ __forceinline__ void dq_rows(bf16 *lds, const DqHead &hd, int qt, float scale_log2,
                                        float scale) {
  using P = DqTile<D>;
  constexpr int BM = P::BM, BN = P::BN, KK = P::KK, DB = P::DB, CH = P::CH, LOADS = P::LOADS;
  const int T = hd.T;

  // An opaque copy of the thread id: values derived from it are computed once and kept,
  // not rematerialised from threadIdx; without it the compiler's allocation of the D = 64
  // kernels spills (8 bytes of scratch; the asm contract test checks for spills).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int q0 = qt * BM + wave * 32;
  const int qrow = q0 + lq;

  const uint32_t head_bytes = (uint32_t)T * D * 2;
  const auto rq = make_rsrc(hd.q, head_bytes);
  const auto ro = make_rsrc(hd.o, head_bytes);
  const auto rdo = make_rsrc(hd.dout, head_bytes);

  // Global -> LDS without registers: lane l of the wave's 1 KB block e0 writes physical
  // chunk (e0 + l) % CH of row (e0 + l) / CH, which holds logical chunk phys ^ swizzle(row).
  // The lane's offset within a tile is fixed; the descriptors are re-based at the tile
  // (scalar work; rows past T still read as zero) and the LDS destinations (M0) come
  // from the scalar wave index.
  const int wave_s = wave_id();
  uint32_t voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int e = 256 * i + 64 * wave + lane, row = e / CH, pc = e % CH;
    voff[i] = (uint32_t)(row * D + swz_l<D, kDqLayout>(row, pc) * 8) * 2;
  }
  auto load_tile = [&](int j, int stage) {
    bf16 *Kt = lds + stage * 2 * BN * D, *Vt = Kt + BN * D;
    const int64_t t0 = (int64_t)j * BN * D;
    const uint32_t left = head_bytes - (uint32_t)t0 * 2;
    const auto rkj = make_rsrc(hd.k + t0, left), rvj = make_rsrc(hd.v + t0, left);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e0 = 256 * i + 64 * wave_s;
      buf_load16_lds(rkj, voff[i], Kt + e0 * 8);
      buf_load16_lds(rvj, voff[i], Vt + e0 * 8);
    }
  };

  // Key tiles run from the diagonal down to key 0.  The row tiles of one head that run
  // at the same time (longest first) then read each K/V tile within a few tiles' time of
  // each other, and a later, shorter row tile of the head starts on tiles the longer
  // ones read recently, so K/V mostly come from L2 (in key order it would restart at
  // key 0, read long before).  The first tile is in flight while this wave's rows load
  // and Delta is formed: both wait on one memory round trip.
  const int n_kv = min((T + BN - 1) / BN, (qt + 1) * (BM / BN));
  load_tile(n_kv - 1, 0);
  bf16x8 qf[KK], dof[KK];
  float dpart = 0.f;
  if constexpr (D == 64) {
    // The row tile's Q and dO go to LDS (stage 1 of the ring, free until the loop's first
    // prefetch, and the 16 KB after the ring) in the coalesced direct-to-LDS form, beside
    // the first K/V tile in stage 0; O stays a register load (it only feeds Delta).
    const uint32_t qbytes = head_bytes - (uint32_t)(qt * BM * D * 2);
    const auto rqt = make_rsrc(hd.q + (int64_t)qt * BM * D, qbytes);
    const auto rdot = make_rsrc(hd.dout + (int64_t)qt * BM * D, qbytes);
    bf16 *Qs = lds + 2 * BN * D, *dOs = lds + 4 * BN * D;
#pragma unroll
    for (int i = 0; i < BM * CH / 256; ++i) {
      const int e = 256 * i + 64 * wave + lane, row = e / CH, pc = e % CH;
      const uint32_t off = (uint32_t)(row * D + swz_l<D, kDqLayout>(row, pc) * 8) * 2;
      buf_load16_lds(rqt, off, Qs + (256 * i + 64 * wave_s) * 8);
      buf_load16_lds(rdot, off, dOs + (256 * i + 64 * wave_s) * 8);
    }
    bf16x8 of[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      of[kk] = __builtin_bit_cast(bf16x8, buf_load16(ro, (uint32_t)(qrow * D + 16 * kk + 8 * lg) * 2));
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qf[kk] = lds_read_row8<D, kDqLayout>(Qs, wave * 32 + lq, 2 * kk + lg);
      dof[kk] = lds_read_row8<D, kDqLayout>(dOs, wave * 32 + lq, 2 * kk + lg);
#pragma unroll
      for (int s = 0; s < 8; ++s) dpart = __builtin_fmaf(bf2f(of[kk][s]), bf2f(dof[kk][s]), dpart);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's Q / dO reads are complete
    __syncthreads();                     // ... in every wave, before stage 1 is refilled
  } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const uint32_t off = (uint32_t)(qrow * D + 16 * kk + 8 * lg) * 2;
      qf[kk] = __builtin_bit_cast(bf16x8, buf_load16(rq, off));
      dof[kk] = __builtin_bit_cast(bf16x8, buf_load16(rdo, off));
      const bf16x8 of = __builtin_bit_cast(bf16x8, buf_load16(ro, off));
#pragma unroll
      for (int s = 0; s < 8; ++s) dpart = __builtin_fmaf(bf2f(of[s]), bf2f(dof[kk][s]), dpart);
    }
  }
  const float delta = xhalf_sum(dpart);
  float lse_t = 0.f;
  if (qrow < T) {
    lse_t = hd.lse[qrow] * kLog2e;
    if (lg == 0) hd.delta[qrow] = delta;
  }
  f32x16 ndelta;
#pragma unroll
  for (int r = 0; r < 16; ++r) ndelta[r] = -delta;

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no register load is pending in the loop
  __syncthreads();

  const int n_full = min((q0 + 1) / BN, T / BN);
  const int n_vis = min(n_kv, (q0 + 31) / BN + 1);

  f32x16 dqacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqacc[db] = f32x16{};

  // No issue-priority steering here (the forward uses it): measured, it slowed both
  // backward passes.
  for (int jj = 0; jj < n_kv; ++jj) {
    const int j = n_kv - 1 - jj;
    if (j > 0) load_tile(j - 1, (jj + 1) & 1);
    const bf16 *Kt = lds + (jj & 1) * 2 * BN * D, *Vt = Kt + BN * D;
    if (j < n_full)
      dq_tile<D, false>(Kt, Vt, qf, dof, ndelta, dqacc, lse_t, scale_log2, j * BN, qrow, T, lane);
    else if (j < n_vis)
      dq_tile<D, true>(Kt, Vt, qf, dof, ndelta, dqacc, lse_t, scale_log2, j * BN, qrow, T, lane);
    wait_vm_all();  // tile j+1 is in LDS before any wave passes the barrier
    __syncthreads();
  }

  // The loop's last barrier freed the LDS ring: each wave stages its dQ tile in its own
  // 32*D slice of it for row-contiguous stores.
  store_rows<D>(dqacc, scale, lds + wave * 32 * D, hd.dq, q0, T, lane);
  __syncthreads();  // the ring is free again for the caller
}

template <int D>
// D = 64: three workgroups per CU (at most 168 VGPRs).
__global__ __launch_bounds__(256, (D == 64 ? 3 : 2)) void fa_bwd_dq_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ O, const bf16 *__restrict__ dO, const float *__restrict__ LSE,
    float *__restrict__ Delta, bf16 *__restrict__ dQ, int B, int Hq, int Hkv, int T,
    float scale_log2, float scale) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];  // [stage 2][K|V][BN*D]
  using P = DqTile<D>;
  const int n_tiles = (T + P::BM - 1) / P::BM;
  // One row tile per workgroup, longest first.  Pairs of row tiles (the forward's
  // schedule) would need a second inlined copy of the row body, which at D = 64 does not
  // fit three workgroups per CU without spills; at D = 128 (two per CU) longest-first
  // single tiles measured 0-4% faster than pairs at T = 500-1536.
  const WorkPair w = single_item(blockIdx.x, n_tiles, B, Hq, Hq / Hkv, false);
  const int G = Hq / Hkv;
  const int b = w.bh / Hq, h = w.bh - b * Hq;
  const int64_t kvh = (int64_t)b * Hkv + h / G, hs = (int64_t)T * D, qb = w.bh * hs;
  const DqHead hd{Q + qb, K + kvh * hs, V + kvh * hs, O + qb, dO + qb,
                  LSE + (int64_t)w.bh * T, Delta + (int64_t)w.bh * T, dQ + qb, T};
  dq_rows<D>(smem, hd, w.first, scale_log2, scale);
}

// Packed variable-length sequences ([H, total, D], sequence s at rows cu_seqlens[s] ..
// cu_seqlens[s+1]-1 of every head; LSE / Delta [H, total]).  Workgroup -> (tile rank,
// sequence, query head), rank-major, longest row tiles first; invalid sequence bounds
// are skipped.
template <int D>
__global__ __launch_bounds__(256, (D == 64 ? 3 : 2)) void fa_bwd_dq_varlen_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ O, const bf16 *__restrict__ dO, const float *__restrict__ LSE,
    float *__restrict__ Delta, bf16 *__restrict__ dQ, const int *__restrict__ cu_seqlens,
    int n_seq, int total, int max_seqlen, int Hq, int Hkv, float scale_log2, float scale) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];
  using P = DqTile<D>;
  const int per_rank = n_seq * Hq;
  const int rank = blockIdx.x / per_rank, rem = blockIdx.x - rank * per_rank;
  const int s = rem / Hq, h = rem - s * Hq;
  const int c0 = cu_seqlens[s], c1 = cu_seqlens[s + 1];
  if (c0 < 0 || c1 < c0 || c1 > total) return;
  const int T = min(c1 - c0, max_seqlen);  // the forward's clamp
  const int n_tiles = (T + P::BM - 1) / P::BM;
  if (rank >= n_tiles) return;
  const int qt = n_tiles - 1 - rank;
  const int hk = h / (Hq / Hkv);
  const int64_t qb = ((int64_t)h * total + c0) * D, kb = ((int64_t)hk * total + c0) * D;
  const int64_t rb = (int64_t)h * total + c0;
  const DqHead hd{Q + qb, K + kb, V + kb, O + qb, dO + qb, LSE + rb, Delta + rb, dQ + qb, T};
  dq_rows<D>(smem, hd, qt, scale_log2, scale);
}

// ---------------------------------------------------------------- pass 2: dK, dV
// The batched and the packed variable-length dK/dV kernels at both head dims are the
// generated stage streams of fa_bwd_dkdv64.hip and fa_bwd_dkdv128.hip (explicit
// specializations declared in fa_bwd.h); their launchers are below.

// 256-row tiles, 64 rows per wave (fa_bwd_dq128.hip): half the LDS and L2 bytes per
// product, but half the workgroups and a longer prologue per workgroup, so only where its
// pairs fill the 256 resident slots of an MI355X and carry at least 18 key stages each
// (T > 1792; measured slower at T = 512 and 1024, faster from T = 2000 up).
bool dq128_uses_wide(int B, int Hq, int T) {
  const int n_wide = (T + 255) / 256;
  return n_wide >= 8 && (int64_t)sched_items(true, n_wide, B, Hq) >= kWideSlots;
}

template <int D>
static hipError_t launch_dq(const void *q, const void *k, const void *v, const void *o,
                            const void *dout, const float *lse, float *delta, void *dq, int B,
                            int Hq, int Hkv, int T, float scale, hipStream_t stream) {
  if constexpr (D == 128) {
    if (dq128_uses_wide(B, Hq, T)) {
      const int n_wide = (T + 255) / 256;
      hipError_t e = allow_lds<fa_bwd_dq_wide_bf16_kernel>(kDq128LdsBytes);  // before the
      if (e != hipSuccess) return e;  // occupancy query, which sees the raised limit
      const int slots = resident_slots<fa_bwd_dq_wide_bf16_kernel>(256, kDq128LdsBytes);
      const bool paired = use_pairs(n_wide, B, Hq, slots);
      const dim3 grid((unsigned)sched_items(paired, n_wide, B, Hq)), block(256);
      fa_bwd_dq_wide_bf16_kernel<<<grid, block, kDq128LdsBytes, stream>>>(
          (const bf16 *)q, (const bf16 *)k, (const bf16 *)v, (const bf16 *)o, (const bf16 *)dout,
          lse, delta, (bf16 *)dq, B, Hq, Hkv, T, scale * kLog2e, scale, (int)paired);
      return hipGetLastError();
    }
  }
  const int n_tiles = (T + DqTile<D>::BM - 1) / DqTile<D>::BM;
  constexpr size_t lds = DqTile<D>::LDS_BYTES;
  auto kern = fa_bwd_dq_bf16_kernel<D>;
  if (lds > 65536) {
    hipError_t e = allow_lds<fa_bwd_dq_bf16_kernel<D>>(lds);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((unsigned)sched_items(false, n_tiles, B, Hq)), block(256);
  kern<<<grid, block, lds, stream>>>((const bf16 *)q, (const bf16 *)k, (const bf16 *)v,
                                     (const bf16 *)o, (const bf16 *)dout, lse, delta, (bf16 *)dq,
                                     B, Hq, Hkv, T, scale * kLog2e, scale);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_dkdv(const void *q, const void *k, const void *v, const void *dout,
                              const float *lse, const float *delta, void *dk, void *dv, int B,
                              int Hq, int Hkv, int T, float scale, hipStream_t stream) {
  const int n_ktiles = (T + 127) / 128;  // 128-key tiles
  constexpr size_t lds = D == 64 ? kDkv64LdsBytes : kDkv128LdsBytes;
  auto kern = fa_bwd_dkdv_bf16_kernel<D>;
  if (lds > 65536) {
    hipError_t e = allow_lds<fa_bwd_dkdv_bf16_kernel<D>>(lds);
    if (e != hipSuccess) return e;
  }
  const bool paired =
      use_pairs(n_ktiles, B, Hkv, resident_slots<fa_bwd_dkdv_bf16_kernel<D>>(256, lds));
  const dim3 grid((unsigned)sched_items(paired, n_ktiles, B, Hkv)), block(256);
  kern<<<grid, block, lds, stream>>>((const bf16 *)q, (const bf16 *)k, (const bf16 *)v,
                                     (const bf16 *)dout, lse, delta, (bf16 *)dk, (bf16 *)dv, B,
                                     Hq, Hkv, T, scale * kLog2e, scale, (int)paired);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_dq_varlen(const void *q, const void *k, const void *v, const void *o,
                                   const void *dout, const float *lse, float *delta, void *dq,
                                   const int *cu_seqlens, int n_seq, int total, int max_seqlen,
                                   int Hq, int Hkv, float scale, hipStream_t stream) {
  const int max_tiles = (max_seqlen + DqTile<D>::BM - 1) / DqTile<D>::BM;
  constexpr size_t lds = DqTile<D>::LDS_BYTES;
  auto kern = fa_bwd_dq_varlen_bf16_kernel<D>;
  if (lds > 65536) {
    hipError_t e = allow_lds<fa_bwd_dq_varlen_bf16_kernel<D>>(lds);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((unsigned)((int64_t)max_tiles * n_seq * Hq)), block(256);
  kern<<<grid, block, lds, stream>>>((const bf16 *)q, (const bf16 *)k, (const bf16 *)v,
                                     (const bf16 *)o, (const bf16 *)dout, lse, delta, (bf16 *)dq,
                                     cu_seqlens, n_seq, total, max_seqlen, Hq, Hkv, scale * kLog2e,
                                     scale);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_dkdv_varlen(const void *q, const void *k, const void *v,
                                     const void *dout, const float *lse, const float *delta,
                                     void *dk, void *dv, const int *cu_seqlens, int n_seq,
                                     int total, int max_seqlen, int Hq, int Hkv, float scale,
                                     hipStream_t stream) {
  const int max_ktiles = (max_seqlen + 127) / 128;  // 128-key tiles
  constexpr size_t lds = D == 64 ? kDkv64LdsBytes : kDkv128LdsBytes;
  auto kern = fa_bwd_dkdv_varlen_bf16_kernel<D>;
  if (lds > 65536) {
    hipError_t e = allow_lds<fa_bwd_dkdv_varlen_bf16_kernel<D>>(lds);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((unsigned)((int64_t)max_ktiles * n_seq * Hkv)), block(256);
  kern<<<grid, block, lds, stream>>>((const bf16 *)q, (const bf16 *)k, (const bf16 *)v,
                                     (const bf16 *)dout, lse, delta, (bf16 *)dk, (bf16 *)dv,
                                     cu_seqlens, n_seq, total, max_seqlen, Hq, Hkv, scale * kLog2e,
                                     scale);
  return hipGetLastError();
}

hipError_t launch_bwd_varlen_bf16(const void *q, const void *k, const void *v, const void *o,
                                  const void *dout, const float *lse, float *delta, void *dq,
                                  void *dk, void *dv, const int *cu_seqlens, int n_seq,
                                  int total, int max_seqlen, int Hq, int Hkv, int D, float scale,
                                  hipStream_t stream) {
  hipError_t e = D == 64 ? launch_dq_varlen<64>(q, k, v, o, dout, lse, delta, dq, cu_seqlens,
                                                n_seq, total, max_seqlen, Hq, Hkv, scale, stream)
                         : launch_dq_varlen<128>(q, k, v, o, dout, lse, delta, dq, cu_seqlens,
                                                 n_seq, total, max_seqlen, Hq, Hkv, scale, stream);
  if (e != hipSuccess) return e;
  return D == 64 ? launch_dkdv_varlen<64>(q, k, v, dout, lse, delta, dk, dv, cu_seqlens, n_seq,
                                          total, max_seqlen, Hq, Hkv, scale, stream)
                 : launch_dkdv_varlen<128>(q, k, v, dout, lse, delta, dk, dv, cu_seqlens, n_seq,
                                           total, max_seqlen, Hq, Hkv, scale, stream);
}

hipError_t launch_bwd_dq_bf16(const void *q, const void *k, const void *v, const void *o,
                              const void *dout, const float *lse, float *delta, void *dq,
                              int B, int Hq, int Hkv, int T, int D, float scale,
                              hipStream_t stream) {
  return D == 64 ? launch_dq<64>(q, k, v, o, dout, lse, delta, dq, B, Hq, Hkv, T, scale, stream)
                 : launch_dq<128>(q, k, v, o, dout, lse, delta, dq, B, Hq, Hkv, T, scale, stream);
}

hipError_t launch_bwd_dkdv_bf16(const void *q, const void *k, const void *v, const void *dout,
                                const float *lse, const float *delta, void *dk, void *dv,
                                int B, int Hq, int Hkv, int T, int D, float scale,
                                hipStream_t stream) {
  return D == 64
             ? launch_dkdv<64>(q, k, v, dout, lse, delta, dk, dv, B, Hq, Hkv, T, scale, stream)
             : launch_dkdv<128>(q, k, v, dout, lse, delta, dk, dv, B, Hq, Hkv, T, scale, stream);
}

}  // namespace ttfa
