// Causal GQA FlashAttention forward, bf16 in / fp32 accumulate, gfx950.
//
// Computes what the reference's fwd_kernel computes (kernels/flash_attn.py:12-67):
// for every query row i of head h, O_i = sum_{j<=i} softmax_j(q_i.k_j * scale) v_j
// with K/V read from KV head h / G, and LSE_i = m_i + ln(l_i) in natural-log units.
//
// Work split: one workgroup = 4 waves; a row tile is 128 query rows of one (batch, head)
// and each wave owns 32 of them.  A workgroup processes a pair of row tiles, the longer
// first, so every workgroup carries the same causal work (pair_item), when pairs fill
// whole rounds of the resident slots; otherwise single tiles, longest first.  K/V stream
// through LDS in 64-key tiles, double-buffered: the next tile's global loads are in
// flight while the current tile is consumed.  The loads go from the buffer straight
// into LDS (buffer_load ... lds, 16 bytes per lane), so no VGPRs stage them.
//
// Per wave and tile, scores are formed transposed, S^T = K Q^T (32x32x16 MFMAs with K
// from LDS as the A operand and the wave's Q rows held in registers as the B operand),
// so every lane owns ONE query row and 16 of the 32 keys of a block: the row max is an
// in-register v_max3 tree plus one v_permlane32_swap.  P^T stays in the result
// registers, is packed to bf16 and feeds O^T += V^T P^T directly as the B operand; V^T
// comes from LDS through ds_read_b64_tr_b16, whose row order matches the MFMA result
// layout.  The row sum is accumulated from the fp32 probabilities (a sum of the
// bf16-rounded values would put up to 2^-9 relative error into LSE for rows that one
// key dominates, more than the 1e-3 LSE tolerance allows).
//
// Softmax runs in the exp2 domain (scale * log2(e) folded into one FMA).  The running
// max is updated lazily: O and l are rescaled only when some row's tile max exceeds
// the running max by more than kRescaleSlack (log2 units), so p <= 2^kRescaleSlack and
// most tiles skip the rescale entirely.  The stored LSE is converted back to natural
// log.  Tiles entirely above the diagonal are never loaded; only tiles that cross the
// diagonal or the ragged end of T run the masked body.
#include "fa_bwd.h"  // allow_lds
#include "fa_common.h"
#include "fa_kernels.h"

namespace ttfa {

namespace {

constexpr float kRescaleSlack = 8.0f;

// K/V tiles use layout 1 (conflict-free K row reads).
constexpr int kFwdLayout = 1;

template <int D>
struct FwdTile {
  static constexpr int BM = 128, BN = 64;
  static constexpr int KK = D / 16;            // MFMA k-steps over D
  static constexpr int DB = D / 32;            // 32-row blocks of O^T
  static constexpr int CH = D / 8;             // 16-byte chunks per row
  static constexpr int LOADS = BN * CH / 256;  // 16-byte loads per thread per K (or V) tile
};

// One 64-key tile for one wave: S^T, online softmax, O^T += V^T P^T.
template <int D, bool MASK>
__device__ __forceinline__ void fwd_tile(const bf16 *Kt, const bf16 *Vt, const bf16x8 (&qf)[D / 16],
                                         f32x16 (&oacc)[D / 32], float &m_t, float &l_part,
                                         float scale_log2, int k0, int qrow, int T, int lane) {
  using P = FwdTile<D>;
  const int lq = lane & 31, lg = lane >> 5;

  // All K operand fragments first, so the LDS reads overlap each other and the MFMAs.
  bf16x8 kf[2][P::KK];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kk = 0; kk < P::KK; ++kk) kf[kb][kk] = lds_read_row8<D, kFwdLayout>(Kt, kb * 32 + lq, 2 * kk + lg);
  f32x16 s[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    s[kb] = mfma32(kf[kb][0], qf[0], f32x16{});
#pragma unroll
    for (int kk = 1; kk < P::KK; ++kk) s[kb] = mfma32(kf[kb][kk], qf[kk], s[kb]);
  }
  if (MASK) {
    if (k0 + P::BN <= T) {
      // Inside T, every 32-key block is either visible, entirely above the wave's 32 rows,
      // or exactly on their diagonal (rows and blocks both start at multiples of 32);
      // which one is wave-uniform, and the diagonal pattern is key slot > row.
      const int q0 = qrow - lq, dl = lq - 4 * lg;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int rel = k0 + 32 * kb - q0;
        if (rel > 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) s[kb][r] = -INFINITY;
        } else if (rel == 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) > dl) s[kb][r] = -INFINITY;
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
          if (key > qrow || key >= T) s[kb][r] = -INFINITY;
        }
    }
  }
  // Row max of this tile (v_max3 tree), then the lazy running-max update.
  float mx = max16(s[1], max16(s[0], -INFINITY));
  mx = xhalf_max(mx) * scale_log2;
  if (__builtin_amdgcn_ballot_w64(mx > m_t + kRescaleSlack)) {  // wave-uniform branch
    const float m_new = fmax2(m_t, mx);
    const float alpha = exp2f_fast(m_t - m_new);
    m_t = m_new;
    l_part *= alpha;
#pragma unroll
    for (int db = 0; db < P::DB; ++db) oacc[db] *= alpha;
  }
  // P = exp2(S * scale*log2e - m) in fp32 (row sum), packed to bf16 for the PV product.
  bf16x8 pb[4];
  float rs0, rs1;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = exp2f_fast(__builtin_fmaf(s[m >> 1][8 * (m & 1) + e], scale_log2, -m_t));
    if (m == 0) {  // the sums start at the first terms (0 + x is not folded: -0)
      rs0 = p[0];
      rs1 = p[1];
    } else {
      rs0 += p[0];
      rs1 += p[1];
    }
#pragma unroll
    for (int e = 2; e < 8; e += 2) {
      rs0 += p[e];
      rs1 += p[e + 1];
    }
    pb[m] = pack8(f32x16{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]}, 0);
  }
  l_part += rs0 + rs1;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    bf16x8 vf[P::DB];
#pragma unroll
    for (int db = 0; db < P::DB; ++db) vf[db] = lds_read_trT<D, kFwdLayout>(Vt, 16 * m, 32 * db, lane);
#pragma unroll
    for (int db = 0; db < P::DB; ++db) oacc[db] = mfma32(vf[db], pb[m], oacc[db]);
  }
}

}  // namespace

// One query head's rows and its KV head's rows for one sequence: T rows of D starting at
// q / k / v / o, and T LSE values at lse.
struct FwdHead {
  const bf16 *q, *k, *v;
  bf16 *o;
  float *lse;
  int T;
};

// All 128 query rows of row tile qt of one head: online softmax over its key tiles.
// Ends with a workgroup barrier, so the caller may reuse the LDS ring right away.
template <int D>
__device__ __forceinline__ void fwd_rows(bf16 (*lds)[2][FwdTile<D>::BN * D], const FwdHead &hd,
                                         int qt, float scale_log2, int work_left, int work_max) {
  using P = FwdTile<D>;
  constexpr int BM = P::BM, BN = P::BN, KK = P::KK, DB = P::DB, CH = P::CH, LOADS = P::LOADS;
  const int T = hd.T;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int q0 = qt * BM + wave * 32;  // first query row of this wave
  const int qrow = q0 + lq;

  const uint32_t head_bytes = (uint32_t)T * D * 2;

  // Global -> LDS without registers: the wave fills 1 KB blocks of the swizzled tile;
  // lane l of block e0 writes physical chunk (e0 + l) % CH of row (e0 + l) / CH, which
  // holds logical chunk phys ^ swizzle(row).  The lane's offset within a tile is fixed
  // (voffset); the tile's start goes into a descriptor re-based per tile (scalar work);
  // the LDS destination (M0) comes from the scalar wave index.
  const int wave_s = wave_id();
  uint32_t voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int e = 256 * i + 64 * wave + lane, row = e / CH, pc = e % CH;
    voff[i] = (uint32_t)(row * D + swz_l<D, kFwdLayout>(row, pc) * 8) * 2;
  }
  auto load_tile = [&](int j, int stage) {
    // descriptors re-based at the tile (scalar work): rows past T still read as zero
    const int64_t t0 = (int64_t)j * BN * D;
    const uint32_t left = head_bytes - (uint32_t)t0 * 2;
    const auto rkj = make_rsrc(hd.k + t0, left), rvj = make_rsrc(hd.v + t0, left);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e0 = 256 * i + 64 * wave_s;
      buf_load16_lds(rkj, voff[i], &lds[stage][0][e0 * 8]);
      buf_load16_lds(rvj, voff[i], &lds[stage][1][e0 * 8]);
    }
  };

  // Q^T as B operand: lane (lq, lg) slot s of step kk holds Q[qrow][16kk + 8lg + s].
  // The row tile's Q goes to LDS stage 1 (free until the loop's first prefetch) in the
  // coalesced direct-to-LDS form, beside the first K/V tile in stage 0, and each wave
  // reads its fragments from there.
  load_tile(0, 0);
  {
    const uint32_t qbytes = head_bytes - (uint32_t)(qt * BM * D * 2);
    const auto rqt = make_rsrc(hd.q + (int64_t)qt * BM * D, qbytes);
    bf16 *Qs = &lds[1][0][0];  // 128 rows x D across stage 1's K and V halves
#pragma unroll
    for (int i = 0; i < 2 * LOADS; ++i) {
      const int e = 256 * i + 64 * wave + lane, row = e / CH, pc = e % CH;
      const uint32_t off = (uint32_t)(row * D + swz_l<D, kFwdLayout>(row, pc) * 8) * 2;
      buf_load16_lds(rqt, off, Qs + (256 * i + 64 * wave_s) * 8);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  bf16x8 qf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
    qf[kk] = lds_read_row8<D, kFwdLayout>(&lds[1][0][0], wave * 32 + lq, 2 * kk + lg);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's Q reads are complete
  __syncthreads();                     // ... in every wave, before stage 1 is refilled

  const int n_kv = min((T + BN - 1) / BN, (qt + 1) * (BM / BN));
  // Tiles [0, n_full) are visible to every row of this wave and lie inside T;
  // tiles [n_full, n_vis) need the mask; later tiles are skipped by this wave.
  const int n_full = min((q0 + 1) / BN, T / BN);
  const int n_vis = min(n_kv, (q0 + 31) / BN + 1);

  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16{};
  float m_t = -INFINITY;  // running row max, in scale*log2(e) units
  float l_part = 0.f;     // this lane's share of the running row sum

  PrioByRemaining prio(work_max);
  for (int j = 0; j < n_kv; ++j) {
    prio.update(work_left - j);
    if (j + 1 < n_kv) load_tile(j + 1, (j + 1) & 1);
    const bf16 *Kt = lds[j & 1][0];
    const bf16 *Vt = lds[j & 1][1];
    if (j < n_full)
      fwd_tile<D, false>(Kt, Vt, qf, oacc, m_t, l_part, scale_log2, j * BN, qrow, T, lane);
    else if (j < n_vis)
      fwd_tile<D, true>(Kt, Vt, qf, oacc, m_t, l_part, scale_log2, j * BN, qrow, T, lane);
    wait_vm_all();  // tile j+1 is in LDS before any wave passes the barrier
    __syncthreads();
  }

  // The loop's last barrier freed the LDS ring: each wave stages its O tile in its own
  // 32*D slice of it for row-contiguous stores.
  const float l = xhalf_sum(l_part);
  store_rows<D>(oacc, 1.f / l, &lds[0][0][0] + wave * 32 * D, hd.o, q0, T, lane);
  if (qrow < T && lg == 0) hd.lse[qrow] = (m_t + __log2f(l)) * kLn2;
  __syncthreads();  // the ring is free again for the caller
}

template <int D>
__global__ __launch_bounds__(256, 2) void fa_fwd_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    bf16 *__restrict__ O, float *__restrict__ LSE, int B, int Hq, int Hkv, int T,
    float scale_log2, int paired) {
  using P = FwdTile<D>;
  __shared__ __attribute__((aligned(16))) bf16 lds[2][2][P::BN * D];  // [stage][K|V]
  const int n_tiles = (T + P::BM - 1) / P::BM;
  const WorkPair w = sched_item(paired, blockIdx.x, n_tiles, B, Hq, Hq / Hkv, false);
  // Key tiles a row tile visits is its work; the priority scales by the largest
  // workgroup's work.
  const int n_kt = (T + P::BN - 1) / P::BN;
  auto work = [&](int qt) { return qt < 0 ? 0 : min(n_kt, (qt + 1) * (P::BM / P::BN)); };
  const int w1 = work(w.first), w2 = work(w.second);
  const int wmax = paired ? work(n_tiles - 1) + work(0) : work(n_tiles - 1);
  const int G = Hq / Hkv;
  const int b = w.bh / Hq, h = w.bh - b * Hq;
  const int64_t kvh = (int64_t)b * Hkv + h / G, hs = (int64_t)T * D;
  const FwdHead hd{Q + w.bh * hs, K + kvh * hs, V + kvh * hs, O + w.bh * hs,
                   LSE + (int64_t)w.bh * T, T};
  // A pair runs its shorter tile first.  The workgroups of one head start together and
  // read key tiles 0, 1, ... of the same K/V, and each then re-reads them in its longer
  // tile within a few tiles of the previous read, so K/V come from L2 (long tile first,
  // the short tile re-read keys from the launch's start, by then evicted).
  if (w.second >= 0) {
    fwd_rows<D>(lds, hd, w.second, scale_log2, w1 + w2, wmax);
    fwd_rows<D>(lds, hd, w.first, scale_log2, w1, wmax);
  } else {
    fwd_rows<D>(lds, hd, w.first, scale_log2, w1, wmax);
  }
}

// Packed variable-length sequences ([H, total, D] per tensor, sequence s at rows
// cu_seqlens[s] .. cu_seqlens[s+1]-1 of every head, causal within each sequence).
// Workgroup -> (tile rank, sequence, query head), rank-major, so every sequence's
// longest row tiles (rank 0 = its last tile) are dispatched first; a rank past a
// sequence's tile count exits at once.  Sequences whose bounds are not
// 0 <= cu[s] <= cu[s+1] <= total are skipped (nothing is read or written for them).
template <int D>
__global__ __launch_bounds__(256, 2) void fa_fwd_varlen_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    bf16 *__restrict__ O, float *__restrict__ LSE, const int *__restrict__ cu_seqlens,
    int n_seq, int total, int Hq, int Hkv, int max_seqlen, float scale_log2) {
  using P = FwdTile<D>;
  __shared__ __attribute__((aligned(16))) bf16 lds[2][2][P::BN * D];
  const int per_rank = n_seq * Hq;
  const int rank = blockIdx.x / per_rank, rem = blockIdx.x - rank * per_rank;
  const int s = rem / Hq, h = rem - s * Hq;
  const int c0 = cu_seqlens[s], c1 = cu_seqlens[s + 1];
  if (c0 < 0 || c1 < c0 || c1 > total) return;
  // A sequence longer than max_seqlen is processed as its first max_seqlen tokens (the
  // same clamp in all three varlen kernels): those rows are exact, later rows unwritten.
  const int T = min(c1 - c0, max_seqlen);
  const int max_tiles = (max_seqlen + P::BM - 1) / P::BM;
  const int n_tiles = (T + P::BM - 1) / P::BM;
  if (rank >= n_tiles) return;
  const int qt = n_tiles - 1 - rank;
  const int n_kt = (T + P::BN - 1) / P::BN;
  const int wmax = min((max_tiles * P::BM + P::BN - 1) / P::BN, max_tiles * (P::BM / P::BN));
  const int hk = h / (Hq / Hkv);
  const int64_t qb = ((int64_t)h * total + c0) * D, kb = ((int64_t)hk * total + c0) * D;
  const FwdHead hd{Q + qb, K + kb, V + kb, O + qb, LSE + (int64_t)h * total + c0, T};
  fwd_rows<D>(lds, hd, qt, scale_log2, min(n_kt, (qt + 1) * (P::BM / P::BN)), wmax);
}

// D = 128 forward over 256-row tiles, 64 rows per wave (fa_fwd128.hip).
__global__ void fa_fwd_wide_bf16_kernel(const bf16 *__restrict__ Q, const bf16 *__restrict__ K,
                                        const bf16 *__restrict__ V, bf16 *__restrict__ O,
                                        float *__restrict__ LSE, int B, int Hq, int Hkv, int T,
                                        float scale_log2, int paired);
constexpr int kFwd128LdsBytes = 2 * 2 * 128 * 128 * 2;  // two 128-key stages of K and V

// 256-row tiles, 64 rows per wave: half the LDS bytes per product, but half the
// workgroups and a longer prologue, so only where its pairs fill the 256 resident slots of
// an MI355X and T > 3840 (measured 5-7% slower at T = 2000-3072, even at 4096, 3-5% faster
// from 8192 up).
bool fwd128_uses_wide(int B, int Hq, int T) {
  const int n_wide = (T + 255) / 256;
  return n_wide >= 16 && (int64_t)sched_items(true, n_wide, B, Hq) >= kWideSlots;
}

hipError_t launch_fwd_bf16(const void *q, const void *k, const void *v, void *o, float *lse,
                           int B, int Hq, int Hkv, int T, int D, float scale,
                           hipStream_t stream) {
  const int n_tiles = (T + FwdTile<64>::BM - 1) / FwdTile<64>::BM;
  const float sl2 = scale * kLog2e;
  if (D == 128 && fwd128_uses_wide(B, Hq, T)) {
    const int n_wide = (T + 255) / 256;
    hipError_t e = allow_lds<fa_fwd_wide_bf16_kernel>(kFwd128LdsBytes);  // before the
    if (e != hipSuccess) return e;  // occupancy query, which sees the raised limit
    const int slots = resident_slots<fa_fwd_wide_bf16_kernel>(256, kFwd128LdsBytes);
    const bool paired = use_pairs(n_wide, B, Hq, slots);
    const dim3 grid((unsigned)sched_items(paired, n_wide, B, Hq)), block(256);
    fa_fwd_wide_bf16_kernel<<<grid, block, kFwd128LdsBytes, stream>>>(
        (const bf16 *)q, (const bf16 *)k, (const bf16 *)v, (bf16 *)o, lse, B, Hq, Hkv, T, sl2,
        (int)paired);
    return hipGetLastError();
  }
  auto go = [&](auto kern, int slots) {
    const bool paired = use_pairs(n_tiles, B, Hq, slots);
    const dim3 grid((unsigned)sched_items(paired, n_tiles, B, Hq)), block(256);
    kern<<<grid, block, 0, stream>>>((const bf16 *)q, (const bf16 *)k, (const bf16 *)v, (bf16 *)o,
                                     lse, B, Hq, Hkv, T, sl2, (int)paired);
    return hipGetLastError();
  };
  return D == 64 ? go(fa_fwd_bf16_kernel<64>, resident_slots<fa_fwd_bf16_kernel<64>>(256, 0))
                 : go(fa_fwd_bf16_kernel<128>, resident_slots<fa_fwd_bf16_kernel<128>>(256, 0));
}

hipError_t launch_fwd_varlen_bf16(const void *q, const void *k, const void *v, void *o,
                                  float *lse, const int *cu_seqlens, int n_seq, int total,
                                  int max_seqlen, int Hq, int Hkv, int D, float scale,
                                  hipStream_t stream) {
  const int max_tiles = (max_seqlen + FwdTile<64>::BM - 1) / FwdTile<64>::BM;
  const dim3 grid((unsigned)((int64_t)max_tiles * n_seq * Hq)), block(256);
  const float sl2 = scale * kLog2e;
  auto go = [&](auto kern) {
    kern<<<grid, block, 0, stream>>>((const bf16 *)q, (const bf16 *)k, (const bf16 *)v,
                                     (bf16 *)o, lse, cu_seqlens, n_seq, total, Hq, Hkv, max_seqlen,
                                     sl2);
    return hipGetLastError();
  };
  return D == 64 ? go(fa_fwd_varlen_bf16_kernel<64>) : go(fa_fwd_varlen_bf16_kernel<128>);
}

}  // namespace ttfa
