// Causal GQA FlashAttention backward, dK/dV pass at D = 128 (bf16 in, fp32 accumulate,
// gfx950): the reference's bwd_dkdv_kernel (kernels/flash_attn.py:93-159) with the work
// split of the D = 64 pass (fa_bwd_dkdv64.hip: a workgroup = 128 keys of one (batch, kv
// head), 4 waves x 32 keys, K and V rows in registers, dK and dV accumulated over the
// head's query-head group in registers: no atomics, bitwise deterministic), the query
// rows streamed in 128-row stages (130 KB of LDS: one workgroup per CU, as the 192 AGPRs
// of accumulators and K/V fragments already allow only one wave per SIMD) and each
// wave's work on a stage issued as one hand-scheduled instruction stream
// (gen_dkdv128_asm.py).  With one wave per SIMD nothing else can issue VALU work while a
// wave's products run, so the stream's overlap of one block's exponentials with its
// neighbours' products is the only overlap the pass gets.
#include "dkdv128_item.inc"
#include "fa_bwd.h"
#include "fa_common.h"

namespace ttfa {

namespace {

// One 128-row stage of the D = 128 dK/dV pass for one wave, as a hand-scheduled
// instruction stream (dkdv128_item.inc, written by gen_dkdv128_asm.py): for each of the
// stage's 32-row query blocks, S - LSE/scale and dP - Delta (accumulators initialised from
// the staged rows), P = exp2(S' * scale*log2e), dS = P (dP - Delta), then dV^T += dO^T P
// and dK^T += Q^T dS over the 4 column blocks, with the blocks software-pipelined against
// each other.  mode (wave-uniform) 0: all four blocks lie below the wave's keys; 1 + w:
// the stage holding the diagonal for wave w.  The accumulators and the K/V fragments stay
// in AGPRs; aR are the lane's LDS byte addresses of the row-fragment reads per k-step, aT
// those of the transposed reads per column block and 8-row half (2db + h), aN that of the
// -LSE/scale rows; dl = lq - 4lg places the diagonal mask.
#define TTFA_DKDV128_OPERANDS                                                                \
  : "+a"(dk[0]), "+a"(dk[1]), "+a"(dk[2]), "+a"(dk[3]), "+a"(dv[0]), "+a"(dv[1]),            \
    "+a"(dv[2]), "+a"(dv[3])                                                                 \
  : "a"(kf[0]), "a"(kf[1]), "a"(kf[2]), "a"(kf[3]), "a"(kf[4]), "a"(kf[5]), "a"(kf[6]),     \
    "a"(kf[7]), "a"(vf[0]), "a"(vf[1]), "a"(vf[2]), "a"(vf[3]), "a"(vf[4]), "a"(vf[5]),     \
    "a"(vf[6]), "a"(vf[7]), "v"(aR[0]), "v"(aR[1]), "v"(aR[2]), "v"(aR[3]), "v"(aR[4]),     \
    "v"(aR[5]), "v"(aR[6]), "v"(aR[7]), "v"(aT[0]), "v"(aT[1]), "v"(aT[2]), "v"(aT[3]),     \
    "v"(aT[4]), "v"(aT[5]), "v"(aT[6]), "v"(aT[7]), "v"(aN), "s"(scale_log2), "v"(dl),      \
    "s"(mode)                                                                                \
  : TTFA_DKDV128_ITEM_CLOBBERS, "memory"
__device__ __forceinline__ void dkdv128_stage(f32x16 (&dk)[4], f32x16 (&dv)[4], const bf16x8 (&kf)[8],
                                              const bf16x8 (&vf)[8], const uint32_t (&aR)[8],
                                              const uint32_t (&aT)[8], uint32_t aN,
                                              float scale_log2, int dl, int mode) {
  asm volatile(TTFA_DKDV128_STAGE_ASM TTFA_DKDV128_OPERANDS);
}
#undef TTFA_DKDV128_OPERANDS

// D = 128: dK and dV for the 128 keys of key tile kt of one KV head, reduced over the
// head's query-head group: 4 waves x 32 keys, the wave's K/V rows in registers, dK/dV
// accumulated over the whole group in registers (no atomics), with 128-row Q/dO stages
// double-buffered through LDS and each stage's compute one hand-scheduled block per wave.  Ends with a
// workgroup barrier, so the caller may reuse the LDS ring right away.
__device__ __forceinline__ void dkdv_rows128(bf16 *lds, const DkvHead &hd, int kt,
                                             float scale_log2, float scale) {
  constexpr int D = 128, BMQ = 128, CH = D / 8, LOADS = BMQ * CH / 256;
  constexpr int TILE_BYTES = BMQ * D * 2, STAGE_BYTES = 2 * TILE_BYTES + 2 * BMQ * 4;
  const int G = hd.G, T = hd.T;
  // An opaque copy of the thread id: the paired kernel inlines this body twice, and
  // without it the compiler shares lane-derived addresses between the two copies, which
  // keeps them live across the first.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int k0w = kt * 128 + wave * 32;  // first key of this wave
  const int krow = k0w + lq;

  const uint32_t head_bytes = (uint32_t)T * D * 2;
  const auto rk = make_rsrc(hd.k, head_bytes);
  const auto rv = make_rsrc(hd.v, head_bytes);
  // K^T, V^T as B operands: lane (key lq, lg) slot s of step kk = row krow, d = 16kk+8lg+s.
  bf16x8 kf[8], vf[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const uint32_t off = (uint32_t)(krow * D + 16 * kk + 8 * lg) * 2;
    kf[kk] = __builtin_bit_cast(bf16x8, buf_load16(rk, off));
    vf[kk] = __builtin_bit_cast(bf16x8, buf_load16(rv, off));
  }

  const int n_qt = (T + BMQ - 1) / BMQ;
  const int per_g = n_qt - kt;  // stages kt..n_qt-1 of each query head (kt holds the diagonal)
  const int n_items = G * per_g;
  const float inv_scale = 1.f / scale;
  // Each thread carries one LSE (tid < 128) or Delta value of the next stage from its load
  // to its staging, so nothing waits on the load until after the current stage's compute.
  float fl = 0.f;
  const uint32_t row_bytes = (uint32_t)T * 4;  // LSE / Delta rows past T read as zero
  int ld_g = 0, ld_qt = kt;
  const int wave_u = wave_id();
  // global -> LDS: thread element e = 256i + tid covers row e / CH, physical chunk e % CH
  uint32_t voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int e = 256 * i + tid, row = e / CH, pc = e % CH;
    voff[i] = (uint32_t)(row * D + swz_rows128(row, pc) * 8) * 2;
  }
  auto load_item = [&](int stage) {
    char *st = reinterpret_cast<char *>(lds) + stage * STAGE_BYTES;
    const int g = ld_g, qt = ld_qt;
    if (++ld_qt == n_qt) {
      ld_qt = kt;
      ++ld_g;
    }
    const int64_t hoff = g * hd.head_stride + (int64_t)qt * BMQ * D;
    const uint32_t left = head_bytes - (uint32_t)(qt * BMQ * D * 2);
    const auto rq = make_rsrc(hd.q + hoff, left), rdo = make_rsrc(hd.dout + hoff, left);
    const float *lse_g = hd.lse + g * hd.row_stride, *delta_g = hd.delta + g * hd.row_stride;
    const auto rfl = make_rsrc(wave_u < 2 ? lse_g : delta_g, row_bytes);  // wave-uniform
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e0 = 256 * i + 64 * wave_u;
      buf_load16_lds(rq, voff[i], reinterpret_cast<bf16 *>(st) + e0 * 8);
      buf_load16_lds(rdo, voff[i], reinterpret_cast<bf16 *>(st + TILE_BYTES) + e0 * 8);
    }
    fl = __uint_as_float(buf_load4(rfl, (uint32_t)(qt * BMQ + (tid & (BMQ - 1))) * 4));
  };
  auto stage_rows = [&](int stage) {
    float *f = reinterpret_cast<float *>(reinterpret_cast<char *>(lds) + stage * STAGE_BYTES +
                                         2 * TILE_BYTES);
    f[tid] = tid < BMQ ? -fl * inv_scale : -fl;
  };

  // The accumulators are zeroed (a product of zeros with a zero addend) and updated only
  // by asm statements with AGPR operands, so they stay in AGPRs between the stages.
  f32x16 dkacc[4], dvacc[4];
  {
    const bf16x8 z = {};
    // (s_nop 1: the compiler may write the zero operand just before, and a VALU result
    // needs 2 wait states before an MFMA reads it; the compiler adds none for asm)
    asm volatile("s_nop 1\n\t"
                 "v_mfma_f32_32x32x16_bf16 %0, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %1, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %2, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %3, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %4, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %5, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %6, %8, %8, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %7, %8, %8, 0\n\t"
                 "s_nop 7\n\ts_nop 7"
                 : "=a"(dkacc[0]), "=a"(dkacc[1]), "=a"(dkacc[2]), "=a"(dkacc[3]),
                   "=a"(dvacc[0]), "=a"(dvacc[1]), "=a"(dvacc[2]), "=a"(dvacc[3])
                 : "v"(z));
  }
  // the lane's LDS addresses in stage 0, query block 0 (stage 1 adds STAGE_BYTES, block
  // lb 8192 lb, the dO tile 32768).  swz_rows128 XORs the chunk with row bits 0-3, so the
  // other query blocks and the 16-row groups of the transposed reads are constant offsets
  // but each k-step and each 8-row half needs an address of its own.
  uint32_t aR[8], aT[8];
  const uint32_t base = lds_addr(lds);
  const int g16 = lane >> 4, r4 = (lane >> 2) & 3, c4 = lane & 3;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) aR[kk] = base + lq * 256 + swz_rows128(lq, 2 * kk + lg) * 16;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 4 * (g16 >> 1) + r4 + 8 * h, col = 32 * db + 16 * (g16 & 1) + 4 * c4;
      aT[2 * db + h] = base + row * 256 + (swz_rows128(row, col >> 3) * 8 + (col & 7)) * 2;
    }
  }
  const uint32_t aN = base + 2 * TILE_BYTES + 16 * lg;
  const int dl = lq - 4 * lg;

  if (n_items > 0) {
    load_item(0);
    stage_rows(0);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K/V registers complete before the loop
  __syncthreads();
  int qt = kt;  // query tile of the current item
  for (int it = 0; it < n_items; ++it) {
    if (it + 1 < n_items) load_item((it + 1) & 1);
    const uint32_t so = (it & 1) * STAGE_BYTES;
    uint32_t r[8], t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      r[i] = aR[i] + so;
      t[i] = aT[i] + so;
    }
    // the stage that holds the diagonal (qt == kt): wave w's keys see its blocks w..3
    const int mode = qt != kt ? 0 : 1 + wave_u;
    dkdv128_stage(dkacc, dvacc, kf, vf, r, t, aN + so, scale_log2, dl, mode);
    if (++qt == n_qt) qt = kt;
    if (it + 1 < n_items) stage_rows((it + 1) & 1);
    wait_vm_all();  // the next stage's Q/dO tiles are in LDS before any wave passes the barrier
    __syncthreads();
  }

  // The loop's last barrier freed the LDS ring: each wave stages its dK and dV tiles in
  // its own two 32*D slices of it for row-contiguous stores.
  store_rows<D>(dkacc, scale, lds + wave * 64 * D, hd.dk, k0w, T, lane);
  store_rows<D>(dvacc, 1.f, lds + wave * 64 * D + 32 * D, hd.dv, k0w, T, lane);
  __syncthreads();  // the ring is free again for the caller
}

}  // namespace

// The paired kernel runs its one or two key tiles through a loop that is not unrolled, so
// the stage body is inlined once.
template <>
__global__ __launch_bounds__(256, 1) void fa_bwd_dkdv_bf16_kernel<128>(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ LSE,
    const float *__restrict__ Delta, bf16 *__restrict__ dK, bf16 *__restrict__ dV, int B,
    int Hq, int Hkv, int T, float scale_log2, float scale, int paired) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];
  const int n_ktiles = (T + 127) / 128;
  // Key tile 0 sees the most query rows, so the longer tile of a pair is the low one.
  const WorkPair w = sched_item(paired, blockIdx.x, n_ktiles, B, Hkv, 1, true);
  const int G = Hq / Hkv;
  const int b = w.bh / Hkv, hk = w.bh - b * Hkv;
  const int64_t hs = (int64_t)T * 128, kvb = w.bh * hs, q0 = (int64_t)b * Hq + hk * G;
  const DkvHead hd{K + kvb, V + kvb, dK + kvb, dV + kvb, Q + q0 * hs, dO + q0 * hs,
                   LSE + q0 * T, Delta + q0 * T, hs, T, G, T};
#pragma nounroll
  for (int p = 0; p < 2; ++p) {
    const int kt = p == 0 ? w.first : w.second;
    if (kt < 0) break;
    dkdv_rows128(smem, hd, kt, scale_log2, scale);
  }
}

// Packed variable-length sequences ([H, total, D] per tensor, sequence s at rows
// cu_seqlens[s] .. cu_seqlens[s+1]-1 of every head): the same stage body per (key tile,
// sequence, KV head), key-tile-major so every sequence's longest key tiles (tile 0 sees
// all of its query rows) are dispatched first; a key tile past a sequence's end exits at
// once.  Sequences whose bounds are not 0 <= cu[s] <= cu[s+1] <= total are skipped, and a
// sequence longer than max_seqlen is processed as its first max_seqlen tokens (the
// forward's clamp).  The per-sequence head view restricts every load to the sequence's
// own rows (the buffer descriptors end at its last row).
template <>
__global__ __launch_bounds__(256, 1) void fa_bwd_dkdv_varlen_bf16_kernel<128>(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ dO, const float *__restrict__ LSE,
    const float *__restrict__ Delta, bf16 *__restrict__ dK, bf16 *__restrict__ dV,
    const int *__restrict__ cu_seqlens, int n_seq, int total, int max_seqlen, int Hq, int Hkv,
    float scale_log2, float scale) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];
  const int per_rank = n_seq * Hkv;
  const int kt = blockIdx.x / per_rank, rem = blockIdx.x - kt * per_rank;
  const int s = rem / Hkv, hk = rem - s * Hkv;
  const int c0 = cu_seqlens[s], c1 = cu_seqlens[s + 1];
  if (c0 < 0 || c1 < c0 || c1 > total) return;
  const int T = min(c1 - c0, max_seqlen);
  if (kt >= (T + 127) / 128) return;
  const int G = Hq / Hkv;
  const int64_t hs = (int64_t)total * 128, kvb = (int64_t)hk * hs + (int64_t)c0 * 128;
  const int64_t q0 = (int64_t)hk * G;
  const DkvHead hd{K + kvb, V + kvb, dK + kvb, dV + kvb, Q + q0 * hs + (int64_t)c0 * 128,
                   dO + q0 * hs + (int64_t)c0 * 128, LSE + q0 * total + c0,
                   Delta + q0 * total + c0, hs, total, G, T};
  dkdv_rows128(smem, hd, kt, scale_log2, scale);
}

}  // namespace ttfa
