// Causal GQA FlashAttention backward, Delta + dQ pass at D = 64 (bf16 in, fp32
// accumulate, gfx950): the reference's bwd_preprocess (kernels/flash_attn.py:70-90)
// fused with its bwd_dq_kernel (:162-217), with the work split of the D = 128 pass in
// fa_bwd.hip (a workgroup = 128 query rows of one (batch, head), 4 waves x 32 rows, the
// wave's Q and dO rows in registers, Delta = rowsum(O * dO) formed in the prologue and
// written for the dK/dV pass), but with the keys streamed in 128-key stages and each
// wave's work on a stage issued as one hand-scheduled instruction stream (gen_dq64_asm.py),
// which overlaps the exponentials of one 32-key block with the matrix products of its
// neighbours.
#include "dq64_stage.inc"
#include "fa_bwd.h"
#include "fa_common.h"

namespace ttfa {

namespace {

// One 128-key stage of the dQ pass for one wave (see dq64_stage.inc for the operands).
// mode 0: every key of the stage precedes every row of the wave; 1 + w: the stage that
// holds wave w's diagonal (blocks 0..w, block w masked); 5: the stage that crosses T
// (every block masked: a key is dropped when its offset in the stage minus 4lg exceeds
// dm = min(row, T - 1) - (first key of the stage) - 4lg).
__device__ __forceinline__ void dq64_stage(f32x16 (&dq)[2], const bf16x8 (&qf)[4],
                                           const bf16x8 (&dof)[4], const uint32_t (&aR)[4],
                                           const uint32_t (&aT)[2][2], float scale_log2,
                                           float nlse, float ndelta, int dm, int mode) {
  asm volatile(TTFA_DQ64_STAGE_ASM
               : "+a"(dq[0]), "+a"(dq[1])
               : "a"(qf[0]), "a"(qf[1]), "a"(qf[2]), "a"(qf[3]), "a"(dof[0]), "a"(dof[1]),
                 "a"(dof[2]), "a"(dof[3]), "v"(aR[0]), "v"(aR[1]), "v"(aR[2]), "v"(aR[3]),
                 "v"(aT[0][0]), "v"(aT[0][1]), "v"(aT[1][0]), "v"(aT[1][1]), "s"(scale_log2),
                 "v"(nlse), "v"(ndelta), "v"(dm), "s"(mode)
               : TTFA_DQ64_STAGE_CLOBBERS, "memory");
}

}  // namespace

// Delta and dQ for the 128 query rows of one row tile (one workgroup per row tile,
// longest first).
template <>
__global__ __launch_bounds__(256, 2) void fa_bwd_dq_bf16_kernel<64>(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ O, const bf16 *__restrict__ dO, const float *__restrict__ LSE,
    float *__restrict__ Delta, bf16 *__restrict__ dQ, int B, int Hq, int Hkv, int T,
    float scale_log2, float scale, int /*paired: unused*/) {
  extern __shared__ __attribute__((aligned(16))) bf16 lds[];  // [stage 2][K|V][128 x 64]
  constexpr int D = 64, BN = 128, CH = D / 8, LOADS = BN * CH / 256;
  constexpr int TILE_BYTES = BN * D * 2, STAGE_BYTES = 2 * TILE_BYTES;
  const int n_tiles = (T + 127) / 128;
  const WorkPair w = sched_item(false, blockIdx.x, n_tiles, B, Hq, Hq / Hkv, false);
  const int qt = w.first;
  const int G = Hq / Hkv;
  const int b = w.bh / Hq, h = w.bh - b * Hq;
  const int64_t kvh = (int64_t)b * Hkv + h / G, hs = (int64_t)T * D, qb = w.bh * hs;
  const bf16 *q = Q + qb, *k = K + kvh * hs, *v = V + kvh * hs, *o = O + qb, *dout = dO + qb;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int wave_u = wave_id();
  const int q0 = qt * 128 + wave * 32;  // first query row of this wave
  const int qrow = q0 + lq;

  const uint32_t head_bytes = (uint32_t)T * D * 2;
  // global -> LDS: thread element e = 256i + tid covers key row e / CH, physical chunk e % CH
  uint32_t voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int e = 256 * i + tid, row = e / CH, pc = e % CH;
    voff[i] = (uint32_t)(row * D + swz_stage64(row, pc) * 8) * 2;
  }
  auto load_stage = [&](int j, int stage) {
    char *st = reinterpret_cast<char *>(lds) + stage * STAGE_BYTES;
    const int64_t t0 = (int64_t)j * BN * D;
    const uint32_t left = head_bytes - (uint32_t)t0 * 2;  // key rows past T read as zero
    const auto rkj = make_rsrc(k + t0, left), rvj = make_rsrc(v + t0, left);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e0 = 256 * i + 64 * wave_u;
      buf_load16_lds(rkj, voff[i], reinterpret_cast<bf16 *>(st) + e0 * 8);
      buf_load16_lds(rvj, voff[i], reinterpret_cast<bf16 *>(st + TILE_BYTES) + e0 * 8);
    }
  };

  // The first K/V stage is in flight while this wave's rows load and Delta is formed.
  load_stage(0, 0);
  const auto rq = make_rsrc(q, head_bytes), ro = make_rsrc(o, head_bytes);
  const auto rdo = make_rsrc(dout, head_bytes);
  bf16x8 qf[4], dof[4];
  float dpart = 0.f;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const uint32_t off = (uint32_t)(qrow * D + 16 * kk + 8 * lg) * 2;
    qf[kk] = __builtin_bit_cast(bf16x8, buf_load16(rq, off));
    dof[kk] = __builtin_bit_cast(bf16x8, buf_load16(rdo, off));
    const bf16x8 of = __builtin_bit_cast(bf16x8, buf_load16(ro, off));
#pragma unroll
    for (int s = 0; s < 8; ++s) dpart = __builtin_fmaf(bf2f(of[s]), bf2f(dof[kk][s]), dpart);
  }
  const float delta = xhalf_sum(dpart);
  float lse_t = 0.f;
  if (qrow < T) {
    lse_t = LSE[(int64_t)w.bh * T + qrow] * kLog2e;
    if (lg == 0) Delta[(int64_t)w.bh * T + qrow] = delta;
  }
  // dQ^T accumulators: zeroed by products of zeros, so they stay in AGPRs (s_nop 1 first:
  // the compiler may write the zero operand just before, and a VALU result needs 2 wait
  // states before an MFMA reads it)
  f32x16 dqacc[2];
  {
    const bf16x8 z = {};
    asm volatile("s_nop 1\n\t"
                 "v_mfma_f32_32x32x16_bf16 %0, %2, %2, 0\n\t"
                 "v_mfma_f32_32x32x16_bf16 %1, %2, %2, 0\n\t"
                 "s_nop 7\n\ts_nop 7"
                 : "=a"(dqacc[0]), "=a"(dqacc[1])
                 : "v"(z));
  }
  // the lane's LDS addresses in stage 0 (stage 1 adds STAGE_BYTES)
  uint32_t aR[4], aT[2][2];
  const uint32_t base = lds_addr(lds);
  const int g16 = lane >> 4, r4 = (lane >> 2) & 3, c4 = lane & 3;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) aR[kk] = base + lq * 128 + swz_stage64(lq, 2 * kk + lg) * 16;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 4 * (g16 >> 1) + r4 + 8 * hh, col = 32 * db + 16 * (g16 & 1) + 4 * c4;
      aT[db][hh] = base + row * 128 + (swz_stage64(row, col >> 3) * 8 + (col & 7)) * 2;
    }
  // a key is masked when its offset in the stage minus 4lg exceeds min(row, T-1) - k0 - 4lg
  const int dm_base = min(qrow, T - 1) - 4 * lg;

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no register load is pending in the loop
  __syncthreads();
  const int n_st = qt + 1;  // key stages 0..qt (the diagonal stage is qt)
  for (int j = 0; j < n_st; ++j) {
    if (j + 1 < n_st) load_stage(j + 1, (j + 1) & 1);
    const uint32_t so = (j & 1) * STAGE_BYTES;
    const uint32_t ra[4] = {aR[0] + so, aR[1] + so, aR[2] + so, aR[3] + so};
    const uint32_t ta[2][2] = {{aT[0][0] + so, aT[0][1] + so}, {aT[1][0] + so, aT[1][1] + so}};
    const int mode = (j + 1) * BN > T ? 5 : j == qt ? 1 + wave_u : 0;
    dq64_stage(dqacc, qf, dof, ra, ta, scale_log2, -lse_t, -delta, dm_base - j * BN, mode);
    wait_vm_all();  // stage j+1 is in LDS before any wave passes the barrier
    __syncthreads();
  }

  // The loop's last barrier freed the LDS ring: each wave stages its dQ tile in its own
  // 32*D slice of it for row-contiguous stores.
  store_rows<D>(dqacc, scale, lds + wave * 32 * D, dQ + qb, q0, T, lane);
}

}  // namespace ttfa
