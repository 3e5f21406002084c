// Causal GQA FlashAttention backward, Delta + dQ pass at D = 128 (bf16 in, fp32
// accumulate, gfx950): the reference's bwd_preprocess (kernels/flash_attn.py:70-90) fused
// with its bwd_dq_kernel (:162-217).  A workgroup takes 256 query rows of one (batch,
// head), 4 waves x 64 rows: each wave keeps the Q and dO fragments of its two 32-row
// groups and their dQ^T accumulators in AGPRs (all 256 of them), forms Delta =
// rowsum(O * dO) in the prologue and writes it for the dK/dV pass.  The keys stream through
// LDS in 128-key stages (K and V tiles, double-buffered: 128 KB), and each wave's work on
// a stage is one hand-scheduled instruction stream (gen_dq128_asm.py) in which every K/V
// fragment read from LDS feeds the products of both row groups: half the LDS bytes per
// product of a 32-row wave, whose LDS delivery bounds that form of the pass.
//
// The AGPR state lives outside every asm operand list, so it is only correct while the
// compiler itself touches no AGPR in this kernel.  Guards that must stay in the test
// suite: tests/test_asm_contracts.py (compiled code: no AGPR access outside the inline
// asm, no spills, no VALU write of an inline MFMA's source within two wait states) and
// the parity tests that select this kernel (test_wide_d128_kernels, which also asserts
// the kernel choice through ttfa_d128_wide, and test_config_parity[C4] / [C5]).
#include "dq128_stage.inc"
#include "fa_bwd.h"
#include "fa_common.h"

namespace ttfa {

namespace {

// One query head's rows (q, o, dout, dq: T rows of D; lse, delta: T values) and its KV
// head's rows (k, v) for one sequence.
struct DqRows128 {
  const bf16 *q, *k, *v, *o, *dout;
  const float *lse;
  float *delta;
  bf16 *dq;
  int T;
};

// One 128-key stage of the dQ pass for one wave (dq128_stage.inc), on the wave's AGPR
// state (dQ^T accumulators, Q and dO fragments in fixed AGPRs).  aR0 / aT0: the
// lane's LDS byte addresses of the stage's k-step 0 row read and (column block 0, half
// 0) transposed read; nlse, ndelta, dm: -LSE*log2(e), -Delta and the mask bound of the
// lane's row in each row group; mode 0: every key visible to both row groups, 1: every
// item masked (a key is dropped when its offset in the stage minus 4lg exceeds dm); ndb:
// -Delta in all 16 registers per row group, the dP^T chains' start value.
#define TTFA_DQ128_OPERANDS                                                              \
  :                                                                                      \
  : "v"(aR0), "v"(aT0), "s"(scale_log2), "v"(nlse[0]), "v"(nlse[1]), "v"(ndelta[0]),     \
    "v"(ndelta[1]), "v"(dm[0]), "v"(dm[1]), "s"(mode), "v"(ndb[0]), "v"(ndb[1])          \
  : TTFA_DQ128_STAGE_CLOBBERS, "memory"
__device__ __forceinline__ void dq128_stage(uint32_t aR0, uint32_t aT0, float scale_log2,
                                            const float (&nlse)[2], const float (&ndelta)[2],
                                            const int (&dm)[2], int mode, const f32x16 (&ndb)[2]) {
  asm volatile(TTFA_DQ128_STAGE_ASM TTFA_DQ128_OPERANDS);
}
#undef TTFA_DQ128_OPERANDS

// The wave's AGPR state for one row tile: Q and dO fragments in, accumulators zeroed.
__device__ __forceinline__ void dq128_init(const bf16x8 (&qf)[2][8], const bf16x8 (&dof)[2][8]) {
  asm volatile(TTFA_DQ128_INIT_ASM
               :
               : "{v[0:3]}"(qf[0][0]), "{v[4:7]}"(qf[0][1]), "{v[8:11]}"(qf[0][2]),
                 "{v[12:15]}"(qf[0][3]), "{v[16:19]}"(qf[0][4]), "{v[20:23]}"(qf[0][5]),
                 "{v[24:27]}"(qf[0][6]), "{v[28:31]}"(qf[0][7]), "{v[32:35]}"(qf[1][0]),
                 "{v[36:39]}"(qf[1][1]), "{v[40:43]}"(qf[1][2]), "{v[44:47]}"(qf[1][3]),
                 "{v[48:51]}"(qf[1][4]), "{v[52:55]}"(qf[1][5]), "{v[56:59]}"(qf[1][6]),
                 "{v[60:63]}"(qf[1][7]),
                 "{v[64:67]}"(dof[0][0]), "{v[68:71]}"(dof[0][1]), "{v[72:75]}"(dof[0][2]),
                 "{v[76:79]}"(dof[0][3]), "{v[80:83]}"(dof[0][4]), "{v[84:87]}"(dof[0][5]),
                 "{v[88:91]}"(dof[0][6]), "{v[92:95]}"(dof[0][7]), "{v[96:99]}"(dof[1][0]),
                 "{v[100:103]}"(dof[1][1]), "{v[104:107]}"(dof[1][2]), "{v[108:111]}"(dof[1][3]),
                 "{v[112:115]}"(dof[1][4]), "{v[116:119]}"(dof[1][5]), "{v[120:123]}"(dof[1][6]),
                 "{v[124:127]}"(dof[1][7])
               : TTFA_DQ128_AGPR_CLOBBERS);
}

// The dQ^T accumulators back from the AGPR state.
__device__ __forceinline__ void dq128_read(f32x16 (&dq)[2][4]) {
  asm volatile(TTFA_DQ128_READ_ASM
               : "={v[0:15]}"(dq[0][0]), "={v[16:31]}"(dq[0][1]), "={v[32:47]}"(dq[0][2]),
                 "={v[48:63]}"(dq[0][3]), "={v[64:79]}"(dq[1][0]), "={v[80:95]}"(dq[1][1]),
                 "={v[96:111]}"(dq[1][2]), "={v[112:127]}"(dq[1][3]));
}

// Delta and dQ for the 256 query rows of row tile qt of one head.  Ends with a workgroup
// barrier, so the caller may reuse the LDS ring right away.
__device__ __forceinline__ void dq_rows256(bf16 *lds, const DqRows128 &hd, int qt,
                                           float scale_log2, float scale) {
  constexpr int D = 128, BN = 128, CH = D / 8, LOADS = BN * CH / 256;
  constexpr int TILE_BYTES = BN * D * 2, STAGE_BYTES = 2 * TILE_BYTES;
  const int T = hd.T;
  // An opaque copy of the thread id: the kernel runs this body for two row tiles, and
  // without it the compiler keeps lane-derived values of the first alive across it.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int wave_u = wave_id();
  const int q0 = qt * 256 + wave * 64;     // first row of this wave (per lane)
  const int q0u = qt * 256 + wave_u * 64;  // the same, wave-uniform (scalar)

  const uint32_t head_bytes = (uint32_t)T * D * 2;
  // global -> LDS: thread element e = 256i + tid covers key row e / CH, physical chunk e % CH
  uint32_t voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int e = 256 * i + tid, row = e / CH, pc = e % CH;
    voff[i] = (uint32_t)(row * D + swz_rows128(row, pc) * 8) * 2;
  }
  auto load_stage = [&](int j, int stage) {
    char *st = reinterpret_cast<char *>(lds) + stage * STAGE_BYTES;
    const int64_t t0 = (int64_t)j * BN * D;
    const uint32_t left = head_bytes - (uint32_t)t0 * 2;  // key rows past T read as zero
    const auto rkj = make_rsrc(hd.k + t0, left), rvj = make_rsrc(hd.v + t0, left);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e0 = 256 * i + 64 * wave_u;
      buf_load16_lds(rkj, voff[i], reinterpret_cast<bf16 *>(st) + e0 * 8);
      buf_load16_lds(rvj, voff[i], reinterpret_cast<bf16 *>(st + TILE_BYTES) + e0 * 8);
    }
  };

  // The first K/V stage is in flight while this wave's rows load and Delta is formed.
  load_stage(0, 0);
  const auto rq = make_rsrc(hd.q, head_bytes), ro = make_rsrc(hd.o, head_bytes);
  const auto rdo = make_rsrc(hd.dout, head_bytes);
  bf16x8 qf[2][8], dof[2][8];
  float nlse[2], ndelta[2];
  int dm[2];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    const int qrow = q0 + 32 * qg + lq;
    float dpart = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const uint32_t off = (uint32_t)(qrow * D + 16 * kk + 8 * lg) * 2;
      qf[qg][kk] = __builtin_bit_cast(bf16x8, buf_load16(rq, off));
      dof[qg][kk] = __builtin_bit_cast(bf16x8, buf_load16(rdo, off));
      const bf16x8 of = __builtin_bit_cast(bf16x8, buf_load16(ro, off));
#pragma unroll
      for (int s = 0; s < 8; ++s) dpart = __builtin_fmaf(bf2f(of[s]), bf2f(dof[qg][kk][s]), dpart);
    }
    const float delta = xhalf_sum(dpart);
    float lse_t = 0.f;
    if (qrow < T) {
      lse_t = hd.lse[qrow] * kLog2e;
      if (lg == 0) hd.delta[qrow] = delta;
    }
    nlse[qg] = -lse_t;
    ndelta[qg] = -delta;
    // a key is masked when its offset in the stage minus 4lg exceeds
    // min(row, T-1) - (first key of the stage) - 4lg
    dm[qg] = min(qrow, T - 1) - 4 * lg;
  }
  dq128_init(qf, dof);
  f32x16 ndb[2];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int r = 0; r < 16; ++r) ndb[qg][r] = ndelta[qg];
  // the lane's LDS addresses of the k-step 0 row read and the (column block 0, half 0)
  // transposed read in stage 0; the stream derives the others (the XOR of swz_rows128)
  const uint32_t base = lds_addr(lds);
  const int g16 = lane >> 4, r4 = (lane >> 2) & 3, c4 = lane & 3;
  const uint32_t aR0 = base + lq * 256 + swz_rows128(lq, lg) * 16;
  const int trow = 4 * (g16 >> 1) + r4, tcol = 16 * (g16 & 1) + 4 * c4;
  const uint32_t aT0 = base + trow * 256 + (swz_rows128(trow, tcol >> 3) * 8 + (tcol & 7)) * 2;

  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no register load is pending in the loop
  __syncthreads();
  // stages 0..n_st-1 hold every key up to the tile's last row
  const int n_st = min((T + BN - 1) / BN, (qt * 256 + 255) / BN + 1);
  for (int j = 0; j < n_st; ++j) {
    if (j + 1 < n_st) load_stage(j + 1, (j + 1) & 1);
    const int k0 = j * BN;
    // wave-uniform: does any key of the stage precede a row of the wave, do all of them
    // precede every row (and lie inside T)?
    if (k0 <= q0u + 63) {
      const int mode = __builtin_amdgcn_readfirstlane(k0 + BN - 1 <= q0u && k0 + BN <= T ? 0 : 1);
      const uint32_t so = (j & 1) * STAGE_BYTES;
      const int dmj[2] = {dm[0] - k0, dm[1] - k0};
      dq128_stage(aR0 + so, aT0 + so, scale_log2, nlse, ndelta, dmj, mode, ndb);
    }
    wait_vm_all();  // stage j+1 is in LDS before any wave passes the barrier
    __syncthreads();
  }

  // The loop's last barrier freed the LDS ring: each wave stages its two dQ tiles in its
  // own 64*D slice of it for row-contiguous stores.
  f32x16 dqacc[2][4];
  dq128_read(dqacc);
  store_rows<D>(dqacc[0], scale, lds + wave * 64 * D, hd.dq, q0, T, lane);
  store_rows<D>(dqacc[1], scale, lds + wave * 64 * D + 32 * D, hd.dq, q0 + 32, T, lane);
  __syncthreads();  // the ring is free again for the caller
}

}  // namespace

// Delta and dQ for one or two 256-row tiles (a pair: the tile of rank p and its mirror,
// so every workgroup sees about the same number of key stages).  The loop is not
// unrolled, so the row body is inlined once.
__global__ __launch_bounds__(256, 1) void fa_bwd_dq_wide_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    const bf16 *__restrict__ O, const bf16 *__restrict__ dO, const float *__restrict__ LSE,
    float *__restrict__ Delta, bf16 *__restrict__ dQ, int B, int Hq, int Hkv, int T,
    float scale_log2, float scale, int paired) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];  // [stage 2][K|V][128 x 128]
  const int n_tiles = (T + 255) / 256;
  const WorkPair w = sched_item(paired, blockIdx.x, n_tiles, B, Hq, Hq / Hkv, false);
  const int G = Hq / Hkv;
  const int b = w.bh / Hq, h = w.bh - b * Hq;
  const int64_t kvh = (int64_t)b * Hkv + h / G, hs = (int64_t)T * 128, qb = w.bh * hs;
  const DqRows128 hd{Q + qb, K + kvh * hs, V + kvh * hs, O + qb, dO + qb,
                     LSE + (int64_t)w.bh * T, Delta + (int64_t)w.bh * T, dQ + qb, T};
#pragma nounroll
  for (int p = 0; p < 2; ++p) {
    const int qt = p == 0 ? w.first : w.second;
    if (qt < 0) break;
    dq_rows256(smem, hd, qt, scale_log2, scale);
  }
}

}  // namespace ttfa
