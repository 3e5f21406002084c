// Causal GQA FlashAttention forward at D = 128 over 256-row tiles (bf16 in, fp32
// accumulate, gfx950): the reference's fwd_kernel (kernels/flash_attn.py:12-67).  A
// workgroup takes 256 query rows of one (batch, head), 4 waves x 64 rows: each wave keeps
// the Q fragments and O^T accumulators of its two 32-row groups in fixed AGPRs.  The keys
// stream through LDS in 128-key stages (K and V tiles, double-buffered: 128 KB), and each
// wave's work on a stage is one hand-scheduled instruction stream (gen_fwd128_asm.py) in
// which every K row and V^T fragment read from LDS feeds the products of both row groups:
// half the LDS bytes per product of the 32-row kernel (fa_fwd.hip).
//
// The AGPR state lives outside every asm operand list, so it is only correct while the
// compiler itself touches no AGPR in this kernel.  Guards that must stay in the test
// suite: tests/test_asm_contracts.py (compiled code: no AGPR access outside the inline
// asm, no spills, no VALU write of an inline MFMA's source within two wait states) and
// the parity tests that select this kernel (test_wide_d128_kernels, which also asserts
// the kernel choice through ttfa_d128_wide, and test_config_parity[C4] / [C5]).
#include "fa_bwd.h"  // lds_addr
#include "fa_common.h"
#include "fwd128_stage.inc"

namespace ttfa {

namespace {

struct FwdRows128 {
  const bf16 *q, *k, *v;
  bf16 *o;
  float *lse;
  int T;
};

// One 128-key stage for one wave (fwd128_stage.inc), on the wave's AGPR state.  m, l:
// the running row max (scale*log2e units) and the lane's share of the row sum, per row
// group; aR0 / aT0: the lane's LDS byte addresses of the stage's k-step 0 K row read and
// (column block 0, half 0) V^T read; dm: the mask bounds; mode 0: every key visible to
// both row groups, 1: every item masked.
__device__ __forceinline__ void fwd128_stage(float (&m)[2], float (&l)[2], uint32_t aR0,
                                             uint32_t aT0, float scale_log2, const int (&dm)[2],
                                             int mode) {
  asm volatile(TTFA_FWD128_STAGE_ASM
               : "+v"(m[0]), "+v"(m[1]), "+v"(l[0]), "+v"(l[1])
               : "v"(aR0), "v"(aT0), "s"(scale_log2), "v"(dm[0]), "v"(dm[1]), "s"(mode)
               : TTFA_FWD128_STAGE_CLOBBERS, "memory");
}

// The wave's AGPR state for one row tile: Q fragments in, accumulators zeroed.
__device__ __forceinline__ void fwd128_init(const bf16x8 (&qf)[2][8]) {
  asm volatile(TTFA_FWD128_INIT_ASM
               :
               : "{v[0:3]}"(qf[0][0]), "{v[4:7]}"(qf[0][1]), "{v[8:11]}"(qf[0][2]),
                 "{v[12:15]}"(qf[0][3]), "{v[16:19]}"(qf[0][4]), "{v[20:23]}"(qf[0][5]),
                 "{v[24:27]}"(qf[0][6]), "{v[28:31]}"(qf[0][7]), "{v[32:35]}"(qf[1][0]),
                 "{v[36:39]}"(qf[1][1]), "{v[40:43]}"(qf[1][2]), "{v[44:47]}"(qf[1][3]),
                 "{v[48:51]}"(qf[1][4]), "{v[52:55]}"(qf[1][5]), "{v[56:59]}"(qf[1][6]),
                 "{v[60:63]}"(qf[1][7])
               : TTFA_FWD128_AGPR_CLOBBERS);
}

// The O^T accumulators back from the AGPR state.
__device__ __forceinline__ void fwd128_read(f32x16 (&o)[2][4]) {
  asm volatile(TTFA_FWD128_READ_ASM
               : "={v[0:15]}"(o[0][0]), "={v[16:31]}"(o[0][1]), "={v[32:47]}"(o[0][2]),
                 "={v[48:63]}"(o[0][3]), "={v[64:79]}"(o[1][0]), "={v[80:95]}"(o[1][1]),
                 "={v[96:111]}"(o[1][2]), "={v[112:127]}"(o[1][3]));
}

// All 256 query rows of row tile qt of one head.  Ends with a workgroup barrier, so the
// caller may reuse the LDS ring right away.
__device__ __forceinline__ void fwd_rows256(bf16 *lds, const FwdRows128 &hd, int qt,
                                            float scale_log2) {
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

  // Q^T as B operand: lane (lq, lg) slot s of step kk holds Q[row][16kk + 8lg + s].
  const auto rq = make_rsrc(hd.q, head_bytes);
  bf16x8 qf[2][8];
  int dm[2];
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    const int qrow = q0 + 32 * qg + lq;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      qf[qg][kk] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(qrow * D + 16 * kk + 8 * lg) * 2));
    // a key is masked when its offset in the stage minus 4lg exceeds
    // min(row, T-1) - (first key of the stage) - 4lg
    dm[qg] = min(qrow, T - 1) - 4 * lg;
  }
  load_stage(0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): Q (and the first stage) complete
  fwd128_init(qf);
  __syncthreads();

  const uint32_t base = lds_addr(lds);
  const int g16 = lane >> 4, r4 = (lane >> 2) & 3, c4 = lane & 3;
  const uint32_t aR0 = base + lq * 256 + swz_rows128(lq, lg) * 16;
  const int trow = 4 * (g16 >> 1) + r4, tcol = 16 * (g16 & 1) + 4 * c4;
  const uint32_t aT0 = base + trow * 256 + (swz_rows128(trow, tcol >> 3) * 8 + (tcol & 7)) * 2;

  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
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
      fwd128_stage(m, l, aR0 + so, aT0 + so, scale_log2, dmj, mode);
    }
    wait_vm_all();  // stage j+1 is in LDS before any wave passes the barrier
    __syncthreads();
  }

  // The loop's last barrier freed the LDS ring: each wave stages its two O tiles in its
  // own 64*D slice of it for row-contiguous stores.
  f32x16 o[2][4];
  fwd128_read(o);
#pragma unroll
  for (int qg = 0; qg < 2; ++qg) {
    const float lt = xhalf_sum(l[qg]);
    store_rows<D>(o[qg], 1.f / lt, lds + wave * 64 * D + 32 * D * qg, hd.o, q0 + 32 * qg, T, lane);
    const int qrow = q0 + 32 * qg + lq;
    if (qrow < T && lg == 0) hd.lse[qrow] = (m[qg] + __log2f(lt)) * kLn2;
  }
  __syncthreads();  // the ring is free again for the caller
}

}  // namespace

// One or two 256-row tiles (a pair: the tile of rank p and its mirror, so every
// workgroup sees about the same number of key stages).  The loop is not unrolled, so the
// row body is inlined once.
__global__ __launch_bounds__(256, 1) void fa_fwd_wide_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    bf16 *__restrict__ O, float *__restrict__ LSE, int B, int Hq, int Hkv, int T,
    float scale_log2, int paired) {
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];  // [stage 2][K|V][128 x 128]
  const int n_tiles = (T + 255) / 256;
  const WorkPair w = sched_item(paired, blockIdx.x, n_tiles, B, Hq, Hq / Hkv, false);
  const int G = Hq / Hkv;
  const int b = w.bh / Hq, h = w.bh - b * Hq;
  const int64_t kvh = (int64_t)b * Hkv + h / G, hs = (int64_t)T * 128;
  const FwdRows128 hd{Q + w.bh * hs, K + kvh * hs, V + kvh * hs, O + w.bh * hs,
                      LSE + (int64_t)w.bh * T, T};
#pragma nounroll
  for (int p = 0; p < 2; ++p) {
    const int qt = p == 0 ? w.first : w.second;
    if (qt < 0) break;
    fwd_rows256(smem, hd, qt, scale_log2);
  }
}

}  // namespace ttfa
