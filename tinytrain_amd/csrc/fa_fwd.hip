// Causal GQA FlashAttention forward, bf16 in / fp32 accumulate, gfx950.
//
// Computes what the reference's fwd_kernel computes (kernels/flash_attn.py:12-67):
// for every query row i of head h, O_i = sum_{j<=i} softmax_j(q_i.k_j * scale) v_j
// with K/V read from KV head h / G, and LSE_i = m_i + ln(l_i) in natural-log units.
//
// Work split: one workgroup = 4 waves = 128 query rows of one (batch, head); each wave
// owns 32 rows.  K/V stream through LDS in 64-key tiles, double-buffered: the next
// tile's global loads are in flight while the current tile is consumed.
//
// Per wave and tile, scores are formed transposed, S^T = K Q^T (32x32x16 MFMAs with K
// from LDS as the A operand and the wave's Q rows held in registers as the B operand),
// so every lane owns ONE query row and 16 of the 32 keys of a block: the row max and
// row sum are in-register reductions plus one v_permlane32_swap.  P^T stays in the
// result registers and feeds O^T += V^T P^T directly as the B operand; V^T comes from
// LDS through ds_read_b64_tr_b16, whose row order matches the MFMA result layout, so
// no register shuffles are needed.  O^T is rescaled per lane (one query per lane).
// Tiles entirely above the diagonal are never loaded; tiles that cross the diagonal
// or the ragged end of T are masked; all others take an unmasked path.
// Softmax runs in the exp2 domain (scale * log2(e) folded into one FMA); the stored
// LSE is converted back to natural log.
#include "fa_common.h"
#include "fa_kernels.h"

namespace ttfa {

template <int D>
__global__ __launch_bounds__(256, 2) void fa_fwd_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ K, const bf16 *__restrict__ V,
    bf16 *__restrict__ O, float *__restrict__ LSE, int B, int Hq, int Hkv, int T,
    float scale_log2) {
  constexpr int BM = 128, BN = 64;
  constexpr int KK = D / 16;           // MFMA k-steps over D
  constexpr int DB = D / 32;           // 32-row blocks of O^T
  constexpr int CH = D / 8;            // 16-byte chunks per row
  constexpr int LOADS = BN * CH / 256; // 16-byte loads per thread per K (or V) tile
  __shared__ __attribute__((aligned(16))) bf16 lds[2][2][BN * D];  // [stage][K|V]

  const int n_tiles = (T + BM - 1) / BM;
  const TileOrder to = order_tiles(blockIdx.x, n_tiles, B, Hq, Hkv);
  const int qt = n_tiles - 1 - to.tile;  // longest rows first
  const int bh = to.bh;
  const int G = Hq / Hkv;
  const int b = bh / Hq, h = bh - b * Hq;
  const int64_t kv_head = (int64_t)b * Hkv + h / G;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int q0 = qt * BM + wave * 32;  // first query row of this wave
  const int qrow = q0 + lq;

  const uint32_t head_bytes = (uint32_t)T * D * 2;
  const bf16 *Qh = Q + (int64_t)bh * T * D;
  const auto rq = make_rsrc(Qh, head_bytes);
  const auto rk = make_rsrc(K + kv_head * T * D, head_bytes);
  const auto rv = make_rsrc(V + kv_head * T * D, head_bytes);

  // Q^T as B operand: lane (lq, lg) slot s of step kk holds Q[qrow][16kk + 8lg + s].
  bf16x8 qf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    u32x4 raw = buf_load16(rq, (uint32_t)(qrow * D + 16 * kk + 8 * lg) * 2);
    qf[kk] = __builtin_bit_cast(bf16x8, raw);
  }

  const int n_kv = min((T + BN - 1) / BN, (qt + 1) * (BM / BN));

  u32x4 kreg[LOADS], vreg[LOADS];
  auto load_tile = [&](int j) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e = tid + 256 * i, row = e / CH, ch = e % CH;
      const uint32_t off = (uint32_t)((j * BN + row) * D + ch * 8) * 2;
      kreg[i] = buf_load16(rk, off);
      vreg[i] = buf_load16(rv, off);
    }
  };
  auto store_tile = [&](int stage) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int e = tid + 256 * i, row = e / CH, ch = e % CH;
      const int off = row * D + (swz(row, ch) << 3);
      *reinterpret_cast<u32x4 *>(&lds[stage][0][off]) = kreg[i];
      *reinterpret_cast<u32x4 *>(&lds[stage][1][off]) = vreg[i];
    }
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16{};
  float m_t = -INFINITY;  // running row max, in scale*log2(e) units
  float l_part = 0.f;     // this lane's share of the running row sum

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int j = 0; j < n_kv; ++j) {
    if (j + 1 < n_kv) load_tile(j + 1);
    const bf16 *Kt = lds[j & 1][0];
    const bf16 *Vt = lds[j & 1][1];
    const int k0 = j * BN;
    if (k0 <= q0 + 31) {  // some key of this tile is visible to some row of the wave
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s[kb] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          s[kb] = mfma32(lds_read_row8<D>(Kt, kb * 32 + lq, 2 * kk + lg), qf[kk], s[kb]);
      }
      if (k0 + BN - 1 > q0 || k0 + BN > T) {  // diagonal or ragged tile
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * lg + (r & 3);
            if (key > qrow || key >= T) s[kb][r] = -INFINITY;
          }
      }
      float mx = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      mx = xhalf_max(mx);
      const float m_new = fmaxf(m_t, mx * scale_log2);
      const float alpha = exp2f_fast(m_t - m_new);
      m_t = m_new;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2f_fast(__builtin_fmaf(s[kb][r], scale_log2, -m_new));
          s[kb][r] = p;
          rs += p;
        }
      l_part = l_part * alpha + rs;
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
#pragma unroll
      for (int m = 0; m < BN / 16; ++m) {
        const bf16x8 pb = pack8(s[m >> 1], 8 * (m & 1));
#pragma unroll
        for (int db = 0; db < DB; ++db)
          oacc[db] = mfma32(lds_read_trT<D>(Vt, 16 * m, 32 * db, lane), pb, oacc[db]);
      }
    }
    if (j + 1 < n_kv) store_tile((j + 1) & 1);
    __syncthreads();
  }

  const float l = xhalf_sum(l_part);
  if (qrow < T) {
    const float inv = 1.f / l;
    bf16 *Orow = O + ((int64_t)bh * T + qrow) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * db + 8 * a + 4 * lg;
        *reinterpret_cast<bf16x4 *>(Orow + d) =
            pack4(oacc[db][4 * a] * inv, oacc[db][4 * a + 1] * inv, oacc[db][4 * a + 2] * inv,
                  oacc[db][4 * a + 3] * inv);
      }
    if (lg == 0) LSE[(int64_t)bh * T + qrow] = m_t * kLn2 + __logf(l);
  }
}

hipError_t launch_fwd_bf16(const void *q, const void *k, const void *v, void *o, float *lse,
                           int B, int Hq, int Hkv, int T, int D, float scale,
                           hipStream_t stream) {
  const int n_tiles = (T + 127) / 128;
  const dim3 grid((unsigned)(n_tiles * B * Hq)), block(256);
  const float sl2 = scale * kLog2e;
  if (D == 64)
    fa_fwd_bf16_kernel<64><<<grid, block, 0, stream>>>(
        (const bf16 *)q, (const bf16 *)k, (const bf16 *)v, (bf16 *)o, lse, B, Hq, Hkv, T, sl2);
  else
    fa_fwd_bf16_kernel<128><<<grid, block, 0, stream>>>(
        (const bf16 *)q, (const bf16 *)k, (const bf16 *)v, (bf16 *)o, lse, B, Hq, Hkv, T, sl2);
  return hipGetLastError();
}

}  // namespace ttfa
