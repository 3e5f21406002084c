// Causal GQA attention forward/backward in fp32 (the reference's fp32 configuration,
// which must agree with the fp32 eager path to 1e-5) on the fp32 matrix cores.
//
// Same contract as the bf16 kernels (kernels/flash_attn.py:12-217): O, natural-log
// LSE, Delta = rowsum(O*dO), dQ, and dK/dV reduced over the query-head group without
// atomics.  The reference feeds fp32 through the same tiled dot products as bf16
// (kernels/flash_attn.py:49,60); here every product is v_mfma_f32_16x16x4_f32 (fp32
// operands, fp32 accumulate) and the exponentials are the accurate expf / logf.
//
// Work split: 16-row blocks.  A workgroup owns one 16-row query block (forward, dQ) or
// one 16-key block (dK/dV); its waves (eight at D = 64, four at D = 128) take the
// block's partner blocks round-robin (the key blocks at or below the diagonal, or the
// query blocks at or above it over the head group), each with its own partial result,
// and the partials are merged through LDS in wave order, so results do not depend on
// timing.
//
// Data path: every 16-row block of Q, K, V, O or dO crosses global memory once per use,
// in fully coalesced 16-byte loads (consecutive lanes read consecutive 16 bytes), into
// registers one block ahead of its use; at its turn the wave writes it to a
// wave-private LDS tile and reads the MFMA operands back from there.  (Loading the
// operands straight from global memory makes every load instruction touch 16 rows,
// which saturates the per-CU load pipeline long before HBM or L2.)
//
// MFMA 16x16x4 lane layout (lane = 16 j + n): A supplies A[n][j], B supplies B[j][n],
// and register r of the result is D[4 j + r][n].  A contraction over D features uses
// feature (D / 4) j + kk at k-step kk, so each lane's operand is one contiguous quarter
// of a row ("row fragment").  A contraction over a block's 16 rows uses row 4 j + r at
// k-step r, which is exactly what the lane holds of a previous product: a product's
// result feeds the next one as its B operand with no data movement; the other operand
// is a column of a block ("column fragment").
#include "fa_common.h"
#include "fa_kernels.h"

namespace ttfa {

namespace {

constexpr int kF32Rows = 16;  // rows per block

// Waves per workgroup: eight at D = 64 (two per SIMD, so one wave's dependent product
// chain overlaps the other's), four at D = 128, whose operand registers do not leave
// room for two waves per SIMD.
template <int D>
constexpr int f32_waves() {
  return D == 64 ? 8 : 4;
}

// One LDS tile: a 16-row block, rows padded to D + 4 floats.
template <int D>
constexpr int tile_floats() {
  return kF32Rows * (D + 4);
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sum / max over the four lanes n, n + 16, n + 32, n + 48 (the lane groups j).
__device__ __forceinline__ float group_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ float group_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

// A 16-row block in registers: load i of lane l holds floats [4 (64 i + l), + 4) of the
// row-major block (rows past the last valid row, last, repeat it).
template <int D>
struct BlockRegs {
  f32x4 v[D / 16];
};

template <int D>
__device__ __forceinline__ void load_block(BlockRegs<D> &b, const float *__restrict__ base,
                                           int row0, int last, int lane) {
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int e = 64 * i + lane, row = e / (D / 4), c4 = e % (D / 4);
    b.v[i] = *reinterpret_cast<const f32x4 *>(base + (int64_t)min(row0 + row, last) * D + 4 * c4);
  }
}

template <int D>
__device__ __forceinline__ void store_block(float *tile, const BlockRegs<D> &b, int lane) {
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int e = 64 * i + lane, row = e / (D / 4), c4 = e % (D / 4);
    *reinterpret_cast<f32x4 *>(tile + row * (D + 4) + 4 * c4) = b.v[i];
  }
}

// Row fragment of tile row n: features (D/4) j .. (D/4) j + D/4 - 1.
template <int D>
__device__ __forceinline__ void read_rowfrag(float (&f)[D / 4], const float *tile, int j, int n) {
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(tile + n * (D + 4) + (D / 4) * j + 4 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * i + e] = x[e];
  }
}

// Column fragment: f[4 db + r] = tile[4 j + r][16 db + n].
template <int D>
__device__ __forceinline__ void read_colfrag(float (&f)[D / 4], const float *tile, int j, int n) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int db = 0; db < D / 16; ++db) f[4 * db + r] = tile[(4 * j + r) * (D + 4) + 16 * db + n];
}

// acc[m][n] = sum over D of a[m][:] b[n][:]: A and B both row fragments.
template <int D>
__device__ __forceinline__ f32x4 dot_block(const float (&a)[D / 4], const float (&b)[D / 4]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < D / 4; ++kk) acc = mfma4(a[kk], b[kk], acc);
  return acc;
}

// acc[db] (features 16 db + 4 j + r', column n) += sum over the block's rows of
// col[row][feature] * w[row][n]; w is a product result (register r = row 4 j + r).
template <int D>
__device__ __forceinline__ void accum_cols(f32x4 (&acc)[D / 16], const float (&col)[D / 4],
                                           const f32x4 &w) {
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[db] = mfma4(col[4 * db + r], w[r], acc[db]);
}

// Write a wave's partial (lane: features 16 db + 4 j + r of row n) into a tile.
template <int D>
__device__ __forceinline__ void put_partial(float *tile, const f32x4 (&acc)[D / 16], int j,
                                            int n) {
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
    *reinterpret_cast<f32x4 *>(tile + n * (D + 4) + 16 * db + 4 * j) = acc[db];
}

// The merge gives each thread of the workgroup a chunk of CH consecutive features of
// one row: 16 rows x D features over 64 NW threads.
template <int D, int NW>
struct Merge {
  static constexpr int CH = D / (4 * NW);
  int row, c0;
  __device__ Merge() : row(threadIdx.x / (4 * NW)), c0((threadIdx.x % (4 * NW)) * CH) {}
};

template <int CH>
__device__ __forceinline__ void store_chunk(float *dst, const float (&x)[CH], float mul) {
  if constexpr (CH == 2) {
    *reinterpret_cast<f32x2 *>(dst) = f32x2{x[0] * mul, x[1] * mul};
  } else {
#pragma unroll
    for (int e = 0; e < CH; e += 4)
      *reinterpret_cast<f32x4 *>(dst + e) =
          f32x4{x[e] * mul, x[e + 1] * mul, x[e + 2] * mul, x[e + 3] * mul};
  }
}

// Workgroup -> (head bh, block) with the longest blocks first: the forward and dQ
// blocks grow with their index, the dK/dV blocks shrink.
__device__ __forceinline__ void block_of(int bid, int n_bh, int n_blk, bool long_is_low,
                                         int &bh, int &blk) {
  const int rank = bid / n_bh;
  bh = bid - rank * n_bh;
  blk = long_is_low ? rank : n_blk - 1 - rank;
}

// LDS of a workgroup: TPW tiles per wave, wave w's at w * TPW tiles.  A wave's merge
// partials go into its own first tiles, after its last block, so no barrier separates
// the loop from the partial writes.
template <int D, int TPW>
__device__ __forceinline__ float *wave_tiles(float *lds, int wave) {
  return lds + wave * TPW * tile_floats<D>();
}

}  // namespace

template <int D>
__global__ __launch_bounds__(64 * f32_waves<D>()) void fa_fwd_f32_kernel(const float *__restrict__ Q,
                                                         const float *__restrict__ K,
                                                         const float *__restrict__ V,
                                                         float *__restrict__ O,
                                                         float *__restrict__ LSE, int Hq,
                                                         int Hkv, int T, int n_bh,
                                                         float scale) {
  constexpr int NW = f32_waves<D>(), TPW = 2;
  __shared__ __attribute__((aligned(16))) float lds[NW * TPW * tile_floats<D>()];
  __shared__ float pm[NW][kF32Rows], pl[NW][kF32Rows];
  const int n_blk = (T + kF32Rows - 1) / kF32Rows;
  int bh, qb;
  block_of(blockIdx.x, n_bh, n_blk, false, bh, qb);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane >> 4, n = lane & 15;
  const int G = Hq / Hkv;
  const int64_t kvh = (int64_t)(bh / Hq) * Hkv + (bh % Hq) / G;
  const float *Kh = K + kvh * T * D, *Vh = V + kvh * T * D;
  const int q0 = qb * kF32Rows, last = T - 1;
  float *tk = wave_tiles<D, TPW>(lds, wave), *tv = tk + tile_floats<D>();

  struct Blk {
    BlockRegs<D> k, v;
  };
  Blk nxt;
  int kb = wave;
  if (kb <= qb) {
    load_block<D>(nxt.k, Kh, kb * kF32Rows, last, lane);
    load_block<D>(nxt.v, Vh, kb * kF32Rows, last, lane);
  }
  float qf[D / 4];
  {
    BlockRegs<D> qr;
    load_block<D>(qr, Q + (int64_t)bh * T * D, q0, last, lane);
    store_block<D>(tk, qr, lane);
    read_rowfrag<D>(qf, tk, j, n);
  }

  float m = -INFINITY, lsum = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (; kb <= qb; kb += NW) {
    const Blk cur = nxt;
    if (kb + NW <= qb) {  // in flight during this block
      load_block<D>(nxt.k, Kh, (kb + NW) * kF32Rows, last, lane);
      load_block<D>(nxt.v, Vh, (kb + NW) * kF32Rows, last, lane);
    }
    store_block<D>(tk, cur.k, lane);
    store_block<D>(tv, cur.v, lane);
    float kf[D / 4];
    read_rowfrag<D>(kf, tk, j, n);
    // S^T block: register r = score of key 16 kb + 4 j + r for query q0 + n.
    const f32x4 st = dot_block<D>(kf, qf);
    f32x4 s;
    float bm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = st[r] * scale;
      if (kb == qb && 4 * j + r > n) s[r] = -INFINITY;  // key after the query
      bm = fmaxf(bm, s[r]);
    }
    const float m_new = fmaxf(m, group_max(bm));  // finite: key 16 kb precedes every query
    const float alpha = expf(m - m_new);
    f32x4 p;
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = expf(s[r] - m_new);
    lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m = m_new;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) acc[db] *= alpha;
    float vc[D / 4];
    read_colfrag<D>(vc, tv, j, n);
    accum_cols<D>(acc, vc, p);
  }
  lsum = group_sum(lsum);

  put_partial<D>(tk, acc, j, n);
  if (j == 0) {
    pm[wave][n] = m;
    pl[wave][n] = lsum;
  }
  __syncthreads();
  // Merge, waves in order.
  using M = Merge<D, NW>;
  const M mg;
  const int row = mg.row, q = q0 + row;
  if (q >= T) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) mx = fmaxf(mx, pm[w][row]);
  float L = 0.f, out[M::CH];
#pragma unroll
  for (int e = 0; e < M::CH; ++e) out[e] = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float cw = pm[w][row] == -INFINITY ? 0.f : expf(pm[w][row] - mx);
    L += cw * pl[w][row];
    const float *src = wave_tiles<D, TPW>(lds, w) + row * (D + 4) + mg.c0;
#pragma unroll
    for (int e = 0; e < M::CH; ++e) out[e] += cw * src[e];
  }
  store_chunk<M::CH>(O + ((int64_t)bh * T + q) * D + mg.c0, out, 1.f / L);
  if (mg.c0 == 0) LSE[(int64_t)bh * T + q] = mx + logf(L);
}

// Arguments of the backward passes.
struct F32Bwd {
  const float *Q, *K, *V, *O, *dO, *LSE;
  float *Delta, *dQ, *dK, *dV;
  int Hq, Hkv, T;
  float scale;
};

// Delta and dQ of query block qb of head bh (LDS: NW * 2 tiles).
template <int D>
__device__ __forceinline__ void dq_block(float *lds, const F32Bwd &a, int bh, int qb) {
  constexpr int NW = f32_waves<D>(), TPW = 2;
  const int Hq = a.Hq, Hkv = a.Hkv, T = a.T;
  const float scale = a.scale;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane >> 4, n = lane & 15;
  const int G = Hq / Hkv;
  const int64_t kvh = (int64_t)(bh / Hq) * Hkv + (bh % Hq) / G;
  const float *Kh = a.K + kvh * T * D, *Vh = a.V + kvh * T * D;
  const int q0 = qb * kF32Rows, last = T - 1;
  float *tk = wave_tiles<D, TPW>(lds, wave), *tv = tk + tile_floats<D>();

  struct Blk {
    BlockRegs<D> k, v;
  };
  Blk nxt;
  int kb = wave;
  if (kb <= qb) {
    load_block<D>(nxt.k, Kh, kb * kF32Rows, last, lane);
    load_block<D>(nxt.v, Vh, kb * kF32Rows, last, lane);
  }
  const int64_t hb = (int64_t)bh * T;
  float qf[D / 4], dof[D / 4], delta;
  {
    BlockRegs<D> qr, dor, orr;
    load_block<D>(qr, a.Q + hb * D, q0, last, lane);
    load_block<D>(dor, a.dO + hb * D, q0, last, lane);
    load_block<D>(orr, a.O + hb * D, q0, last, lane);
    store_block<D>(tk, qr, lane);
    store_block<D>(tv, dor, lane);
    read_rowfrag<D>(qf, tk, j, n);
    read_rowfrag<D>(dof, tv, j, n);
    float of[D / 4];
    store_block<D>(tk, orr, lane);
    read_rowfrag<D>(of, tk, j, n);
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < D / 4; ++i) d = __builtin_fmaf(of[i], dof[i], d);
    delta = group_sum(d);
  }
  const int64_t qrow = hb + min(q0 + n, last);
  const float lse = a.LSE[qrow];
  if (wave == 0 && j == 0 && q0 + n < T) a.Delta[qrow] = delta;

  f32x4 acc[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (; kb <= qb; kb += NW) {
    const Blk cur = nxt;
    if (kb + NW <= qb) {  // in flight during this block
      load_block<D>(nxt.k, Kh, (kb + NW) * kF32Rows, last, lane);
      load_block<D>(nxt.v, Vh, (kb + NW) * kF32Rows, last, lane);
    }
    store_block<D>(tk, cur.k, lane);
    store_block<D>(tv, cur.v, lane);
    float kf[D / 4], vf[D / 4];
    read_rowfrag<D>(kf, tk, j, n);
    read_rowfrag<D>(vf, tv, j, n);
    const f32x4 st = dot_block<D>(kf, qf);   // S^T: key 16 kb + 4 j + r, query q0 + n
    const f32x4 dpt = dot_block<D>(vf, dof);  // dP^T, same layout
    f32x4 ds;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = (kb == qb && 4 * j + r > n) ? 0.f : expf(st[r] * scale - lse);
      ds[r] = p * (dpt[r] - delta);
    }
    float kc[D / 4];
    read_colfrag<D>(kc, tk, j, n);
    accum_cols<D>(acc, kc, ds);  // dQ^T += K^T dS^T
  }

  put_partial<D>(tk, acc, j, n);
  __syncthreads();
  using M = Merge<D, NW>;
  const M mg;
  const int q = q0 + mg.row;
  if (q >= T) return;
  float out[M::CH];
#pragma unroll
  for (int e = 0; e < M::CH; ++e) out[e] = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float *src = wave_tiles<D, TPW>(lds, w) + mg.row * (D + 4) + mg.c0;
#pragma unroll
    for (int e = 0; e < M::CH; ++e) out[e] += src[e];
  }
  store_chunk<M::CH>(a.dQ + (hb + q) * D + mg.c0, out, scale);
}

template <bool OWN_DELTA>
constexpr int dkdv_tiles() {
  return OWN_DELTA ? 3 : 2;
}

// dK and dV of key block kb of KV head bhk (LDS: NW * dkdv_tiles tiles).  OWN_DELTA:
// form each query row's Delta from O and dO (the same sums, in the same order, as
// dq_block) instead of reading it, so this pass need not wait for the dQ pass.
template <int D, bool OWN_DELTA>
__device__ __forceinline__ void dkdv_block(float *lds, const F32Bwd &a, int bhk, int kb) {
  constexpr int NW = f32_waves<D>(), TPW = dkdv_tiles<OWN_DELTA>();
  const int Hq = a.Hq, Hkv = a.Hkv, T = a.T;
  const float scale = a.scale;
  const int n_blk = (T + kF32Rows - 1) / kF32Rows;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane >> 4, n = lane & 15;
  const int G = Hq / Hkv;
  const int b = bhk / Hkv, hk = bhk - b * Hkv;
  const int k0 = kb * kF32Rows, last = T - 1;
  float *tq = wave_tiles<D, TPW>(lds, wave), *tdo = tq + tile_floats<D>();
  float *to = tdo + tile_floats<D>();  // OWN_DELTA only

  // Items: (query head g of the group, query block qb >= kb), g-major; wave w takes the
  // items w, w + NW, ...
  const int per_g = n_blk - kb, n_items = G * per_g;
  struct Item {
    BlockRegs<D> q, dout;
    BlockRegs<OWN_DELTA ? D : 16> o;
    float lse[4], delta[4];
  };
  auto load_item = [&](Item &it, int i) {
    const int g = i / per_g, qb = kb + (i - g * per_g);
    const int64_t qh = (int64_t)b * Hq + hk * G + g;
    const int q0 = qb * kF32Rows;
    load_block<D>(it.q, a.Q + qh * T * D, q0, last, lane);
    load_block<D>(it.dout, a.dO + qh * T * D, q0, last, lane);
    if constexpr (OWN_DELTA) load_block<D>(it.o, a.O + qh * T * D, q0, last, lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t x = qh * T + min(q0 + 4 * j + r, last);
      it.lse[r] = a.LSE[x];
      if constexpr (!OWN_DELTA) it.delta[r] = a.Delta[x];
    }
  };
  Item nxt;
  int i = wave;
  if (i < n_items) load_item(nxt, i);

  // K^T, V^T as B operands: row fragments of key k0 + n.
  float kf[D / 4], vf[D / 4];
  {
    BlockRegs<D> kr, vr;
    const int64_t hb = (int64_t)bhk * T * D;
    load_block<D>(kr, a.K + hb, k0, last, lane);
    load_block<D>(vr, a.V + hb, k0, last, lane);
    store_block<D>(tq, kr, lane);
    store_block<D>(tdo, vr, lane);
    read_rowfrag<D>(kf, tq, j, n);
    read_rowfrag<D>(vf, tdo, j, n);
  }

  f32x4 dk[D / 16], dv[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) dk[db] = dv[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (; i < n_items; i += NW) {
    const Item cur = nxt;
    if (i + NW < n_items) load_item(nxt, i + NW);  // in flight during this item
    const int g = i / per_g, qb = kb + (i - g * per_g), q0 = qb * kF32Rows;
    store_block<D>(tq, cur.q, lane);
    store_block<D>(tdo, cur.dout, lane);
    float qa[D / 4], doa[D / 4];
    read_rowfrag<D>(qa, tq, j, n);
    read_rowfrag<D>(doa, tdo, j, n);
    // S and dP: register r = query q0 + 4 j + r, key k0 + n.
    const f32x4 s = dot_block<D>(qa, kf);
    const f32x4 dp = dot_block<D>(doa, vf);
    float delta[4];
    if constexpr (OWN_DELTA) {
      // Delta of row q0 + n in every lane of column n, then row q0 + 4 j + r from lane 4 j + r.
      float oa[D / 4];
      store_block<D>(to, cur.o, lane);
      read_rowfrag<D>(oa, to, j, n);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < D / 4; ++e) d = __builtin_fmaf(oa[e], doa[e], d);
      d = group_sum(d);
#pragma unroll
      for (int r = 0; r < 4; ++r) delta[r] = __shfl(d, 4 * j + r);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) delta[r] = cur.delta[r];
    }
    f32x4 p, ds;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = q0 + 4 * j + r;
      const bool keep = q < T && (qb != kb || n <= 4 * j + r);
      p[r] = keep ? expf(s[r] * scale - cur.lse[r]) : 0.f;
      ds[r] = p[r] * (dp[r] - delta[r]);
    }
    float col[D / 4];
    read_colfrag<D>(col, tdo, j, n);
    accum_cols<D>(dv, col, p);   // dV^T += dO^T P
    read_colfrag<D>(col, tq, j, n);
    accum_cols<D>(dk, col, ds);  // dK^T += Q^T dS
  }

  put_partial<D>(tq, dk, j, n);
  put_partial<D>(tdo, dv, j, n);
  __syncthreads();
  using M = Merge<D, NW>;
  const M mg;
  const int key = k0 + mg.row;
  if (key >= T) return;
  float ok[M::CH], ov[M::CH];
#pragma unroll
  for (int e = 0; e < M::CH; ++e) ok[e] = ov[e] = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float *src = wave_tiles<D, TPW>(lds, w) + mg.row * (D + 4) + mg.c0;
#pragma unroll
    for (int e = 0; e < M::CH; ++e) {
      ok[e] += src[e];
      ov[e] += src[tile_floats<D>() + e];
    }
  }
  const int64_t o = ((int64_t)bhk * T + key) * D + mg.c0;
  store_chunk<M::CH>(a.dK + o, ok, scale);
  store_chunk<M::CH>(a.dV + o, ov, 1.f);
}

template <int D>
__global__ __launch_bounds__(64 * f32_waves<D>()) void fa_bwd_dq_f32_kernel(F32Bwd a,
                                                                             int n_bh) {
  __shared__ __attribute__((aligned(16))) float lds[f32_waves<D>() * 2 * tile_floats<D>()];
  int bh, qb;
  block_of(blockIdx.x, n_bh, (a.T + kF32Rows - 1) / kF32Rows, false, bh, qb);
  dq_block<D>(lds, a, bh, qb);
}

template <int D>
__global__ __launch_bounds__(64 * f32_waves<D>()) void fa_bwd_dkdv_f32_kernel(F32Bwd a,
                                                                               int n_bhk) {
  __shared__ __attribute__((aligned(16))) float lds[f32_waves<D>() * 2 * tile_floats<D>()];
  int bhk, kb;
  block_of(blockIdx.x, n_bhk, (a.T + kF32Rows - 1) / kF32Rows, true, bhk, kb);
  dkdv_block<D, false>(lds, a, bhk, kb);
}

// Both backward passes in one launch: the dK/dV workgroups form Delta themselves, so
// they run beside the dQ workgroups instead of after them.  Workgroups go rank-major,
// longest first in both roles: rank r holds the dK/dV blocks of key block r, then the
// dQ blocks of query block n_blk - 1 - r.
template <int D>
__global__ __launch_bounds__(64 * f32_waves<D>()) void fa_bwd_f32_kernel(F32Bwd a, int n_bh,
                                                                          int n_bhk) {
  __shared__ __attribute__((aligned(16))) float lds[f32_waves<D>() * 3 * tile_floats<D>()];
  const int n_blk = (a.T + kF32Rows - 1) / kF32Rows;
  const int per_rank = n_bhk + n_bh;
  const int rank = blockIdx.x / per_rank, x = blockIdx.x - rank * per_rank;
  if (x < n_bhk)
    dkdv_block<D, true>(lds, a, x, rank);
  else
    dq_block<D>(lds, a, x - n_bhk, n_blk - 1 - rank);
}

static unsigned blocks_grid(int n_bh, int T) {
  return (unsigned)((int64_t)n_bh * ((T + kF32Rows - 1) / kF32Rows));
}

static dim3 f32_block(int D) { return dim3(64 * (D == 64 ? f32_waves<64>() : f32_waves<128>())); }

static F32Bwd bwd_args(const void *q, const void *k, const void *v, const void *o,
                       const void *dout, const float *lse, float *delta, void *dq, void *dk,
                       void *dv, int Hq, int Hkv, int T, float scale) {
  return F32Bwd{(const float *)q, (const float *)k, (const float *)v, (const float *)o,
                (const float *)dout, lse, delta, (float *)dq, (float *)dk, (float *)dv,
                Hq, Hkv, T, scale};
}

hipError_t launch_fwd_f32(const void *q, const void *k, const void *v, void *o, float *lse,
                          int B, int Hq, int Hkv, int T, int D, float scale, hipStream_t stream) {
  const dim3 grid(blocks_grid(B * Hq, T)), block = f32_block(D);
  if (D == 64)
    fa_fwd_f32_kernel<64><<<grid, block, 0, stream>>>((const float *)q, (const float *)k,
                                                      (const float *)v, (float *)o, lse, Hq,
                                                      Hkv, T, B * Hq, scale);
  else
    fa_fwd_f32_kernel<128><<<grid, block, 0, stream>>>((const float *)q, (const float *)k,
                                                       (const float *)v, (float *)o, lse, Hq,
                                                       Hkv, T, B * Hq, scale);
  return hipGetLastError();
}

hipError_t launch_bwd_dq_f32(const void *q, const void *k, const void *v, const void *o,
                             const void *dout, const float *lse, float *delta, void *dq,
                             int B, int Hq, int Hkv, int T, int D, float scale,
                             hipStream_t stream) {
  const F32Bwd a = bwd_args(q, k, v, o, dout, lse, delta, dq, nullptr, nullptr, Hq, Hkv, T, scale);
  const dim3 grid(blocks_grid(B * Hq, T)), block = f32_block(D);
  if (D == 64)
    fa_bwd_dq_f32_kernel<64><<<grid, block, 0, stream>>>(a, B * Hq);
  else
    fa_bwd_dq_f32_kernel<128><<<grid, block, 0, stream>>>(a, B * Hq);
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_f32(const void *q, const void *k, const void *v, const void *dout,
                               const float *lse, const float *delta, void *dk, void *dv,
                               int B, int Hq, int Hkv, int T, int D, float scale,
                               hipStream_t stream) {
  const F32Bwd a = bwd_args(q, k, v, nullptr, dout, lse, const_cast<float *>(delta), nullptr,
                            dk, dv, Hq, Hkv, T, scale);
  const dim3 grid(blocks_grid(B * Hkv, T)), block = f32_block(D);
  if (D == 64)
    fa_bwd_dkdv_f32_kernel<64><<<grid, block, 0, stream>>>(a, B * Hkv);
  else
    fa_bwd_dkdv_f32_kernel<128><<<grid, block, 0, stream>>>(a, B * Hkv);
  return hipGetLastError();
}

hipError_t launch_bwd_f32(const void *q, const void *k, const void *v, const void *o,
                          const void *dout, const float *lse, float *delta, void *dq, void *dk,
                          void *dv, int B, int Hq, int Hkv, int T, int D, float scale,
                          hipStream_t stream) {
  const F32Bwd a = bwd_args(q, k, v, o, dout, lse, delta, dq, dk, dv, Hq, Hkv, T, scale);
  const dim3 grid(blocks_grid(B * Hq + B * Hkv, T)), block = f32_block(D);
  if (D == 64)
    fa_bwd_f32_kernel<64><<<grid, block, 0, stream>>>(a, B * Hq, B * Hkv);
  else
    fa_bwd_f32_kernel<128><<<grid, block, 0, stream>>>(a, B * Hq, B * Hkv);
  return hipGetLastError();
}

}  // namespace ttfa
