// KV-cache decode attention (bf16 in / fp32 accumulate), gfx950: Tq new query rows per
// (batch, head) against a cache of L_b keys, split over the cache length.
//
// The reference has no decode kernel: generate.py:7-20 recomputes the whole prefix for
// every token, and its roadmap lists a KV-cache inference engine (README.md:158).  What
// is computed is the reference's causal attention (model.py:94-98) restricted to the
// last Tq rows: query i of the new tokens sits at position L_b - Tq + i and sees keys
// 0 .. L_b - Tq + i of the cache, O = softmax(q k^T * scale) v, LSE = m + ln(l).
//
// Work split (split-K, "flash decoding"): the cache of every (batch, KV head) is cut into
// ranges of `wkeys` keys, one range per wave; a 256-thread workgroup runs 4 ranges.  All
// G query heads of the KV head and all Tq rows form the R = G * Tq <= 32 query columns
// of one 32x32 MFMA tile (columns past R repeat valid ones and are not stored), so the K
// and V bytes of a range are read once for the whole group.  A wave streams its range in
// 32-key blocks: the block's K fragments load straight into the MFMA A-operand registers
// (row-major rows are the A layout), V goes into a wave-private, swizzled, double-
// buffered LDS block for the transposed operand reads, and the next block's loads are in
// flight while the current one is computed (the wave waits on its own vmcnt only; no
// workgroup barriers).  Per block: S^T = K Q^T, online softmax in the exp2 domain
// (lazy rescale as in the forward kernel), O^T += V^T P^T.  Each wave writes an fp32
// partial (unnormalised O, running max m in log2 units, sum l) per query row; a second
// kernel merges the partials of a row with the log-sum-exp rule.  The memory traffic is
// the cache bytes (the roofline of decode), read once.
#include "fa_common.h"
#include "fa_kernels.h"

namespace ttfa {

namespace {

constexpr float kDecodeSlack = 8.0f;
constexpr int kDecBlock = 32;  // keys per block
constexpr int kDecWaves = 4;   // ranges (waves) per workgroup
constexpr int kDecMaxSplits = 512;  // partials per query row, at most
constexpr int kCombinePrefetch = 16;  // partial rows per merge thread loaded up front ...
constexpr int kCombinePrefetchMin = 64;  // ... when a row has at least this many partials

template <int D>
struct DecShape {
  static constexpr int KK = D / 16, DB = D / 32, CH = D / 8;
  static constexpr int VLOADS = kDecBlock * CH / 64;            // 1 KB DMA blocks per V block
  static constexpr int VMEM_PER_BLOCK = VLOADS + KK;            // vector memory ops per block
  static constexpr int WAVE_LDS = 2 * kDecBlock * D;            // bf16 elements, two stages
};

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt, lgkmcnt at max)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x0F70 | ((N >> 4) << 14));
}

// One 32-key block of one wave: S^T = K Q^T, mask, online softmax, O^T += V^T P^T.
template <int D, bool MASK>
__device__ __forceinline__ void decode_block(const bf16x8 (&kf)[D / 16], const bf16 *Vt,
                                             const bf16x8 (&qf)[D / 16], f32x16 (&oacc)[D / 32],
                                             float &m_t, float &l_part, float scale_log2, int k0,
                                             int pos, int L, int lane) {
  using P = DecShape<D>;
  const int lg = lane >> 5;
  f32x16 s = mfma32(kf[0], qf[0], f32x16{});
#pragma unroll
  for (int kk = 1; kk < P::KK; ++kk) s = mfma32(kf[kk], qf[kk], s);
  if (MASK) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + 8 * (r >> 2) + 4 * lg + (r & 3);
      if (key > pos || key >= L) s[r] = -INFINITY;
    }
  }
  const float mx = xhalf_max(max16(s, -INFINITY)) * scale_log2;
  if (__builtin_amdgcn_ballot_w64(mx > m_t + kDecodeSlack)) {
    const float m_new = fmax2(m_t, mx);
    // 0 when m_t is still -inf; 1 for a column that stays all-masked (m_new = -inf; its
    // sums are still 0), where exp2(-inf - -inf) would be NaN
    const float alpha = m_new == -INFINITY ? 1.f : exp2f_fast(m_t - m_new);
    m_t = m_new;
    l_part *= alpha;
#pragma unroll
    for (int db = 0; db < P::DB; ++db) oacc[db] *= alpha;
  }
  // A column none of whose keys so far is visible keeps m = -inf; its p are all 0.
  const float m_use = m_t == -INFINITY ? 0.f : m_t;
  bf16x8 pb[2];
  float rs = 0.f;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = exp2f_fast(__builtin_fmaf(s[8 * m + e], scale_log2, -m_use));
      rs += p[e];
    }
    pb[m] = pack8(f32x16{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]}, 0);
  }
  l_part += rs;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    bf16x8 vf[P::DB];
#pragma unroll
    for (int db = 0; db < P::DB; ++db) vf[db] = lds_read_trT<D>(Vt, 16 * m, 32 * db, lane);
#pragma unroll
    for (int db = 0; db < P::DB; ++db) oacc[db] = mfma32(vf[db], pb[m], oacc[db]);
  }
}

}  // namespace

// Grid: B * Hkv * n_chunks workgroups of 4 waves; wave w of chunk c owns keys
// [(4c + w) * wkeys, (4c + w + 1) * wkeys) of its (batch, KV head).  Partial rows are
// indexed (b * Hq + h) * Tq + i, each with n_splits = 4 * n_chunks slots.
template <int D>
__global__ __launch_bounds__(256, 2) void fa_decode_bf16_kernel(
    const bf16 *__restrict__ Q, const bf16 *__restrict__ Kc, const bf16 *__restrict__ Vc,
    const int *__restrict__ cache_seqlens, float *__restrict__ part_o,
    float *__restrict__ part_ml, int B, int Hq, int Hkv, int Tq, int Lmax, int n_chunks,
    int wkeys, float scale_log2) {
  using P = DecShape<D>;
  constexpr int KK = P::KK, DB = P::DB, CH = P::CH;
  __shared__ __attribute__((aligned(16))) bf16 lds[kDecWaves][P::WAVE_LDS];
  const int chunk = blockIdx.x % n_chunks, bhk = blockIdx.x / n_chunks;
  const int b = bhk / Hkv, hk = bhk - b * Hkv;
  const int G = Hq / Hkv, R = G * Tq;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lq = lane & 31, lg = lane >> 5;
  const int split = chunk * kDecWaves + wave, n_splits = n_chunks * kDecWaves;
  const int L = min(max(cache_seqlens[b], 0), Lmax);

  // this lane's query column
  const int col = lq % R, g = col / Tq, i = col - g * Tq;
  const int h = hk * G + g;
  const int pos = L - Tq + i;  // last visible key of this column
  const int64_t qrow = ((int64_t)b * Hq + h) * Tq + i;

  const int k_lo = split * wkeys;
  const int k_hi = min(k_lo + wkeys, L);  // keys past L do not exist
  bf16 *wl = lds[wave];

  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16{};
  float m_t = -INFINITY, l_part = 0.f;

  if (k_lo < k_hi) {
    const auto rq = make_rsrc(Q + qrow * D, (uint32_t)D * 2);
    const int64_t kvbase = ((int64_t)b * Hkv + hk) * Lmax * D;
    const uint32_t kv_bytes = (uint32_t)L * D * 2;  // keys >= L read as zero
    const auto rk = make_rsrc(Kc + kvbase, kv_bytes);
    const auto rv = make_rsrc(Vc + kvbase, kv_bytes);
    bf16x8 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      qf[kk] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(16 * kk + 8 * lg) * 2));

    auto load_k = [&](bf16x8 (&kf)[KK], int k0) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        kf[kk] = __builtin_bit_cast(
            bf16x8, buf_load16(rk, (uint32_t)((k0 + lq) * D + 16 * kk + 8 * lg) * 2));
    };
    auto load_v = [&](int k0, int stage) {  // V rows k0..k0+31 -> the wave's LDS stage
      bf16 *dst = wl + stage * kDecBlock * D;
#pragma unroll
      for (int j = 0; j < P::VLOADS; ++j) {
        const int e0 = 64 * j, e = e0 + lane, row = e / CH, pc = e % CH;
        const uint32_t off = (uint32_t)((k0 + row) * D + swz<D>(row, pc) * 8) * 2;
        buf_load16_lds(rv, off, dst + e0 * 8);
      }
    };

    bf16x8 kf[KK], kn[KK];
    load_v(k_lo, 0);
    load_k(kf, k_lo);
    const int n_blk = (k_hi - k_lo + kDecBlock - 1) / kDecBlock;
    const int first_masked = L - Tq;  // keys past this need the mask for some column
#pragma unroll 1
    for (int t = 0; t < n_blk; ++t) {
      const int k0 = k_lo + t * kDecBlock;
      const bool more = t + 1 < n_blk;
      if (more) {
        load_v(k0 + kDecBlock, (t + 1) & 1);
        load_k(kn, k0 + kDecBlock);
        wait_vmcnt<P::VMEM_PER_BLOCK>();  // block t's V (LDS) and K are in
      } else {
        wait_vmcnt<0>();
      }
      __builtin_amdgcn_sched_barrier(0);
      const bf16 *Vt = wl + (t & 1) * kDecBlock * D;
      if (k0 + kDecBlock - 1 > first_masked || k0 + kDecBlock > k_hi)
        decode_block<D, true>(kf, Vt, qf, oacc, m_t, l_part, scale_log2, k0, pos, L, lane);
      else
        decode_block<D, false>(kf, Vt, qf, oacc, m_t, l_part, scale_log2, k0, pos, L, lane);
      if (more) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) kf[kk] = kn[kk];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // partial of this wave's range for the columns it owns (lanes lq < R)
  const float l = xhalf_sum(l_part);
  if (lq < R) {
    const int64_t slot = qrow * n_splits + split;
    float *po = part_o + slot * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<f32x4 *>(po + 32 * db + 8 * a + 4 * lg) =
            f32x4{oacc[db][4 * a], oacc[db][4 * a + 1], oacc[db][4 * a + 2], oacc[db][4 * a + 3]};
    if (lg == 0) *reinterpret_cast<f32x2 *>(part_ml + slot * 2) = f32x2{m_t, l};
  }
}

// Merge the n_splits partials of every query row: M = max m over partials with l > 0,
// O = sum o_s 2^(m_s - M) / sum l_s 2^(m_s - M), LSE = (M + log2 sum) ln 2; a row with no
// visible key gets O = 0, LSE = -inf.  One 256-thread workgroup per row: thread t sums
// float4 column t % (D/4) over the partials s = t / (D/4) (mod 256 / (D/4)).  With PF > 0
// (rows with many partials) its first PF partial rows and its (m, l) pair are loaded
// before anything waits, so the row takes one memory round trip; then the threads reduce
// M and the weights (kept in LDS), and the partials are weighted (a partial without keys
// holds zeros and weight 0) and the groups added in a fixed order, so the result does not
// depend on timing (nor on PF).
template <int D, int PF>
__global__ __launch_bounds__(256) void fa_decode_combine_kernel(
    const float *__restrict__ part_o, const float *__restrict__ part_ml, bf16 *__restrict__ O,
    float *__restrict__ LSE, int rows, int n_splits) {
  constexpr int C4 = D / 4, SG = 256 / C4;
  __shared__ float wts[kDecMaxSplits];
  __shared__ float red[8];
  __shared__ f32x4 accs[SG][C4];
  const int row = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float *ml = part_ml + (int64_t)row * n_splits * 2;
  const int c = tid % C4, sg = tid / C4;
  const f32x4 *po = reinterpret_cast<const f32x4 *>(part_o + (int64_t)row * n_splits * D) + c;
  f32x4 xs[PF > 0 ? PF : 1];
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const int s = sg + j * SG;
    xs[j] = s < n_splits ? po[(int64_t)s * C4] : f32x4{};
  }
  const f32x2 v0 = tid < n_splits ? *reinterpret_cast<const f32x2 *>(ml + 2 * tid) : f32x2{0.f, 0.f};
  float M = v0[1] > 0.f ? v0[0] : -INFINITY;
  for (int s = tid + 256; s < n_splits; s += 256) {
    const f32x2 v = *reinterpret_cast<const f32x2 *>(ml + 2 * s);
    if (v[1] > 0.f) M = fmax2(M, v[0]);
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) M = fmax2(M, __shfl_xor(M, m));
  if (lane == 0) red[wave] = M;
  __syncthreads();
  M = fmax2(fmax2(red[0], red[1]), fmax2(red[2], red[3]));
  float lsum = 0.f;
  for (int s = tid; s < n_splits; s += 256) {
    const f32x2 v = s == tid ? v0 : *reinterpret_cast<const f32x2 *>(ml + 2 * s);
    const float w = (v[1] > 0.f && M != -INFINITY) ? exp2f_fast(v[0] - M) : 0.f;
    wts[s] = w;
    lsum = __builtin_fmaf(v[1] > 0.f ? v[1] : 0.f, w, lsum);
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) lsum += __shfl_xor(lsum, m);
  if (lane == 0) red[4 + wave] = lsum;
  __syncthreads();  // wts and the sums are visible
  lsum = (red[4] + red[5]) + (red[6] + red[7]);
  f32x4 acc{};
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const int s = sg + j * SG;
    const float w = s < n_splits ? wts[s] : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = w != 0.f ? __builtin_fmaf(xs[j][e], w, acc[e]) : acc[e];
  }
#pragma unroll 4
  for (int s = sg + PF * SG; s < n_splits; s += SG) {
    const f32x4 x = po[(int64_t)s * C4];
    const float w = wts[s];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = w != 0.f ? __builtin_fmaf(x[e], w, acc[e]) : acc[e];
  }
  accs[sg][c] = acc;
  __syncthreads();
  if (tid < C4) {
    f32x4 t = accs[0][tid];
#pragma unroll
    for (int g = 1; g < SG; ++g) t += accs[g][tid];
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    bf16 *out = O + (int64_t)row * D + 4 * tid;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (bf16)(t[e] * inv);
  }
  if (tid == 0) LSE[row] = lsum > 0.f ? (M + __log2f(lsum)) * kLn2 : -INFINITY;
}

// Keys per wave: enough waves to fill the device (about 2048), at least 128 keys per
// wave (so the block prefetch has work to hide behind), a multiple of 32, and at most
// kDecMaxSplits partials per query row.
DecodeSplit decode_split(int B, int Hkv, int Lmax) {
  const int64_t units = (int64_t)B * Hkv;
  const int64_t target_waves = 2048;
  int64_t per = ((int64_t)Lmax * units + target_waves - 1) / target_waves;
  per = ((per + kDecBlock - 1) / kDecBlock) * kDecBlock;
  if (per < 128) per = 128;
  int64_t waves_per_unit = ((int64_t)Lmax + per - 1) / per;
  while ((waves_per_unit + kDecWaves - 1) / kDecWaves * kDecWaves > kDecMaxSplits) {
    per *= 2;
    waves_per_unit = ((int64_t)Lmax + per - 1) / per;
  }
  DecodeSplit s;
  s.wkeys = (int)per;
  s.n_chunks = (int)((waves_per_unit + kDecWaves - 1) / kDecWaves);
  s.n_splits = s.n_chunks * kDecWaves;
  return s;
}

hipError_t launch_decode_bf16(const void *q, const void *k_cache, const void *v_cache,
                              const int *cache_seqlens, void *o, float *lse, float *workspace,
                              int B, int Hq, int Hkv, int Tq, int Lmax, int D, float scale,
                              hipStream_t stream) {
  const DecodeSplit sp = decode_split(B, Hkv, Lmax);
  const int rows = B * Hq * Tq;
  float *part_o = workspace;
  float *part_ml = workspace + (int64_t)rows * sp.n_splits * D;
  const float sl2 = scale * kLog2e;
  const dim3 grid((unsigned)((int64_t)B * Hkv * sp.n_chunks)), block(256);
  const dim3 cgrid((unsigned)rows), cblock(256);
  const bool prefetch = sp.n_splits >= kCombinePrefetchMin;
  auto combine = [&](auto kern) {
    kern<<<cgrid, cblock, 0, stream>>>(part_o, part_ml, (bf16 *)o, lse, rows, sp.n_splits);
  };
  if (D == 64) {
    fa_decode_bf16_kernel<64><<<grid, block, 0, stream>>>(
        (const bf16 *)q, (const bf16 *)k_cache, (const bf16 *)v_cache, cache_seqlens, part_o,
        part_ml, B, Hq, Hkv, Tq, Lmax, sp.n_chunks, sp.wkeys, sl2);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (prefetch)
      combine(fa_decode_combine_kernel<64, kCombinePrefetch>);
    else
      combine(fa_decode_combine_kernel<64, 0>);
  } else {
    fa_decode_bf16_kernel<128><<<grid, block, 0, stream>>>(
        (const bf16 *)q, (const bf16 *)k_cache, (const bf16 *)v_cache, cache_seqlens, part_o,
        part_ml, B, Hq, Hkv, Tq, Lmax, sp.n_chunks, sp.wkeys, sl2);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (prefetch)
      combine(fa_decode_combine_kernel<128, kCombinePrefetch>);
    else
      combine(fa_decode_combine_kernel<128, 0>);
  }
  return hipGetLastError();
}

}  // namespace ttfa
