// Causal GQA attention forward/backward in fp32 (the reference's fp32 CPU-eager
// configuration, which must agree with the fp32 eager path to 1e-5).
//
// Same contract as the bf16 kernels (kernels/flash_attn.py:12-217): O, natural-log
// LSE, Delta = rowsum(O*dO), dQ, and dK/dV reduced over the query-head group inside
// one wave without atomics.  Arithmetic is plain fp32 FMA with accurate expf/logf.
//
// Work split: one wave per row.  A wave scores 64 keys (or, for dK/dV, 64 queries) at
// a time, one per lane, does the chunk's softmax statistics with two wave reductions,
// then accumulates the D-wide row with lane = feature (D/64 features per lane).  The
// row vectors a lane dots against live in LDS.  This path favours exactness and
// simplicity over speed: fp32 attention is a correctness configuration here.
#include "fa_common.h"
#include "fa_kernels.h"

namespace ttfa {

namespace {

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <int D>
__device__ __forceinline__ float dot_row(const float *__restrict__ a_lds, const float *__restrict__ row) {
  float acc = 0.f;
#pragma unroll 8
  for (int d = 0; d < D; d += 4) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(row + d);
    acc = __builtin_fmaf(a_lds[d], x[0], acc);
    acc = __builtin_fmaf(a_lds[d + 1], x[1], acc);
    acc = __builtin_fmaf(a_lds[d + 2], x[2], acc);
    acc = __builtin_fmaf(a_lds[d + 3], x[3], acc);
  }
  return acc;
}

}  // namespace

constexpr int kF32Waves = 4;

template <int D>
__global__ __launch_bounds__(256) void fa_fwd_f32_kernel(const float *__restrict__ Q,
                                                         const float *__restrict__ K,
                                                         const float *__restrict__ V,
                                                         float *__restrict__ O,
                                                         float *__restrict__ LSE, int Hq,
                                                         int Hkv, int T, int64_t rows,
                                                         float scale) {
  constexpr int PL = D / 64;  // features per lane
  __shared__ float qs[kF32Waves][D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // Waves past the last row redo the last row and store nothing (uniform barriers).
  const int64_t wid = (int64_t)blockIdx.x * kF32Waves + wave;
  const bool valid = wid < rows;
  const int64_t rowid = valid ? wid : rows - 1;  // bh * T + i
  const int G = Hq / Hkv;
  const int bh = (int)(rowid / T), i = (int)(rowid - (int64_t)bh * T);
  const int64_t kvh = (int64_t)(bh / Hq) * Hkv + (bh % Hq) / G;
  const float *Kh = K + kvh * T * D, *Vh = V + kvh * T * D;
  const float *qrow = Q + rowid * D;
#pragma unroll
  for (int e = 0; e < PL; ++e) qs[wave][lane + 64 * e] = qrow[lane + 64 * e];
  __syncthreads();
  float m = -INFINITY, l = 0.f, acc[PL];
#pragma unroll
  for (int e = 0; e < PL; ++e) acc[e] = 0.f;
  for (int j0 = 0; j0 <= i; j0 += 64) {
    const int key = j0 + lane;
    float s = -INFINITY;
    if (key <= i) s = dot_row<D>(qs[wave], Kh + (int64_t)key * D) * scale;
    const float m_new = fmaxf(m, wave_max(s));
    const float p = key <= i ? expf(s - m_new) : 0.f;
    const float alpha = expf(m - m_new);
    l = l * alpha + wave_sum(p);
    m = m_new;
#pragma unroll
    for (int e = 0; e < PL; ++e) acc[e] *= alpha;
    const int n = min(64, i + 1 - j0);
    for (int jj = 0; jj < n; ++jj) {
      const float pj = __shfl(p, jj);
      const float *vr = Vh + (int64_t)(j0 + jj) * D;
#pragma unroll
      for (int e = 0; e < PL; ++e) acc[e] = __builtin_fmaf(pj, vr[lane + 64 * e], acc[e]);
    }
  }
  if (!valid) return;
  const float inv = 1.f / l;
#pragma unroll
  for (int e = 0; e < PL; ++e) O[rowid * D + lane + 64 * e] = acc[e] * inv;
  if (lane == 0) LSE[rowid] = m + logf(l);
}

template <int D>
__global__ __launch_bounds__(256) void fa_bwd_dq_f32_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    const float *__restrict__ O, const float *__restrict__ dO, const float *__restrict__ LSE,
    float *__restrict__ Delta, float *__restrict__ dQ, int Hq, int Hkv, int T, int64_t rows,
    float scale) {
  constexpr int PL = D / 64;
  __shared__ float qs[kF32Waves][D], dos[kF32Waves][D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * kF32Waves + wave;
  const bool valid = wid < rows;
  const int64_t rowid = valid ? wid : rows - 1;
  const int G = Hq / Hkv;
  const int bh = (int)(rowid / T), i = (int)(rowid - (int64_t)bh * T);
  const int64_t kvh = (int64_t)(bh / Hq) * Hkv + (bh % Hq) / G;
  const float *Kh = K + kvh * T * D, *Vh = V + kvh * T * D;
  float dpart = 0.f;
#pragma unroll
  for (int e = 0; e < PL; ++e) {
    const int64_t x = rowid * D + lane + 64 * e;
    qs[wave][lane + 64 * e] = Q[x];
    dos[wave][lane + 64 * e] = dO[x];
    dpart = __builtin_fmaf(O[x], dO[x], dpart);
  }
  const float delta = wave_sum(dpart);
  const float lse = LSE[rowid];
  if (lane == 0 && valid) Delta[rowid] = delta;
  __syncthreads();
  float acc[PL];
#pragma unroll
  for (int e = 0; e < PL; ++e) acc[e] = 0.f;
  for (int j0 = 0; j0 <= i; j0 += 64) {
    const int key = j0 + lane;
    float ds = 0.f;
    if (key <= i) {
      const float s = dot_row<D>(qs[wave], Kh + (int64_t)key * D) * scale;
      const float dp = dot_row<D>(dos[wave], Vh + (int64_t)key * D);
      ds = expf(s - lse) * (dp - delta);
    }
    const int n = min(64, i + 1 - j0);
    for (int jj = 0; jj < n; ++jj) {
      const float dsj = __shfl(ds, jj);
      const float *kr = Kh + (int64_t)(j0 + jj) * D;
#pragma unroll
      for (int e = 0; e < PL; ++e) acc[e] = __builtin_fmaf(dsj, kr[lane + 64 * e], acc[e]);
    }
  }
  if (!valid) return;
#pragma unroll
  for (int e = 0; e < PL; ++e) dQ[rowid * D + lane + 64 * e] = acc[e] * scale;
}

template <int D>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_f32_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    const float *__restrict__ dO, const float *__restrict__ LSE,
    const float *__restrict__ Delta, float *__restrict__ dK, float *__restrict__ dV, int Hq,
    int Hkv, int T, int64_t rows, float scale) {
  constexpr int PL = D / 64;
  __shared__ float ks[kF32Waves][D], vs[kF32Waves][D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * kF32Waves + wave;
  const bool valid = wid < rows;
  const int64_t rowid = valid ? wid : rows - 1;  // bhk * T + j
  const int G = Hq / Hkv;
  const int bhk = (int)(rowid / T), j = (int)(rowid - (int64_t)bhk * T);
  const int b = bhk / Hkv, hk = bhk % Hkv;
#pragma unroll
  for (int e = 0; e < PL; ++e) {
    ks[wave][lane + 64 * e] = K[rowid * D + lane + 64 * e];
    vs[wave][lane + 64 * e] = V[rowid * D + lane + 64 * e];
  }
  __syncthreads();
  float dk[PL], dv[PL];
#pragma unroll
  for (int e = 0; e < PL; ++e) dk[e] = dv[e] = 0.f;
  for (int g = 0; g < G; ++g) {
    const int64_t bhq = (int64_t)b * Hq + hk * G + g;
    const float *Qh = Q + bhq * T * D, *dOh = dO + bhq * T * D;
    for (int i0 = j; i0 < T; i0 += 64) {
      const int qi = i0 + lane;
      float p = 0.f, ds = 0.f;
      if (qi < T) {
        const float s = dot_row<D>(ks[wave], Qh + (int64_t)qi * D) * scale;
        const float dp = dot_row<D>(vs[wave], dOh + (int64_t)qi * D);
        p = expf(s - LSE[bhq * T + qi]);
        ds = p * (dp - Delta[bhq * T + qi]);
      }
      const int n = min(64, T - i0);
      for (int ii = 0; ii < n; ++ii) {
        const float pi = __shfl(p, ii), dsi = __shfl(ds, ii);
        const float *qr = Qh + (int64_t)(i0 + ii) * D, *dor = dOh + (int64_t)(i0 + ii) * D;
#pragma unroll
        for (int e = 0; e < PL; ++e) {
          dv[e] = __builtin_fmaf(pi, dor[lane + 64 * e], dv[e]);
          dk[e] = __builtin_fmaf(dsi, qr[lane + 64 * e], dk[e]);
        }
      }
    }
  }
  if (!valid) return;
#pragma unroll
  for (int e = 0; e < PL; ++e) {
    dK[rowid * D + lane + 64 * e] = dk[e] * scale;
    dV[rowid * D + lane + 64 * e] = dv[e];
  }
}

static unsigned rows_grid(int B, int H, int T) {
  return (unsigned)(((int64_t)B * H * T + kF32Waves - 1) / kF32Waves);
}

hipError_t launch_fwd_f32(const void *q, const void *k, const void *v, void *o, float *lse,
                          int B, int Hq, int Hkv, int T, int D, float scale, hipStream_t stream) {
  const dim3 grid(rows_grid(B, Hq, T)), block(256);
  if (D == 64)
    fa_fwd_f32_kernel<64><<<grid, block, 0, stream>>>((const float *)q, (const float *)k,
                                                      (const float *)v, (float *)o, lse, Hq,
                                                      Hkv, T, (int64_t)B * Hq * T, scale);
  else
    fa_fwd_f32_kernel<128><<<grid, block, 0, stream>>>((const float *)q, (const float *)k,
                                                       (const float *)v, (float *)o, lse, Hq,
                                                       Hkv, T, (int64_t)B * Hq * T, scale);
  return hipGetLastError();
}

hipError_t launch_bwd_dq_f32(const void *q, const void *k, const void *v, const void *o,
                             const void *dout, const float *lse, float *delta, void *dq,
                             int B, int Hq, int Hkv, int T, int D, float scale,
                             hipStream_t stream) {
  const dim3 grid(rows_grid(B, Hq, T)), block(256);
  if (D == 64)
    fa_bwd_dq_f32_kernel<64><<<grid, block, 0, stream>>>(
        (const float *)q, (const float *)k, (const float *)v, (const float *)o,
        (const float *)dout, lse, delta, (float *)dq, Hq, Hkv, T, (int64_t)B * Hq * T, scale);
  else
    fa_bwd_dq_f32_kernel<128><<<grid, block, 0, stream>>>(
        (const float *)q, (const float *)k, (const float *)v, (const float *)o,
        (const float *)dout, lse, delta, (float *)dq, Hq, Hkv, T, (int64_t)B * Hq * T, scale);
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_f32(const void *q, const void *k, const void *v, const void *dout,
                               const float *lse, const float *delta, void *dk, void *dv,
                               int B, int Hq, int Hkv, int T, int D, float scale,
                               hipStream_t stream) {
  const dim3 grid(rows_grid(B, Hkv, T)), block(256);
  if (D == 64)
    fa_bwd_dkdv_f32_kernel<64><<<grid, block, 0, stream>>>(
        (const float *)q, (const float *)k, (const float *)v, (const float *)dout, lse, delta,
        (float *)dk, (float *)dv, Hq, Hkv, T, (int64_t)B * Hkv * T, scale);
  else
    fa_bwd_dkdv_f32_kernel<128><<<grid, block, 0, stream>>>(
        (const float *)q, (const float *)k, (const float *)v, (const float *)dout, lse, delta,
        (float *)dk, (float *)dv, Hq, Hkv, T, (int64_t)B * Hkv * T, scale);
  return hipGetLastError();
}

}  // namespace ttfa
