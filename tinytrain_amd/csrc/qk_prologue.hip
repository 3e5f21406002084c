// Fused attention prologue for bf16 models: q/k RMSNorm + rotate-half RoPE + the
// [B, T, H, D] -> [B, H, T, D] layout change, forward and backward, gfx950.
//
// Computes what the reference's Attention.forward does between the projections and the
// attention call (model.py:83-93): RMSNorm over D per (b, t, head) in fp32 with the
// result rounded to bf16 (model.py:30-35: (w * x) * rsqrt(mean(x^2) + eps)), the
// transpose to [B, H, T, D], then apply_rope in bf16 arithmetic (model.py:48-56:
// cos/sin rounded to bf16, x*cos and cat(-x2, x1)*sin each rounded to bf16, their sum
// rounded to bf16), and the .contiguous() copies the attention kernels need.  V only
// changes layout.  One pass reads each input row once and writes it once in the
// attention layout, instead of separate norm, transpose, rotate, multiply, add and copy
// passes.
//
// Work split: a row is one (b, t, head) vector of D bf16, handled by D/8 lanes holding
// 8 consecutive elements (16 bytes) each; the RoPE partner of element i (i +- D/2) sits
// in lane ^ D/16 of the same row group.  A 256-thread workgroup runs 256/(D/8) rows at a
// time for kRounds (forward) or kBwdRounds (backward) rounds; workgroups are ordered q
// rows, then k rows, then v rows, each in the inputs' [B, T, H] row order (contiguous
// 16-byte loads).
//
// Backward (autograd of the same expressions; the bf16 roundings pass gradients
// through unchanged): RoPE^T, dy_i = g_i c_i + (i < D/2 ? g_{i+D/2} s_{i+D/2}
// : -g_{i-D/2} s_{i-D/2}); RMSNorm^T, dx = r (w dy) - x r^3 mean(w dy x), and the norm
// weight gradient sum over rows of dy x r.  The weight gradients are reduced without
// atomics: each workgroup writes its partial sum over its rows to the workspace, and a
// second kernel adds the partials in a fixed order, so results are bitwise reproducible.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_common.h"
#include "ttfa.h"

// The forward repeats the reference's bf16 roundings operation by operation.  With
// contraction on, the compiler turns round_bf16(y * c) + round_bf16(rot * s) into
// fma(y, c, round_bf16(rot * s)), dropping the first rounding (the bf16 product is
// widened back to fp32 and fused into the add), which changes about one element in ten.
#pragma clang fp contract(off)

namespace ttfa {

namespace {

constexpr int kRounds = 4;      // forward: row-group rounds per workgroup
constexpr int kBwdRounds = 8;   // backward: more rows per workgroup, fewer weight-gradient
                                // partials for the second kernel to add

template <int D, int R = kRounds>
struct PShape {
  static constexpr int L = D / 8;               // lanes per row
  static constexpr int GROUPS = 256 / L;         // rows in flight per workgroup
  static constexpr int ROUNDS = R;
  static constexpr int ROWS = GROUPS * R;        // rows per workgroup
};

__device__ __forceinline__ float bf16_round(float x) { return (float)(bf16)x; }

__device__ __forceinline__ void unpack8(u32x4 u, float (&f)[8]) {
  const bf16x8 b = __builtin_bit_cast(bf16x8, u);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)b[i];
}

__device__ __forceinline__ u32x4 pack8f(const float (&f)[8]) {
  bf16x8 b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (bf16)f[i];
  return __builtin_bit_cast(u32x4, b);
}

template <int L>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int m = 1; m < L; m <<= 1) v += __shfl_xor(v, m, L);
  return v;
}

// Which tensor workgroup `wg` works on, and its index within that tensor's workgroups.
__device__ __forceinline__ int split_wg(int &wg, int nq_wg, int nk_wg) {
  if (wg < nq_wg) return 0;
  wg -= nq_wg;
  if (wg < nk_wg) return 1;
  wg -= nk_wg;
  return 2;
}

template <int D>
__global__ __launch_bounds__(256) void qk_prologue_fwd_kernel(
    const bf16 *__restrict__ q_raw, const bf16 *__restrict__ k_raw, const bf16 *__restrict__ v_raw,
    const float *__restrict__ wq, const float *__restrict__ wk, const bf16 *__restrict__ cosb,
    const bf16 *__restrict__ sinb, bf16 *__restrict__ q, bf16 *__restrict__ k,
    bf16 *__restrict__ v, float *__restrict__ rstd_q, float *__restrict__ rstd_k, int B, int T,
    int Hq, int Hkv, float eps, int nq_wg, int nk_wg) {
  using S = PShape<D>;
  constexpr int L = S::L;
  const int lane = threadIdx.x % L, group = threadIdx.x / L;
  int wg = blockIdx.x;
  const int kind = split_wg(wg, nq_wg, nk_wg);
  const int H = kind == 0 ? Hq : Hkv;
  const bf16 *src = kind == 0 ? q_raw : kind == 1 ? k_raw : v_raw;
  bf16 *dst = kind == 0 ? q : kind == 1 ? k : v;
  const float *w = kind == 0 ? wq : wk;
  float *rstd = kind == 0 ? rstd_q : rstd_k;
  const int64_t n_rows = (int64_t)B * T * H;
  const bool first_half = lane < L / 2;

  float wl[8];
  if (kind < 2) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(w + lane * 8);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(w + lane * 8 + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wl[i] = a[i];
      wl[i + 4] = b[i];
    }
  }
#pragma unroll 1
  for (int rd = 0; rd < kRounds; ++rd) {
    const int64_t row = (int64_t)wg * S::ROWS + rd * S::GROUPS + group;
    if (row >= n_rows) break;  // whole row groups leave together
    const int h = (int)(row % H);
    const int64_t bt = row / H;
    const int t = (int)(bt % T);
    const int64_t b = bt / T;
    const u32x4 raw = *reinterpret_cast<const u32x4 *>(src + row * D + lane * 8);
    bf16 *out = dst + ((b * H + h) * T + t) * D + lane * 8;
    if (kind == 2) {
      *reinterpret_cast<u32x4 *>(out) = raw;
      continue;
    }
    float x[8];
    unpack8(raw, x);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = row_sum<L>(ss);
    const float r = rsqrtf(ss / (float)D + eps);
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = bf16_round((wl[i] * x[i]) * r);
    // partner half of the row (bf16-exact values travel as packed pairs)
    const u32x4 yp = pack8f(y);
    u32x4 pp;
#pragma unroll
    for (int i = 0; i < 4; ++i) pp[i] = (uint32_t)__shfl_xor((int)yp[i], L / 2, L);
    float py[8];
    unpack8(pp, py);
    float c[8], s[8];
    unpack8(*reinterpret_cast<const u32x4 *>(cosb + (int64_t)t * D + lane * 8), c);
    unpack8(*reinterpret_cast<const u32x4 *>(sinb + (int64_t)t * D + lane * 8), s);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float rot = first_half ? -py[i] : py[i];
      o[i] = bf16_round(y[i] * c[i]) + bf16_round(rot * s[i]);
    }
    *reinterpret_cast<u32x4 *>(out) = pack8f(o);
    if (lane == 0) rstd[row] = r;
  }
}

template <int D>
__global__ __launch_bounds__(256) void qk_prologue_bwd_kernel(
    const bf16 *__restrict__ gq, const bf16 *__restrict__ gk, const bf16 *__restrict__ gv,
    const bf16 *__restrict__ q_raw, const bf16 *__restrict__ k_raw, const float *__restrict__ wq,
    const float *__restrict__ wk, const bf16 *__restrict__ cosb, const bf16 *__restrict__ sinb,
    const float *__restrict__ rstd_q, const float *__restrict__ rstd_k, bf16 *__restrict__ dq_raw,
    bf16 *__restrict__ dk_raw, bf16 *__restrict__ dv_raw, float *__restrict__ partial, int B,
    int T, int Hq, int Hkv, int nq_wg, int nk_wg) {
  using S = PShape<D, kBwdRounds>;
  constexpr int L = S::L;
  __shared__ float red[S::GROUPS][D + 4];
  const int lane = threadIdx.x % L, group = threadIdx.x / L;
  int wg = blockIdx.x;
  const int wg_all = blockIdx.x;
  const int kind = split_wg(wg, nq_wg, nk_wg);
  const int H = kind == 0 ? Hq : Hkv;
  const bf16 *g_src = kind == 0 ? gq : kind == 1 ? gk : gv;
  const bf16 *x_src = kind == 0 ? q_raw : k_raw;
  bf16 *dst = kind == 0 ? dq_raw : kind == 1 ? dk_raw : dv_raw;
  const float *w = kind == 0 ? wq : wk;
  const float *rstd = kind == 0 ? rstd_q : rstd_k;
  const int64_t n_rows = (int64_t)B * T * H;
  const bool first_half = lane < L / 2;

  float wl[8], dw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) dw[i] = 0.f;
  if (kind < 2) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(w + lane * 8);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(w + lane * 8 + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wl[i] = a[i];
      wl[i + 4] = b[i];
    }
  }
#pragma unroll 1
  for (int rd = 0; rd < S::ROUNDS; ++rd) {
    const int64_t row = (int64_t)wg * S::ROWS + rd * S::GROUPS + group;
    if (row >= n_rows) break;
    const int h = (int)(row % H);
    const int64_t bt = row / H;
    const int t = (int)(bt % T);
    const int64_t b = bt / T;
    const u32x4 graw = *reinterpret_cast<const u32x4 *>(g_src + ((b * H + h) * T + t) * D + lane * 8);
    bf16 *out = dst + row * D + lane * 8;
    if (kind == 2) {
      *reinterpret_cast<u32x4 *>(out) = graw;
      continue;
    }
    float g[8], x[8], c[8], s[8];
    unpack8(graw, g);
    unpack8(*reinterpret_cast<const u32x4 *>(x_src + row * D + lane * 8), x);
    unpack8(*reinterpret_cast<const u32x4 *>(cosb + (int64_t)t * D + lane * 8), c);
    unpack8(*reinterpret_cast<const u32x4 *>(sinb + (int64_t)t * D + lane * 8), s);
    const float r = rstd[row];
    float gs[8], pgs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) gs[i] = g[i] * s[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) pgs[i] = __shfl_xor(gs[i], L / 2, L);
    float dy[8], a[8];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dy[i] = __builtin_fmaf(g[i], c[i], first_half ? pgs[i] : -pgs[i]);
      a[i] = wl[i] * dy[i];
      dot = __builtin_fmaf(a[i], x[i], dot);
      dw[i] = __builtin_fmaf(dy[i] * x[i], r, dw[i]);
    }
    dot = row_sum<L>(dot);
    const float k3 = r * r * r * dot / (float)D;
    float dx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dx[i] = r * a[i] - x[i] * k3;
    *reinterpret_cast<u32x4 *>(out) = pack8f(dx);
  }
  if (kind == 2) return;  // v workgroups have no weight gradient (uniform per workgroup)
  // Partial weight gradient of this workgroup: sum over its row groups, fixed order.
#pragma unroll
  for (int i = 0; i < 8; ++i) red[group][lane * 8 + i] = dw[i];
  __syncthreads();
  if (threadIdx.x < D) {
    float acc = 0.f;
    for (int gi = 0; gi < S::GROUPS; ++gi) acc += red[gi][threadIdx.x];
    partial[(int64_t)wg_all * D + threadIdx.x] = acc;
  }
}

// dw_q = sum of the q workgroups' partials, dw_k of the k workgroups'.  2 * D / 16
// workgroups of 1024 threads; workgroup (vector, column slice) owns 16 columns of one
// weight vector: thread (slice, col) adds partials slice, slice + 64, ... in index order
// (independent loads, unrolled, so many are in flight), then the 64 slice sums of each
// column are added in slice order through LDS.  Every column's summation order is fixed,
// so the result is the same on every call; spreading the columns over 16 workgroups
// reads the partials with 16 CUs instead of 2.
template <int D>
__global__ __launch_bounds__(1024) void qk_prologue_dw_kernel(const float *__restrict__ partial,
                                                              float *__restrict__ dwq,
                                                              float *__restrict__ dwk, int nq_wg,
                                                              int nk_wg) {
  constexpr int C = 16, S = 1024 / C;
  __shared__ float red[S][C + 1];
  const int which = blockIdx.x / (D / C), c0 = (blockIdx.x % (D / C)) * C;
  const int col = threadIdx.x % C, slice = threadIdx.x / C;
  const int lo = which == 0 ? 0 : nq_wg, n = which == 0 ? nq_wg : nk_wg;
  float acc = 0.f;
#pragma unroll 8
  for (int i = slice; i < n; i += S) acc += partial[(int64_t)(lo + i) * D + c0 + col];
  red[slice][col] = acc;
  __syncthreads();
  if (threadIdx.x < C) {
    float tot = 0.f;
    for (int j = 0; j < S; ++j) tot += red[j][threadIdx.x];
    (which == 0 ? dwq : dwk)[c0 + threadIdx.x] = tot;
  }
}

struct Grid {
  int nq, nk, nv;
};

template <int D, int R = kRounds>
Grid prologue_grid(int B, int T, int Hq, int Hkv) {
  const int64_t rows = PShape<D, R>::ROWS;
  auto n = [&](int H) { return (int)(((int64_t)B * T * H + rows - 1) / rows); };
  return {n(Hq), n(Hkv), n(Hkv)};
}

int check_prologue(int B, int T, int Hq, int Hkv, int D) {
  if (D != 64 && D != 128) return TTFA_E_HEAD_DIM;
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return TTFA_E_GROUP;
  if (B < 1 || T < 1) return TTFA_E_SEQ;
  // workgroup counts must fit the grid
  const int64_t rows = 256 / (D / 8) * kRounds;
  if (((int64_t)B * T * (Hq + 2 * Hkv) + rows - 1) / rows > (int64_t)0x7fffffff) return TTFA_E_SEQ;
  return TTFA_OK;
}

int check_ptrs16(const void *const *ptrs, int n) {
  for (int i = 0; i < n; ++i)
    if (ptrs[i] == nullptr) return TTFA_E_NULL;
  for (int i = 0; i < n; ++i)
    if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15u) return TTFA_E_ALIGN;
  return TTFA_OK;
}

}  // namespace

}  // namespace ttfa

using namespace ttfa;

extern "C" {

int ttfa_qk_prologue_fwd(const void *q_raw, const void *k_raw, const void *v_raw,
                         const float *q_norm_w, const float *k_norm_w, const void *cos,
                         const void *sin, void *q, void *k, void *v, float *rstd_q,
                         float *rstd_k, int B, int T, int Hq, int Hkv, int D, float eps,
                         void *hip_stream) {
  const void *ptrs[] = {q_raw, k_raw, v_raw, q_norm_w, k_norm_w, cos, sin, q, k, v, rstd_q, rstd_k};
  int rc = check_ptrs16(ptrs, 12);
  if (rc) return rc;
  if ((rc = check_prologue(B, T, Hq, Hkv, D))) return rc;
  if (!(eps >= 0.f) || !(eps < 1.f)) return TTFA_E_EPS;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  auto go = [&](auto kern, Grid g) {
    kern<<<dim3((unsigned)(g.nq + g.nk + g.nv)), dim3(256), 0, st>>>(
        (const bf16 *)q_raw, (const bf16 *)k_raw, (const bf16 *)v_raw, q_norm_w, k_norm_w,
        (const bf16 *)cos, (const bf16 *)sin, (bf16 *)q, (bf16 *)k, (bf16 *)v, rstd_q, rstd_k, B,
        T, Hq, Hkv, eps, g.nq, g.nk);
    return (int)hipGetLastError();
  };
  return D == 64 ? go(qk_prologue_fwd_kernel<64>, prologue_grid<64>(B, T, Hq, Hkv))
                 : go(qk_prologue_fwd_kernel<128>, prologue_grid<128>(B, T, Hq, Hkv));
}

long long ttfa_qk_prologue_workspace_bytes(int B, int T, int Hq, int Hkv, int D) {
  if (check_prologue(B, T, Hq, Hkv, D)) return -1;
  const Grid g = D == 64 ? prologue_grid<64, kBwdRounds>(B, T, Hq, Hkv)
                         : prologue_grid<128, kBwdRounds>(B, T, Hq, Hkv);
  return (long long)(g.nq + g.nk) * D * (long long)sizeof(float);
}

int ttfa_qk_prologue_bwd(const void *dq, const void *dk, const void *dv, const void *q_raw,
                         const void *k_raw, const float *q_norm_w, const float *k_norm_w,
                         const void *cos, const void *sin, const float *rstd_q,
                         const float *rstd_k, void *dq_raw, void *dk_raw, void *dv_raw,
                         float *dq_norm_w, float *dk_norm_w, float *workspace, int B, int T,
                         int Hq, int Hkv, int D, void *hip_stream) {
  const void *ptrs[] = {dq, dk, dv, q_raw, k_raw, q_norm_w, k_norm_w, cos, sin, rstd_q,
                        rstd_k, dq_raw, dk_raw, dv_raw, dq_norm_w, dk_norm_w, workspace};
  int rc = check_ptrs16(ptrs, 17);
  if (rc) return rc;
  if ((rc = check_prologue(B, T, Hq, Hkv, D))) return rc;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  auto go = [&](auto kern, auto dwk_kern, Grid g) {
    kern<<<dim3((unsigned)(g.nq + g.nk + g.nv)), dim3(256), 0, st>>>(
        (const bf16 *)dq, (const bf16 *)dk, (const bf16 *)dv, (const bf16 *)q_raw,
        (const bf16 *)k_raw, q_norm_w, k_norm_w, (const bf16 *)cos, (const bf16 *)sin, rstd_q,
        rstd_k, (bf16 *)dq_raw, (bf16 *)dk_raw, (bf16 *)dv_raw, workspace, B, T, Hq, Hkv, g.nq,
        g.nk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    dwk_kern<<<dim3(2 * D / 16), dim3(1024), 0, st>>>(workspace, dq_norm_w, dk_norm_w, g.nq,
                                                       g.nk);
    return (int)hipGetLastError();
  };
  return D == 64 ? go(qk_prologue_bwd_kernel<64>, qk_prologue_dw_kernel<64>,
                      prologue_grid<64, kBwdRounds>(B, T, Hq, Hkv))
                 : go(qk_prologue_bwd_kernel<128>, qk_prologue_dw_kernel<128>,
                      prologue_grid<128, kBwdRounds>(B, T, Hq, Hkv));
}

}  // extern "C"
