// Device-side building blocks shared by the gfx950 attention kernels.
//
// Layout facts used throughout (checked on gfx950 hardware with a one-wave probe):
//  * v_mfma_f32_32x32x16_bf16  D[32x32] += A[32x16] * B[16x32]
//      A[i][k] sits in lane i + 32*(k/8), slot k%8 (8 bf16 per lane)
//      B[k][j] sits in lane j + 32*(k/8), slot k%8
//      D[i][j] sits in lane j + 32*((i/4)%2), register 4*(i/8) + i%4
//    so a lane owns one column j and 16 rows {8a + 4*(lane/32) + e : a<4, e<4}.
//  * ds_read_b64_tr_b16 (16-lane groups): lane i of a group receives, in slot r,
//    element i%4 of the 8-byte chunk addressed by lane 4r + i/4 of the same group.
//    Pointing lane 4r+c at row R0+r, column C0+4c of a row-major [row][col] LDS tile
//    hands lane i the column C0+i for rows R0..R0+3: a transposed 4x16 read.
//  * v_permlane32_swap(x, x): lanes < 32 get (x[l], x[l+32]), lanes >= 32 get
//    (x[l-32], x[l]); max/add of the pair is the cross-half reduction.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ttfa {

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define TTFA_LDS __attribute__((address_space(3)))

constexpr float kLn2 = 0.693147180559945309f;
constexpr float kLog2e = 1.442695040888963407f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Buffer resource over [base, base + bytes): loads past the end return zero, which is
// how tiles handle the ragged tail of T without branches or out-of-bounds reads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}

// LDS tiles are row-major [rows][D] bf16, stored in 16-byte chunks whose index is
// XOR-swizzled by the row: 8 consecutive rows read at one logical chunk (b128 MFMA
// operand reads) and 4 consecutive rows read at two adjacent chunks (the transposed
// b64 reads) both land on distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ (((row & 3) << 1) | ((row >> 2) & 1));
}

template <int D>
__device__ __forceinline__ int lds_off(int row, int col) {  // element offset of (row, col)
  return row * D + (swz(row, col >> 3) << 3) + (col & 7);
}

template <int D>
__device__ __forceinline__ bf16x8 lds_read_row8(const bf16 *tile, int row, int chunk) {
  return *reinterpret_cast<const bf16x8 *>(tile + row * D + (swz(row, chunk) << 3));
}

__device__ __forceinline__ bf16x4 lds_read_tr(const bf16 *p) {
  typedef TTFA_LDS bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p));
}

// A-operand (32 rows = columns C0..C0+31 of the tile, 16 k = tile rows R0..R0+15)
// read transposed from a row-major [row][col] LDS tile.  Slot s of lane l holds
// tile[R0 + 8*(s/4) + 4*(l/32) + s%4][C0 + l%32], i.e. the row set a lane owns in a
// 32x32 MFMA result, which is what lets a result tile feed the next MFMA as-is.
template <int D>
__device__ __forceinline__ bf16x8 lds_read_trT(const bf16 *tile, int R0, int C0, int lane) {
  const int g16 = lane >> 4, r = (lane >> 2) & 3, c = lane & 3;
  const int row = R0 + 4 * (g16 >> 1) + r;
  const int col = C0 + 16 * (g16 & 1) + 4 * c;
  bf16x4 lo = lds_read_tr(tile + lds_off<D>(row, col));
  bf16x4 hi = lds_read_tr(tile + lds_off<D>(row + 8, col));
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// IEEE maximum (NaN-propagating): lowers to v_maximum3_f32 trees with no per-input
// canonicalisation, unlike fmaxf (maxnum), which quiets every MFMA result first.
__device__ __forceinline__ float fmax2(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmax3(float a, float b, float c) { return fmax2(a, fmax2(b, c)); }

// max over the 16 values of one MFMA result register block
__device__ __forceinline__ float max16(const f32x16 &v, float init) {
  float m = fmax3(init, v[0], v[1]);
#pragma unroll
  for (int r = 2; r < 16; r += 2) m = fmax3(m, v[r], v[r + 1]);
  return m;
}

__device__ __forceinline__ float xhalf_max(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax2(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

__device__ __forceinline__ float xhalf_sum(float x) {
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

__device__ __forceinline__ float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 fp32 -> 8 bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 pack8(f32x16 v, int base) {
  bf16x2 a = __builtin_convertvector((f32x2{v[base + 0], v[base + 1]}), bf16x2);
  bf16x2 b = __builtin_convertvector((f32x2{v[base + 2], v[base + 3]}), bf16x2);
  bf16x2 c = __builtin_convertvector((f32x2{v[base + 4], v[base + 5]}), bf16x2);
  bf16x2 d = __builtin_convertvector((f32x2{v[base + 6], v[base + 7]}), bf16x2);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ bf16x4 pack4(float a, float b, float c, float d) {
  bf16x2 x = __builtin_convertvector((f32x2{a, b}), bf16x2);
  bf16x2 y = __builtin_convertvector((f32x2{c, d}), bf16x2);
  return bf16x4{x[0], x[1], y[0], y[1]};
}

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }

// Workgroup -> work-item order.  Hardware hands consecutive workgroup ids to the 8
// XCDs round-robin (id % 8), and each XCD has its own L2.  When the number of
// (batch, kv-head) groups is a multiple of 8, every group is pinned to one XCD so
// the Hq/Hkv query heads and all row tiles that read the same K/V share one L2;
// within an XCD, the longest causal tiles go first.  Otherwise: longest tiles
// first, heads interleaved.
struct TileOrder {
  int tile;  // row-tile index in the "longest first" sense is resolved by the caller
  int bh;    // batch * Hq + query head
};

__device__ __forceinline__ TileOrder order_tiles(int bid, int n_tiles, int B, int Hq, int Hkv) {
  const int G = Hq / Hkv;
  const int BHkv = B * Hkv;
  TileOrder t;
  if ((BHkv & 7) == 0) {
    const int x = bid & 7, i = bid >> 3;
    const int per_rank = (BHkv >> 3) * G;  // work items per tile rank on one XCD
    t.tile = i / per_rank;
    const int rem = i - t.tile * per_rank;
    const int z = (rem / G) * 8 + x;      // batch * Hkv + kv head
    const int hq = (z % Hkv) * G + rem % G;
    t.bh = (z / Hkv) * Hq + hq;
  } else {
    const int BH = B * Hq;
    t.tile = bid / BH;
    t.bh = bid - t.tile * BH;
  }
  return t;
}

}  // namespace ttfa
