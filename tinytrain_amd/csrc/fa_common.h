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

#include <atomic>

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

__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0);
}

// 16 bytes per lane straight from a buffer into LDS: the wave's 64 lanes fill the
// 1 KB at lds_wave (wave-uniform) in lane order.
__device__ __forceinline__ void buf_load16_lds(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, void *lds_wave) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (TTFA_LDS void *)lds_wave, 16, byte_off, 0, 0, 0);
}

// s_waitcnt vmcnt(0): every vector memory load of this wave (direct-to-LDS included) done.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Index of the calling wave in its workgroup as a wave-uniform (scalar) value, so LDS
// addresses derived from it stay in SGPRs (M0 of the LDS-direct loads needs no
// v_readfirstlane per load).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// LDS tiles are row-major [rows][D] bf16, stored in 16-byte chunks whose index is
// XOR-swizzled by the row.  gfx950's LDS serves 256 bytes (64 banks) per clock: a
// ds_read_b128 in four groups of 16 consecutive lanes, a ds_read_b64_tr_b16 in two
// groups of 32; a group runs at full rate when its 16-byte pieces fall on distinct
// 16-byte bank groups (address bits 4..7).  The access shapes are
//  * transposed operand reads: rows 4k..4k+3 x chunks 4m..4m+3, and the same 8 rows
//    further down (lds_read_trT), and
//  * row operand reads: 16 consecutive rows at one logical chunk (lds_read_row8).
// The swizzle depends on row bits 0-2 only, so the second half of a transposed read
// (8 rows down) has the same XOR and its address is the first one plus an immediate;
// a swizzle that also separates 16 consecutive rows needs row bit 3 (swz_stage64 and
// swz_rows128 below: layout 1 of the read helpers, used by the forward's K/V tiles, the
// dQ pass's K/V tiles and the batched dK/dV passes' Q/dO tiles).  swz<D> (layout 0)
// serves the Q/dO tiles of the D = 64 varlen dK/dV pass, decode and the O staging of
// store_rows.
//  D = 64 (128-byte rows, row bit 0 picks the half of a 256-byte window): row bit 1 ->
//    chunk bit 2, row bit 0 -> bit 1, row bit 2 -> bit 0; rows 4k and 4k+2 (4k+1, 4k+3)
//    get disjoint chunk groups, so transposed reads are conflict-free; row reads are
//    2-way.
//  D = 128 (256-byte rows): row bits 0-1 -> chunk bits 2-3, row bit 2 -> bit 0; the
//    4 rows of a transposed read get 4 disjoint chunk groups (conflict-free); row reads
//    are 2-way.
// Measured read rates of these shapes on MI355X (B/clk/CU at 2.4 GHz, 4 waves/SIMD;
// linear b128 reads: 213): transposed D=64 188, D=128 190 (121 with row bits 0-1 ->
// chunk bits 1-2, the D=64 mapping); row reads 122-124 (2-way), 219-221 with a swizzle
// that uses row bit 3.
template <int D>
__device__ __forceinline__ int swz(int row, int chunk) {
  if constexpr (D == 128) return chunk ^ (((row & 3) << 2) | ((row >> 2) & 1));
  else return chunk ^ (((row & 3) << 1) | ((row >> 2) & 1));
}

// Swizzle of the D = 64 tiles that are read as row fragments by 16 consecutive rows (K
// in the forward, Q/dO in the dK/dV pass, K/V in the dQ pass): 16-byte chunk c of row r
// is stored at chunk c ^ (r bit 1 -> bit 2, r bits 2-3 -> bits 0-1).  A row-fragment read
// serves 16 lanes (rows r0..r0+15 at one logical chunk) per clock; row bit 0 picks the
// half of the 256-byte bank window and bits 1-3 the chunk, so the 16 pieces land on 16
// distinct 16-byte bank groups (conflict-free: 224 B/clk/CU measured on MI355X against
// 122 for swz<64>, which leaves row bit 3 out).  The transposed reads run at the same
// rate with either (165 B/clk/CU).  Row bit 3 changes the swizzle, so the two 8-row
// halves of a transposed read have separate lane addresses.
__device__ __forceinline__ int swz_stage64(int row, int chunk) {
  return chunk ^ ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}

// The D = 128 counterpart (256-byte rows): row bits 0-1 -> chunk bits 2-3, row bits 2-3 ->
// bits 0-1, so a row-fragment read's 16 rows land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz_rows128(int row, int chunk) {
  return chunk ^ (((row & 3) << 2) | ((row >> 2) & 3));
}

// Tile layout L: 0 = swz<D>, 1 = the swizzle of D with conflict-free row reads
// (swz_stage64 / swz_rows128).  Loads and reads of one tile use the same L.
template <int D, int L>
__device__ __forceinline__ int swz_l(int row, int chunk) {
  if constexpr (L == 0) return swz<D>(row, chunk);
  else if constexpr (D == 64) return swz_stage64(row, chunk);
  else return swz_rows128(row, chunk);
}

template <int D, int L = 0>
__device__ __forceinline__ int lds_off(int row, int col) {  // element offset of (row, col)
  return row * D + (swz_l<D, L>(row, col >> 3) << 3) + (col & 7);
}

template <int D, int L = 0>
__device__ __forceinline__ bf16x8 lds_read_row8(const bf16 *tile, int row, int chunk) {
  return *reinterpret_cast<const bf16x8 *>(tile + row * D + (swz_l<D, L>(row, chunk) << 3));
}

// The pointer is __restrict__ so that, once inlined, the read carries alias-scope
// metadata: without it the compiler makes every transposed read wait (vmcnt) for all
// direct-to-LDS loads in flight, including the next tile's prefetch into the other LDS
// stage.  The kernels order each stage's loads before its reads explicitly (vmcnt(0)
// and a barrier between the two).
__device__ __forceinline__ bf16x4 lds_read_tr(const bf16 *__restrict__ p) {
  typedef TTFA_LDS bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p));
}

// A-operand (32 rows = columns C0..C0+31 of the tile, 16 k = tile rows R0..R0+15)
// read transposed from a row-major [row][col] LDS tile.  Slot s of lane l holds
// tile[R0 + 8*(s/4) + 4*(l/32) + s%4][C0 + l%32], i.e. the row set a lane owns in a
// 32x32 MFMA result, which is what lets a result tile feed the next MFMA as-is.
template <int D, int L = 0>
__device__ __forceinline__ bf16x8 lds_read_trT(const bf16 *tile, int R0, int C0, int lane) {
  const int g16 = lane >> 4, r = (lane >> 2) & 3, c = lane & 3;
  const int row = R0 + 4 * (g16 >> 1) + r;
  const int col = C0 + 16 * (g16 & 1) + 4 * c;
  bf16x4 lo = lds_read_tr(tile + lds_off<D, L>(row, col));
  bf16x4 hi = lds_read_tr(tile + lds_off<D, L>(row + 8, col));
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// IEEE maximum (NaN-propagating): lowers to v_maximum3_f32 trees with no per-input
// canonicalisation, unlike fmaxf (maxnum), which quiets every MFMA result first.
__device__ __forceinline__ float fmax2(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmax3(float a, float b, float c) { return fmax2(fmax2(a, b), c); }

// max over the 16 values of one MFMA result register block
__device__ __forceinline__ float max16(const f32x16 &v, float init) {
  float m = fmax3(init, v[0], v[1]);
#pragma unroll
  for (int r = 2; r < 16; r += 2) m = fmax3(m, v[r], v[r + 1]);
  return m;
}

// Stores a wave's 32 x D result tile held in MFMA result layout (lane l owns row l%32;
// register 4a+e of block db holds column 32db + 8a + 4(l/32) + e), times `mul` and
// rounded to bf16, to rows row0.. of a row-major [T][D] output.  The tile goes through
// the wave's own LDS scratch (32*D bf16, swizzled like the operand tiles), so every
// global store instruction writes whole rows: 64 lanes x 16 contiguous bytes, instead of
// 8-byte pieces of 32 different rows.  Rows at or past T are not written.
template <int D>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[D / 32], float mul, bf16 *scratch,
                                           bf16 *out, int row0, int T, int lane) {
  const int lq = lane & 31, lg = lane >> 5;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int col = 32 * db + 8 * a + 4 * lg;
      const bf16x2 x = __builtin_convertvector((f32x2{acc[db][4 * a] * mul, acc[db][4 * a + 1] * mul}), bf16x2);
      const bf16x2 y = __builtin_convertvector((f32x2{acc[db][4 * a + 2] * mul, acc[db][4 * a + 3] * mul}), bf16x2);
      *reinterpret_cast<bf16x4 *>(scratch + lq * D + (swz<D>(lq, col >> 3) << 3) + (col & 7)) =
          bf16x4{x[0], x[1], y[0], y[1]};
    }
  constexpr int CH = D / 8;
#pragma unroll
  for (int i = 0; i < 32 * CH / 64; ++i) {
    const int e = lane + 64 * i, row = e / CH, ch = e % CH;
    const u32x4 v = *reinterpret_cast<const u32x4 *>(scratch + row * D + (swz<D>(row, ch) << 3));
    if (row0 + row < T) *reinterpret_cast<u32x4 *>(out + (int64_t)(row0 + row) * D + ch * 8) = v;
  }
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

// Workgroup -> work item.  Causal row tiles carry very different amounts of work (tile t
// of n sees t+1 key tiles), so every workgroup takes a PAIR of row tiles (n-1-p, p):
// the pair's total work is the same for every p, and a grid of pairs is one balanced
// round instead of a long tail behind the diagonal's longest tiles.  `first` is the
// longer tile of the pair; each kernel chooses which of the two it runs first.  When n
// is odd the middle tile forms a pair of its own.
//
// Hardware hands consecutive workgroup ids to the 8 XCDs round-robin (id % 8), and each
// XCD has its own L2.  (This holds for a whole MI355X, SPX mode.  The grouping below is
// a bijection from workgroup ids to items for any XCD count, so another partition mode
// changes only which L2 serves an item, never the results.)  When the number of (batch, kv-head) groups is a multiple of 8,
// each group's items (its G query heads x pairs) are placed on one XCD and numbered
// consecutively there, so the workgroups that read the same K/V run at the same time
// on the same L2.  Otherwise items are numbered group-major in plain id order.
struct WorkPair {
  int bh;      // batch * H + head (H = the caller's head count)
  int first;   // longer row tile
  int second;  // shorter row tile, or -1
};

// n_tiles: row tiles per head; H heads per batch, grouped by Hg heads per group
// (Hg = Hq / Hkv for query-row kernels, 1 for the kv-row kernel); long_first_low: the
// longest tile is tile n-1 (query rows) when false, tile 0 (key rows) when true.
__device__ __forceinline__ WorkPair pair_item(int bid, int n_tiles, int B, int H, int Hg,
                                              bool long_is_low) {
  const int n_pairs = (n_tiles + 1) / 2;
  const int per_group = Hg * n_pairs;
  const int n_groups = B * (H / Hg);
  int z, i;
  if ((n_groups & 7) == 0) {
    const int x = bid & 7, k = bid >> 3;
    z = (k / per_group) * 8 + x;
    i = k - (k / per_group) * per_group;
  } else {
    z = bid / per_group;
    i = bid - z * per_group;
  }
  const int g = i / n_pairs, p = i - g * n_pairs;
  WorkPair w;
  w.bh = z * Hg + g;  // groups are consecutive heads: bh = b*H + hk*Hg + g
  const int lo = p, hi = n_tiles - 1 - p;
  w.first = long_is_low ? lo : hi;
  w.second = lo == hi ? -1 : (long_is_low ? hi : lo);
  return w;
}

// Single-tile schedule: one row tile per workgroup, longest tiles first (tile-rank
// major), with the same XCD grouping as pair_item.  Used when pairs would not fill whole
// rounds of the resident workgroup slots.
__device__ __forceinline__ WorkPair single_item(int bid, int n_tiles, int B, int H, int Hg,
                                                bool long_is_low) {
  const int n_groups = B * (H / Hg);
  int rank, z, g;
  if ((n_groups & 7) == 0) {
    const int x = bid & 7, k = bid >> 3;
    const int per_rank = (n_groups >> 3) * Hg;  // items of one tile rank on one XCD
    rank = k / per_rank;
    const int rem = k - rank * per_rank;
    z = (rem / Hg) * 8 + x;
    g = rem - (rem / Hg) * Hg;
  } else {
    const int per_rank = n_groups * Hg;
    rank = bid / per_rank;
    const int rem = bid - rank * per_rank;
    z = rem / Hg;
    g = rem - z * Hg;
  }
  WorkPair w;
  w.bh = z * Hg + g;
  w.first = long_is_low ? rank : n_tiles - 1 - rank;
  w.second = -1;
  return w;
}

__device__ __forceinline__ WorkPair sched_item(bool paired, int bid, int n_tiles, int B, int H,
                                               int Hg, bool long_is_low) {
  return paired ? pair_item(bid, n_tiles, B, H, Hg, long_is_low)
                : single_item(bid, n_tiles, B, H, Hg, long_is_low);
}

// Workgroups a launch needs for n_tiles row tiles per head: paired or single.
inline int sched_items(bool paired, int n_tiles, int B, int H) {
  return (paired ? (n_tiles + 1) / 2 : n_tiles) * B * H;
}

// Workgroups of kernel KERN resident on the current device at once: CUs x blocks per CU,
// from the runtime's occupancy calculator, cached per kernel and device (devices 0..63;
// a higher id is asked every time).  The value only picks the work schedule (pairs or
// single row tiles), never the results: which kernel a shape runs is a rule on the shape
// alone (fwd128_uses_wide, dq128_uses_wide).
template <auto KERN>
inline int resident_slots(int block, size_t lds) {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  int v = dev >= 0 && dev < 64 ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (v) return v;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(KERN),
                                                   block, lds) != hipSuccess ||
      cus <= 0 || per_cu <= 0)
    return 1;  // unknown: then pairs are used only when they fill rounds of one slot
  v = cus * per_cu;
  if (dev >= 0 && dev < 64) cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

// Pairs only when they fill whole rounds of the resident slots (or nearly: the last
// round at least 7/8 full); otherwise single tiles, longest first, keep slots busy.
inline bool use_pairs(int n_tiles, int B, int H, int slots) {
  const int items = sched_items(true, n_tiles, B, H);
  const int rem = items % slots;
  return n_tiles > 1 && (rem == 0 || 8 * rem >= 7 * slots);
}

// Wave issue priority from the workgroup's remaining work.  A CU's SIMDs issue from
// the oldest wave first, so of several equal workgroups sharing a CU the oldest races
// ahead and the youngest drains alone at the end.  Giving the workgroup with more work
// left the higher priority (0..3, by quarters of its total) keeps them in step, so the
// CU stays fully occupied until all of them finish.
struct PrioByRemaining {
  int total, lvl = -1, floor_r = 0;  // the level holds while remaining >= floor_r
  __device__ explicit PrioByRemaining(int total_) : total(total_ > 0 ? total_ : 1) {}
  // remaining >= total * k/4 for k = 1, 2, 3 gives level k; s_setprio runs only when the
  // level changes (its operand is an immediate, hence the branches).  Remaining work only
  // decreases, so the common case is one scalar compare against the current level's
  // floor.
  __device__ __forceinline__ void update(int remaining) {
    if (lvl >= 0 && remaining >= floor_r) return;
    const int r4 = 4 * remaining;
    const int l = r4 >= 3 * total ? 3 : r4 >= 2 * total ? 2 : r4 >= total ? 1 : 0;
    floor_r = (l * total + 3) / 4;  // smallest remaining with 4 * remaining >= l * total
    if (l == lvl) return;
    lvl = l;
    if (l == 3)
      __builtin_amdgcn_s_setprio(3);
    else if (l == 2)
      __builtin_amdgcn_s_setprio(2);
    else if (l == 1)
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
  }
};

}  // namespace ttfa
