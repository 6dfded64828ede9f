// Device-side building blocks shared by the gfx950 attention kernels.
//
// MFMA used throughout: v_mfma_f32_32x32x16_bf16 (wave64).
//   A operand (8 bf16 per lane): row i = lane % 32, k = 8*(lane/32) + e.
//   B operand (8 bf16 per lane): col j = lane % 32, k = 8*(lane/32) + e.
//   C/D (16 fp32 per lane):      col j = lane % 32,
//                                row i = 8*(r/4) + 4*(lane/32) + (r%4).
// Only the pairing of A's and B's (lane/32, e) slots matters for the sum, so a
// kernel may assign any bijection of key/query indices to the k slots as long
// as both operands use the same one.  The kernels exploit this to feed the C
// layout of one product straight into the B operand of the next without a
// register shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace avattn {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Combine a value with the one held by the lane 32 positions away.
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with the
// lower 32 lanes of its second; with both operands equal, every lane ends up
// holding its own value in one result and its partner's in the other, so the
// symmetric combinations below do not depend on which is which.
__device__ __forceinline__ float halves_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }

__device__ __forceinline__ float bf16_to_f32(bf16 x) { return (float)x; }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v;
  v[0] = (bf16)lo;
  v[1] = (bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ bf16x8 bits_to_bf16x8(const u32x4& u) {
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ u32x4 bf16x8_to_bits(const bf16x8& v) {
  return __builtin_bit_cast(u32x4, v);
}

__device__ __forceinline__ bf16x8 cat4(const u32x2& lo, const u32x2& hi) {
  u32x4 u;
  u[0] = lo[0];
  u[1] = lo[1];
  u[2] = hi[0];
  u[3] = hi[1];
  return __builtin_bit_cast(bf16x8, u);
}

// Pack the low (hi == 0) or high (hi == 1) 16-bit halves of a and b as
// (a.half, b.half).
__device__ __forceinline__ uint32_t pack_halves(uint32_t a, uint32_t b, int hi) {
  return hi ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
}

// Interleaved-pair rotation of 8 consecutive channels (4 pairs) in fp32 with
// every product rounded separately (no FMA contraction), then rounded to
// bf16.  Matches src/avgen/models/rope.py:332-338 bit for bit.
__device__ __forceinline__ u32x4 rotate8(const u32x4& x, const f32x4& c, const f32x4& s, bool inverse) {
  // Contraction off: with -ffp-contract=fast the compiler would fuse a
  // product with the following add/sub into one FMA (one rounding instead of
  // two).  HIP's __fmul_rn/__fadd_rn are plain operators defined in a header
  // compiled with contraction on, so the operators are written out here,
  // inside the pragma's scope.
#pragma clang fp contract(off)
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float e = __uint_as_float(x[p] << 16);
    const float o = __uint_as_float(x[p] & 0xffff0000u);
    const float ec = e * c[p], os = o * s[p], es = e * s[p], oc = o * c[p];
    float a, b;
    if (!inverse) {
      a = ec - os;
      b = es + oc;
    } else {
      a = ec + os;
      b = oc - es;
    }
    r[p] = pack_bf16x2(a, b);
  }
  return r;
}

// Map a linear block id so that consecutive *logical* ids land on the same
// XCD.  The dispatcher places block i on XCD (i % 8); logical neighbours (the
// query tiles of one head) then share that XCD's L2 for their K/V reads.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  constexpr int kXcds = 8;
  const int xcd = bid % kXcds;
  const int local = bid / kXcds;
  const int per = total / kXcds;
  const int rem = total % kXcds;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// ---------------------------------------------------------------------------
// LDS tile layout
// ---------------------------------------------------------------------------
// Row-major tile of RL-element (2*RL-byte) bf16 rows, unpadded, whose
// 16-byte chunks are XOR-swizzled: chunk c of row r sits at chunk slot
// c ^ f(r).
//   RL == 128 (256-byte rows): f(r) = 4*(r%4) + (r/4)%4
//   RL == 64  (128-byte rows): f(r) = 4*((r/2)%2) + (r/4)%4
//   RL == 32  ( 64-byte rows): f(r) = (r/4)%4
// With these, sixteen lanes reading one chunk each of 16 distinct rows in an
// aligned group of 16 (ds_read_b128) touch all 64 banks exactly once, and a
// 1 KB block of consecutive rows can be filled by one direct global->LDS
// wave load (stage_direct).  Row-major sequence tiles use RL = head_dim;
// head_dim-major ("transposed") tiles use RL = the tile's sequence length.
template <int RL>
struct TileLayout {
  static_assert(RL == 32 || RL == 64 || RL == 128, "row length 32, 64 or 128 elements");
  static constexpr int kRowElems = RL;
  static __device__ __forceinline__ int swz(int row) {
    if constexpr (RL == 128) return ((row & 3) << 2) | ((row >> 2) & 3);
    if constexpr (RL == 64) return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
    return (row >> 2) & 3;
  }
  // Element offset of (row, col); col must be a multiple of 4.
  static __device__ __forceinline__ int off(int row, int col) {
    return row * RL + (((col >> 3) ^ swz(row)) << 3) + (col & 7);
  }
};

// Row index permutation that swaps bits 2 and 3 (an involution on 0..15 in
// every aligned group of 16).  When lane l supplies row perm23(l % 32) of a
// 32-row MFMA operand, the C-layout registers 8*k2 + e of lane l hold rows
// 16*k2 + 8*(l/32) + e, e = 0..7: eight *consecutive* rows per 16-row k-step,
// which is exactly the k order of an A (or B) operand read as one 16-byte
// chunk from a transposed (sequence-contiguous) tile.
__device__ __forceinline__ int perm23(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

// 8 consecutive elements (one 16-byte chunk) of one row of a TileLayout<RL>
// tile: an MFMA operand whose k index runs along the row.
template <int RL>
__device__ __forceinline__ bf16x8 row_operand(const bf16* tile, int row, int col) {
  return *reinterpret_cast<const bf16x8*>(tile + TileLayout<RL>::off(row, col));
}

// 16 bytes per lane from global memory straight into LDS at
// lds_block + 16*lane (global_load_lds_dwordx4; lds_block is wave-uniform).
__device__ __forceinline__ void direct_load16(const void* src, void* lds_block) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_block, 16, 0, 0);
}

// 4 bytes per lane from global memory straight into LDS at lds_block + 4*lane.
__device__ __forceinline__ void direct_load4(const void* src, void* lds_block) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_block, 4, 0, 0);
}

// Direct global->LDS staging of a ROWS x RL tile (global rows of RL
// contiguous bf16 at `row_stride` elements) into TileLayout<RL> with
// global_load_lds_dwordx4.  One wave instruction moves 1 KB: lane j's 16
// bytes land at LDS block base + 16*j, i.e. row row0 + j/(RL/8), chunk slot
// j%(RL/8); the lane therefore loads the logical chunk the swizzle maps to
// that slot.  Rows at or past rows_valid (>= 1) re-read row rows_valid-1:
// callers never use those rows unmasked.  The NW waves of a workgroup split
// the tile's instructions; completion is tracked by vmcnt (callers wait with
// vmcnt(0) and a barrier before reading).
template <int ROWS, int RL, int NW>
__device__ __forceinline__ void stage_direct(bf16* lds, const bf16* g, int64_t row_stride, int rows_valid, int wave,
                                             int lane) {
  constexpr int kCpr = RL / 8;      // 16-byte chunks per row
  constexpr int kRpi = 64 / kCpr;   // rows per wave instruction
  constexpr int kNi = ROWS / kRpi;  // instructions per tile
  static_assert(kNi % NW == 0, "tile must split evenly over the waves");
#pragma unroll
  for (int i = 0; i < kNi / NW; ++i) {
    const int row0 = (wave * (kNi / NW) + i) * kRpi;
    const int row = row0 + lane / kCpr;
    const int chunk = (lane % kCpr) ^ TileLayout<RL>::swz(row);
    const int srow = min(row, rows_valid - 1);
    direct_load16(g + (int64_t)srow * row_stride + chunk * 8, lds + row0 * RL);
  }
}

// stage_direct with the per-lane source offsets precomputed (they depend only
// on the lane, the wave and the row stride): for full tiles each load is a
// uniform tile base plus a 32-bit lane offset, with no per-tile address math.
// The row stride times ROWS must fit in 31 bits.
template <int ROWS, int RL, int NW>
struct DirectStager {
  static constexpr int kCpr = RL / 8;
  static constexpr int kRpi = 64 / kCpr;
  static constexpr int kNi = ROWS / kRpi;
  static constexpr int kPer = kNi / NW;
  static_assert(kNi % NW == 0, "tile must split evenly over the waves");
  int off[kPer];  // element offset of this lane's source chunk, per instruction

  __device__ __forceinline__ void init(int64_t row_stride, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int row0 = (wave * kPer + i) * kRpi;
      const int row = row0 + lane / kCpr;
      off[i] = (int)(row * row_stride) + ((lane % kCpr) ^ TileLayout<RL>::swz(row)) * 8;
    }
  }
  __device__ __forceinline__ static int lds_row0(int i, int wave) { return (wave * kPer + i) * kRpi; }
  // Every row valid; `g` points at the tile's first row.
  __device__ __forceinline__ void stage_full(bf16* lds, const bf16* g, int wave) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) direct_load16(g + off[i], lds + lds_row0(i, wave) * RL);
  }
  // rows_valid in [1, ROWS].
  __device__ __forceinline__ void stage(bf16* lds, const bf16* g, int64_t row_stride, int rows_valid, int wave,
                                        int lane) const {
    if (rows_valid >= ROWS)
      stage_full(lds, g, wave);
    else
      stage_direct<ROWS, RL, NW>(lds, g, row_stride, rows_valid, wave, lane);
  }
};

// Wait for this wave's outstanding global loads (including direct-to-LDS
// ones); a following barrier makes every wave's tile visible.
__device__ __forceinline__ void wait_vmem() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace avattn
