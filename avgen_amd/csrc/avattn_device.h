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

#include <type_traits>
#include <utility>

namespace avattn {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));  // 32 fp8 values

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 32x32x64 product of e4m3 (OCP fp8) operands: lane l supplies row (A) or
// column (B) l % 32 as 32 bytes; A and B use the same byte -> k mapping, so a
// lane's bytes j of A and B meet in the sum whatever that mapping is.  With
// zero scale operands the compiler selects the unscaled
// v_mfma_f32_32x32x64_f8f6f4 (format 0 = e4m3 for both operands), which
// computes the plain product (checked on the GPU against the layout-free sum
// of per-lane byte products).
__device__ __forceinline__ f32x16 mfma32_fp8(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// The same product with block scales: c + 2^(sa-127) * 2^(sb-127) * (a . b),
// sa and sb E8M0 exponents (byte 0 of the operand, 127 = 1.0) applied to the
// products only, c added unscaled (checked on the GPU against the unscaled
// product for exponents -27..13 with a nonzero c).
__device__ __forceinline__ f32x16 mfma32_fp8_scaled(const i32x8& a, const i32x8& b, const f32x16& c, int sa,
                                                    int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

// The smallest e with 2^e >= |t|, clamped to [-126, 127] (E8M0's range of
// finite scales with a normal fp32 2^-e): a zero or subnormal t gives -126,
// an infinite or NaN one 127.
__device__ __forceinline__ int ceil_log2_clamped(float t) {
  const uint32_t u = __float_as_uint(t) & 0x7fffffffu;
  const int field = (int)(u >> 23);
  if (field == 0) return -126;
  const int e = field - 127 + ((u & 0x7fffffu) != 0u ? 1 : 0);
  return e > 127 ? 127 : (e < -126 ? -126 : e);
}

// Four fp32 values -> four e4m3 bytes (byte i = value i), round to nearest
// even, no saturation (|x| < 464 stays finite; the callers scale into
// [-448, 448]); v_cvt_pk_fp8_f32 matches torch's float8_e4m3fn cast bit for
// bit, subnormals included.
__device__ __forceinline__ uint32_t pack_fp8x4(float x0, float x1, float x2, float x3) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, w, true);
  return (uint32_t)w;
}

// The two bf16 halves of a 32-bit word as fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// The same value, opaque to the optimizer at this point of the program: an
// LDS offset or address passed through it is added to a stage's base where
// it is used (folded into the instruction's 16-bit offset field when that
// fits) instead of being hoisted out of the loop as one extra register per
// (offset, stage) pair.
template <class T>
__device__ __forceinline__ T opaque(T x) {
  __asm__ volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ f32x16 splat16(float x) {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = x;
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

// Rotation of 2 interleaved pairs (4 consecutive channels) held as two bf16x2
// words: the same arithmetic as rotate8, for the epilogues whose lanes own 4
// consecutive channels of a row.
__device__ __forceinline__ u32x2 rotate4(const u32x2& x, float c0, float s0, float c1, float s1, bool inverse) {
#pragma clang fp contract(off)
  u32x2 r;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float c = p ? c1 : c0, s = p ? s1 : s0;
    const float e = __uint_as_float(x[p] << 16);
    const float o = __uint_as_float(x[p] & 0xffff0000u);
    const float ec = e * c, os = o * s, es = e * s, oc = o * c;
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

// One step of the ring merge (torch/.../_context_parallel/_attention.py
// :182-183) for a row with accumulated LSE `la` and block LSE `lb`:
//   out <- out - sigmoid(lb - la) * (out - out_b),  lse <- la - logsigmoid(la - lb)
// with sigmoid = 1 / (1 + exp(-x)) and logsigmoid = min(x, 0) - log1p(exp(-|x|))
// (PyTorch's closed forms).  A -inf LSE (a row with no valid key) is the
// identity element: a -inf block keeps the accumulator (mode 0), a -inf
// accumulator takes the block (mode 1).  Anything else, NaN included, goes
// through the formula (mode 2), so a NaN on either side stays NaN.  Returns
// the merged LSE; lse_merge_elem gives each merged output element.  Every
// kernel that merges uses these two functions, so the separate merge kernel
// and the forward's fused merge round identically.
__device__ __forceinline__ float lse_merge_coeffs(float la, float lb, int& mode, float& w) {
  if (lb == kNegInf) {
    mode = 0;
    w = 0.f;
    return la;
  }
  if (la == kNegInf) {
    mode = 1;
    w = 1.f;
    return lb;
  }
  mode = 2;
  w = 1.f / (1.f + expf(-(lb - la)));
  const float x = la - lb;
  const float ls = fminf(x, 0.f) - log1pf(expf(-fabsf(x)));
  return la - ls;
}
__device__ __forceinline__ float lse_merge_elem(float o, float ob, int mode, float w) {
  return mode == 0 ? o : (mode == 1 ? ob : o - w * (o - ob));
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

// An int of device memory the kernel only reads, loaded through the constant
// address space: with a wave-uniform address this is a scalar load.  (The
// kernels' inline-asm stores clobber "memory", so the compiler cannot prove
// such data unchanged and keeps a plain load a vector load, counted with the
// hand-counted tile loads and waited for with them.)
__device__ __forceinline__ int load_const_i32(const int* p, int64_t i) {
  typedef __attribute__((address_space(4))) const int const_int;
  return reinterpret_cast<const_int*>(reinterpret_cast<uintptr_t>(p))[i];
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
// wave load (TileStager).  Row-major sequence tiles use RL = head_dim;
// head_dim-major ("transposed") tiles use RL = the tile's sequence length.
template <int RL>
struct TileLayout {
  static_assert(RL == 32 || RL == 64 || RL == 128, "row length 32, 64 or 128 elements");
  static constexpr int kRowElems = RL;
  static __host__ __device__ __forceinline__ int swz(int row) {
    if constexpr (RL == 128) return ((row & 3) << 2) | ((row >> 2) & 3);
    if constexpr (RL == 64) return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
    return (row >> 2) & 3;
  }
  // Element offset of (row, col); col must be a multiple of 4.
  static __host__ __device__ __forceinline__ int off(int row, int col) {
    return row * RL + (((col >> 3) ^ swz(row)) << 3) + (col & 7);
  }
};

// Row index permutation that swaps bits 2 and 3 (an involution on 0..15 in
// every aligned group of 16).  When lane l supplies row perm23(l % 32) of a
// 32-row MFMA operand, the C-layout registers 8*k2 + e of lane l hold rows
// 16*k2 + 8*(l/32) + e, e = 0..7: eight *consecutive* rows per 16-row k-step,
// which is exactly the k order of an A (or B) operand read as one 16-byte
// chunk from a transposed (sequence-contiguous) tile.
__host__ __device__ __forceinline__ int perm23(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

// Element offset lane `lane` passes to transposed read h (0, 1) of a
// row-major TileLayout<RL> tile, for the A operand of a product contracting
// over the tile's rows (ds_read_b64_tr_b16: in each 16-lane group lane i
// points at four consecutive elements of "row" i/4 and lane j receives
// element j of the four rows).  Lane i of group g points at channels
// 32*dt + 16*(g%2) + 4*(i%4) .. +3 of row 8*(g/2) + 4*h + i/4, so lane l
// receives channel 32*dt + l%32 of rows 8*(l/32) + 4*h .. +3: the two reads
// give the eight consecutive rows of its k slots.  For the 16-row step s add
// 16*s*RL: the row swizzle repeats every 16 rows.
template <int RL>
__host__ __device__ __forceinline__ int tr_read_off(int lane, int dt, int h) {
  return TileLayout<RL>::off(8 * (lane >> 5) + 4 * h + ((lane & 15) >> 2), 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3));
}

// 8 consecutive elements (one 16-byte chunk) of one row of a TileLayout<RL>
// tile: an MFMA operand whose k index runs along the row.
template <int RL>
__device__ __forceinline__ bf16x8 row_operand(const bf16* tile, int row, int col) {
  return *reinterpret_cast<const bf16x8*>(tile + TileLayout<RL>::off(row, col));
}

// ---------------------------------------------------------------------------
// Staged dS units (backward with the dS stored to HBM)
// ---------------------------------------------------------------------------
// A unit is the bf16 dS of 32 query rows x 128 keys, 8 KB ordered
// [k2 (2)][128 keys][16 rows]: row 16*k2 + r of key j at element
// (k2*128 + j)*16 + r.  The units of one (query head, 32-row group) follow
// each other for the 128-key blocks kt = 0, 1, ...; the two units of a
// 64-row tile are nkt*8192 bytes apart.
struct DsUnit {
  // Writer (a dS wave of the dK/dV kernel; its lane owns key j of the block,
  // j = 32*kw + lane % 32): the 16 bytes of rows 16*k2 + 8*(lane/32) .. +7
  // of the tile's half `sub` go to this byte offset from the tile's first
  // unit.
  static __host__ __device__ __forceinline__ uint32_t store_offset(int j, int lane, int sub, int k2, int nkt) {
    return (uint32_t)(sub ? nkt * 8192 : 0) + (uint32_t)k2 * 4096 + (uint32_t)j * 32 + 16 * (lane >> 5);
  }
  // Reader (the dQ kernel; a wave owns one 32-row group): stage s holds keys
  // [BK*s, BK*s + BK); its 1 KB load i (of BK/16) brings lane `lane`'s 16
  // bytes from this byte offset of the group's units to LDS byte 1024*i +
  // 16*lane, so the stage sits in LDS as [k2][BK keys][16 rows].
  template <int BK>
  static __host__ __device__ __forceinline__ uint32_t stage_src(int s, int i, int lane) {
    constexpr int per_k2 = BK / 32;
    return (uint32_t)(s * BK / 128) * 8192 + (uint32_t)((s * BK) % 128) * 32 + (uint32_t)lane * 16 +
           (uint32_t)(i % per_k2) * 1024 + (uint32_t)(i / per_k2) * 4096;
  }
  // Element offset (in the wave's [k2][BK][16] stage) that lane `lane`
  // passes to the transposed read `half` (0, 1) of 16-key step ks: in its
  // 16-lane group G (k2 = G % 2, key half G / 2) lane i points at rows
  // 16*k2 + 4*(i%4) .. +3 of key 16*ks + 8*(G/2) + 4*half + i/4.
  template <int BK>
  static __host__ __device__ __forceinline__ int tr_elem(int lane, int ks, int half) {
    const int g = lane >> 4, i = lane & 15;
    return ((g & 1) * BK + 8 * (g >> 1) + (i >> 2)) * 16 + 4 * (i & 3) + ks * 256 + half * 64;
  }
};

// ---------------------------------------------------------------------------
// Direct global->LDS tile loads (buffer_load_dword{,x4} ... lds).
// ---------------------------------------------------------------------------
// Issued through inline assembly on purpose: the kernels order these loads
// themselves (a counted vmcnt wait, then a workgroup barrier, before a stage
// is read; a barrier before a stage is refilled).  Seen as compiler builtins
// they are LDS writes whose aliasing with later LDS reads the compiler can
// only track for a few buffers at a time, and it then inserts vmcnt waits
// that also wait for tiles loaded ahead.  Addressing: a raw buffer resource
// (scalar base + byte range), a 32-bit per-lane byte offset and a scalar byte
// offset; M0 holds the LDS destination of lane 0 (lane j writes +4*j or
// +16*j bytes).

// Raw buffer over [base, base + bytes): descriptor words for the gfx9 family
// (32-bit data format in word 3, no swizzle, stride 0), in scalar registers.
__device__ __forceinline__ u32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000u;
  return r;
}

// Byte address of an LDS location (the value M0 takes).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p);
}

// 16 bytes per lane from base + voff + soff into LDS at lds + 16*lane.
__device__ __forceinline__ void dma16(const u32x4& r, uint32_t lds, uint32_t voff, uint32_t soff) {
  __asm__ volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds),
      "v"(voff), "s"(r), "s"(soff)
      : "memory", "m0");
}

// 4 bytes per lane into LDS at lds + 4*lane.
__device__ __forceinline__ void dma4(const u32x4& r, uint32_t lds, uint32_t voff, uint32_t soff) {
  __asm__ volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, %3 offen lds" ::"s"(lds),
      "v"(voff), "s"(r), "s"(soff)
      : "memory", "m0");
}

// Full ROWS x RL tile (rows of RL contiguous bf16, `row_stride` elements
// apart in the source) into TileLayout<RL> with dma16.  One wave instruction
// moves 1 KB: lane j's 16 bytes land at LDS block base + 16*j, i.e. row
// row0 + j/(RL/8), chunk slot j%(RL/8), so the lane loads the logical chunk
// the swizzle maps to that slot.  The NW waves of a workgroup split the
// tile's instructions; the per-lane byte offsets depend only on the lane, the
// wave and the row stride, so they are computed once.
template <int ROWS, int RL, int NW>
struct TileStager {
  static constexpr int kCpr = RL / 8;      // 16-byte chunks per row
  static constexpr int kRpi = 64 / kCpr;   // rows per wave instruction
  static constexpr int kNi = ROWS / kRpi;  // instructions per tile
  // Instructions per wave.  With fewer instructions than waves, wave w
  // repeats instruction w % kNi (the same bytes to the same place), so every
  // wave issues the same number of loads and can wait on a fixed count.
  static constexpr int kPer = kNi >= NW ? kNi / NW : 1;
  static_assert(kNi % NW == 0 || NW % kNi == 0, "tile must split evenly over the waves");
  uint32_t off[kPer];  // byte offset of this lane's source chunk, per instruction
  uint32_t lds0;       // byte offset of this wave's first LDS block in the tile

  // First instruction of wave `wave` (instructions first .. first+kPer-1).
  static __host__ __device__ __forceinline__ int first_instr(int wave) { return (wave * kPer) % kNi; }
  // Tile row whose chunk lane `lane` moves in instruction `instr`.
  static __host__ __device__ __forceinline__ int row_of(int instr, int lane) {
    return instr * kRpi + lane / kCpr;
  }
  // Byte offset (from the tile's first source row) of the 16-byte source chunk
  // lane `lane` moves in instruction `instr`: the logical chunk stored at
  // physical slot lane % kCpr of its row.
  static __host__ __device__ __forceinline__ uint32_t src_offset(int instr, int lane, int64_t row_stride) {
    const int row = row_of(instr, lane);
    return (uint32_t)((row * row_stride + ((lane % kCpr) ^ TileLayout<RL>::swz(row)) * 8) * 2);
  }
  __device__ __forceinline__ void init(int64_t row_stride, int wave, int lane) {
    const int first = first_instr(wave);
    lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(first * kRpi * RL * 2));
#pragma unroll
    for (int i = 0; i < kPer; ++i) off[i] = src_offset(first + i, lane, row_stride);
  }
  // `soff`: byte offset of the tile's first row in the buffer.
  __device__ __forceinline__ void stage(bf16* lds, const u32x4& r, uint32_t soff) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) stage_one(lds, r, soff, i);
  }
  // Instruction i of stage() alone (i < kPer), for spreading a tile's loads
  // between other work.
  __device__ __forceinline__ void stage_one(bf16* lds, const u32x4& r, uint32_t soff, int i) const {
    dma16(r, lds_addr(lds) + lds0 + i * kRpi * RL * 2, off[i], soff);
  }
};

// 16 bytes per lane at byte base + voff + soff of a raw buffer, non-temporal
// (streamed past the caches, so a large write does not evict the reader's
// cached tiles).  Inline assembly like the loads above: the caller counts
// these stores in its vmcnt waits.  A store of more than 8 bytes with an
// SGPR offset reads its data registers for one more cycle: the next
// instruction must not be a VALU write of them (one wait state).  The
// compiler inserts that wait state after the stores it emits itself, not
// after inline assembly, so the s_nop is part of the statement.
__device__ __forceinline__ void store_b128_nt(const u32x4& r, uint32_t voff, uint32_t soff, const u32x4& data) {
  __asm__ volatile(
      "buffer_store_dwordx4 %0, %1, %2, %3 offen nt\n\t"
      "s_nop 0" ::"v"(data),
      "v"(voff), "s"(r), "s"(soff)
      : "memory");
}

// dma16 with a non-temporal load (data read once).
__device__ __forceinline__ void dma16_nt(const u32x4& r, uint32_t lds, uint32_t voff, uint32_t soff) {
  __asm__ volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen nt lds" ::"s"(lds),
      "v"(voff), "s"(r), "s"(soff)
      : "memory", "m0");
}

// Four bf16 of a transposed LDS read (ds_read_b64_tr_b16): in each group of
// 16 lanes, lane i supplies the address of 4 consecutive elements, the
// piece (i % 4) of "row" i / 4 of a 4 x 16 block, and lane j receives
// element j of rows 0..3 (checked on the GPU).
__device__ __forceinline__ bf16x4 lds_read_tr16(const bf16* p) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(const_cast<bf16*>(p)));
}

// LDS accesses at a byte address (lds_addr) held in a register; with the
// address made opaque, a constant added to it goes into the offset field.
template <class T>
__device__ __forceinline__ T lds_ld(uint32_t a) {
  return *(const __attribute__((address_space(3))) T*)(uintptr_t)a;
}
template <class T>
__device__ __forceinline__ void lds_st(uint32_t a, const T& v) {
  *(__attribute__((address_space(3))) T*)(uintptr_t)a = v;
}
__device__ __forceinline__ bf16x4 lds_read_tr16_at(uint32_t a) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(uintptr_t)a);
}

// Retire every outstanding memory operation of this wave, as an instruction
// the compiler's wait-count bookkeeping sees: a loop that issues its tile
// loads as inline assembly calls this first, so no compiler-inserted wait for
// a prologue load lands inside the loop (where, counting the loop's own tile
// loads too, it would wait for tiles loaded ahead).
__device__ __forceinline__ void retire_prologue_loads() { __builtin_amdgcn_s_waitcnt(0); }

// Wait until at most N of this wave's vector-memory loads are outstanding
// (loads complete in issue order, so every load issued before the last N has
// landed).
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait for this wave's outstanding global loads (including direct-to-LDS
// ones); a following barrier makes every wave's tile visible.
__device__ __forceinline__ void wait_vmem() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier that orders this wave's LDS writes before every wave's
// later LDS reads, without waiting for outstanding global loads (unlike
// __syncthreads, whose release fence also waits for the next tile's direct
// global->LDS loads still in flight).
__device__ __forceinline__ void barrier_lds() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// Instruction-class masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedValu = 0x002;
constexpr int kSchedDsRead = 0x100;
constexpr int kSchedDsWrite = 0x200;
constexpr int kSchedVmem = 0x010;
constexpr int kSchedSalu = 0x004;

// f(std::integral_constant<int, u>()) for u = 0 .. N-1 in order while f
// returns true (a loop body unrolled with its iteration index as a
// compile-time constant); returns whether every call did.
template <class F, int... U>
__device__ __forceinline__ bool unrolled_while(F&& f, std::integer_sequence<int, U...>) {
  return (f(std::integral_constant<int, U>()) && ...);
}
template <int N, class F>
__device__ __forceinline__ bool unrolled_while(F&& f) {
  return unrolled_while(f, std::make_integer_sequence<int, N>());
}

}  // namespace avattn
