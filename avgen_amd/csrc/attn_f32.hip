// Attention on float32 tensors.  The reference's attention() computes in the
// caller's dtype (src/avgen/models/attention.py:227-273 hands q, k, v to
// F.scaled_dot_product_attention as they come), and its fp32 tensors are
// rotated in fp32 (src/avgen/models/rope.py:332-338, a cast back to fp32 is
// the identity).  These kernels keep every operand and every product in
// fp32, the products on the fp32 matrix cores (v_mfma_f32_32x32x2f32: its
// peak, 157.3 TFLOP/s, equals the vector ALUs', but it takes one operand
// float per lane per 4,096 FLOP where vector FMAs need LDS reads for every
// four):
//   * forward: one wave per 32 query rows, 32-key tiles of K and V through
//     LDS, the online softmax in the exp2 domain;
//   * backward, without atomics: row statistics (lse2 = lse*log2 e, +inf
//     for a row without keys; ndelta = -rowsum(dO*O)), then dK/dV with a
//     pair of waves per 32 keys looping over 32-row query tiles of every
//     query head of its group, and dQ either from the dS the dK/dV kernel
//     staged (one product, in passes of (batch, kv head) pairs) or with a
//     pair of waves per 32 query rows recomputing S and dP;
//   * per-row key windows in all of them (the temporal neighbour and packed
//     varlen masks of src/avgen/models/blocks.py:54-104 and
//     src/avgen/data/packing.py:181-200), visiting only the tiles that meet;
//   * the interleaved-pair rotation of fp32 tensors (and its transpose),
//     with the reference's operation order (two products, one sum, no FMA),
//     and the per-head RMSNorm fused with it (q_norm/k_norm, fp32 gain).
// Every attention kernel is sized for two waves per SIMD (at most 256
// registers).
// They are the exact-dtype path for fp32 callers; the bf16 kernels are the
// fast path.
#include "avattn.h"

#include <math.h>

#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {
namespace {

struct F32Args {
  const float *q, *k, *v;
  int64_t qsb, qsh, qsl, ksb, ksh, ksl, vsb, vsh, vsl;
  int B, Hq, Hkv, Lq, Lk, D;
  const uint8_t* mask;
  int64_t msb;
  float scale, c;  // c = scale * log2(e)
  // forward
  float* o;
  int64_t osb, osh, osl;
  float* lse;
  // backward
  const float *dout, *out, *lse_in;
  int64_t dosb, dosh, dosl, oisb, oish, oisl;
  float *dq, *dk, *dv;
  int64_t dqsb, dqsh, dqsl, dksb, dksh, dksl, dvsb, dvsh, dvsl;
  float *lse2, *ndelta;  // workspace, (B, Hq, Lq) each
  // staged dS: pairs pair0 .. of this pass, dsp floats per (batch, kv head)
  // pair, 32x32 row-major blocks ordered (query head of the group, row tile,
  // key tile) with ceil(Lq/32) row tiles and 4*ceil(Lk/128) key tiles
  float* ds;
  int64_t dsp;
  int pair0;
  // per-row key windows (WIN kernels): row r of batch b attends keys in
  // [wlo[b*wsb + r], whi[b*wsb + r]), clamped into 0 <= lo <= hi <= Lk
  const int32_t *wlo, *whi;
  int64_t wsb;
};

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, const f32x4& v) { *reinterpret_cast<f32x4*>(p) = v; }

__device__ __forceinline__ bool key_ok(const F32Args& a, int b, int key) {
  return key < a.Lk && (a.mask == nullptr || a.mask[b * a.msb + key] != 0);
}

// The clamped key window of row r of batch b.
__device__ __forceinline__ void row_window(const F32Args& a, int b, int r, int& lo, int& hi) {
  const int64_t i = (int64_t)b * a.wsb + r;
  lo = min(max(a.wlo[i], 0), a.Lk);
  hi = min(max(a.whi[i], lo), a.Lk);
}

// The 32-key tiles [t0, t1) meeting the union of the non-empty windows held
// by the lanes of a workgroup's NW waves (every thread calls it: it holds a
// barrier; red: 2*NW ints of LDS).
template <int NW>
__device__ __forceinline__ void window_tiles(int lo, int hi, bool use, int* red, int& t0, int& t1) {
  int mn = use && lo < hi ? lo : 0x7fffffff, mx = use && lo < hi ? hi : -1;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mn = min(mn, __shfl_xor(mn, o)), mx = max(mx, __shfl_xor(mx, o));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = mn, red[NW + wave] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) mn = min(mn, red[w]), mx = max(mx, red[NW + w]);
  // the same in every lane; said so, so the tile loops run on scalar
  // counters and uniform branches (barriers inside them)
  t0 = __builtin_amdgcn_readfirstlane(mn < mx ? mn / 32 : 0);
  t1 = __builtin_amdgcn_readfirstlane(mn < mx ? (mx + 31) / 32 : 0);
}

// Does any of the wave's rows (lanes' windows, both halves alike) meet key
// block kb (keys [128*kb, min(128*kb + 128, Lk))?  Wave-uniform.
__device__ __forceinline__ bool rows_meet_block(const F32Args& a, int lo, int hi, bool use, int kb) {
  const int k0 = 128 * kb, k1 = min(k0 + 128, a.Lk);
  return __builtin_amdgcn_ballot_w64(use && lo < k1 && hi > k0) != 0;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// On the fp32 matrix cores (v_mfma_f32_32x32x2f32: A one float per lane,
// A[m = l%32][k = l/32]; B[k = l/32][n = l%32]; D register i of lane l at
// [8*(i/4) + 4*(l/32) + i%4][l%32], checked on the GPU).  One wave per 32
// query rows, four per workgroup, 32-key tiles.  Scores are formed
// transposed, S^T = K Q^T, k-step j contracting channels j and D/2 + j (the
// lane's half of head_dim, held in registers as B operands), so lane l holds
// 16 keys of query l%32; those are exactly the keys its B operand of
// O^T += V^T P^T needs in k-step j (key 8*(j/4) + 4*(l/32) + j%4), so P
// never moves.  K tiles sit in LDS row-major with rows padded by 4 floats
// (the 32 lanes of a K read hit different banks); V tiles with channel
// 32*t + m of a key at m*(D/32) + t, so one read gives a lane the D/32
// channels its products for one key take.  Both are staged one tile ahead
// through registers, and the next operands are read while the current
// ones' products issue.  The running maximum is raised only when a score
// exceeds it by more than 2^8 in the exp2 domain (any lane of the wave: the
// branch is uniform), so the rescale of the output accumulator is rare;
// the probabilities stay at most 2^8 and out = O / l is unchanged in exact
// arithmetic.  WIN: per-row key windows (F32Args::wlo/whi): the workgroup
// visits the tiles meeting its rows' windows and masks each score outside
// its row's window.
template <int D, bool WIN>
__global__ __launch_bounds__(256, 2) void fwd_f32_kernel(F32Args a) {
  constexpr int KT = 32, ROWS = 128, PITCH = D + 4, HD = D / 2, DT = D / 32;
  constexpr int PER = KT * D / 4 / 256;  // K float4 chunks per thread and tile
  constexpr int VPER = KT * 32 / 256;    // V (key, lane) slots per thread and tile
  using vdt = float __attribute__((ext_vector_type(DT)));
  __shared__ __attribute__((aligned(16))) float ks[2][KT * PITCH];
  __shared__ __attribute__((aligned(16))) float vs[2][KT * D];
  __shared__ __attribute__((aligned(16))) float bias[2][KT];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int nqb = (a.Lq + ROWS - 1) / ROWS;
  const int qb = blockIdx.x % nqb, bh = blockIdx.x / nqb;
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int row = qb * ROWS + wave * 32 + l32;
  const bool valid = row < a.Lq;

  float q[HD];  // channels hh*HD .. +HD-1 of this lane's query row
  {
    const float* qp = a.q + b * a.qsb + h * a.qsh + (int64_t)row * a.qsl + hh * HD;
#pragma unroll
    for (int d = 0; d < HD; d += 4) {
      const f32x4 x = valid ? ld4(qp + d) : f32x4{0.f, 0.f, 0.f, 0.f};
      q[d] = x[0], q[d + 1] = x[1], q[d + 2] = x[2], q[d + 3] = x[3];
    }
  }
  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = zero16();
  float m = kNegInf, l = 0.f;
  const float* kb = a.k + b * a.ksb + hk * a.ksh;
  const float* vb = a.v + b * a.vsb + hk * a.vsh;

  // Tile staging: thread tid moves K float4 chunks u = tid + 256*i (key u /
  // (D/4), channels 4*(u % (D/4)) ..) and V slots u = tid + 256*i (key u/32,
  // channels 32*t + u%32).
  f32x4 pk[PER];
  float pv[VPER][DT];
  float pbias = 0.f;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + 256 * i, j = u / (D / 4), c4 = 4 * (u % (D / 4)), key = k0 + j;
      pk[i] = key < a.Lk ? ld4(kb + (int64_t)key * a.ksl + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < VPER; ++i) {
      const int u = tid + 256 * i, key = k0 + u / 32;
      const float* vp = vb + (int64_t)key * a.vsl + (u % 32);
#pragma unroll
      for (int t = 0; t < DT; ++t) pv[i][t] = key < a.Lk ? vp[32 * t] : 0.f;
    }
    if (tid < KT) pbias = key_ok(a, b, k0 + tid) ? 0.f : kNegInf;
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = tid + 256 * i, j = u / (D / 4), c4 = 4 * (u % (D / 4));
      st4(&ks[buf][j * PITCH + c4], pk[i]);
    }
#pragma unroll
    for (int i = 0; i < VPER; ++i) {
      const int u = tid + 256 * i;
      vdt x;
#pragma unroll
      for (int t = 0; t < DT; ++t) x[t] = pv[i][t];
      *reinterpret_cast<vdt*>(&vs[buf][(u / 32) * D + (u % 32) * DT]) = x;
    }
    if (tid < KT) bias[buf][tid] = pbias;
  };

  int t0 = 0, ntile = (a.Lk + KT - 1) / KT, wl = 0, wh = a.Lk;
  if constexpr (WIN) {
    __shared__ int red[8];
    if (valid) row_window(a, b, row, wl, wh);
    window_tiles<4>(wl, wh, valid, red, t0, ntile);
  }
  if (t0 < ntile) {
    fetch(t0 * KT);
    store(0);
  }
  for (int t = t0; t < ntile; ++t) {
    const int buf = (t - t0) & 1;
    __syncthreads();  // tile t stored; every wave is done with tile t - 1
    if (t + 1 < ntile) fetch((t + 1) * KT);
    // S^T = K Q^T: k-step j takes channels j (lanes 0-31) and HD + j (32-63)
    const float* kr = ks[buf] + l32 * PITCH + hh * HD;
    f32x16 s = zero16();
    f32x4 k0 = ld4(kr), k1 = ld4(kr + 4);
#pragma unroll
    for (int j = 0; j < HD; j += 8) {
      f32x4 n0 = k0, n1 = k1;
      if (j + 8 < HD) n0 = ld4(kr + j + 8), n1 = ld4(kr + j + 12);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(k0[e], q[j + e], s, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(k1[e], q[j + 4 + e], s, 0, 0, 0);
      k0 = n0, k1 = n1;
    }
    // register i: key 8*(i/4) + 4*hh + i%4 of the tile, query l32
    float mt = kNegInf;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 bb = ld4(&bias[buf][8 * g + 4 * hh]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[4 * g + r] += bb[r];
        if constexpr (WIN) {
          const int key = t * KT + 8 * g + 4 * hh + r;
          if (key < wl || key >= wh) s[4 * g + r] = kNegInf;
        }
        mt = fmaxf(mt, s[4 * g + r]);
      }
    }
    mt = halves_max(mt);  // the query's other 16 keys
    // (mt - m)*c is NaN when both are -inf (no key yet: nothing to raise)
    if (__builtin_amdgcn_ballot_w64((mt - m) * a.c > 8.f)) {
      const float mn = fmaxf(m, mt);
      const float alpha = (m == kNegInf || mn == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m - mn) * a.c);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
      m = mn;
    }
    const float mc = m * a.c;
    f32x16 p;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[i] = m == kNegInf ? 0.f : __builtin_amdgcn_exp2f(fmaf(s[i], a.c, -mc));
      l += p[i];
    }
    // O^T += V^T P^T: k-step j takes key 8*(j/4) + 4*hh + j%4, this lane's
    // register j of P; A is channel 32*dt + l32 of that key.
    const float* vr = vs[buf] + 4 * hh * D + l32 * DT;
    auto vkey = [&](int j) { return *reinterpret_cast<const vdt*>(vr + (8 * (j / 4) + (j % 4)) * D); };
    vdt v0 = vkey(0), v1 = vkey(1);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      vdt n0 = v0, n1 = v1;
      if (j + 2 < 16) n0 = vkey(j + 2), n1 = vkey(j + 3);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[dt], p[j], o[dt], 0, 0, 0);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[dt], p[j + 1], o[dt], 0, 0, 0);
      v0 = n0, v1 = n1;
    }
    if (t + 1 < ntile) store(buf ^ 1);
  }

  // The row sum over both halves of the keys; l > 0: normal row; l == 0: no
  // valid key (out 0, lse -inf); NaN: a NaN or +inf score reached the row.
  l = halves_sum(l);
  if (!valid) return;
  const float nan = __builtin_nanf("");
  const float inv = l > 0.f ? 1.f / l : (l == 0.f ? 0.f : nan);
  float* op = a.o + b * a.osb + h * a.osh + (int64_t)row * a.osl;
  // o[dt] register i: channel 32*dt + 8*(i/4) + 4*hh + i%4 of this lane's query
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      st4(op + 32 * dt + 8 * g + 4 * hh,
          f32x4{o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv});
  if (hh == 0) a.lse[(int64_t)bh * a.Lq + row] = l > 0.f ? fmaf(m, a.scale, logf(l)) : (l == 0.f ? kNegInf : nan);
}

// Zeros to out and -inf to lse (no keys at all).
__global__ void empty_f32_kernel(F32Args a) {
  const int64_t n = (int64_t)a.B * a.Hq * a.Lq;
  const int D = a.D;
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < n; r += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(r % a.Lq);
    const int h = (int)((r / a.Lq) % a.Hq);
    const int b = (int)(r / ((int64_t)a.Lq * a.Hq));
    float* op = a.o + b * a.osb + h * a.osh + (int64_t)i * a.osl;
    for (int d = 0; d < D; d += 4) st4(op + d, f32x4{0.f, 0.f, 0.f, 0.f});
    a.lse[r] = kNegInf;
  }
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_pre_f32_kernel(F32Args a) {
  const int64_t n = (int64_t)a.B * a.Hq * a.Lq;
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int i = (int)(r % a.Lq);
  const int h = (int)((r / a.Lq) % a.Hq);
  const int b = (int)(r / ((int64_t)a.Lq * a.Hq));
  const float* dp = a.dout + b * a.dosb + h * a.dosh + (int64_t)i * a.dosl;
  const float* op = a.out + b * a.oisb + h * a.oish + (int64_t)i * a.oisl;
  float acc = 0.f;
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    const f32x4 x = ld4(dp + d), y = ld4(op + d);
    acc = fmaf(x[0], y[0], fmaf(x[1], y[1], fmaf(x[2], y[2], fmaf(x[3], y[3], acc))));
  }
  a.ndelta[r] = -acc;
  const float l = a.lse_in[r];
  a.lse2[r] = l == kNegInf ? kPosInf : l * kLog2e;
}


// Backward tiles of 32 rows sit in LDS with channel 32*t + m of a row at
// m*(D/32) + t (rows padded by 4 floats), so one read gives a lane either the
// D/32 channels 32*t + m its products against a row take, or, for the
// contraction over head_dim, the channels of D/32 k-steps: k-step D/32*u + e
// contracts channels 32*e + u (lanes 0-31) and 32*e + u + 16 (lanes 32-63),
// and the operands held in registers follow the same order.
template <int D>
__device__ __forceinline__ void load_row_ksteps(float (&r)[D / 2], const float* p, bool in, int hh) {
  constexpr int DT = D / 32;
#pragma unroll
  for (int u = 0; u < 16; ++u)
#pragma unroll
    for (int e = 0; e < DT; ++e) r[DT * u + e] = in ? p[32 * e + u + 16 * hh] : 0.f;
}

// Staging of one 32-row tile in that layout by 512 threads: thread slot v =
// tid + 512*i holds row v/32, channels 32*t + v%32.
template <int D>
struct Tile32 {
  static constexpr int DT = D / 32, PITCH = D + 4, SL = 32 * 32 / 512;
  using vdt = float __attribute__((ext_vector_type(DT)));
  float x[SL][DT];
  __device__ __forceinline__ void fetch(const float* base, int64_t rs, int r0, int n, int tid) {
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const int v = tid + 512 * i, row = r0 + v / 32;
      const float* p = base + (int64_t)row * rs + (v % 32);
#pragma unroll
      for (int t = 0; t < DT; ++t) x[i][t] = row < n ? p[32 * t] : 0.f;
    }
  }
  __device__ __forceinline__ void store(float* tile, int tid) const {
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const int v = tid + 512 * i;
      vdt y;
#pragma unroll
      for (int t = 0; t < DT; ++t) y[t] = x[i][t];
      *reinterpret_cast<vdt*>(tile + (v / 32) * PITCH + (v % 32) * DT) = y;
    }
  }
};

// dK/dV on the fp32 matrix cores: per 32 keys a pair of waves on one SIMD,
// eight waves per workgroup.  The P wave holds the keys' K halves (B
// operands) and the dV accumulators: S = Q K^T, P = exp2(S*c - lse2), dV +=
// P^T dO.  The dS wave holds the V halves and the dK accumulators: dP = dO
// V^T, dS = P*(dP + ndelta) with P handed over through LDS (the two waves
// hold the same key and rows in the same lanes and registers), dK += dS^T Q.
// S and dP put row 8*(i/4) + 4*(l/32) + i%4 of the tile in register i of lane
// l, against the lane's key, so P and dS registers j are the A operands of
// the second products in k-step j as they stand.  The dS wave runs its dS
// step one tile behind (Q tiles in three slots, P in two), so one barrier
// per tile serves the staging and the hand-over.  STAGE: the dS wave also
// stores dS (0 for masked keys) for bwd_dq_ds_f32_kernel.  WIN: per-row key
// windows, non-decreasing in the row: the workgroup visits the query tiles
// holding the rows whose windows meet its keys (a contiguous range, found
// by binary search) and P is 0 outside each row's window.
template <int D, bool STAGE, bool WIN>
__global__ __launch_bounds__(512) void bwd_dkdv_f32_kernel(F32Args a) {
  constexpr int QT = 32, KPB = 128, PITCH = D + 4, HD = D / 2, DT = D / 32;
  using vdt = float __attribute__((ext_vector_type(DT)));
  __shared__ __attribute__((aligned(16))) float qs[3][QT * PITCH];
  __shared__ __attribute__((aligned(16))) float dos[2][QT * PITCH];
  __shared__ __attribute__((aligned(16))) float l2s[2][QT];
  __shared__ __attribute__((aligned(16))) float nds[3][QT];
  __shared__ __attribute__((aligned(16))) float px[2][4][16 * 64];
  __shared__ __attribute__((aligned(16))) int wls[WIN ? 2 : 1][QT], whs[WIN ? 2 : 1][QT];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int pair = wave & 3, role = wave >> 2;  // role 0: P wave, 1: dS wave
  const int nkb = (a.Lk + KPB - 1) / KPB;
  const int kb = blockIdx.x % nkb, bhk = a.pair0 + blockIdx.x / nkb;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.Hq / a.Hkv;
  const int k0 = kb * KPB + pair * 32;  // the pair's first key
  const int key = k0 + l32;
  const bool kvalid = key_ok(a, b, key);
  float kv[HD];  // K (P wave) or V (dS wave) of the lane's key, k-step order
  load_row_ksteps<D>(kv,
                     role == 0 ? a.k + b * a.ksb + hk * a.ksh + (int64_t)key * a.ksl
                               : a.v + b * a.vsb + hk * a.vsh + (int64_t)key * a.vsl,
                     key < a.Lk, hh);
  f32x16 acc[DT];  // dV (P wave) or dK (dS wave)
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = zero16();

  // dV += P^T dO (P wave) or dK += dS^T Q (dS wave) over one tile; k-step j:
  // rows 8*(j/4) + j%4 (+4 for lanes 32-63), registers j
  auto second = [&](const f32x16& w, const float* tile) {
    const float* bt = tile + l32 * DT;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const vdt y = *reinterpret_cast<const vdt*>(bt + (8 * (j / 4) + 4 * hh + (j % 4)) * PITCH);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[j], y[dt], acc[dt], 0, 0, 0);
    }
  };
  // dS of tile u from its P (LDS) and dP (registers), then dK; staged: dS
  // row 8*(i/4) + 4*hh + i%4, this lane's key, to block (gi, u, key tile)
  const int nrt = (a.Lq + 31) / 32, nkt = 4 * nkb;
  float* dsw = nullptr;
  if constexpr (STAGE) dsw = a.ds + (bhk - a.pair0) * a.dsp + (int64_t)(kb * 4 + pair) * 1024 + l32;
  auto ds_step = [&](const f32x16& dp, int u, int gi) {
    const float* pp = px[u & 1][pair] + lane * 4;
    f32x16 w;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 N = ld4(&nds[u % 3][8 * g + 4 * hh]);
      const f32x4 P = ld4(pp + 256 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) w[4 * g + r] = P[r] * (dp[4 * g + r] + N[r]);
    }
    if constexpr (STAGE) {
      float* o = dsw + ((int64_t)gi * nrt + u) * nkt * 1024;
#pragma unroll
      for (int i = 0; i < 16; ++i) o[(8 * (i / 4) + 4 * hh + (i % 4)) * 32] = kvalid ? w[i] : 0.f;
    }
    second(w, qs[u % 3]);
  };

  // query tiles [tb, ntile)
  int tb = 0, ntile = (a.Lq + QT - 1) / QT;
  if constexpr (WIN) {
    // rows meeting keys [K0, K1): from the first row with hi > K0 to the
    // first with lo >= K1 (both bounds non-decreasing in the row)
    const int K0 = kb * KPB, K1 = min(K0 + KPB, a.Lk);
    int lo = 0, hi = a.Lq, wl, wh;
    while (lo < hi) {
      const int m = (lo + hi) >> 1;
      row_window(a, b, m, wl, wh);
      if (wh > K0) hi = m; else lo = m + 1;
    }
    const int r1 = lo;
    hi = a.Lq;
    while (lo < hi) {
      const int m = (lo + hi) >> 1;
      row_window(a, b, m, wl, wh);
      if (wl >= K1) hi = m; else lo = m + 1;
    }
    tb = __builtin_amdgcn_readfirstlane(r1 / QT);
    ntile = __builtin_amdgcn_readfirstlane(lo > r1 ? (lo + QT - 1) / QT : r1 / QT);
  }
  for (int gi = 0; gi < group; ++gi) {
    const int h = hk * group + gi;
    const int64_t rbase = ((int64_t)b * a.Hq + h) * a.Lq;
    const float* qb = a.q + b * a.qsb + h * a.qsh;
    const float* db = a.dout + b * a.dosb + h * a.dosh;
    Tile32<D> sq, sd;
    float pl2 = kPosInf, pnd = 0.f;
    int pwl = 0, pwh = 0;
    auto fetch = [&](int r0) {
      sq.fetch(qb, a.qsl, r0, a.Lq, tid);
      sd.fetch(db, a.dosl, r0, a.Lq, tid);
      if (tid < QT) {
        const int row = r0 + tid;
        pl2 = row < a.Lq ? a.lse2[rbase + row] : kPosInf;  // rows past the end get P = 0
        pnd = row < a.Lq ? a.ndelta[rbase + row] : 0.f;
        if constexpr (WIN) {
          if (row < a.Lq) row_window(a, b, row, pwl, pwh);
        }
      }
    };
    auto store = [&](int u) {
      sq.store(qs[u % 3], tid);
      sd.store(dos[u & 1], tid);
      if (tid < QT) {
        l2s[u & 1][tid] = pl2, nds[u % 3][tid] = pnd;
        if constexpr (WIN) wls[u & 1][tid] = pwl, whs[u & 1][tid] = pwh;
      }
    };
    __syncthreads();  // the previous head's last tiles are consumed
    if (tb < ntile) {
      fetch(tb * QT);
      store(tb);
    }
    f32x16 s;
    for (int t = tb; t < ntile; ++t) {
      // tile t stored, P of tile t-1 handed over; every wave is done with
      // the slots the next store reuses
      __syncthreads();
      if (t + 1 < ntile) fetch((t + 1) * QT);
      if (role == 1 && t > tb) ds_step(s, t - 1, gi);
      // S = Q K^T (P wave) or dP = dO V^T (dS wave)
      const float* at = (role == 0 ? qs[t % 3] : dos[t & 1]) + l32 * PITCH + 16 * hh * DT;
      s = zero16();
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const vdt x = *reinterpret_cast<const vdt*>(at + u * DT);
#pragma unroll
        for (int e = 0; e < DT; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(x[e], kv[DT * u + e], s, 0, 0, 0);
      }
      if (role == 0) {
        // register i: row 8*(i/4) + 4*hh + i%4 of the tile, this lane's key
        f32x16 w;
        float* pw = px[t & 1][pair] + lane * 4;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 L = ld4(&l2s[t & 1][8 * g + 4 * hh]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bool in = kvalid;
            if constexpr (WIN) {
              const int rr = 8 * g + 4 * hh + r;
              in = in && key >= wls[t & 1][rr] && key < whs[t & 1][rr];
            }
            w[4 * g + r] = in ? __builtin_amdgcn_exp2f(fmaf(s[4 * g + r], a.c, -L[r])) : 0.f;
          }
          st4(pw + 256 * g, f32x4{w[4 * g], w[4 * g + 1], w[4 * g + 2], w[4 * g + 3]});
        }
        second(w, dos[t & 1]);
      }
      if (t + 1 < ntile) store(t + 1);
    }
    __syncthreads();  // P of the last tile handed over
    if (role == 1 && ntile > tb) ds_step(s, ntile - 1, gi);
  }
  // acc[d] register i: key k0 + 8*(i/4) + 4*hh + i%4, channel 32*d + l32.
  // Masked keys: exactly zero (their P is 0; a non-finite dO or V elsewhere
  // in the row must not reach them through 0 * inf).
  float* const gb = role == 0 ? a.dv + b * a.dvsb + hk * a.dvsh : a.dk + b * a.dksb + hk * a.dksh;
  const int64_t gs = role == 0 ? a.dvsl : a.dksl;
  const float f = role == 0 ? 1.f : a.scale;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int kk = k0 + 8 * (i / 4) + 4 * hh + (i % 4);
    if (kk >= a.Lk) continue;
    const bool ok = key_ok(a, b, kk);
    float* gp = gb + (int64_t)kk * gs + l32;
#pragma unroll
    for (int d = 0; d < DT; ++d) gp[32 * d] = ok ? acc[d][i] * f : 0.f;
  }
}

// dQ on the fp32 matrix cores: per 32 query rows a pair of waves on one
// SIMD, eight waves per workgroup, 32-key tiles of K and V through LDS.  One
// wave holds the rows' q halves and forms S^T = K Q^T and P, the other holds
// the dO halves and forms dP^T = V dO^T; both put key 8*(i/4) + 4*(l/32) +
// i%4 in register i of lane l against the lane's row.  They exchange P and dP
// through LDS, both form dS = P*(dP + ndelta) (the same bits), and each adds
// dS K into half of dQ's channel blocks, dS register j being the A operand
// in k-step j.  The dS step runs one tile behind (K tiles in three slots,
// the exchange in two), so one barrier per tile serves both.  WIN: per-row
// key windows; the workgroup visits the tiles meeting its rows' windows and
// dS is 0 outside each row's window.
template <int D, bool WIN>
__global__ __launch_bounds__(512) void bwd_dq_f32_kernel(F32Args a) {
  constexpr int KT = 32, ROWS = 128, PITCH = D + 4, HD = D / 2, DT = D / 32, DH = DT / 2;
  using vdt = float __attribute__((ext_vector_type(DT)));
  __shared__ __attribute__((aligned(16))) float ks[3][KT * PITCH];
  __shared__ __attribute__((aligned(16))) float vs[2][KT * PITCH];
  __shared__ __attribute__((aligned(16))) float kok[3][KT];  // 1: valid key, 0: masked or past the end
  __shared__ __attribute__((aligned(16))) float xs[2][2][4][16 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int pair = wave & 3, role = wave >> 2;  // role 0: q and P, 1: dO and dP
  const int nqb = (a.Lq + ROWS - 1) / ROWS;
  const int qb = blockIdx.x % nqb, bh = blockIdx.x / nqb;
  const int b = bh / a.Hq, h = bh % a.Hq, hk = h / (a.Hq / a.Hkv);
  const int r0 = qb * ROWS + pair * 32;  // the pair's first row
  const int row = r0 + l32;
  const bool valid = row < a.Lq;
  float qg[HD];  // q (role 0) or dO (role 1) of the lane's row, k-step order
  load_row_ksteps<D>(qg,
                     role == 0 ? a.q + b * a.qsb + h * a.qsh + (int64_t)row * a.qsl
                               : a.dout + b * a.dosb + h * a.dosh + (int64_t)row * a.dosl,
                     valid, hh);
  const int64_t rr = (int64_t)bh * a.Lq + row;
  const float l2 = valid ? a.lse2[rr] : kPosInf;
  const float nd = valid ? a.ndelta[rr] : 0.f;
  int wl = 0, wh = a.Lk;
  if constexpr (WIN) {
    if (valid) row_window(a, b, row, wl, wh);
  }
  f32x16 dq[DH];  // channel blocks role*DH .. +DH-1
#pragma unroll
  for (int d = 0; d < DH; ++d) dq[d] = zero16();
  const float* kb = a.k + b * a.ksb + hk * a.ksh;
  const float* vb = a.v + b * a.vsb + hk * a.vsh;

  // dS of tile u from this wave's P or dP (registers) and the partner's
  // (LDS), then dQ += dS K over this wave's channel blocks.  Masked keys add
  // nothing (dS exactly 0).  The K reads take a lane's D/32 channels whole
  // (conflict-free) and keep this wave's half.
  auto ds_step = [&](const f32x16& mine, int u) {
    const float* other = xs[u & 1][role ^ 1][pair] + lane * 4;
    f32x16 ds;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 ok = ld4(&kok[u % 3][8 * g + 4 * hh]);
      const f32x4 o = ld4(other + 256 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = role == 0 ? mine[4 * g + r] : o[r], dp = role == 0 ? o[r] : mine[4 * g + r];
        bool in = ok[r] != 0.f;
        if constexpr (WIN) {
          const int key = u * KT + 8 * g + 4 * hh + r;
          in = in && key >= wl && key < wh;
        }
        ds[4 * g + r] = in ? p * (dp + nd) : 0.f;
      }
    }
    const float* bt = ks[u % 3] + l32 * DT;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const vdt y = *reinterpret_cast<const vdt*>(bt + (8 * (j / 4) + 4 * hh + (j % 4)) * PITCH);
#pragma unroll
      for (int d = 0; d < DH; ++d)
        dq[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[j], role == 0 ? y[d] : y[DH + d], dq[d], 0, 0, 0);
    }
  };

  Tile32<D> sk, sv;
  float pok = 0.f;
  auto fetch = [&](int c0) {
    sk.fetch(kb, a.ksl, c0, a.Lk, tid);
    sv.fetch(vb, a.vsl, c0, a.Lk, tid);
    if (tid < KT) pok = key_ok(a, b, c0 + tid) ? 1.f : 0.f;
  };
  auto store = [&](int u) {
    sk.store(ks[u % 3], tid);
    sv.store(vs[u & 1], tid);
    if (tid < KT) kok[u % 3][tid] = pok;
  };
  int t0 = 0, ntile = (a.Lk + KT - 1) / KT;
  if constexpr (WIN) {
    __shared__ int red[16];
    window_tiles<8>(wl, wh, valid, red, t0, ntile);
  }
  if (t0 < ntile) {
    fetch(t0 * KT);
    store(t0);
  }
  f32x16 s;
  for (int t = t0; t < ntile; ++t) {
    // tile t stored, tile t-1's P and dP exchanged; every wave is done with
    // the slots the next store reuses
    __syncthreads();
    if (t + 1 < ntile) fetch((t + 1) * KT);
    if (t > t0) ds_step(s, t - 1);
    // S^T = K Q^T (role 0) or dP^T = V dO^T (role 1)
    const float* at = (role == 0 ? ks[t % 3] : vs[t & 1]) + l32 * PITCH + 16 * hh * DT;
    s = zero16();
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const vdt x = *reinterpret_cast<const vdt*>(at + u * DT);
#pragma unroll
      for (int e = 0; e < DT; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(x[e], qg[DT * u + e], s, 0, 0, 0);
    }
    // register i: key 8*(i/4) + 4*hh + i%4 of the tile, this lane's row
    if (role == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = __builtin_amdgcn_exp2f(fmaf(s[i], a.c, -l2));
    }
    float* mine = xs[t & 1][role][pair] + lane * 4;
#pragma unroll
    for (int g = 0; g < 4; ++g) st4(mine + 256 * g, f32x4{s[4 * g], s[4 * g + 1], s[4 * g + 2], s[4 * g + 3]});
    if (t + 1 < ntile) store(t + 1);
  }
  __syncthreads();  // the last tile's P and dP exchanged
  if (ntile > t0) ds_step(s, ntile - 1);
  // dq[d] register i: row r0 + 8*(i/4) + 4*hh + i%4, channel 32*(role*DH + d) + l32
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rw = r0 + 8 * (i / 4) + 4 * hh + (i % 4);
    if (rw >= a.Lq) continue;
    float* op = a.dq + b * a.dqsb + h * a.dqsh + (int64_t)rw * a.dqsl + l32 + 32 * role * DH;
#pragma unroll
    for (int d = 0; d < DH; ++d) op[32 * d] = dq[d][i] * a.scale;
  }
}

// dQ = scale * dS K from the staged dS: eight waves per workgroup, 32 query
// rows each, 32-key tiles of K in LDS (the backward tile layout).  A lane
// reads its row's dS over keys 16*(l/32) .. +15 of a tile (64 contiguous
// bytes of the tile's 32x32 block) straight into registers, a tile ahead;
// k-step j contracts keys j and 16 + j, so one LDS read gives the lane its
// D/32 channel blocks of K's row 16*(l/32) + j.  WIN: the workgroup stages
// the tiles meeting its rows' windows, and a wave multiplies only the key
// blocks its rows meet (the blocks the windowed dK/dV kernel wrote).
template <int D, bool WIN>
__global__ __launch_bounds__(512) void bwd_dq_ds_f32_kernel(F32Args a) {
  constexpr int KT = 32, ROWS = 256, PITCH = D + 4, DT = D / 32;
  using vdt = float __attribute__((ext_vector_type(DT)));
  __shared__ __attribute__((aligned(16))) float ks[2][KT * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int group = a.Hq / a.Hkv;
  const int nrb = (a.Lq + ROWS - 1) / ROWS;
  const int rb = blockIdx.x % nrb, pg = blockIdx.x / nrb;
  const int gi = pg % group, bhk = a.pair0 + pg / group;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv, h = hk * group + gi;
  const int r0 = rb * ROWS + wave * 32;  // this wave's first row
  const int nrt = (a.Lq + 31) / 32, nkt = 4 * ((a.Lk + 127) / 128), ntile = (a.Lk + KT - 1) / KT;
  const bool rows_in = r0 < a.Lq;
  const bool valid = r0 + l32 < a.Lq;
  int wl = 0, wh = a.Lk, t0 = 0, ntile_w = ntile;
  if constexpr (WIN) {
    __shared__ int red[16];
    if (valid) row_window(a, b, r0 + l32, wl, wh);
    window_tiles<8>(wl, wh, valid, red, t0, ntile_w);
  }
  // does this wave multiply key tile t
  auto takes = [&](int t) {
    if constexpr (WIN) return rows_meet_block(a, wl, wh, valid, t / 4);
    return rows_in;
  };
  // this lane's dS: row r0 + l32, keys 16*hh .. of key tile t at dsr + 1024*t
  const float* dsr = a.ds + (bhk - a.pair0) * a.dsp + ((int64_t)gi * nrt + r0 / 32) * nkt * 1024 + l32 * 32 + 16 * hh;
  f32x16 dq[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) dq[d] = zero16();
  const float* kb = a.k + b * a.ksb + hk * a.ksh;
  Tile32<D> sk;
  f32x4 pa[4];
  auto fetch = [&](int t) {
    sk.fetch(kb, a.ksl, t * KT, a.Lk, tid);
    const bool take = takes(t);
#pragma unroll
    for (int e = 0; e < 4; ++e) pa[e] = take ? ld4(dsr + (int64_t)t * 1024 + 4 * e) : f32x4{0.f, 0.f, 0.f, 0.f};
  };
  if (t0 < ntile_w) {
    fetch(t0);
    sk.store(ks[0], tid);
  }
  for (int t = t0; t < ntile_w; ++t) {
    const int buf = (t - t0) & 1;
    __syncthreads();  // tile t stored; every wave is done with tile t - 1
    f32x4 ca[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) ca[e] = pa[e];
    const bool take = takes(t);
    if (t + 1 < ntile_w) fetch(t + 1);
    if (take) {
      const float* bt = ks[buf] + (16 * hh) * PITCH + l32 * DT;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const vdt y = *reinterpret_cast<const vdt*>(bt + j * PITCH);
#pragma unroll
        for (int d = 0; d < DT; ++d)
          dq[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[j / 4][j % 4], y[d], dq[d], 0, 0, 0);
      }
    }
    if (t + 1 < ntile_w) sk.store(ks[buf ^ 1], tid);
  }
  // dq[d] register i: row r0 + 8*(i/4) + 4*hh + i%4, channel 32*d + l32
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rw = r0 + 8 * (i / 4) + 4 * hh + (i % 4);
    if (rw >= a.Lq) continue;
    float* op = a.dq + b * a.dqsb + h * a.dqsh + (int64_t)rw * a.dqsl + l32;
#pragma unroll
    for (int d = 0; d < DT; ++d) op[32 * d] = dq[d][i] * a.scale;
  }
}

// Zeros over a (B, H, L, D) fp32 tensor (gradients of an empty side).
__global__ void zero_f32_kernel(float* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D) {
  const int64_t n = (int64_t)B * H * L * (D / 4);
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < n; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % (D / 4));
    const int64_t rw = u / (D / 4);
    const int i = (int)(rw % L);
    const int h = (int)((rw / L) % H);
    const int b = (int)(rw / ((int64_t)L * H));
    st4(x + b * sb + h * sh + (int64_t)i * sl + 4 * c, f32x4{0.f, 0.f, 0.f, 0.f});
  }
}

// ---------------------------------------------------------------------------
// Rotation of fp32 tensors: channels 4c .. 4c+3 of a row are pairs 2c, 2c+1;
// (e, o) -> (e*cos - o*sin, e*sin + o*cos), or the transpose with `inverse`,
// each product and sum rounded on its own as the reference's fp32 torch ops
// round them.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_apply_f32_kernel(const float* __restrict__ x, int64_t xsb, int64_t xsh,
                                                             int64_t xsl, int B, int H, int L, int D,
                                                             const float* __restrict__ ct,
                                                             const float* __restrict__ st, int64_t tsb, int inverse,
                                                             float* __restrict__ out, int64_t osb, int64_t osh,
                                                             int64_t osl) {
#pragma clang fp contract(off)
  const int cpr = D / 4;
  const int64_t n = (int64_t)B * H * L * cpr;
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < n; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % cpr);
    const int64_t rw = u / cpr;
    const int i = (int)(rw % L);
    const int h = (int)((rw / L) % H);
    const int b = (int)(rw / ((int64_t)L * H));
    const f32x4 v = ld4(x + b * xsb + h * xsh + (int64_t)i * xsl + 4 * c);
    const int64_t t = b * tsb + (int64_t)i * (D / 2) + 2 * c;
    f32x4 r;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const float e = v[2 * p], od = v[2 * p + 1], cs = ct[t + p], sn = st[t + p];
      const float ec = e * cs, os = od * sn, es = e * sn, oc = od * cs;
      if (!inverse) {
        r[2 * p] = ec - os;
        r[2 * p + 1] = es + oc;
      } else {
        r[2 * p] = ec + os;
        r[2 * p + 1] = oc - es;
      }
    }
    st4(out + b * osb + h * osh + (int64_t)i * osl + 4 * c, r);
  }
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm + rotation on float32 rows (a float32 model's q_norm /
// k_norm then apply_rotary, src/avgen/models/layers.py:106-118, 530-536:
// F.rms_norm with the gain in the activation's dtype, then the fp32
// rotation of src/avgen/models/rope.py:332-338).  Forward per row:
//   rstd = 1/sqrt(mean(x^2) + eps),  n = (x*rstd)*w,  y = rotate(n)
// backward given dy: g = rotate^T(dy), xh = x*rstd, wg = w*g,
//   dx = rstd*(wg - xh*mean(wg*xh)),  dw = sum over rows of g*xh (per-block
//   partials, then one fixed-order reduction: deterministic).
// One wave per token, D/4 lanes per head row holding 4 floats (16 bytes)
// each, 64/(D/4) heads at a time; the token's rotation values are read
// once.  HBM-bound: one read and one write of the rows (two reads back).
// ---------------------------------------------------------------------------
struct NormF32Args {
  const float* x;
  int64_t xsb, xsh, xsl;
  int B, H, L;
  const float* w;  // (head_dim) gain, or null
  float eps;
  const float *ct, *st;  // rotation tables at b*tsb + i*head_dim/2 + pair; null: no rotation
  int64_t tsb;
  float* out;
  int64_t osb, osh, osl;
  const float* dy;
  int64_t dsb, dsh, dsl;
  float* dx;
  int64_t xgb, xgh, xgl;
  float* wpart;  // backward: per-block dW partials, null without a gain
};
constexpr int kNormF32Blocks = 4096;  // fixed grid of the backward (dW partials per block)

template <int R>
__device__ __forceinline__ float lane_group_sum(float v) {
#pragma unroll
  for (int off = R / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// The rotation of a lane's two interleaved pairs (as rope_apply_f32_kernel).
__device__ __forceinline__ f32x4 rotate4(const f32x4& v, const float* cs, const float* sn, bool inverse) {
#pragma clang fp contract(off)
  f32x4 r;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float e = v[2 * p], od = v[2 * p + 1];
    const float ec = e * cs[p], os = od * sn[p], es = e * sn[p], oc = od * cs[p];
    r[2 * p] = inverse ? ec + os : ec - os;
    r[2 * p + 1] = inverse ? oc - es : es + oc;
  }
  return r;
}

template <int D>
__global__ __launch_bounds__(64) void qk_norm_f32_fwd_kernel(NormF32Args a) {
#pragma clang fp contract(off)
  constexpr int R = D / 4, HPW = 64 / R;
  const int c = threadIdx.x % R, hg = threadIdx.x / R;
  const f32x4 w = a.w ? ld4(a.w + 4 * c) : f32x4{1.f, 1.f, 1.f, 1.f};
  const int64_t ntok = (int64_t)a.B * a.L;
  for (int64_t tok = blockIdx.x; tok < ntok; tok += gridDim.x) {
    const int b = (int)(tok / a.L), i = (int)(tok % a.L);
    float cs[2] = {1.f, 1.f}, sn[2] = {0.f, 0.f};
    if (a.ct) {
      const int64_t t = b * a.tsb + (int64_t)i * (D / 2) + 2 * c;
      cs[0] = a.ct[t], cs[1] = a.ct[t + 1], sn[0] = a.st[t], sn[1] = a.st[t + 1];
    }
    const float* xrow = a.x + b * a.xsb + (int64_t)i * a.xsl + 4 * c;
    for (int h = hg; h < a.H; h += HPW) {  // uniform over the row's lanes
      const f32x4 x = ld4(xrow + h * a.xsh);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += x[j] * x[j];
      ss = lane_group_sum<R>(ss);
      const float rstd = 1.f / __builtin_sqrtf(ss / (float)D + a.eps);
      f32x4 n;
#pragma unroll
      for (int j = 0; j < 4; ++j) n[j] = (x[j] * rstd) * w[j];
      if (a.ct) n = rotate4(n, cs, sn, false);
      st4(a.out + b * a.osb + h * a.osh + (int64_t)i * a.osl + 4 * c, n);
    }
  }
}

template <int D>
__global__ __launch_bounds__(64) void qk_norm_f32_bwd_kernel(NormF32Args a) {
#pragma clang fp contract(off)
  constexpr int R = D / 4, HPW = 64 / R;
  __shared__ float red[HPW][D];
  const int c = threadIdx.x % R, hg = threadIdx.x / R;
  const f32x4 w = a.w ? ld4(a.w + 4 * c) : f32x4{1.f, 1.f, 1.f, 1.f};
  float dw[4] = {0.f, 0.f, 0.f, 0.f};
  const int64_t ntok = (int64_t)a.B * a.L;
  for (int64_t tok = blockIdx.x; tok < ntok; tok += gridDim.x) {
    const int b = (int)(tok / a.L), i = (int)(tok % a.L);
    float cs[2] = {1.f, 1.f}, sn[2] = {0.f, 0.f};
    if (a.ct) {
      const int64_t t = b * a.tsb + (int64_t)i * (D / 2) + 2 * c;
      cs[0] = a.ct[t], cs[1] = a.ct[t + 1], sn[0] = a.st[t], sn[1] = a.st[t + 1];
    }
    const float* xrow = a.x + b * a.xsb + (int64_t)i * a.xsl + 4 * c;
    const float* grow = a.dy + b * a.dsb + (int64_t)i * a.dsl + 4 * c;
    for (int h = hg; h < a.H; h += HPW) {
      const f32x4 x = ld4(xrow + h * a.xsh);
      f32x4 g = ld4(grow + h * a.dsh);
      if (a.ct) g = rotate4(g, cs, sn, true);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += x[j] * x[j];
      ss = lane_group_sum<R>(ss);
      const float rstd = 1.f / __builtin_sqrtf(ss / (float)D + a.eps);
      float xh[4], wg[4], dot = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xh[j] = x[j] * rstd;
        wg[j] = w[j] * g[j];
        dot += wg[j] * xh[j];
        dw[j] += g[j] * xh[j];
      }
      const float m = lane_group_sum<R>(dot) / (float)D;
      f32x4 dx;
#pragma unroll
      for (int j = 0; j < 4; ++j) dx[j] = rstd * (wg[j] - xh[j] * m);
      st4(a.dx + b * a.xgb + h * a.xgh + (int64_t)i * a.xgl + 4 * c, dx);
    }
  }
  if (!a.wpart) return;  // uniform: no gain, no dW
#pragma unroll
  for (int j = 0; j < 4; ++j) red[hg][4 * c + j] = dw[j];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 64) {
    float s = 0.f;
    for (int r = 0; r < HPW; ++r) s += red[r][d];
    a.wpart[(int64_t)blockIdx.x * D + d] = s;
  }
}

// dw[d] = the backward blocks' partials summed in a fixed order (one
// workgroup per d: strided shares, then a tree over the threads).
__global__ __launch_bounds__(256) void qk_norm_f32_dw_kernel(const float* __restrict__ part, int nblocks, int D,
                                                             float* __restrict__ dw) {
  __shared__ float red[256];
  const int d = blockIdx.x;
  float s = 0.f;
  for (int k = threadIdx.x; k < nblocks; k += 256) s += part[(int64_t)k * D + d];
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) dw[d] = red[0];
}

__global__ void qk_norm_f32_dw_zero_kernel(int D, float* __restrict__ dw) {
  if ((int)threadIdx.x < D) dw[threadIdx.x] = 0.f;
}

int grid_of(int64_t n, int per = 256) {
  const int64_t g = (n + per - 1) / per;
  return (int)(g < 1 ? 1 : (g > 65535 ? 65535 : g));
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool str4(const int64_t* s) { return s && s[0] % 4 == 0 && s[1] % 4 == 0 && s[2] % 4 == 0; }

int check_f32_dims(int32_t B, int32_t Hq, int32_t Hkv, int32_t Lq, int32_t Lk, int32_t D) {
  if (B < 0 || Hq < 0 || Hkv < 0 || Lq < 0 || Lk < 0) return AVATTN_ERR_BAD_SHAPE;
  if (D != 64 && D != 128) return AVATTN_ERR_HEAD_DIM;
  if (Hkv == 0 || Hq == 0) return (B == 0) ? AVATTN_OK : AVATTN_ERR_GQA;
  if (Hq % Hkv != 0) return AVATTN_ERR_GQA;
  // Grids: B*Hq*ceil(Lq/64) and B*Hkv*ceil(Lk/64) workgroups; row indices
  // (b*Hq + h)*Lq + i in 64 bits.
  const int64_t lim = 2147483647;
  if ((int64_t)B * Hq * (((int64_t)Lq + 63) / 64) > lim || (int64_t)B * Hkv * (((int64_t)Lk + 63) / 64) > lim)
    return AVATTN_ERR_TOO_LARGE;
  if ((int64_t)B * Hq * Lq > ((int64_t)1 << 40)) return AVATTN_ERR_TOO_LARGE;
  return AVATTN_OK;
}

size_t r256(size_t x) { return (x + 255) / 256 * 256; }

template <int D, bool WIN>
void launch_fwd_f32(const F32Args& a, hipStream_t s) {
  const int nqb = (a.Lq + 127) / 128;
  hipLaunchKernelGGL((fwd_f32_kernel<D, WIN>), dim3((unsigned)(nqb * a.B * a.Hq)), dim3(256), 0, s, a);
}

// Staged dS floats per (batch, kv head) pair (see F32Args::ds).
int64_t ds_floats_per_pair(int group, int Lq, int Lk) {
  return (int64_t)group * ((Lq + 31) / 32) * 32 * ((Lk + 127) / 128) * 128;
}

// pairs_per_pass 0: dQ recomputes S and dP; else dS is staged for that many
// (batch, kv head) pairs at a time.
template <int D, bool WIN>
void launch_bwd_f32(F32Args a, int pairs_per_pass, hipStream_t s) {
  const int64_t rows = (int64_t)a.B * a.Hq * a.Lq;
  hipLaunchKernelGGL(bwd_pre_f32_kernel<D>, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, a);
  const int nkb = (a.Lk + 127) / 128;
  const int pairs = a.B * a.Hkv;
  if (pairs_per_pass == 0) {
    a.pair0 = 0;
    hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, false, WIN>), dim3((unsigned)(nkb * pairs)), dim3(512), 0, s, a);
    const int nqb = (a.Lq + 127) / 128;
    hipLaunchKernelGGL((bwd_dq_f32_kernel<D, WIN>), dim3((unsigned)(nqb * a.B * a.Hq)), dim3(512), 0, s, a);
    return;
  }
  const int group = a.Hq / a.Hkv, nrb = (a.Lq + 255) / 256;
  for (int p0 = 0; p0 < pairs; p0 += pairs_per_pass) {
    const int np = pairs - p0 < pairs_per_pass ? pairs - p0 : pairs_per_pass;
    a.pair0 = p0;
    hipLaunchKernelGGL((bwd_dkdv_f32_kernel<D, true, WIN>), dim3((unsigned)(nkb * np)), dim3(512), 0, s, a);
    hipLaunchKernelGGL((bwd_dq_ds_f32_kernel<D, WIN>), dim3((unsigned)(nrb * np * group)), dim3(512), 0, s, a);
  }
}

// Optional key windows: both null (none) or both given, 4-byte aligned,
// batch stride 0 or >= len_q.
int check_f32_windows(const int32_t* lo, const int32_t* hi, int64_t batch_stride, int32_t len_q) {
  if (!lo && !hi) return AVATTN_OK;
  if (!lo || !hi) return AVATTN_ERR_NULL_POINTER;
  if (((reinterpret_cast<uintptr_t>(lo) | reinterpret_cast<uintptr_t>(hi)) & 3u) != 0) return AVATTN_ERR_LAYOUT;
  if (batch_stride != 0 && batch_stride < len_q) return AVATTN_ERR_ARGUMENT;
  return AVATTN_OK;
}

}  // namespace
}  // namespace avattn

using namespace avattn;

extern "C" {

static int fwd_f32_entry(const float* q, const float* k, const float* v, const int64_t* q_strides,
                         const int64_t* k_strides, const int64_t* v_strides, int32_t batch, int32_t heads_q,
                         int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
                         int64_t key_mask_batch_stride, const int32_t* window_lo, const int32_t* window_hi,
                         int64_t window_batch_stride, float scale, float* out, const int64_t* out_strides,
                         float* lse, avattn_stream_t stream) {
  int st = check_f32_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (st != AVATTN_OK) return st;
  st = check_f32_windows(window_lo, window_hi, window_batch_stride, len_q);
  if (st != AVATTN_OK) return st;
  if (!q_strides || !k_strides || !v_strides || !out_strides) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads_q * len_q == 0) return AVATTN_OK;
  if (!q || !out || !lse) return AVATTN_ERR_NULL_POINTER;
  if (!al16(q) || !al16(out) || !str4(q_strides) || !str4(out_strides)) return AVATTN_ERR_LAYOUT;
  if (!(scale > 0.f) || !isfinite(scale)) return AVATTN_ERR_ARGUMENT;
  F32Args a{};
  a.q = q, a.k = k, a.v = v;
  a.qsb = q_strides[0], a.qsh = q_strides[1], a.qsl = q_strides[2];
  a.ksb = k_strides[0], a.ksh = k_strides[1], a.ksl = k_strides[2];
  a.vsb = v_strides[0], a.vsh = v_strides[1], a.vsl = v_strides[2];
  a.B = batch, a.Hq = heads_q, a.Hkv = heads_kv, a.Lq = len_q, a.Lk = len_k, a.D = head_dim;
  a.mask = key_mask, a.msb = key_mask_batch_stride;
  a.o = out, a.osb = out_strides[0], a.osh = out_strides[1], a.osl = out_strides[2];
  a.lse = lse;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (len_k == 0) {  // src/avgen/models/attention.py:261-262: zeros
    hipLaunchKernelGGL(empty_f32_kernel, dim3(grid_of((int64_t)batch * heads_q * len_q)), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
  }
  if (!k || !v) return AVATTN_ERR_NULL_POINTER;
  if (!al16(k) || !al16(v) || !str4(k_strides) || !str4(v_strides)) return AVATTN_ERR_LAYOUT;
  if (key_mask && key_mask_batch_stride != 0 && key_mask_batch_stride < len_k) return AVATTN_ERR_ARGUMENT;
  a.scale = scale, a.c = scale * kLog2e;
  a.wlo = window_lo, a.whi = window_hi, a.wsb = window_batch_stride;
  if (window_lo) {
    if (head_dim == 128)
      launch_fwd_f32<128, true>(a, s);
    else
      launch_fwd_f32<64, true>(a, s);
  } else if (head_dim == 128) {
    launch_fwd_f32<128, false>(a, s);
  } else {
    launch_fwd_f32<64, false>(a, s);
  }
  return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
}

int avattn_fwd_f32(const float* q, const float* k, const float* v, const int64_t* q_strides,
                   const int64_t* k_strides, const int64_t* v_strides, int32_t batch, int32_t heads_q,
                   int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
                   int64_t key_mask_batch_stride, float scale, float* out, const int64_t* out_strides, float* lse,
                   avattn_stream_t stream) {
  return fwd_f32_entry(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                       key_mask, key_mask_batch_stride, nullptr, nullptr, 0, scale, out, out_strides, lse, stream);
}

int avattn_fwd_windowed_f32(const float* q, const float* k, const float* v, const int64_t* q_strides,
                            const int64_t* k_strides, const int64_t* v_strides, int32_t batch, int32_t heads_q,
                            int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim,
                            const uint8_t* key_mask, int64_t key_mask_batch_stride, const int32_t* window_lo,
                            const int32_t* window_hi, int64_t window_batch_stride, float scale, float* out,
                            const int64_t* out_strides, float* lse, avattn_stream_t stream) {
  return fwd_f32_entry(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                       key_mask, key_mask_batch_stride, window_lo, window_hi, window_batch_stride, scale, out,
                       out_strides, lse, stream);
}

size_t avattn_bwd_f32_workspace_size(int32_t batch, int32_t heads_q, int32_t len_q) {
  if (batch <= 0 || heads_q <= 0 || len_q <= 0) return 0;
  return 2 * r256((size_t)batch * heads_q * len_q * sizeof(float));
}

size_t avattn_bwd_f32_staged_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q,
                                            int32_t len_k, int32_t kv_pairs_per_pass) {
  const size_t base = avattn_bwd_f32_workspace_size(batch, heads_q, len_q);
  if (base == 0 || heads_kv <= 0 || heads_q % heads_kv != 0 || len_k <= 0 || kv_pairs_per_pass <= 0) return base;
  const int64_t pairs = (int64_t)batch * heads_kv;
  const int64_t pp = kv_pairs_per_pass < pairs ? kv_pairs_per_pass : pairs;
  return (base + 4095) / 4096 * 4096 +
         (size_t)pp * (size_t)ds_floats_per_pair(heads_q / heads_kv, len_q, len_k) * sizeof(float);
}

static int bwd_f32_entry(const float* dout, const float* q, const float* k, const float* v, const float* out,
                         const float* lse, const int64_t* dout_strides, const int64_t* q_strides,
                         const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                         int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                         int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
                         const int32_t* window_lo, const int32_t* window_hi, int64_t window_batch_stride,
                         float scale, float* dq, const int64_t* dq_strides, float* dk, const int64_t* dk_strides,
                         float* dv, const int64_t* dv_strides, void* workspace, size_t workspace_bytes,
                         avattn_stream_t stream) {
  int st = check_f32_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (st != AVATTN_OK) return st;
  st = check_f32_windows(window_lo, window_hi, window_batch_stride, len_q);
  if (st != AVATTN_OK) return st;
  if (!dout_strides || !q_strides || !k_strides || !v_strides || !out_strides || !dq_strides || !dk_strides ||
      !dv_strides)
    return AVATTN_ERR_NULL_POINTER;
  if (!(scale > 0.f) || !isfinite(scale)) return AVATTN_ERR_ARGUMENT;
  const bool qside = (int64_t)batch * heads_q * len_q > 0, kside = (int64_t)batch * heads_kv * len_k > 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (qside && !kside) {  // no keys: dq = 0
    if (!dq) return AVATTN_ERR_NULL_POINTER;
    if (!al16(dq) || !str4(dq_strides)) return AVATTN_ERR_LAYOUT;
    hipLaunchKernelGGL(zero_f32_kernel, dim3(grid_of((int64_t)batch * heads_q * len_q * (head_dim / 4))), dim3(256),
                       0, s, dq, dq_strides[0], dq_strides[1], dq_strides[2], batch, heads_q, len_q, head_dim);
    return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
  }
  if (kside && !qside) {  // no queries: dk = dv = 0
    if (!dk || !dv) return AVATTN_ERR_NULL_POINTER;
    if (!al16(dk) || !al16(dv) || !str4(dk_strides) || !str4(dv_strides)) return AVATTN_ERR_LAYOUT;
    hipLaunchKernelGGL(zero_f32_kernel, dim3(grid_of((int64_t)batch * heads_kv * len_k * (head_dim / 4))), dim3(256),
                       0, s, dk, dk_strides[0], dk_strides[1], dk_strides[2], batch, heads_kv, len_k, head_dim);
    hipLaunchKernelGGL(zero_f32_kernel, dim3(grid_of((int64_t)batch * heads_kv * len_k * (head_dim / 4))), dim3(256),
                       0, s, dv, dv_strides[0], dv_strides[1], dv_strides[2], batch, heads_kv, len_k, head_dim);
    return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
  }
  if (!qside) return AVATTN_OK;
  if (!dout || !q || !k || !v || !out || !lse || !dq || !dk || !dv) return AVATTN_ERR_NULL_POINTER;
  for (const void* p : {(const void*)dout, (const void*)q, (const void*)k, (const void*)v, (const void*)out,
                        (const void*)dq, (const void*)dk, (const void*)dv})
    if (!al16(p)) return AVATTN_ERR_LAYOUT;
  for (const int64_t* sp : {dout_strides, q_strides, k_strides, v_strides, out_strides, dq_strides, dk_strides,
                            dv_strides})
    if (!str4(sp)) return AVATTN_ERR_LAYOUT;
  if (key_mask && key_mask_batch_stride != 0 && key_mask_batch_stride < len_k) return AVATTN_ERR_ARGUMENT;
  const size_t need = avattn_bwd_f32_workspace_size(batch, heads_q, len_q);
  if (!workspace || workspace_bytes < need) return AVATTN_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return AVATTN_ERR_LAYOUT;
  F32Args a{};
  a.q = q, a.k = k, a.v = v;
  a.qsb = q_strides[0], a.qsh = q_strides[1], a.qsl = q_strides[2];
  a.ksb = k_strides[0], a.ksh = k_strides[1], a.ksl = k_strides[2];
  a.vsb = v_strides[0], a.vsh = v_strides[1], a.vsl = v_strides[2];
  a.B = batch, a.Hq = heads_q, a.Hkv = heads_kv, a.Lq = len_q, a.Lk = len_k, a.D = head_dim;
  a.mask = key_mask, a.msb = key_mask_batch_stride;
  a.scale = scale, a.c = scale * kLog2e;
  a.dout = dout, a.out = out, a.lse_in = lse;
  a.dosb = dout_strides[0], a.dosh = dout_strides[1], a.dosl = dout_strides[2];
  a.oisb = out_strides[0], a.oish = out_strides[1], a.oisl = out_strides[2];
  a.dq = dq, a.dqsb = dq_strides[0], a.dqsh = dq_strides[1], a.dqsl = dq_strides[2];
  a.dk = dk, a.dksb = dk_strides[0], a.dksh = dk_strides[1], a.dksl = dk_strides[2];
  a.dv = dv, a.dvsb = dv_strides[0], a.dvsh = dv_strides[1], a.dvsl = dv_strides[2];
  a.lse2 = static_cast<float*>(workspace);
  a.ndelta = a.lse2 + need / 2 / sizeof(float);
  // Workspace beyond the statistics (from the next 4 KB) holding the staged
  // dS of at least one (batch, kv head) pair: stage dS, in equal passes of
  // as many pairs as fit.
  int pp = 0;
  {
    const size_t off = (need + 4095) / 4096 * 4096;
    const size_t per = (size_t)ds_floats_per_pair(heads_q / heads_kv, len_q, len_k) * sizeof(float);
    const int64_t pairs = (int64_t)batch * heads_kv;
    if (workspace_bytes >= off + per) {
      int64_t fit = (int64_t)((workspace_bytes - off) / per);
      if (fit > pairs) fit = pairs;
      const int64_t npass = (pairs + fit - 1) / fit;
      pp = (int)((pairs + npass - 1) / npass);
      a.ds = reinterpret_cast<float*>(static_cast<char*>(workspace) + off);
      a.dsp = (int64_t)(per / sizeof(float));
    }
  }
  a.wlo = window_lo, a.whi = window_hi, a.wsb = window_batch_stride;
  if (window_lo) {
    if (head_dim == 128)
      launch_bwd_f32<128, true>(a, pp, s);
    else
      launch_bwd_f32<64, true>(a, pp, s);
  } else if (head_dim == 128) {
    launch_bwd_f32<128, false>(a, pp, s);
  } else {
    launch_bwd_f32<64, false>(a, pp, s);
  }
  return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
}

int avattn_bwd_f32(const float* dout, const float* q, const float* k, const float* v, const float* out,
                   const float* lse, const int64_t* dout_strides, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* out_strides, int32_t batch, int32_t heads_q,
                   int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
                   int64_t key_mask_batch_stride, float scale, float* dq, const int64_t* dq_strides, float* dk,
                   const int64_t* dk_strides, float* dv, const int64_t* dv_strides, void* workspace,
                   size_t workspace_bytes, avattn_stream_t stream) {
  return bwd_f32_entry(dout, q, k, v, out, lse, dout_strides, q_strides, k_strides, v_strides, out_strides, batch,
                       heads_q, heads_kv, len_q, len_k, head_dim, key_mask, key_mask_batch_stride, nullptr, nullptr,
                       0, scale, dq, dq_strides, dk, dk_strides, dv, dv_strides, workspace, workspace_bytes, stream);
}

int avattn_bwd_windowed_f32(const float* dout, const float* q, const float* k, const float* v, const float* out,
                            const float* lse, const int64_t* dout_strides, const int64_t* q_strides,
                            const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                            int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                            int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
                            const int32_t* window_lo, const int32_t* window_hi, int64_t window_batch_stride,
                            float scale, float* dq, const int64_t* dq_strides, float* dk, const int64_t* dk_strides,
                            float* dv, const int64_t* dv_strides, void* workspace, size_t workspace_bytes,
                            avattn_stream_t stream) {
  return bwd_f32_entry(dout, q, k, v, out, lse, dout_strides, q_strides, k_strides, v_strides, out_strides, batch,
                       heads_q, heads_kv, len_q, len_k, head_dim, key_mask, key_mask_batch_stride, window_lo,
                       window_hi, window_batch_stride, scale, dq, dq_strides, dk, dk_strides, dv, dv_strides,
                       workspace, workspace_bytes, stream);
}

int avattn_rope_apply_f32(const float* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                          int32_t head_dim, const float* cos_tab, const float* sin_tab, int64_t table_batch_stride,
                          int32_t inverse, float* out, const int64_t* out_strides, avattn_stream_t stream) {
  if (batch < 0 || heads < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim < 4 || head_dim > 128 || head_dim % 4 != 0) return AVATTN_ERR_HEAD_DIM;
  if (!x_strides || !out_strides) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!x || !out || !cos_tab || !sin_tab) return AVATTN_ERR_NULL_POINTER;
  if (!al16(x) || !al16(out) || !str4(x_strides) || !str4(out_strides) || table_batch_stride < 0)
    return AVATTN_ERR_LAYOUT;
  if ((int64_t)batch * heads > 2147483647 || len > 2147483647) return AVATTN_ERR_TOO_LARGE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t n = (int64_t)batch * heads * len * (head_dim / 4);
  hipLaunchKernelGGL(rope_apply_f32_kernel, dim3(grid_of(n)), dim3(256), 0, s, x, x_strides[0], x_strides[1],
                     x_strides[2], batch, heads, len, head_dim, cos_tab, sin_tab, table_batch_stride,
                     inverse ? 1 : 0, out, out_strides[0], out_strides[1], out_strides[2]);
  return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
}


// Arguments of the float32 q/k norm entry points (as check_qk_norm of the
// bf16 ones).
static int check_norm_f32(const float* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                          int32_t head_dim, const float* weight, float eps, const float* cos_tab,
                          const float* sin_tab, int64_t table_batch_stride) {
  if (batch < 0 || heads < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim != 64 && head_dim != 128) return AVATTN_ERR_HEAD_DIM;
  if (!x_strides) return AVATTN_ERR_NULL_POINTER;
  if (!(eps >= 0.f) || !isfinite(eps)) return AVATTN_ERR_ARGUMENT;
  if (!cos_tab != !sin_tab) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!x) return AVATTN_ERR_NULL_POINTER;
  if (!al16(x) || !str4(x_strides) || (weight && !al16(weight))) return AVATTN_ERR_LAYOUT;
  if (cos_tab && (!al16(cos_tab) || !al16(sin_tab) || table_batch_stride % 4 != 0)) return AVATTN_ERR_LAYOUT;
  if ((int64_t)batch * heads > 2147483647 || (int64_t)batch * len > ((int64_t)1 << 40)) return AVATTN_ERR_TOO_LARGE;
  return AVATTN_OK;
}

static NormF32Args norm_f32_args(const float* x, const int64_t* xs, int32_t batch, int32_t heads, int32_t len,
                                 const float* weight, float eps, const float* cos_tab, const float* sin_tab,
                                 int64_t tsb) {
  NormF32Args a{};
  a.x = x, a.xsb = xs[0], a.xsh = xs[1], a.xsl = xs[2];
  a.B = batch, a.H = heads, a.L = len;
  a.w = weight, a.eps = eps;
  a.ct = cos_tab, a.st = sin_tab, a.tsb = tsb;
  return a;
}

int avattn_qk_norm_rope_f32(const float* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                            int32_t head_dim, const float* weight, float eps, const float* cos_tab,
                            const float* sin_tab, int64_t table_batch_stride, float* out,
                            const int64_t* out_strides, avattn_stream_t stream) {
  int st = check_norm_f32(x, x_strides, batch, heads, len, head_dim, weight, eps, cos_tab, sin_tab,
                          table_batch_stride);
  if (st != AVATTN_OK) return st;
  if (!out_strides) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!out) return AVATTN_ERR_NULL_POINTER;
  if (!al16(out) || !str4(out_strides)) return AVATTN_ERR_LAYOUT;
  NormF32Args a = norm_f32_args(x, x_strides, batch, heads, len, weight, eps, cos_tab, sin_tab, table_batch_stride);
  a.out = out, a.osb = out_strides[0], a.osh = out_strides[1], a.osl = out_strides[2];
  const int64_t tokens = (int64_t)batch * len;
  const dim3 grid((unsigned)(tokens > (1 << 20) ? (1 << 20) : tokens));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 128)
    hipLaunchKernelGGL(qk_norm_f32_fwd_kernel<128>, grid, dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL(qk_norm_f32_fwd_kernel<64>, grid, dim3(64), 0, s, a);
  return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
}

int avattn_qk_norm_rope_bwd_f32(const float* x, const int64_t* x_strides, const float* dy,
                                const int64_t* dy_strides, int32_t batch, int32_t heads, int32_t len,
                                int32_t head_dim, const float* weight, float eps, const float* cos_tab,
                                const float* sin_tab, int64_t table_batch_stride, float* dx,
                                const int64_t* dx_strides, float* dweight, void* workspace, size_t workspace_bytes,
                                avattn_stream_t stream) {
  int st = check_norm_f32(x, x_strides, batch, heads, len, head_dim, weight, eps, cos_tab, sin_tab,
                          table_batch_stride);
  if (st != AVATTN_OK) return st;
  if (!dy_strides || !dx_strides) return AVATTN_ERR_NULL_POINTER;
  if (weight && !dweight) return AVATTN_ERR_NULL_POINTER;
  if (weight && (!workspace || workspace_bytes < (size_t)kNormF32Blocks * head_dim * sizeof(float) ||
                 !al16(workspace)))
    return AVATTN_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if ((int64_t)batch * heads * len == 0) {
    if (!weight) return AVATTN_OK;
    // no rows: the gain's gradient is zero (the reduction over no blocks)
    hipLaunchKernelGGL(qk_norm_f32_dw_zero_kernel, dim3(1), dim3(128), 0, s, head_dim, dweight);
    return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
  }
  if (!dy || !dx) return AVATTN_ERR_NULL_POINTER;
  if (!al16(dy) || !al16(dx) || !str4(dy_strides) || !str4(dx_strides)) return AVATTN_ERR_LAYOUT;
  NormF32Args a = norm_f32_args(x, x_strides, batch, heads, len, weight, eps, cos_tab, sin_tab, table_batch_stride);
  a.dy = dy, a.dsb = dy_strides[0], a.dsh = dy_strides[1], a.dsl = dy_strides[2];
  a.dx = dx, a.xgb = dx_strides[0], a.xgh = dx_strides[1], a.xgl = dx_strides[2];
  a.wpart = weight ? static_cast<float*>(workspace) : nullptr;
  const int64_t tokens = (int64_t)batch * len;
  const int nb = (int)(tokens > kNormF32Blocks ? kNormF32Blocks : tokens);
  if (head_dim == 128)
    hipLaunchKernelGGL(qk_norm_f32_bwd_kernel<128>, dim3(nb), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL(qk_norm_f32_bwd_kernel<64>, dim3(nb), dim3(64), 0, s, a);
  if (weight) hipLaunchKernelGGL(qk_norm_f32_dw_kernel, dim3(head_dim), dim3(256), 0, s, a.wpart, nb, head_dim, dweight);
  return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
}

}  // extern "C"
