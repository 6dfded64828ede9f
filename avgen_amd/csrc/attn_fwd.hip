// Flash-style attention forward for gfx950.  K streams through LDS in 64-key
// row-major tiles and V in 64-key head_dim-major tiles, both from the padded
// copies made by prep.hip.
//
// Per wave and tile the scores are computed transposed, S^T = K Q^T, so that
// each lane owns one query column (query = lane % 32) and holds 32 of that
// query's 64 scores: the row max and row sum are in-lane plus one exchange
// with the partner lane (lane ^ 32).  Lane l reads K row perm23(l % 32) of
// each 32-key half, so the probabilities in the MFMA C layout are exactly the
// B operand of O^T += V^T P^T with eight consecutive keys per k slot group,
// and the matching V^T operand is one 16-byte LDS read.  P never leaves
// registers.  Q stays in registers for the whole kernel (optionally rotated on
// load, src/avgen/models/rope.py:332-338).  Softmax runs in the exp2 domain on
// raw scores with a running max; the LSE is natural-log
// (aten::_scaled_dot_product_flash_attention's logsumexp output).
#include <type_traits>

#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

// One workgroup = 256 query rows of one (batch, head), 8 waves x 32 rows, one
// workgroup per CU; K/V tiles of 64 keys.  Waves 0-3 (group A) and 4-7
// (group B) share the SIMDs pairwise and run the same per-tile work
//   S = K Q^T (16 MFMAs), softmax (VALU), O^T += V^T P^T (16 MFMAs)
// in a staggered order: in iteration t group A does PV(t-1), QK^T(t) and then
// softmax(t) (its probabilities are carried in registers across the
// barrier), group B does softmax(t-1) and then PV(t-1), QK^T(t) (its scores
// are carried).  Each iteration of each wave is thus one MFMA phase and one
// VALU phase, in opposite order in the two groups, so on every SIMD one
// wave's softmax runs while the other wave's MFMAs keep the matrix pipe busy;
// wave priorities (s_setprio) give the MFMA phases first claim on issue.  (With
// group A in the order QK^T(t), softmax(t), PV(t) the two softmax phases
// overlapped each other instead: 6.80 vs 5.84 ms per c3 chunk.)  K rows and
// V^T come from padded copies through four LDS stages: tile t+2 is loaded
// during iteration t (spread between MFMAs), tile t-1 stays resident for the
// PV products.
//
// FP8: q k^T on e4m3 operands (v_mfma_scale_f32_32x32x64_f8f6f4, twice the
// bf16 rate) producing the scores in log2 units with the lane's running
// maximum already subtracted, so the softmax is one exp2 per score.  q is
// quantized on load against the softmax constant and k's scale:
// q8 = e4m3(q * g * 2^-eq), g = scale_log2 * k_scale[hk] and 2^eq the
// smallest power of two >= g * q_scale[h] (fp32; so |q8| <= 448 wherever
// |q| <= 448 * q_scale[h]); the MFMA's block scale restores 2^eq and its
// accumulator starts from -m.  K comes from the e4m3 copy (fp8.hip).  P, V
// and O^T += V^T P^T stay bf16 / fp32 as above.
//
// WIN: per-query-row key windows [wlo, whi) (FwdArgs::wlo/whi).  The
// workgroup visits only the tiles that meet the union of its rows' windows,
// and a tile half that is not inside every window of the wave masks each
// score outside its row's window to -inf (before the key bias and softmax).
template <int D, bool ROPE, bool FP8, bool WIN>
__global__ __launch_bounds__(512, 1) void attn_fwd_kernel(FwdArgs a) {
  static_assert(!(ROPE && FP8), "the fp8 variant takes rotated q");
  static_assert(!(WIN && FP8), "windows on the bf16 path only");
  constexpr int NW = 8, BM = 32 * NW, BN = 64;
  // k-steps of q k^T: 16 bf16 channels (32x32x16 bf16) or 64 fp8 channels
  // (32x32x64 e4m3) per MFMA.
  constexpr int KS = FP8 ? D / 64 : D / 16;
  constexpr int KRL = FP8 ? D / 2 : D;  // K tile row in 2-byte units (an fp8 row is D bytes)
  constexpr int DT = D / 32;  // 32-channel row tiles of O^T
  constexpr int TE = BN * D;  // tile elements
  // One LDS object per stage (the compiler never sees the tile loads, which
  // are ordered by the explicit waits and barriers below).
  struct Stage {
    bf16 k[BN * KRL];  // K rows: TileLayout<KRL> (bf16, or e4m3 byte pairs)
    bf16 vt[TE];       // V^T rows (channel-major): TileLayout<BN>
    float bias[BN];  // key bias
    int flags[64];   // "all attended" flags of the tile's two 32-key halves (and beyond)
  };
  __shared__ __attribute__((aligned(16))) Stage st0, st1, st2, st3;
  auto stage_ref = [&](auto bufc) __attribute__((always_inline)) -> Stage& {
    constexpr int buf = decltype(bufc)::value;
    return buf == 0 ? st0 : (buf == 1 ? st1 : (buf == 2 ? st2 : st3));
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int prow = perm23(l32);  // K row this lane supplies to S^T = K Q^T

  const int nqt = (a.Lq + BM - 1) / BM;
  const int total = nqt * a.B * a.Hq;
  const int bid = xcd_remap(blockIdx.x, total);
  const int qt = bid % nqt;
  const int bh = bid / nqt;
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);

  const int qrow = qt * BM + wave * 32 + l32;
  const bool qvalid = qrow < a.Lq;

  // Key windows: this lane's row's [wlo, whi) (every key for a row past the
  // end); the wave's largest lo and smallest hi (a tile half inside both is
  // inside every row's window); the workgroup's tile range [t0, t0 + ntile).
  int wlo = 0, whi = a.Lkp, wlo_max = 0, whi_min = a.Lkp;
  int t0 = 0;
  int ntile = a.Lkp / BN;
  if constexpr (WIN) {
    __shared__ int wred[NW][2];
    int rlo = 0x7fffffff, rhi = -1;  // range contribution (none for empty or past-the-end rows)
    int mlo = -1, mhi = 0x7fffffff;  // interior test contribution
    if (qvalid) {
      // Clamped into 0 <= lo <= hi <= Lk, so any values stay in bounds.
      wlo = min(max(a.wlo[b * a.wsb + qrow], 0), a.Lk);
      whi = min(max(a.whi[b * a.wsb + qrow], wlo), a.Lk);
      mlo = wlo;
      mhi = whi;
      if (wlo < whi) {
        rlo = wlo;
        rhi = whi;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      rlo = min(rlo, __shfl_xor(rlo, off));
      rhi = max(rhi, __shfl_xor(rhi, off));
      mlo = max(mlo, __shfl_xor(mlo, off));
      mhi = min(mhi, __shfl_xor(mhi, off));
    }
    wlo_max = __builtin_amdgcn_readfirstlane(mlo);
    whi_min = __builtin_amdgcn_readfirstlane(mhi);
    if (lane == 0) {
      wred[wave][0] = rlo;
      wred[wave][1] = rhi;
    }
    __syncthreads();
    int glo = 0x7fffffff, ghi = -1;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      glo = min(glo, wred[w][0]);
      ghi = max(ghi, wred[w][1]);
    }
    glo = __builtin_amdgcn_readfirstlane(glo);
    ghi = __builtin_amdgcn_readfirstlane(ghi);
    t0 = ghi > glo ? glo / BN : 0;
    ntile = ghi > glo ? (ghi + BN - 1) / BN - t0 : 0;
  }

  const int64_t bhk = (int64_t)(b * a.Hkv + hk);
  const uint32_t slice = (uint32_t)a.Lkp * D * 2;  // bytes of one (b, h) slice of a copy
  const bf16* kcopy = FP8 ? reinterpret_cast<const bf16*>(a.k8) : a.kr;
  const u32x4 rk = make_rsrc(kcopy + bhk * a.Lkp * KRL, (uint32_t)a.Lkp * KRL * 2);
  const u32x4 rv = make_rsrc(a.vt + bhk * D * a.Lkp, slice);
  const u32x4 rb = make_rsrc(a.kbias + (int64_t)b * a.Lkp, (uint32_t)(a.Lkp + 64) * 4);
  // Flags are padded by 64 entries: the 64 read from a tile start stay inside.
  const u32x4 rf = make_rsrc(a.kfull + (int64_t)b * (a.Lkp / 32), (uint32_t)(a.Lkp / 32 + 64) * 4);
  const int tend = t0 + ntile;  // tiles t0 .. tend-1 (all of them without windows)

  using KSt = TileStager<BN, KRL, NW>;  // 64 K rows of D channels
  using VSt = TileStager<D, BN, NW>;  // D V^T rows of 64 keys (row stride Lkp)
  KSt kst;
  VSt vst;
  kst.init(KRL, wave, lane);
  vst.init(a.Lkp, wave, lane);
  constexpr int kStageOps = KSt::kPer + VSt::kPer + 2;  // loads per wave per tile
  auto stage_op = [&](int t, auto bufc, int i) __attribute__((always_inline)) {
    Stage& sg = stage_ref(bufc);
    const uint32_t k0 = (uint32_t)t * BN;
    if (i < KSt::kPer)
      kst.stage_one(sg.k, rk, k0 * KRL * 2, i);
    else if (i < KSt::kPer + VSt::kPer)
      vst.stage_one(sg.vt, rv, k0 * 2, i - KSt::kPer);
    else if (i == kStageOps - 2)
      dma4(rb, lds_addr(sg.bias), lane * 4, k0 * 4);
    else
      dma4(rf, lds_addr(sg.flags), lane * 4, (uint32_t)t * 8);
  };

  // Q fragments: B operand of S^T = K Q^T; lane holds row qrow, channels
  // 16*ks + 8*hh + [0, 8) (bf16), or 64*ks + 32*hh + [0, 32) (e4m3 bytes in
  // channel order, the same order the K operand reads).
  using QFrag = std::conditional_t<FP8, i32x8, bf16x8>;
  QFrag qf[KS];
  float c = a.scale_log2, sc = a.scale;  // softmax constants on raw q.k (bf16 path)
  int qe8 = 127;                         // fp8: E8M0 block scale of the q operand, 127 + eq
  int eq = 0;
  float qn2 = 0.f;  // this lane's share of the squared q row norm (fp8: of q8, e4m3 units)
  if constexpr (FP8) {
    const float g = a.scale_log2 * a.k_scale[hk];
    eq = ceil_log2_clamped(g * a.q_scale[h]);
    const float qm = ldexpf(g, -eq);
    qe8 = 127 + eq;
    const bf16* qp = a.q + b * a.qsb + h * a.qsh + (int64_t)qrow * a.qsl + 32 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      i32x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
      if (qvalid) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const u32x4 w = *reinterpret_cast<const u32x4*>(qp + 64 * ks + 8 * q4);
          x[2 * q4] = (int)pack_fp8x4(bf16_lo(w[0]) * qm, bf16_hi(w[0]) * qm, bf16_lo(w[1]) * qm,
                                      bf16_hi(w[1]) * qm);
          x[2 * q4 + 1] = (int)pack_fp8x4(bf16_lo(w[2]) * qm, bf16_hi(w[2]) * qm, bf16_lo(w[3]) * qm,
                                          bf16_hi(w[3]) * qm);
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v0 = __builtin_amdgcn_cvt_f32_fp8(x[i], 0), v1 = __builtin_amdgcn_cvt_f32_fp8(x[i], 1);
        const float v2 = __builtin_amdgcn_cvt_f32_fp8(x[i], 2), v3 = __builtin_amdgcn_cvt_f32_fp8(x[i], 3);
        qn2 = fmaf(v0, v0, fmaf(v1, v1, fmaf(v2, v2, fmaf(v3, v3, qn2))));
      }
      qf[ks] = x;
    }
  } else {
    const bf16* qp = a.q + b * a.qsb + h * a.qsh + (int64_t)qrow * a.qsl + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (qvalid) {
        x = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
        if constexpr (ROPE) {
          const int64_t t = b * a.rsb + (int64_t)qrow * (D / 2) + 8 * ks + 4 * hh;
          const f32x4 c = *reinterpret_cast<const f32x4*>(a.cos_q + t);
          const f32x4 s = *reinterpret_cast<const f32x4*>(a.sin_q + t);
          x = rotate8(x, c, s, false);
        }
      }
      qf[ks] = bits_to_bf16x8(x);
    }
  }

  // Loop-invariant per-lane LDS element offsets.
  constexpr int KC = FP8 ? 2 : 1;  // 16-byte chunks per K operand
  int ko[KS * KC];  // K row perm23(l32): chunk 16*ks + 8*hh, or chunks 32*ks + 16*hh + {0, 8} (fp8)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int cc = 0; cc < KC; ++cc)
      ko[KC * ks + cc] = FP8 ? TileLayout<KRL>::off(prow, 32 * ks + 16 * hh + 8 * cc)
                             : TileLayout<KRL>::off(prow, 16 * ks + 8 * hh);
  int vo[4];  // V^T row l32 (+32*dt), key chunk 16*j + 8*hh (j = 2*half + k2)
#pragma unroll
  for (int j = 0; j < 4; ++j) vo[j] = TileLayout<BN>::off(l32, 16 * j + 8 * hh);

  // Lazy rescaling: the reference max m_run only moves when a half-tile's
  // max exceeds it by more than 8 in log2 units, so probabilities stay
  // <= 2^8 (exact in fp32/bf16 range) and the O rescale is rare after the
  // first tiles.  The result is the same softmax; only roundings differ.
  const float tau = 8.f / c;
  // Score bound (bf16 path): |s| <= |q_row| * max_k |k| (Cauchy-Schwarz; the
  // fp32 accumulation error is far below the 1/1024 margin).  Once
  // (bound - m_run) * c <= kBoundTau for every row of the wave, no later
  // score can make a probability exceed 2^kBoundTau (far inside fp32/bf16
  // range, and O, l stay finite), so the wave stops tracking row maxima:
  // m_run is then final and the per-tile max and rescale test are skipped.
  // The fp8 path bounds its log2-unit scores by 2^eq * |q8_row| * max_k |k8|
  // (the products of e4m3 values are exact; same margin) against a maximum
  // kept in log2 units.
  constexpr float kBoundTau = 32.f;
  float bound = kPosInf;
  if constexpr (FP8) {
    if (a.kmax2 != nullptr) {
      qn2 = halves_sum(qn2);
      const int ntk = a.Lkp / 64;
      const uint32_t* km = a.kmax2 + bhk * ntk;
      float km2 = 0.f;
      for (int i = lane; i < ntk; i += 64) km2 = fmaxf(km2, __uint_as_float(km[i]));
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) km2 = fmaxf(km2, __shfl_xor(km2, off));
      bound = ldexpf(sqrtf(qn2) * sqrtf(km2) * (1.f + 1.f / 1024.f), eq);
    }
  } else {
    if (a.kmax2 != nullptr) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (float)qf[ks][e];
          qn2 = fmaf(x, x, qn2);
        }
      qn2 = halves_sum(qn2);
      // Largest squared k row norm of the head: a wave maximum over its tiles.
      const int ntk = a.Lkp / 64;
      const uint32_t* km = a.kmax2 + bhk * ntk;
      float km2 = 0.f;
      for (int i = lane; i < ntk; i += 64) km2 = fmaxf(km2, __uint_as_float(km[i]));
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) km2 = fmaxf(km2, __shfl_xor(km2, off));
      bound = sqrtf(qn2) * sqrtf(km2) * (1.f + 1.f / 1024.f);
    }
  }
  int bounded = 0;  // wave-uniform
  // Reference max for this lane's query: of the raw scores (bf16 path), of
  // the log2-unit scores (fp8, where cneg holds -m_run in every register, 0
  // while m_run is -inf: the accumulator the q k^T products start from).
  float m_run = kNegInf;
  f32x16 cneg = zero16();
  float l_run0 = 0.f, l_run1 = 0.f;  // this lane's share of the row sum
  f32x16 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = zero16();

  // The 2*KS QK^T MFMAs of a tile: sh[half][8*k2 + e] is the score of key
  // 32*half + 16*k2 + 8*hh + e against this lane's query.  K operand reads
  // run four MFMAs ahead; `slot(j)` runs extra work after MFMA j.
  // sched_barrier(0) pins the order (the scheduler would otherwise sink each
  // read next to its MFMA).
  auto scores = [&](const Stage& sg, f32x16* sh, auto&& slot) __attribute__((always_inline)) {
    constexpr int NS = 2 * KS;
    constexpr int R = NS < 4 ? NS : 4;  // operand reads in flight
    auto kop = [&](int j) __attribute__((always_inline)) {
      const bf16* base = sg.k + (j / KS) * 32 * KRL;
      if constexpr (FP8) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(base + ko[2 * (j % KS)]);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(base + ko[2 * (j % KS) + 1]);
        return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      } else {
        return *reinterpret_cast<const bf16x8*>(base + ko[j % KS]);
      }
    };
    QFrag ka[R];
#pragma unroll
    for (int j = 0; j < R; ++j) ka[j] = kop(j);
    if constexpr (!FP8) {
      sh[0] = zero16();
      sh[1] = zero16();
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      if constexpr (FP8)
        sh[j / KS] = mfma32_fp8_scaled(ka[j % R], qf[j % KS], j % KS == 0 ? cneg : sh[j / KS], 127, qe8);
      else
        sh[j / KS] = mfma32(ka[j % R], qf[j % KS], sh[j / KS]);
      if (j + R < NS) ka[j % R] = kop(j + R);
      slot(j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Softmax of one tile's scores (both halves) into the bf16 PV operands.
  auto softmax = [&](const Stage& sg, f32x16* sh, bf16x8 (*pf)[2], int t) __attribute__((always_inline)) {
    if constexpr (FP8) {
      // sh: the tile's log2-unit scores minus m_run (plain scores while m_run
      // is -inf), both halves formed against the same m_run, so one maximum
      // per tile: a new reference moves m_run by the excess mx and shifts
      // both halves by it (the next tiles' products start from the new
      // -m_run).
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        if (!__builtin_amdgcn_readfirstlane(sg.flags[hf])) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 bb =
                *reinterpret_cast<const f32x4*>(sg.bias + hf * 32 + 16 * (g >> 1) + 8 * hh + 4 * (g & 1));
#pragma unroll
            for (int r = 0; r < 4; ++r) sh[hf][4 * g + r] += bb[r];
          }
        }
      }
      if (!bounded) {
        float mx = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sh[0][r], sh[1][r]));
        mx = halves_max(mx);
        const bool first = m_run == kNegInf;
        if (first ? mx > kNegInf : mx > 8.f) {
          if (first) {
            m_run = mx;
          } else {
            const float alpha = __builtin_amdgcn_exp2f(-mx);
            l_run0 *= alpha;
            l_run1 *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
            m_run += mx;
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            sh[0][r] -= mx;
            sh[1][r] -= mx;
          }
          cneg = splat16(-m_run);
        }
        bounded = __all(bound - m_run <= kBoundTau);
      }
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          u32x4 u;
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int r = 8 * k2 + 2 * e2;
            const float p0 = __builtin_amdgcn_exp2f(sh[hf][r]);
            const float p1 = __builtin_amdgcn_exp2f(sh[hf][r + 1]);
            if (e2 & 1)
              l_run1 += p0 + p1;
            else
              l_run0 += p0 + p1;
            u[e2] = pack_bf16x2(p0, p1);
          }
          pf[hf][k2] = bits_to_bf16x8(u);
        }
      return;
    }
    // Masks of both halves first, then one reference max for the tile: the
    // probabilities of both halves are formed against the same m_run (a
    // half processed against a reference the other half then moves would
    // enter P V at the wrong scale while the row sum is rescaled).
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f32x16& s_cur = sh[hf];
      if constexpr (WIN) {
        // Register 8*k2 + e holds key 64*t + 32*hf + 16*k2 + 8*hh + e.
        const int kh = BN * t + 32 * hf;
        if (kh < wlo_max || kh + 32 > whi_min) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kh + 16 * (r >> 3) + 8 * hh + (r & 7);
            if (key < wlo || key >= whi) s_cur[r] = kNegInf;
          }
        }
      }
      if (!__builtin_amdgcn_readfirstlane(sg.flags[hf])) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bb = *reinterpret_cast<const f32x4*>(sg.bias + hf * 32 + 16 * (g >> 1) + 8 * hh + 4 * (g & 1));
#pragma unroll
          for (int r = 0; r < 4; ++r) s_cur[4 * g + r] += bb[r];
        }
      }
    }
    if (!bounded) {
      float mx = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sh[0][r], sh[1][r]));
      mx = halves_max(mx);
      if (mx > m_run + tau) {
        // New reference max (both lanes of a query agree: mx is shared).
        const float alpha = __builtin_amdgcn_exp2f((m_run - mx) * c);
        l_run0 *= alpha;
        l_run1 *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
        m_run = mx;
      }
      bounded = __all((bound - m_run) * c <= kBoundTau);
    }
    const float mc = (m_run == kNegInf) ? 0.f : m_run * c;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        u32x4 u;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int r = 8 * k2 + 2 * e2;
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sh[hf][r], c, -mc));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sh[hf][r + 1], c, -mc));
          if (e2 & 1)
            l_run1 += p0 + p1;
          else
            l_run0 += p0 + p1;
          u[e2] = pack_bf16x2(p0, p1);
        }
        pf[hf][k2] = bits_to_bf16x8(u);
      }
  };
  // O^T += V^T P^T over the (half, k2, dt) steps; B operand slot (hh, e) of
  // pf[hf][k2] is key 32*hf + 16*k2 + 8*hh + e: one 16-byte chunk of a V^T
  // row.  Reads four MFMAs ahead; `slot(j)` runs extra work after MFMA j.
  auto pv = [&](const Stage& sg, bf16x8 (*pf)[2], auto&& slot) __attribute__((always_inline)) {
    constexpr int NJ = 4 * DT;
    auto vop = [&](int j) __attribute__((always_inline)) {
      const int sk = j / DT, dt = j % DT;
      return *reinterpret_cast<const bf16x8*>(sg.vt + dt * 32 * BN + vo[sk]);
    };
    bf16x8 va[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) va[j] = vop(j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int sk = j / DT, dt = j % DT;
      acc[dt] = mfma32(va[j & 3], pf[sk >> 1][sk & 1], acc[dt]);
      if (j + 4 < NJ) va[j & 3] = vop(j + 4);
      slot(j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto no_slot = [](int) __attribute__((always_inline)) {};

  // Top of iteration t: tile t has landed (its loads were issued two
  // iterations ago; only tile t+1's may still be in flight) for every wave;
  // the stage tile t-2 used is free for tile t+2.
  auto top = [&]() __attribute__((always_inline)) {
    wait_vmem_n<kStageOps>();
    barrier_lds();
  };
  // Tile t's loads, spread over a loop's MFMA slots: slot kLoad0 +
  // kLoadStep*i issues load i (measured ~2% faster than one load in each of
  // the first slots, which crowds the loop's first operand reads); loads whose
  // slot lies past the end of the loop follow it (loads_after).  Every wave
  // issues exactly kStageOps loads per iteration: the counted waits rely on
  // it.  The fp8 q k^T has only 4 MFMAs per tile, so there the loads ride on
  // PV.
  constexpr int kLoad0 = 2, kLoadStep = 3;
  auto loads_in = [&](int t, auto nextc) __attribute__((always_inline)) {
    return [&, t, nextc](int j) __attribute__((always_inline)) {
      if (j >= kLoad0 && (j - kLoad0) % kLoadStep == 0 && (j - kLoad0) / kLoadStep < kStageOps)
        stage_op(t, nextc, (j - kLoad0) / kLoadStep);
    };
  };
  auto loads_after = [&](int t, auto nextc, int nslots) __attribute__((always_inline)) {
    const int done = nslots > kLoad0 ? (nslots - kLoad0 + kLoadStep - 1) / kLoadStep : 0;
#pragma unroll
    for (int i = done; i < kStageOps; ++i) stage_op(t, nextc, i);
  };

  retire_prologue_loads();
  // ntile is the same for every wave of the workgroup (0: every row's window
  // is empty, nothing to visit).
  if (ntile > 0) {
    {
      using B0 = std::integral_constant<int, 0>;
      using B1 = std::integral_constant<int, 1>;
#pragma unroll
      for (int i = 0; i < kStageOps; ++i) stage_op(t0, B0(), i);
#pragma unroll
      for (int i = 0; i < kStageOps; ++i) stage_op(min(t0 + 1, tend - 1), B1(), i);
    }

    f32x16 sh[2];
    bf16x8 pf[2][2];
    // Tile t0 + i uses stage i % 4.
    if (wave < NW / 2) {
      // Group A: PV(t-1), QK^T(t), softmax(t); the probabilities of tile t
      // are carried to the next iteration.  Each iteration is one MFMA
      // phase (PV, QK^T) and then one VALU phase (softmax), the reverse of
      // group B's, so on each SIMD one wave's softmax runs beside the other
      // wave's MFMAs.
      auto body = [&](int t, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        using Prev = std::integral_constant<int, (buf + 3) % 4>;
        using Next2 = std::integral_constant<int, (buf + 2) % 4>;
        top();
        const Stage& sg = stage_ref(bufc);
        __builtin_amdgcn_s_setprio(2);
        const int tl = min(t + 2, tend - 1);
        if constexpr (FP8) {
          pv(stage_ref(Prev()), pf, loads_in(tl, Next2()));
          loads_after(tl, Next2(), 4 * DT);
          scores(sg, sh, no_slot);
        } else {
          pv(stage_ref(Prev()), pf, no_slot);
          scores(sg, sh, loads_in(tl, Next2()));
          loads_after(tl, Next2(), 2 * KS);
        }
        __builtin_amdgcn_s_setprio(0);
        softmax(sg, sh, pf, t);
      };
      {
        // Iteration 0: QK^T(t0), softmax(t0).
        using B0 = std::integral_constant<int, 0>;
        using B2 = std::integral_constant<int, 2>;
        top();
        __builtin_amdgcn_s_setprio(2);
        if constexpr (FP8) {
          scores(stage_ref(B0()), sh, no_slot);
#pragma unroll
          for (int i = 0; i < kStageOps; ++i) stage_op(min(t0 + 2, tend - 1), B2(), i);
        } else {
          scores(stage_ref(B0()), sh, loads_in(min(t0 + 2, tend - 1), B2()));
          loads_after(min(t0 + 2, tend - 1), B2(), 2 * KS);
        }
        __builtin_amdgcn_s_setprio(0);
        softmax(stage_ref(B0()), sh, pf, t0);
      }
      for (int t = t0 + 1; t < tend; t += 4) {
        body(t, std::integral_constant<int, 1>());
        if (t + 1 < tend) body(t + 1, std::integral_constant<int, 2>());
        if (t + 2 < tend) body(t + 2, std::integral_constant<int, 3>());
        if (t + 3 < tend) body(t + 3, std::integral_constant<int, 0>());
      }
      // Tail: PV of the last tile (its stage is not refilled).
      const int bl = (ntile - 1) % 4;
      const Stage& sl = bl == 0 ? st0 : (bl == 1 ? st1 : (bl == 2 ? st2 : st3));
      __builtin_amdgcn_s_setprio(2);
      pv(sl, pf, no_slot);
    } else {
      // Group B: softmax(t-1), PV(t-1), QK^T(t); the scores of tile t are
      // carried to the next iteration.
      auto body = [&](int t, auto bufc) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        using Prev = std::integral_constant<int, (buf + 3) % 4>;
        using Next2 = std::integral_constant<int, (buf + 2) % 4>;
        top();
        const Stage& sp = stage_ref(Prev());
        __builtin_amdgcn_s_setprio(0);
        softmax(sp, sh, pf, t - 1);
        __builtin_amdgcn_s_setprio(2);
        pv(sp, pf, loads_in(min(t + 2, tend - 1), Next2()));
        loads_after(min(t + 2, tend - 1), Next2(), 4 * DT);
        scores(stage_ref(bufc), sh, no_slot);
      };
      {
        // Iteration 0: only QK^T(t0).
        using B0 = std::integral_constant<int, 0>;
        using B2 = std::integral_constant<int, 2>;
        top();
        if constexpr (FP8) {
          scores(stage_ref(B0()), sh, no_slot);
#pragma unroll
          for (int i = 0; i < kStageOps; ++i) stage_op(min(t0 + 2, tend - 1), B2(), i);
        } else {
          scores(stage_ref(B0()), sh, loads_in(min(t0 + 2, tend - 1), B2()));
          loads_after(min(t0 + 2, tend - 1), B2(), 2 * KS);
        }
      }
      for (int t = t0 + 1; t < tend; t += 4) {
        body(t, std::integral_constant<int, 1>());
        if (t + 1 < tend) body(t + 1, std::integral_constant<int, 2>());
        if (t + 2 < tend) body(t + 2, std::integral_constant<int, 3>());
        if (t + 3 < tend) body(t + 3, std::integral_constant<int, 0>());
      }
      // Tail: softmax and PV of the last tile (its stage is not refilled).
      const int bl = (ntile - 1) % 4;
      const Stage& sl = bl == 0 ? st0 : (bl == 1 ? st1 : (bl == 2 ? st2 : st3));
      __builtin_amdgcn_s_setprio(0);
      softmax(sl, sh, pf, tend - 1);
      pv(sl, pf, no_slot);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  wait_vmem();  // the last (re-staged) tile loads

  // Three row states: l_tot > 0; l_tot == 0, no valid key (out 0 as SDPA
  // returns, lse -inf); NaN, a NaN (or +inf) score reached the row (out and
  // lse NaN, as the softmax of such a row gives).
  const float l_tot = halves_sum(l_run0 + l_run1);
  const float nan = __builtin_nanf("");
  const float inv = l_tot > 0.f ? 1.f / l_tot : (l_tot == 0.f ? 0.f : nan);
  // m_run is in raw score units (bf16 path) or log2 units (fp8).
  const float lse = l_tot > 0.f ? fmaf(m_run, FP8 ? kLn2 : sc, logf(l_tot)) : (l_tot == 0.f ? kNegInf : nan);
  if (qvalid) {
    bf16* op = a.o + b * a.osb + h * a.osh + (int64_t)qrow * a.osl;
    if (a.o_acc == nullptr) {
      if (hh == 0) a.lse[(int64_t)bh * a.Lq + qrow] = lse;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 w;
          w[0] = pack_bf16x2(acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv);
          w[1] = pack_bf16x2(acc[dt][4 * g + 2] * inv, acc[dt][4 * g + 3] * inv);
          *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
        }
    } else {
      // Ring step: merge this chunk's bf16-rounded output and lse into the
      // fp32 accumulator, exactly as lse_merge_kernel would merge them
      // (torch/.../_context_parallel/_attention.py:182-183).
      const int64_t row = (int64_t)bh * a.Lq + qrow;
      float* accp = a.o_acc + row * D;
      int mode = 1;
      float w = 1.f;
      float nl = lse;
      if (!a.acc_first) nl = lse_merge_coeffs(a.lse_acc[row], lse, mode, w);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ch = dt * 32 + 8 * g + 4 * hh;
          const u32x2 ob = {pack_bf16x2(acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv),
                            pack_bf16x2(acc[dt][4 * g + 2] * inv, acc[dt][4 * g + 3] * inv)};
          f32x4 m = {bf16_lo(ob[0]), bf16_hi(ob[0]), bf16_lo(ob[1]), bf16_hi(ob[1])};
          if (mode != 1) {
            const f32x4 prev = *reinterpret_cast<const f32x4*>(accp + ch);
#pragma unroll
            for (int r = 0; r < 4; ++r) m[r] = lse_merge_elem(prev[r], m[r], mode, w);
          }
          *reinterpret_cast<f32x4*>(accp + ch) = m;
          if (a.acc_final) {
            const u32x2 fo = {pack_bf16x2(m[0], m[1]), pack_bf16x2(m[2], m[3])};
            *reinterpret_cast<u32x2*>(op + ch) = fo;
          }
        }
      // Both lanes of the row read lse_acc above (one wave, program order)
      // before this write.
      if (hh == 0) a.lse_acc[row] = nl;
    }
  }
}

// Writes zeros to out and -inf to lse: attention over an empty key set
// (src/avgen/models/attention.py:261-262 returns zeros_like(query)).
__global__ void attn_empty_kernel(bf16* o, int64_t osb, int64_t osh, int64_t osl, int B, int H, int L, int D,
                                  float* lse) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % (D / 8));
    const int64_t row = u / (D / 8);
    const int i = (int)(row % L);
    const int h = (int)((row / L) % H);
    const int b = (int)(row / ((int64_t)L * H));
    *reinterpret_cast<u32x4*>(o + b * osb + h * osh + (int64_t)i * osl + 8 * c) = u32x4{0u, 0u, 0u, 0u};
    if (c == 0) lse[row] = kNegInf;
  }
}

template <int D>
static hipError_t launch_fwd_d(const FwdArgs& a, hipStream_t stream) {
  const bool fp8 = a.k8 != nullptr;
  {
    LaunchTimer timer(kKidTranspose, stream);
    hipError_t e = launch_key_prep(a.mask, a.msb, a.B, a.Lk, a.kbias, a.kfull, stream);
    if (e == hipSuccess)
      e = fp8 ? launch_quantize_rows(a.k, a.ksb, a.ksh, a.ksl, a.B, a.Hkv, a.Lk, D, a.k_scale, a.k8, a.kmax2,
                                     stream)
              : launch_prep_copies(a.k, a.ksb, a.ksh, a.ksl, a.B, a.Hkv, a.Lk, D, a.kr, nullptr, stream, a.kmax2,
                                   a.cos_k, a.sin_k, a.rksb);
    if (e == hipSuccess) e = launch_prep_copies(a.v, a.vsb, a.vsh, a.vsl, a.B, a.Hkv, a.Lk, D, nullptr, a.vt, stream);
    if (e != hipSuccess) return e;
  }
  const int nqt = (a.Lq + 255) / 256;
  const dim3 grid(nqt * a.B * a.Hq);
  const dim3 block(512);
  LaunchTimer timer(fp8 ? kKidFwdFp8 : kKidFwd, stream);
  if (fp8)
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, true, false>), grid, block, 0, stream, a);
  else if (a.wlo != nullptr)
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, false, true>), grid, block, 0, stream, a);
  else if (a.cos_q != nullptr)
    hipLaunchKernelGGL((attn_fwd_kernel<D, true, false, false>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdArgs& a, int head_dim, hipStream_t stream) {
  return head_dim == 128 ? launch_fwd_d<128>(a, stream) : launch_fwd_d<64>(a, stream);
}

hipError_t launch_empty(bf16* o, int64_t osb, int64_t osh, int64_t osl, int B, int H, int L, int D, float* lse,
                        hipStream_t stream) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  const int blocks = (int)((units + 255) / 256 < 65536 ? (units + 255) / 256 : 65536);
  hipLaunchKernelGGL(attn_empty_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, stream, o, osb, osh, osl, B, H,
                     L, D, lse);
  return hipGetLastError();
}

}  // namespace avattn
