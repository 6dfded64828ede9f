// Attention backward for gfx950, recomputing the probabilities from (q, k,
// lse) instead of storing them.  No atomics (bitwise reproducible):
//   1. preprocess: per query row, lse2 = lse * log2(e) and
//      ndelta = -rowsum(dout * out) (the `D` term of dS = P * (dP - D)), in
//      arrays padded to whole 64-row tiles (+inf / 0 past the end so padded
//      rows get P = 0); plus head_dim-major copies of q, dout and k
//      (transpose.hip);
//   2. dK/dV: one workgroup per 128 keys (32 per wave, kept in registers as
//      MFMA operands); loops over 64-row query tiles of every query head
//      that reads this KV head;
//   3. dQ: one workgroup per 128 query rows (32 per wave); loops over 32-key
//      tiles.
// Every MFMA operand read from LDS is one 16-byte chunk of a tile row: the
// products contracting over the sequence read head_dim-major tiles of the
// copies, and the rows feeding the first product are read in perm23 order so
// that their C layout lines up with those chunks.
// With out/lse the merged result over all KV chunks, the outputs are one
// chunk's contributions, which is how the ring backward calls the op
// (torch/.../_context_parallel/_attention.py:567-575).
#include <type_traits>

#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

// ---------------------------------------------------------------------------
// 1. lse2 / ndelta
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdArgs a) {
  constexpr int TPR = D / 8;  // threads per row
  constexpr int RPB = 256 / TPR;
  const int64_t rows = (int64_t)a.B * a.Hq * a.Lqp;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int c = threadIdx.x % TPR;
  const int i = (int)(row % a.Lqp);
  const int64_t bh = row / a.Lqp;
  const bool valid = row < rows && i < a.Lq;
  float acc = 0.f;
  if (valid) {
    const int h = (int)(bh % a.Hq);
    const int b = (int)(bh / a.Hq);
    const u32x4 x = *reinterpret_cast<const u32x4*>(a.dout + b * a.dosb + h * a.dosh + (int64_t)i * a.dosl + 8 * c);
    const u32x4 y = *reinterpret_cast<const u32x4*>(a.out + b * a.osb + h * a.osh + (int64_t)i * a.osl + 8 * c);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      acc = fmaf(__uint_as_float(x[w] << 16), __uint_as_float(y[w] << 16), acc);
      acc = fmaf(__uint_as_float(x[w] & 0xffff0000u), __uint_as_float(y[w] & 0xffff0000u), acc);
    }
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, TPR);
  if (row < rows && c == 0) {
    a.ndelta[row] = -acc;
    if (valid) {
      const float l = a.lse[bh * a.Lq + i];
      a.lse2[row] = (l == kNegInf) ? kPosInf : l * kLog2e;
    } else {
      a.lse2[row] = kPosInf;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. dK / dV
// ---------------------------------------------------------------------------
// Per wave: 32 keys (lane % 32 owns key column k0w + lane % 32).  For each
// 32-row half `sub` of a 64-row query tile (lane l supplies query row
// 32*sub + perm23(l % 32) to the first two products):
//   S  = Q K^T    A = Q rows (LDS)              B = K^T (registers)
//   dP = dO V^T   A = dO rows (LDS)             B = V^T (registers)
//   P  = exp2(S*c - lse2[q]),  dS = P * (dP + ndelta[q])        (fp32)
//   dV^T += dO^T P   A = dO^T (LDS, head_dim-major)   B = P  (C layout reused)
//   dK^T += Q^T dS   A = Q^T  (LDS, head_dim-major)   B = dS (C layout reused)
// C-layout register 8*k2 + e of lane l holds query 32*sub + 16*k2 + 8*(l/32)
// + e, so the A operands of the last two products and the row statistics are
// 16-byte / 32-byte LDS reads.  Keys that are masked (or past the end) are
// not special-cased in the loop: each key's dK/dV column depends only on that
// key, and those columns are written as zeros (or not at all) at the end.
//
// Tiles come from the padded copies (every load full, per-lane offsets loop
// invariant); the loop body is branch-free and unrolled over the two LDS
// buffers so that every LDS address is a per-lane base plus an immediate.
// Order inside one tile: S/dP of half 0; S/dP of half 1 (the softmax of half
// 0 fills the VALU meanwhile); dV/dK of half 0 (softmax of half 1); dV/dK of
// half 1.
template <int D, bool MASK>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_kernel(BwdArgs a) {
  constexpr int BK = 128, BQ = 64, NW = 4;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int TE = BQ * D;
  // Each buffer of the double-buffered tiles is its own LDS object, so the
  // compiler knows the next tile's direct loads do not alias this tile's reads.
  __shared__ __attribute__((aligned(16))) bf16 sq0[TE], sq1[TE];      // Q rows: TileLayout<D>
  __shared__ __attribute__((aligned(16))) bf16 sdo0[TE], sdo1[TE];    // dO rows: TileLayout<D>
  __shared__ __attribute__((aligned(16))) bf16 sqt0[TE], sqt1[TE];    // Q^T: D rows of BQ, TileLayout<BQ>
  __shared__ __attribute__((aligned(16))) bf16 sdot0[TE], sdot1[TE];  // dO^T: TileLayout<BQ>
  __shared__ __attribute__((aligned(16))) float slse0[BQ], slse1[BQ];
  __shared__ __attribute__((aligned(16))) float sndl0[BQ], sndl1[BQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int prow = perm23(l32);

  const int nkt = (a.Lk + BK - 1) / BK;
  const int total = nkt * a.B * a.Hkv;
  const int bid = xcd_remap(blockIdx.x, total);
  const int kt = bid % nkt;
  const int bhk = bid / nkt;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.Hq / a.Hkv;

  const int key = kt * BK + wave * 32 + l32;

  // K/V of this lane's key (zeros past the end).
  bf16x8 kf[KS], vf[KS];
  {
    const bool in = key < a.Lk;
    const int64_t kr = ((int64_t)bhk * a.Lkp + key) * D + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
      if (in) {
        x = *reinterpret_cast<const u32x4*>(a.kr + kr + 16 * ks);
        y = *reinterpret_cast<const u32x4*>(a.vr + kr + 16 * ks);
      }
      kf[ks] = bits_to_bf16x8(x);
      vf[ks] = bits_to_bf16x8(y);
    }
  }

  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) {
    dk[i] = zero16();
    dv[i] = zero16();
  }

  // Loop-invariant per-lane LDS element offsets.
  int ro[KS];  // row tiles: chunk (16*ks + 8*hh) of row perm23(l32)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) ro[ks] = TileLayout<D>::off(prow, 16 * ks + 8 * hh);
  int to[4];  // head_dim-major tiles: chunk (32*sub + 16*k2 + 8*hh) of row l32 (+32*dt rows)
#pragma unroll
  for (int j = 0; j < 4; ++j) to[j] = TileLayout<BQ>::off(l32, 16 * j + 8 * hh);

  const int nqt = a.Lqp / BQ;
  const int niter = nqt * group;
  DirectStager<BQ, D, NW> rst;  // 64 rows of D channels (row stride D)
  DirectStager<D, BQ, NW> tst;  // D rows of 64 queries (row stride Lqp)
  rst.init(D, wave, lane);
  tst.init(a.Lqp, wave, lane);

  auto stage = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int hq = hk * group + it / nqt;
    const int q0 = (it % nqt) * BQ;
    const int64_t bq = (int64_t)(b * a.Hq + hq);
    const int64_t rb = (bq * a.Lqp + q0) * D;
    rst.stage_full(buf == 0 ? sq0 : sq1, a.qr + rb, wave);
    rst.stage_full(buf == 0 ? sdo0 : sdo1, a.dor + rb, wave);
    const int64_t tb = bq * D * a.Lqp + q0;
    tst.stage_full(buf == 0 ? sqt0 : sqt1, a.qt + tb, wave);
    tst.stage_full(buf == 0 ? sdot0 : sdot1, a.dot + tb, wave);
    const int64_t sr = bq * a.Lqp + q0 + lane;
    direct_load4(a.lse2 + sr, buf == 0 ? slse0 : slse1);
    direct_load4(a.ndelta + sr, buf == 0 ? sndl0 : sndl1);
  };

  const float c = a.scale_log2;

  // P and dS of one 32-row half from its S/dP accumulators.
  auto softmax = [&](const f32x16& s, const f32x16& dp, const float* ll, const float* lnd, bf16x8* pb,
                     bf16x8* dsb) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const f32x4 l2a = *reinterpret_cast<const f32x4*>(ll + 16 * k2 + 8 * hh);
      const f32x4 l2b = *reinterpret_cast<const f32x4*>(ll + 16 * k2 + 8 * hh + 4);
      const f32x4 nda = *reinterpret_cast<const f32x4*>(lnd + 16 * k2 + 8 * hh);
      const f32x4 ndb = *reinterpret_cast<const f32x4*>(lnd + 16 * k2 + 8 * hh + 4);
      u32x4 up, ud;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int e = 2 * e2;
        const float l0 = e < 4 ? l2a[e] : l2b[e - 4], l1 = e < 4 ? l2a[e + 1] : l2b[e - 3];
        const float n0 = e < 4 ? nda[e] : ndb[e - 4], n1 = e < 4 ? nda[e + 1] : ndb[e - 3];
        const float p0 = __builtin_amdgcn_exp2f(fmaf(s[8 * k2 + e], c, -l0));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(s[8 * k2 + e + 1], c, -l1));
        up[e2] = pack_bf16x2(p0, p1);
        ud[e2] = pack_bf16x2(p0 * (dp[8 * k2 + e] + n0), p1 * (dp[8 * k2 + e + 1] + n1));
      }
      pb[k2] = bits_to_bf16x8(up);
      dsb[k2] = bits_to_bf16x8(ud);
    }
  };

  auto body = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    wait_vmem();
    __syncthreads();  // tile `it` visible in `buf`; tile it-1 fully consumed everywhere
    // the last iteration re-stages a tile nobody reads
    stage(min(it + 1, niter - 1), std::integral_constant<int, buf ^ 1>());
    const bf16* tq = buf == 0 ? sq0 : sq1;
    const bf16* tdo = buf == 0 ? sdo0 : sdo1;
    const bf16* tqt = buf == 0 ? sqt0 : sqt1;
    const bf16* tdot = buf == 0 ? sdot0 : sdot1;
    const float* tl = buf == 0 ? slse0 : slse1;
    const float* tn = buf == 0 ? sndl0 : sndl1;

    bf16x8 qa[KS], da[KS];
    f32x16 s0 = zero16(), dp0 = zero16(), s1 = zero16(), dp1 = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qa[ks] = *reinterpret_cast<const bf16x8*>(tq + ro[ks]);
      da[ks] = *reinterpret_cast<const bf16x8*>(tdo + ro[ks]);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s0 = mfma32(qa[ks], kf[ks], s0);
      dp0 = mfma32(da[ks], vf[ks], dp0);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qa[ks] = *reinterpret_cast<const bf16x8*>(tq + 32 * D + ro[ks]);
      da[ks] = *reinterpret_cast<const bf16x8*>(tdo + 32 * D + ro[ks]);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s1 = mfma32(qa[ks], kf[ks], s1);
      dp1 = mfma32(da[ks], vf[ks], dp1);
    }
    bf16x8 pb[2], dsb[2];
    softmax(s0, dp0, tl, tn, pb, dsb);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dv[dt] = mfma32(*reinterpret_cast<const bf16x8*>(tdot + dt * 32 * BQ + to[k2]), pb[k2], dv[dt]);
        dk[dt] = mfma32(*reinterpret_cast<const bf16x8*>(tqt + dt * 32 * BQ + to[k2]), dsb[k2], dk[dt]);
      }
    softmax(s1, dp1, tl + 32, tn + 32, pb, dsb);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        dv[dt] = mfma32(*reinterpret_cast<const bf16x8*>(tdot + dt * 32 * BQ + to[2 + k2]), pb[k2], dv[dt]);
        dk[dt] = mfma32(*reinterpret_cast<const bf16x8*>(tqt + dt * 32 * BQ + to[2 + k2]), dsb[k2], dk[dt]);
      }
  };

  stage(0, std::integral_constant<int, 0>());
  for (int it = 0; it < niter; it += 2) {
    body(it, std::integral_constant<int, 0>());
    if (it + 1 < niter) body(it + 1, std::integral_constant<int, 1>());
  }

  if (key < a.Lk) {
    bool kvalid = true;
    if (MASK) kvalid = a.mask[b * a.msb + key] != 0;
    bf16* kp = a.dk + b * a.dksb + hk * a.dksh + (int64_t)key * a.dksl;
    bf16* vp = a.dv + b * a.dvsb + hk * a.dvsh + (int64_t)key * a.dvsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 wk = {0u, 0u}, wv = {0u, 0u};
        if (kvalid) {
          wk[0] = pack_bf16x2(dk[dt][4 * g] * a.scale, dk[dt][4 * g + 1] * a.scale);
          wk[1] = pack_bf16x2(dk[dt][4 * g + 2] * a.scale, dk[dt][4 * g + 3] * a.scale);
          wv[0] = pack_bf16x2(dv[dt][4 * g], dv[dt][4 * g + 1]);
          wv[1] = pack_bf16x2(dv[dt][4 * g + 2], dv[dt][4 * g + 3]);
        }
        *reinterpret_cast<u32x2*>(kp + dt * 32 + 8 * g + 4 * hh) = wk;
        *reinterpret_cast<u32x2*>(vp + dt * 32 + 8 * g + 4 * hh) = wv;
      }
  }
}

// ---------------------------------------------------------------------------
// 3. dQ
// ---------------------------------------------------------------------------
// Per wave: 32 query rows (lane % 32 owns query column q0w + lane % 32).  For
// each 32-key tile (lane l supplies key row perm23(l % 32) to the first two
// products):
//   S^T  = K Q^T    A = K rows (LDS)          B = Q^T (registers)
//   dP^T = V dO^T   A = V rows (LDS)          B = dO^T (registers)
//   dS^T = P^T * (dP^T + ndelta[q])           (fp32, key bias masks P^T)
//   dQ^T += K^T dS^T   A = K^T (LDS, head_dim-major)  B = dS^T (C layout reused)
// Tiles come from the padded copies; the body is unrolled over the two LDS
// buffers and branch-free apart from the masked-tile bias.
template <int D>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(BwdArgs a) {
  constexpr int BM = 128, BN = 32, NW = 4;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int TE = BN * D;
  // One LDS object per buffer (see bwd_dkdv_kernel).
  __shared__ __attribute__((aligned(16))) bf16 sk0[TE], sk1[TE];    // K rows: TileLayout<D>
  __shared__ __attribute__((aligned(16))) bf16 sv0[TE], sv1[TE];    // V rows: TileLayout<D>
  __shared__ __attribute__((aligned(16))) bf16 skt0[TE], skt1[TE];  // K^T: D rows of BN keys, TileLayout<BN>
  __shared__ __attribute__((aligned(16))) float sb0[64], sb1[64];   // key bias (this tile and the next)

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int prow = perm23(l32);

  const int nqt = (a.Lq + BM - 1) / BM;
  const int total = nqt * a.B * a.Hq;
  const int bid = xcd_remap(blockIdx.x, total);
  const int qt = bid % nqt;
  const int bh = bid / nqt;
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);

  const int qrow = qt * BM + wave * 32 + l32;
  const bool qvalid = qrow < a.Lq;
  const int64_t srow = (int64_t)bh * a.Lqp + qrow;
  const float lse2 = qvalid ? a.lse2[srow] : kPosInf;
  const float ndelta = qvalid ? a.ndelta[srow] : 0.f;

  bf16x8 qf[KS], df[KS];
  {
    const bf16* qp = a.q + b * a.qsb + h * a.qsh + (int64_t)qrow * a.qsl + 8 * hh;
    const bf16* dp = a.dout + b * a.dosb + h * a.dosh + (int64_t)qrow * a.dosl + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
      if (qvalid) {
        x = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
        y = *reinterpret_cast<const u32x4*>(dp + 16 * ks);
      }
      qf[ks] = bits_to_bf16x8(x);
      df[ks] = bits_to_bf16x8(y);
    }
  }

  const int64_t bhk = (int64_t)(b * a.Hkv + hk);
  const bf16* krbase = a.kr + bhk * a.Lkp * D;
  const bf16* vrbase = a.vr + bhk * a.Lkp * D;
  const bf16* ktbase = a.kt + bhk * D * a.Lkp;
  const float* kbias = a.kbias + (int64_t)b * a.Lkp;
  const int* kfull = a.kfull + (int64_t)b * (a.Lkp / 32);

  DirectStager<BN, D, NW> rst;   // 32 rows of D channels (row stride D)
  DirectStager<D, BN, NW> ktst;  // D rows of 32 keys (row stride Lkp)
  rst.init(D, wave, lane);
  ktst.init(a.Lkp, wave, lane);
  // Stages tile t and loads its "all attended" flag into a register that is
  // consumed one iteration later (after the wait that covers the tile).
  int full_next = 1;
  auto stage = [&](int t, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int k0 = t * BN;
    full_next = kfull[t];
    rst.stage_full(buf == 0 ? sk0 : sk1, krbase + (int64_t)k0 * D, wave);
    rst.stage_full(buf == 0 ? sv0 : sv1, vrbase + (int64_t)k0 * D, wave);
    ktst.stage_full(buf == 0 ? skt0 : skt1, ktbase + k0, wave);
    // 64 biases (this tile and the next; the array is padded to whole
    // 64-key tiles, so k0 + 63 < Lkp for every even tile and the read for an
    // odd last tile stays inside the next batch row or the 64-float pad).
    direct_load4(kbias + k0 + lane, buf == 0 ? sb0 : sb1);
  };

  int ko[KS];  // K/V row perm23(l32), chunk 16*ks + 8*hh
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) ko[ks] = TileLayout<D>::off(prow, 16 * ks + 8 * hh);
  int to[2];  // K^T row l32 (+32*dt), key chunk 16*k2 + 8*hh
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) to[k2] = TileLayout<BN>::off(l32, 16 * k2 + 8 * hh);

  f32x16 dq[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dq[i] = zero16();

  const float c = a.scale_log2;
  const int nkt = (a.Lk + BN - 1) / BN;

  auto body = [&](int t, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    wait_vmem();
    __syncthreads();  // tile t visible in `buf`; tile t-1 fully consumed everywhere
    const int full = __builtin_amdgcn_readfirstlane(full_next);
    stage(min(t + 1, nkt - 1), std::integral_constant<int, buf ^ 1>());
    const bf16* tk = buf == 0 ? sk0 : sk1;
    const bf16* tv = buf == 0 ? sv0 : sv1;
    const bf16* tkt = buf == 0 ? skt0 : skt1;
    const float* tb = buf == 0 ? sb0 : sb1;

    bf16x8 ka[KS], va[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      ka[ks] = *reinterpret_cast<const bf16x8*>(tk + ko[ks]);
      va[ks] = *reinterpret_cast<const bf16x8*>(tv + ko[ks]);
    }
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s = mfma32(ka[ks], qf[ks], s);
      dp = mfma32(va[ks], df[ks], dp);
    }
    // registers 8*k2 + e hold key 16*k2 + 8*hh + e
    if (!full) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 bb = *reinterpret_cast<const f32x4*>(tb + 16 * (g >> 1) + 8 * hh + 4 * (g & 1));
#pragma unroll
        for (int r = 0; r < 4; ++r) s[4 * g + r] += bb[r];
      }
    }
    bf16x8 dsb[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      u32x4 u;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int r = 8 * k2 + 2 * e2;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(s[r], c, -lse2));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(s[r + 1], c, -lse2));
        u[e2] = pack_bf16x2(p0 * (dp[r] + ndelta), p1 * (dp[r + 1] + ndelta));
      }
      dsb[k2] = bits_to_bf16x8(u);
    }
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        dq[dt] = mfma32(*reinterpret_cast<const bf16x8*>(tkt + dt * 32 * BN + to[k2]), dsb[k2], dq[dt]);
  };

  stage(0, std::integral_constant<int, 0>());
  for (int t = 0; t < nkt; t += 2) {
    body(t, std::integral_constant<int, 0>());
    if (t + 1 < nkt) body(t + 1, std::integral_constant<int, 1>());
  }

  if (qvalid) {
    bf16* op = a.dq + b * a.dqsb + h * a.dqsh + (int64_t)qrow * a.dqsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w[0] = pack_bf16x2(dq[dt][4 * g] * a.scale, dq[dt][4 * g + 1] * a.scale);
        w[1] = pack_bf16x2(dq[dt][4 * g + 2] * a.scale, dq[dt][4 * g + 3] * a.scale);
        *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
      }
  }
}

// Zero-fill rows of a strided (B, H, L, D) bf16 tensor (gradients of an empty
// attention).
__global__ void zero_rows_kernel(bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % (D / 8));
    const int64_t row = u / (D / 8);
    const int i = (int)(row % L);
    const int h = (int)((row / L) % H);
    const int b = (int)(row / ((int64_t)L * H));
    *reinterpret_cast<u32x4*>(x + b * sb + h * sh + (int64_t)i * sl + 8 * c) = u32x4{0u, 0u, 0u, 0u};
  }
}

template <int D>
static hipError_t launch_bwd_d(const BwdArgs& a, hipStream_t stream) {
  const bool mask = a.mask != nullptr;
  {
    LaunchTimer timer(kKidTranspose, stream);
    hipError_t e = launch_prep_copies(a.q, a.qsb, a.qsh, a.qsl, a.B, a.Hq, a.Lq, D, a.qr, a.qt, stream);
    if (e == hipSuccess)
      e = launch_prep_copies(a.dout, a.dosb, a.dosh, a.dosl, a.B, a.Hq, a.Lq, D, a.dor, a.dot, stream);
    if (e == hipSuccess) e = launch_prep_copies(a.k, a.ksb, a.ksh, a.ksl, a.B, a.Hkv, a.Lk, D, a.kr, a.kt, stream);
    if (e == hipSuccess) e = launch_prep_copies(a.v, a.vsb, a.vsh, a.vsl, a.B, a.Hkv, a.Lk, D, a.vr, nullptr, stream);
    if (e == hipSuccess) e = launch_key_prep(a.mask, a.msb, a.B, a.Lk, a.kbias, a.kfull, stream);
    if (e != hipSuccess) return e;
  }
  {
    constexpr int RPB = 256 / (D / 8);
    const int64_t rows = (int64_t)a.B * a.Hq * a.Lqp;
    LaunchTimer timer(kKidBwdPre, stream);
    hipLaunchKernelGGL(bwd_pre_kernel<D>, dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, stream, a);
  }
  {
    const int nkt = (a.Lk + 127) / 128;
    const dim3 grid(nkt * a.B * a.Hkv);
    LaunchTimer timer(kKidBwdDkdv, stream);  // 1 workgroup per CU (LDS-bound occupancy)
    if (mask)
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, false>), grid, dim3(256), 0, stream, a);
  }
  {
    const int nqt = (a.Lq + 127) / 128;
    const dim3 grid(nqt * a.B * a.Hq);
    LaunchTimer timer(kKidBwdDq, stream);
    hipLaunchKernelGGL(bwd_dq_kernel<D>, grid, dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdArgs& a, int head_dim, hipStream_t stream) {
  return head_dim == 128 ? launch_bwd_d<128>(a, stream) : launch_bwd_d<64>(a, stream);
}

hipError_t launch_zero_rows(bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                            hipStream_t stream) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  if (units == 0) return hipSuccess;
  const int64_t blocks = (units + 255) / 256;
  hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, stream, x,
                     sb, sh, sl, B, H, L, D);
  return hipGetLastError();
}

}  // namespace avattn
