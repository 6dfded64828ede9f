// Attention backward for gfx950, recomputing the probabilities from (q, k,
// lse) instead of storing them.  Three launches, no atomics (bitwise
// reproducible):
//   1. preprocess: delta = rowsum(dout * out) and lse2 = lse * log2(e) per
//      query row (the `D` term of dS = P * (dP - D));
//   2. dK/dV: one workgroup per 128 keys (32 per wave, kept in registers as
//      MFMA operands); loops over 64-row query tiles of every query head
//      that reads this KV head;
//   3. dQ: one workgroup per 128 query rows (32 per wave); loops over 64-key
//      tiles.
// Tiles live in LDS row-major only; the transposed operands (Q^T, dO^T,
// K^T) come from ds_read_b64_tr_b16 reads of the same tiles.  Each step
// works on two independent 32-row halves so the MFMA chains of one half
// overlap the softmax-gradient VALU work of the other.
// With out/lse the merged result over all KV chunks, the outputs are one
// chunk's contributions, which is how the ring backward calls the op
// (torch/.../_context_parallel/_attention.py:567-575).
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

// ---------------------------------------------------------------------------
// 1. delta / lse2
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdArgs a) {
  constexpr int TPR = D / 8;  // threads per row
  constexpr int RPB = 256 / TPR;
  const int64_t rows = (int64_t)a.B * a.Hq * a.Lq;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int c = threadIdx.x % TPR;
  float acc = 0.f;
  if (row < rows) {
    const int i = (int)(row % a.Lq);
    const int h = (int)((row / a.Lq) % a.Hq);
    const int b = (int)(row / ((int64_t)a.Lq * a.Hq));
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
    a.delta[row] = acc;
    const float l = a.lse[row];
    a.lse2[row] = (l == kNegInf) ? kPosInf : l * kLog2e;
  }
}

// ---------------------------------------------------------------------------
// 2. dK / dV
// ---------------------------------------------------------------------------
// Per wave: 32 keys (lane % 32 owns key column k0w + lane % 32).  For each
// 32-row half of a 64-row query tile:
//   S  = Q K^T    A = Q rows (LDS)             B = K^T (registers)
//   dP = dO V^T   A = dO rows (LDS)            B = V^T (registers)
//   P  = exp2(S*c - lse2[q]),  dS = P * (dP - delta[q])        (fp32)
//   dV^T += dO^T P   A = dO^T (LDS, tr read)   B = P  (C layout reused)
//   dK^T += Q^T dS   A = Q^T  (LDS, tr read)   B = dS (C layout reused)
// The C layout of S puts query 8*(r/4) + 4*hh + r%4 in register r; the
// 16-row k-step k2 uses registers 8*k2 + e for slot (hh, e) <-> query
// 16*k2 + 8*(e/4) + 4*hh + e%4, which is the order tr_operand reads.
template <int D, bool MASK>
__global__ __launch_bounds__(256, 1) void bwd_dkdv_kernel(BwdArgs a) {
  constexpr int BK = 128, BQ = 64, NT = 256;
  constexpr int KS = D / 16, DT = D / 32;
  using Tile = RowTile<BQ, D, NT>;
  __shared__ __attribute__((aligned(16))) bf16 sq[2][Tile::kElems];
  __shared__ __attribute__((aligned(16))) bf16 sdo[2][Tile::kElems];
  __shared__ __attribute__((aligned(16))) float slse[2][BQ];
  __shared__ __attribute__((aligned(16))) float sdel[2][BQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;

  const int nkt = (a.Lk + BK - 1) / BK;
  const int total = nkt * a.B * a.Hkv;
  const int bid = xcd_remap(blockIdx.x, total);
  const int kt = bid % nkt;
  const int bhk = bid / nkt;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.Hq / a.Hkv;

  const int key = kt * BK + wave * 32 + l32;
  bool kvalid = key < a.Lk;
  if (MASK && kvalid) kvalid = a.mask[b * a.msb + key] != 0;

  bf16x8 kf[KS], vf[KS];
  {
    const bool in = key < a.Lk;
    const bf16* kp = a.k + b * a.ksb + hk * a.ksh + (int64_t)key * a.ksl + 8 * hh;
    const bf16* vp = a.v + b * a.vsb + hk * a.vsh + (int64_t)key * a.vsl + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
      if (in) {
        x = *reinterpret_cast<const u32x4*>(kp + 16 * ks);
        y = *reinterpret_cast<const u32x4*>(vp + 16 * ks);
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

  const int nqt = (a.Lq + BQ - 1) / BQ;
  const int niter = nqt * group;
  Tile qreg, oreg;
  float stat_reg = 0.f;

  auto load_tile = [&](int it) {
    const int hq = hk * group + it / nqt;
    const int q0 = (it % nqt) * BQ;
    const int rows = min(BQ, a.Lq - q0);
    qreg.load(a.q + b * a.qsb + hq * a.qsh + (int64_t)q0 * a.qsl, a.qsl, rows, tid);
    oreg.load(a.dout + b * a.dosb + hq * a.dosh + (int64_t)q0 * a.dosl, a.dosl, rows, tid);
    // Row statistics: threads [0, 64) lse2, [64, 128) delta.
    if (tid < 2 * BQ) {
      const int i = tid % BQ;
      const int64_t row = ((int64_t)(b * a.Hq + hq)) * a.Lq + q0 + i;
      if (tid < BQ)
        stat_reg = (i < rows) ? a.lse2[row] : kPosInf;
      else
        stat_reg = (i < rows) ? a.delta[row] : 0.f;
    }
  };
  auto store_tile = [&](int buf) {
    qreg.store(sq[buf], tid);
    oreg.store(sdo[buf], tid);
    if (tid < BQ)
      slse[buf][tid] = stat_reg;
    else if (tid < 2 * BQ)
      sdel[buf][tid - BQ] = stat_reg;
  };

  const float c = a.scale_log2;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int it = 0; it < niter; ++it) {
    const int buf = it & 1;
    if (it + 1 < niter) load_tile(it + 1);
    const bf16* tq = sq[buf];
    const bf16* tdo = sdo[buf];

    f32x16 s[2], dp[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      s[sub] = zero16();
      dp[sub] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 qa = row_operand<D>(tq, sub * 32 + l32, 16 * ks + 8 * hh);
        const bf16x8 da = row_operand<D>(tdo, sub * 32 + l32, 16 * ks + 8 * hh);
        s[sub] = mfma32(qa, kf[ks], s[sub]);
        dp[sub] = mfma32(da, vf[ks], dp[sub]);
      }
    }

    bf16x8 pb[2][2], dsb[2][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        u32x4 up, ud;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          // registers 8*k2 + 4*half + [0,4) hold queries
          // 32*sub + 16*k2 + 8*half + 4*hh + [0,4)
          const int g = 2 * k2 + half;
          const f32x4 l2 = *reinterpret_cast<const f32x4*>(&slse[buf][sub * 32 + 8 * g + 4 * hh]);
          const f32x4 dl = *reinterpret_cast<const f32x4*>(&sdel[buf][sub * 32 + 8 * g + 4 * hh]);
          float p[4], ds[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pr = kvalid ? __builtin_amdgcn_exp2f(fmaf(s[sub][4 * g + r], c, -l2[r])) : 0.f;
            p[r] = pr;
            ds[r] = pr * (dp[sub][4 * g + r] - dl[r]);
          }
          up[2 * half] = pack_bf16x2(p[0], p[1]);
          up[2 * half + 1] = pack_bf16x2(p[2], p[3]);
          ud[2 * half] = pack_bf16x2(ds[0], ds[1]);
          ud[2 * half + 1] = pack_bf16x2(ds[2], ds[3]);
        }
        pb[sub][k2] = bits_to_bf16x8(up);
        dsb[sub][k2] = bits_to_bf16x8(ud);
      }

#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int r0 = sub * 32 + 16 * k2;
          const bf16x8 da = tr_operand<D>(tdo, r0, dt * 32, lane);
          const bf16x8 qa = tr_operand<D>(tq, r0, dt * 32, lane);
          dv[dt] = mfma32(da, pb[sub][k2], dv[dt]);
          dk[dt] = mfma32(qa, dsb[sub][k2], dk[dt]);
        }

    if (it + 1 < niter) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (key < a.Lk) {
    bf16* kp = a.dk + b * a.dksb + hk * a.dksh + (int64_t)key * a.dksl;
    bf16* vp = a.dv + b * a.dvsb + hk * a.dvsh + (int64_t)key * a.dvsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 wk, wv;
        wk[0] = pack_bf16x2(dk[dt][4 * g] * a.scale, dk[dt][4 * g + 1] * a.scale);
        wk[1] = pack_bf16x2(dk[dt][4 * g + 2] * a.scale, dk[dt][4 * g + 3] * a.scale);
        wv[0] = pack_bf16x2(dv[dt][4 * g], dv[dt][4 * g + 1]);
        wv[1] = pack_bf16x2(dv[dt][4 * g + 2], dv[dt][4 * g + 3]);
        *reinterpret_cast<u32x2*>(kp + dt * 32 + 8 * g + 4 * hh) = wk;
        *reinterpret_cast<u32x2*>(vp + dt * 32 + 8 * g + 4 * hh) = wv;
      }
  }
}

// ---------------------------------------------------------------------------
// 3. dQ
// ---------------------------------------------------------------------------
// Per wave: 32 query rows (lane % 32 owns query column q0w + lane % 32).  For
// each 32-key half of a 64-key tile:
//   S^T  = K Q^T    A = K rows (LDS)          B = Q^T (registers)
//   dP^T = V dO^T   A = V rows (LDS)          B = dO^T (registers)
//   dS^T = P^T * (dP^T - delta[q])            (fp32, key bias masks P^T)
//   dQ^T += K^T dS^T   A = K^T (LDS, tr read)  B = dS^T (C layout reused)
#ifndef AVATTN_DQ_BN
#define AVATTN_DQ_BN 32  // keys per dQ step: 32 or 64 (two 32-key halves)
#endif

template <int D, bool MASK>
__global__ __launch_bounds__(256, AVATTN_DQ_BN == 64 ? 1 : 2) void bwd_dq_kernel(BwdArgs a) {
  constexpr int BM = 128, BN = AVATTN_DQ_BN, NT = 256, NSUB = BN / 32;
  constexpr int KS = D / 16, DT = D / 32;
  using Tile = RowTile<BN, D, NT>;
  __shared__ __attribute__((aligned(16))) bf16 sk[2][Tile::kElems];
  __shared__ __attribute__((aligned(16))) bf16 sv[2][Tile::kElems];
  __shared__ __attribute__((aligned(16))) float sbias[2][BN];
  __shared__ int sfull[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;

  const int nqt = (a.Lq + BM - 1) / BM;
  const int total = nqt * a.B * a.Hq;
  const int bid = xcd_remap(blockIdx.x, total);
  const int qt = bid % nqt;
  const int bh = bid / nqt;
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);

  const int qrow = qt * BM + wave * 32 + l32;
  const bool qvalid = qrow < a.Lq;
  const int64_t srow = (int64_t)bh * a.Lq + qrow;
  const float lse2 = qvalid ? a.lse2[srow] : kPosInf;
  const float delta = qvalid ? a.delta[srow] : 0.f;

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

  const bf16* kbase = a.k + b * a.ksb + hk * a.ksh;
  const bf16* vbase = a.v + b * a.vsb + hk * a.vsh;
  const uint8_t* mbase = MASK ? a.mask + b * a.msb : nullptr;

  Tile kreg, vreg;
  float bias_reg = 0.f;

  auto load_tile = [&](int t) {
    const int k0 = t * BN;
    const int rows = min(BN, a.Lk - k0);
    kreg.load(kbase + (int64_t)k0 * a.ksl, a.ksl, rows, tid);
    vreg.load(vbase + (int64_t)k0 * a.vsl, a.vsl, rows, tid);
    if (tid < BN) {
      bool valid = tid < rows;
      if (MASK && valid) valid = mbase[k0 + tid] != 0;
      bias_reg = valid ? 0.f : kNegInf;
    }
  };
  auto store_tile = [&](int buf) {
    kreg.store(sk[buf], tid);
    vreg.store(sv[buf], tid);
    if (tid < 64) {
      if (tid < BN) sbias[buf][tid] = bias_reg;
      const unsigned long long ball = __ballot(tid >= BN || bias_reg == 0.f);
      if (tid == 0) sfull[buf] = (ball == ~0ull) ? 1 : 0;
    }
  };

  f32x16 dq[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dq[i] = zero16();

  const float c = a.scale_log2;
  const int nkt = (a.Lk + BN - 1) / BN;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < nkt; ++t) {
    const int buf = t & 1;
    if (t + 1 < nkt) load_tile(t + 1);
    const bf16* tk = sk[buf];
    const bf16* tv = sv[buf];

    f32x16 s[NSUB], dp[NSUB];
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      s[sub] = zero16();
      dp[sub] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 ka = row_operand<D>(tk, sub * 32 + l32, 16 * ks + 8 * hh);
        const bf16x8 va = row_operand<D>(tv, sub * 32 + l32, 16 * ks + 8 * hh);
        s[sub] = mfma32(ka, qf[ks], s[sub]);
        dp[sub] = mfma32(va, df[ks], dp[sub]);
      }
    }
    if (!sfull[buf]) {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bb = *reinterpret_cast<const f32x4*>(&sbias[buf][sub * 32 + 8 * g + 4 * hh]);
#pragma unroll
          for (int r = 0; r < 4; ++r) s[sub][4 * g + r] += bb[r];
        }
    }
    bf16x8 dsb[NSUB][2];
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        u32x4 u;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int r = 8 * k2 + 2 * e2;
          const float p0 = __builtin_amdgcn_exp2f(fmaf(s[sub][r], c, -lse2));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(s[sub][r + 1], c, -lse2));
          u[e2] = pack_bf16x2(p0 * (dp[sub][r] - delta), p1 * (dp[sub][r + 1] - delta));
        }
        dsb[sub][k2] = bits_to_bf16x8(u);
      }
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 ka = tr_operand<D>(tk, sub * 32 + 16 * k2, dt * 32, lane);
          dq[dt] = mfma32(ka, dsb[sub][k2], dq[dt]);
        }

    if (t + 1 < nkt) store_tile(buf ^ 1);
    __syncthreads();
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
    constexpr int RPB = 256 / (D / 8);
    const int64_t rows = (int64_t)a.B * a.Hq * a.Lq;
    LaunchTimer timer(kKidBwdPre, stream);
    hipLaunchKernelGGL(bwd_pre_kernel<D>, dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, stream, a);
  }
  {
    const int nkt = (a.Lk + 127) / 128;
    const dim3 grid(nkt * a.B * a.Hkv);
    LaunchTimer timer(kKidBwdDkdv, stream);
    if (mask)
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, false>), grid, dim3(256), 0, stream, a);
  }
  {
    const int nqt = (a.Lq + 127) / 128;
    const dim3 grid(nqt * a.B * a.Hq);
    LaunchTimer timer(kKidBwdDq, stream);
    if (mask)
      hipLaunchKernelGGL((bwd_dq_kernel<D, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((bwd_dq_kernel<D, false>), grid, dim3(256), 0, stream, a);
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
