// Flash-style attention forward for gfx950: one workgroup = 128 query rows of
// one (batch, head); four waves own 32 rows each; K/V stream through LDS in
// 64-key row-major tiles, double-buffered (V^T operands come from LDS
// transpose reads).
//
// Per wave and tile the scores are computed transposed, S^T = K Q^T, so that
// each lane owns one query column (query = lane % 32) and holds 32 of that
// query's 64 scores: the row max and row sum are in-lane plus one exchange
// with the partner lane (lane ^ 32).  The probabilities, in the MFMA C
// layout, are exactly the B operand of O^T += V^T P^T, so P never leaves
// registers.  Q stays in registers for the whole kernel (optionally rotated
// on load, src/avgen/models/rope.py:332-338).  Softmax runs in the exp2
// domain on raw scores with a running max; the LSE is natural-log
// (aten::_scaled_dot_product_flash_attention's logsumexp output).
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

// One workgroup = 128 query rows, 4 waves x 32 rows; K/V tiles of 64 keys.
//
// Per tile the waves issue both 32-key halves' QK^T MFMAs, then run each
// half's softmax on the VALU while the other half's MFMAs (QK^T of half 1,
// then PV of half 0) execute.  K and V are double-buffered in LDS: right
// after the barrier that opens iteration t, tile t+1 is loaded straight from
// global memory into buffer (t+1)%2 (tile t-1 was fully consumed before that
// barrier) and lands before the next one.  One barrier per tile.
template <int D, bool MASK, bool ROPE>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(FwdArgs a) {
  constexpr int BM = 128, BN = 64, NW = 4;
  constexpr int KS = D / 16;  // 16-channel k-steps of q k^T
  constexpr int DT = D / 32;  // 32-channel row tiles of O^T
  constexpr int TE = BN * D;  // tile elements
  __shared__ __attribute__((aligned(16))) bf16 sk[2][TE];
  __shared__ __attribute__((aligned(16))) bf16 sv[2][TE];
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

  const bf16* kbase = a.k + b * a.ksb + hk * a.ksh;
  const bf16* vbase = a.v + b * a.vsb + hk * a.vsh;
  const uint8_t* mbase = MASK ? a.mask + b * a.msb : nullptr;
  const int nkt = (a.Lk + BN - 1) / BN;

  DirectStager<BN, D, NW> kst, vst;
  kst.init(a.ksl, wave, lane);
  vst.init(a.vsl, wave, lane);
  // Key bias of tile t (0 or -inf) into sbias[t & 1]; wave 0 only.
  float bias_reg = 0.f;
  auto load_bias = [&](int t) {
    if (wave == 0) {
      const int key = t * BN + lane;
      bool valid = key < a.Lk;
      if (MASK && valid) valid = mbase[key] != 0;
      bias_reg = valid ? 0.f : kNegInf;
    }
  };
  auto store_bias = [&](int t) {
    if (wave == 0) {
      sbias[t & 1][lane] = bias_reg;
      const unsigned long long ball = __ballot(bias_reg == 0.f);
      if (lane == 0) sfull[t & 1] = (ball == ~0ull) ? 1 : 0;
    }
  };

  // Prologue loads, then Q (rotated on load) while they fly.
  kst.stage(sk[0], kbase, a.ksl, min(BN, a.Lk), wave, lane);
  vst.stage(sv[0], vbase, a.vsl, min(BN, a.Lk), wave, lane);
  load_bias(0);

  // Q fragments: B operand of S^T = K Q^T; lane holds row qrow, channels
  // 16*ks + 8*hh + [0, 8).
  bf16x8 qf[KS];
  {
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

  // S^T of one 32-key half of a tile: s[r] is the score of key
  // 32*half + 8*(r/4) + 4*hh + r%4 against this lane's query.
  auto scores = [&](const bf16* kl, int half) {
    f32x16 s = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s = mfma32(row_operand<D>(kl, half * 32 + l32, 16 * ks + 8 * hh), qf[ks], s);
    return s;
  };

  const float c = a.scale_log2;
  // Lazy rescaling: the reference max m_run only moves when a half-tile's
  // max exceeds it by more than 8 in log2 units, so probabilities stay
  // <= 2^8 (exact in fp32/bf16 range) and the O rescale is rare after the
  // first tiles.  The result is the same softmax; only roundings differ.
  const float tau = 8.f / c;
  float m_run = kNegInf;             // reference max of raw scores for this lane's query
  float l_run0 = 0.f, l_run1 = 0.f;  // this lane's share of the row sum
  f32x16 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = zero16();

  wait_vmem();
  store_bias(0);

  for (int t = 0; t < nkt; ++t) {
    const int buf = t & 1;
    wait_vmem();
    __syncthreads();  // K(t), V(t), bias(t) visible; tile t-1 fully consumed everywhere
    if (t + 1 < nkt) {
      const int k1 = (t + 1) * BN;
      kst.stage(sk[buf ^ 1], kbase + (int64_t)k1 * a.ksl, a.ksl, min(BN, a.Lk - k1), wave, lane);
      vst.stage(sv[buf ^ 1], vbase + (int64_t)k1 * a.vsl, a.vsl, min(BN, a.Lk - k1), wave, lane);
      load_bias(t + 1);
    }
    const bf16* kl = sk[buf];
    const bf16* vl = sv[buf];
    const bool full = sfull[buf] != 0;

    // Both halves' QK^T MFMAs are issued up front; the softmax of half 0
    // then runs on the VALU while half 1's MFMAs execute, and the softmax of
    // half 1 while half 0's PV MFMAs execute.
    f32x16 sh[2];
    sh[0] = scores(kl, 0);
    sh[1] = scores(kl, 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f32x16& s_cur = sh[hf];
      if (!full) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bb = *reinterpret_cast<const f32x4*>(&sbias[buf][hf * 32 + 8 * g + 4 * hh]);
#pragma unroll
          for (int r = 0; r < 4; ++r) s_cur[4 * g + r] += bb[r];
        }
      }
      float mx = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_cur[r]);
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
      const float mc = (m_run == kNegInf) ? 0.f : m_run * c;

      bf16x8 pf[2];
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        u32x4 u;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int r = 8 * k2 + 2 * e2;
          const float p0 = __builtin_amdgcn_exp2f(fmaf(s_cur[r], c, -mc));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(s_cur[r + 1], c, -mc));
          if (e2 & 1)
            l_run1 += p0 + p1;
          else
            l_run0 += p0 + p1;
          u[e2] = pack_bf16x2(p0, p1);
        }
        pf[k2] = bits_to_bf16x8(u);
      }

      // O^T += V^T P^T.  B operand slot (hh, e) of pf[k2] is key
      // 32*hf + 16*k2 + 8*(e/4) + 4*hh + e%4; tr_operand reads V^T in that
      // key order from the row-major V tile.
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          acc[dt] = mfma32(tr_operand<D>(vl, hf * 32 + 16 * k2, dt * 32, lane), pf[k2], acc[dt]);
    }

    if (t + 1 < nkt) store_bias(t + 1);
  }

  const float l_tot = halves_sum(l_run0 + l_run1);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qvalid) {
    if (hh == 0) {
      const float lse = l_tot > 0.f ? fmaf(m_run, a.scale, logf(l_tot)) : kNegInf;
      a.lse[(int64_t)bh * a.Lq + qrow] = lse;
    }
    bf16* op = a.o + b * a.osb + h * a.osh + (int64_t)qrow * a.osl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w[0] = pack_bf16x2(acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv);
        w[1] = pack_bf16x2(acc[dt][4 * g + 2] * inv, acc[dt][4 * g + 3] * inv);
        *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
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
  const int nqt = (a.Lq + 127) / 128;
  const dim3 grid(nqt * a.B * a.Hq);
  const dim3 block(256);
  const bool mask = a.mask != nullptr;
  const bool rope = a.cos_q != nullptr;
  LaunchTimer timer(kKidFwd, stream);
  if (mask && rope)
    hipLaunchKernelGGL((attn_fwd_kernel<D, true, true>), grid, block, 0, stream, a);
  else if (mask)
    hipLaunchKernelGGL((attn_fwd_kernel<D, true, false>), grid, block, 0, stream, a);
  else if (rope)
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, false>), grid, block, 0, stream, a);
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
