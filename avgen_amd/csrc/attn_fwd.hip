// Flash-style attention forward for gfx950: one workgroup = 128 query rows of
// one (batch, head); four waves own 32 rows each; K/V stream through LDS in
// 64-key tiles, double-buffered.
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

template <int D, bool MASK, bool ROPE>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(FwdArgs a) {
  constexpr int BM = 128, BN = 64, NT = 256;
  constexpr int KS = D / 16;  // 16-channel k-steps of q k^T
  constexpr int DT = D / 32;  // 32-channel row tiles of O^T
  using KTile = RowTile<BN, D, NT>;
  using VTile = TransTile<BN, D, NT>;
  __shared__ __attribute__((aligned(16))) bf16 sk[2][BN * KTile::kStride];
  __shared__ __attribute__((aligned(16))) bf16 svt[2][D * VTile::kStride];
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

  const bf16* kbase = a.k + b * a.ksb + hk * a.ksh;
  const bf16* vbase = a.v + b * a.vsb + hk * a.vsh;
  const uint8_t* mbase = MASK ? a.mask + b * a.msb : nullptr;

  KTile kreg;
  VTile vreg;
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
    vreg.store(svt[buf], tid);
    if (tid < BN) {
      sbias[buf][tid] = bias_reg;
      const unsigned long long ball = __ballot(bias_reg == 0.f);
      if (tid == 0) sfull[buf] = (ball == ~0ull) ? 1 : 0;
    }
  };

  const float c = a.scale_log2;
  float m_run = kNegInf;  // running max of raw scores for this lane's query
  float l_run = 0.f;      // this lane's share of the running row sum
  f32x16 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = zero16();

  const int nkt = (a.Lk + BN - 1) / BN;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < nkt; ++t) {
    const int buf = t & 1;
    if (t + 1 < nkt) load_tile(t + 1);
    const bf16* kl = sk[buf];
    const bf16* vl = svt[buf];

    // S^T for the two 32-key halves: s[sub][r] is the score of key
    // 32*sub + 8*(r/4) + 4*hh + r%4 against this lane's query.
    f32x16 s[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      s[sub] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kf =
            *reinterpret_cast<const bf16x8*>(kl + (sub * 32 + l32) * KTile::kStride + 16 * ks + 8 * hh);
        s[sub] = mfma32(kf, qf[ks], s[sub]);
      }
    }
    if (!sfull[buf]) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bb = *reinterpret_cast<const f32x4*>(&sbias[buf][sub * 32 + 8 * g + 4 * hh]);
#pragma unroll
          for (int r = 0; r < 4; ++r) s[sub][4 * g + r] += bb[r];
        }
    }

    float mx = kNegInf;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sub][r]);
    mx = halves_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * c);
    const float mc = m_use * c;

    float rs = 0.f;
    bf16x8 pf[2][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        u32x4 u;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int r = 8 * k2 + 2 * e2;
          const float p0 = __builtin_amdgcn_exp2f(fmaf(s[sub][r], c, -mc));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(s[sub][r + 1], c, -mc));
          rs += p0 + p1;
          u[e2] = pack_bf16x2(p0, p1);
        }
        pf[sub][k2] = bits_to_bf16x8(u);
      }
    l_run = l_run * alpha + rs;
    m_run = m_new;
    if (alpha != 1.f) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    }

    // O^T += V^T P^T.  B operand slot (hh, e) of pf[sub][k2] is key
    // 32*sub + 16*k2 + 8*(e/4) + 4*hh + e%4; the A operand reads the same keys
    // of channel row d from the transposed V tile.
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16* vr = vl + (dt * 32 + l32) * VTile::kStride + sub * 32 + 16 * k2 + 4 * hh;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vr);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + 8);
          acc[dt] = mfma32(cat4(lo, hi), pf[sub][k2], acc[dt]);
        }

    if (t + 1 < nkt) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = halves_sum(l_run);
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
