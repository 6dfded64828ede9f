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

#ifndef AVATTN_FWD_QH
#define AVATTN_FWD_QH 1  // 32-row query halves per wave (1 or 2)
#endif

// QH = query halves per wave: each wave owns 32*QH query rows and reuses every
// K/V operand it reads from LDS for all of them (QH = 2 halves the LDS reads
// per MFMA and gives the scheduler two independent softmax/MFMA chains).
template <int D, bool MASK, bool ROPE, int QH>
__global__ __launch_bounds__(256, QH == 1 ? 2 : 1) void attn_fwd_kernel(FwdArgs a) {
  constexpr int BM = 128 * QH, BN = 64, NT = 256;
  constexpr int KS = D / 16;  // 16-channel k-steps of q k^T
  constexpr int DT = D / 32;  // 32-channel row tiles of O^T
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

  int qrow[QH];
  bool qvalid[QH];
#pragma unroll
  for (int qh = 0; qh < QH; ++qh) {
    qrow[qh] = qt * BM + (wave * QH + qh) * 32 + l32;
    qvalid[qh] = qrow[qh] < a.Lq;
  }

  // Q fragments: B operand of S^T = K Q^T; lane holds row qrow, channels
  // 16*ks + 8*hh + [0, 8).
  bf16x8 qf[QH][KS];
#pragma unroll
  for (int qh = 0; qh < QH; ++qh) {
    const bf16* qp = a.q + b * a.qsb + h * a.qsh + (int64_t)qrow[qh] * a.qsl + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (qvalid[qh]) {
        x = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
        if constexpr (ROPE) {
          const int64_t t = b * a.rsb + (int64_t)qrow[qh] * (D / 2) + 8 * ks + 4 * hh;
          const f32x4 c = *reinterpret_cast<const f32x4*>(a.cos_q + t);
          const f32x4 s = *reinterpret_cast<const f32x4*>(a.sin_q + t);
          x = rotate8(x, c, s, false);
        }
      }
      qf[qh][ks] = bits_to_bf16x8(x);
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
    if (tid < BN) {
      sbias[buf][tid] = bias_reg;
      const unsigned long long ball = __ballot(bias_reg == 0.f);
      if (tid == 0) sfull[buf] = (ball == ~0ull) ? 1 : 0;
    }
  };

  const float c = a.scale_log2;
  // Lazy rescaling: the reference max m_run only moves when a tile's max
  // exceeds it by more than 8 in log2 units, so probabilities stay <= 2^8
  // (exact in fp32/bf16 range) and the O rescale is rare after the first
  // tile.  The result is the same softmax; only roundings differ.
  const float tau = 8.f / c;
  float m_run[QH], l_run[QH][2];
  f32x16 acc[QH][DT];
#pragma unroll
  for (int qh = 0; qh < QH; ++qh) {
    m_run[qh] = kNegInf;  // reference max of raw scores for this lane's query
    l_run[qh][0] = l_run[qh][1] = 0.f;  // this lane's share of the row sum
#pragma unroll
    for (int i = 0; i < DT; ++i) acc[qh][i] = zero16();
  }

  const int nkt = (a.Lk + BN - 1) / BN;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < nkt; ++t) {
    const int buf = t & 1;
    if (t + 1 < nkt) load_tile(t + 1);
    const bf16* kl = sk[buf];
    const bf16* vl = sv[buf];
    const bool full = sfull[buf] != 0;

    // S^T for the two 32-key halves: s[qh][sub][r] is the score of key
    // 32*sub + 8*(r/4) + 4*hh + r%4 against this lane's query of half qh.
    f32x16 s[QH][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int qh = 0; qh < QH; ++qh) s[qh][sub] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kf = row_operand<D>(kl, sub * 32 + l32, 16 * ks + 8 * hh);
#pragma unroll
        for (int qh = 0; qh < QH; ++qh) s[qh][sub] = mfma32(kf, qf[qh][ks], s[qh][sub]);
      }
    }

    bf16x8 pf[QH][2][2];
#pragma unroll
    for (int qh = 0; qh < QH; ++qh) {
      if (!full) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 bb = *reinterpret_cast<const f32x4*>(&sbias[buf][sub * 32 + 8 * g + 4 * hh]);
#pragma unroll
            for (int r = 0; r < 4; ++r) s[qh][sub][4 * g + r] += bb[r];
          }
      }
      float mx = kNegInf;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qh][sub][r]);
      mx = halves_max(mx);
      if (mx > m_run[qh] + tau) {
        // New reference max (both lanes of a query agree: mx is shared).
        const float alpha = __builtin_amdgcn_exp2f((m_run[qh] - mx) * c);
        l_run[qh][0] *= alpha;
        l_run[qh][1] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[qh][dt][r] *= alpha;
        m_run[qh] = mx;
      }
      const float mc = (m_run[qh] == kNegInf) ? 0.f : m_run[qh] * c;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          u32x4 u;
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int r = 8 * k2 + 2 * e2;
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[qh][sub][r], c, -mc));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[qh][sub][r + 1], c, -mc));
            l_run[qh][e2 & 1] += p0 + p1;
            u[e2] = pack_bf16x2(p0, p1);
          }
          pf[qh][sub][k2] = bits_to_bf16x8(u);
        }
    }

    // O^T += V^T P^T.  B operand slot (hh, e) of pf[qh][sub][k2] is key
    // 32*sub + 16*k2 + 8*(e/4) + 4*hh + e%4; tr_operand reads V^T in that
    // key order from the row-major V tile.
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 va = tr_operand<D>(vl, sub * 32 + 16 * k2, dt * 32, lane);
#pragma unroll
          for (int qh = 0; qh < QH; ++qh) acc[qh][dt] = mfma32(va, pf[qh][sub][k2], acc[qh][dt]);
        }

    if (t + 1 < nkt) store_tile(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int qh = 0; qh < QH; ++qh) {
    const float l_tot = halves_sum(l_run[qh][0] + l_run[qh][1]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qvalid[qh]) {
      if (hh == 0) {
        const float lse = l_tot > 0.f ? fmaf(m_run[qh], a.scale, logf(l_tot)) : kNegInf;
        a.lse[(int64_t)bh * a.Lq + qrow[qh]] = lse;
      }
      bf16* op = a.o + b * a.osb + h * a.osh + (int64_t)qrow[qh] * a.osl;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 w;
          w[0] = pack_bf16x2(acc[qh][dt][4 * g] * inv, acc[qh][dt][4 * g + 1] * inv);
          w[1] = pack_bf16x2(acc[qh][dt][4 * g + 2] * inv, acc[qh][dt][4 * g + 3] * inv);
          *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
        }
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
  constexpr int QH = AVATTN_FWD_QH;
  const int nqt = (a.Lq + 128 * QH - 1) / (128 * QH);
  const dim3 grid(nqt * a.B * a.Hq);
  const dim3 block(256);
  const bool mask = a.mask != nullptr;
  const bool rope = a.cos_q != nullptr;
  LaunchTimer timer(kKidFwd, stream);
  if (mask && rope)
    hipLaunchKernelGGL((attn_fwd_kernel<D, true, true, QH>), grid, block, 0, stream, a);
  else if (mask)
    hipLaunchKernelGGL((attn_fwd_kernel<D, true, false, QH>), grid, block, 0, stream, a);
  else if (rope)
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, true, QH>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<D, false, false, QH>), grid, block, 0, stream, a);
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
