// Operand preparation for the attention kernels: padded copies of the
// sequence tensors and the padded key bias.
//
// The attention kernels stream sequence tiles through LDS with direct
// global->LDS loads.  Two kinds of copy of a (B, H, L, D) strided tensor are
// made here, once per call, each padded with zeros to Lp = L rounded up to a
// whole 64-row tile (transpose_padded_len), so that every tile load is a
// full, branch-free load with loop-invariant per-lane offsets and padded
// positions hold finite values:
//   rows: xr[((b*H + h)*Lp + i)*D + d] = x[b, h, i, d]      (row-major)
//   cols: xt[((b*H + h)*D + d)*Lp + i] = x[b, h, i, d]      (head_dim-major)
// The head_dim-major copy serves the products that contract over the
// sequence (O += P V, dV += P^T dO, dK += dS^T Q, dQ += dS K): their MFMA
// operand then has its k index along a contiguous row and is one 16-byte LDS
// read, instead of transpose reads, which run at a fraction of the rate on
// gfx950.  Each copy is HBM-bound: one read of x, one write per copy.
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

// One workgroup copies 64 sequence rows x D channels of one (b, h), rotating
// each row first when rotation tables are given (the copies then hold the
// rotated rows src/avgen/models/rope.py:332-338 produces).  With
// rowmax2 set, it also writes the largest squared norm of its (valid) rows to
// rowmax2[(b*H + h)*(Lp/64) + tile] as float bits (one plain store per
// workgroup; an atomic per wave into one word per head serialised badly).
template <int D>
__global__ __launch_bounds__(256) void prep_copies_kernel(const bf16* __restrict__ x, int64_t sb, int64_t sh,
                                                          int64_t sl, int H, int L, int Lp, bf16* __restrict__ xr,
                                                          bf16* __restrict__ xt, uint32_t* __restrict__ rowmax2,
                                                          const float* __restrict__ ct, const float* __restrict__ st,
                                                          int64_t tsb) {
  constexpr int S = 64;       // sequence rows per workgroup
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  constexpr int LD = D + 2;   // LDS row pitch in bf16 (odd word count: column reads spread over banks)
  __shared__ bf16 tile[S * LD];
  const int tid = threadIdx.x;
  const int ntiles = Lp / S;
  const int s0 = (blockIdx.x % ntiles) * S;
  const int bh = blockIdx.x / ntiles;
  const int b = bh / H, h = bh % H;
  const bf16* src = x + b * sb + h * sh;

  // Load 64 rows (zeros past L) as 16-byte chunks; write the row-major copy
  // and scatter into the pitched tile for the head_dim-major one.
  float nmax = 0.f;  // largest squared row norm seen by this thread's rows
#pragma unroll
  for (int i = 0; i < S * CPR / 256; ++i) {
    const int c = tid + i * 256;
    const int row = c / CPR, ch = c % CPR;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (s0 + row < L) {
      v = *reinterpret_cast<const u32x4*>(src + (int64_t)(s0 + row) * sl + ch * 8);
      if (ct) {
        // Channels 8*ch .. +7 are pairs 4*ch .. +3 of row s0 + row.
        const int64_t t = b * tsb + (int64_t)(s0 + row) * (D / 2) + 4 * ch;
        v = rotate8(v, *reinterpret_cast<const f32x4*>(ct + t), *reinterpret_cast<const f32x4*>(st + t), false);
      }
    }
    if (xr) *reinterpret_cast<u32x4*>(xr + ((int64_t)bh * Lp + s0 + row) * D + ch * 8) = v;
    uint32_t* dst = reinterpret_cast<uint32_t*>(tile + row * LD + ch * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) dst[w] = v[w];
    if (rowmax2) {
      // A row's CPR chunks sit in CPR consecutive lanes: sum their squares.
      float n = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) n = fmaf(bf16_lo(v[w]), bf16_lo(v[w]), fmaf(bf16_hi(v[w]), bf16_hi(v[w]), n));
#pragma unroll
      for (int off = 1; off < CPR; off <<= 1) n += __shfl_xor(n, off);
      nmax = fmaxf(nmax, n);
    }
  }
  if (rowmax2) {
    __shared__ float wmax[4];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) nmax = fmaxf(nmax, __shfl_xor(nmax, off));
    if ((tid & 63) == 0) wmax[tid >> 6] = nmax;
    __syncthreads();
    if (tid == 0) rowmax2[blockIdx.x] = __float_as_uint(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
  }
  if (!xt) return;
  __syncthreads();

  // Each thread writes 16-byte chunks of head_dim-major rows: 8 consecutive
  // sequence positions of one channel.
  bf16* dst = xt + (int64_t)bh * D * Lp + s0;
#pragma unroll
  for (int i = 0; i < D * (S / 8) / 256; ++i) {
    const int c = tid + i * 256;
    const int d = c / (S / 8), j = c % (S / 8);
    u32x4 v;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint16_t lo = __builtin_bit_cast(uint16_t, tile[(8 * j + 2 * w) * LD + d]);
      const uint16_t hi = __builtin_bit_cast(uint16_t, tile[(8 * j + 2 * w + 1) * LD + d]);
      v[w] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<u32x4*>(dst + (int64_t)d * Lp + 8 * j) = v;
  }
}

// Key bias and tile flags: kbias[b*Lkp + j] = 0 if key j < Lk is attended
// (mask nonzero, or no mask) else -inf, for j < Lkp; kfull[b*(Lkp/32) + t] = 1
// if all 32 keys of tile t are attended.  One thread per 32-key tile.
__global__ __launch_bounds__(256) void key_prep_kernel(const uint8_t* __restrict__ mask, int64_t msb, int B, int Lk,
                                                       int Lkp, float* __restrict__ kbias, int* __restrict__ kfull) {
  const int tiles = Lkp / 32;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)B * tiles) return;
  const int b = (int)(t / tiles), j0 = (int)(t % tiles) * 32;
  int all = 1;
  for (int j = j0; j < j0 + 32; ++j) {
    const bool valid = j < Lk && (mask == nullptr || mask[b * msb + j] != 0);
    kbias[(int64_t)b * Lkp + j] = valid ? 0.f : kNegInf;
    all &= valid ? 1 : 0;
  }
  kfull[t] = all;
}

hipError_t launch_key_prep(const uint8_t* mask, int64_t msb, int B, int Lk, float* kbias, int* kfull,
                           hipStream_t stream) {
  const int Lkp = transpose_padded_len(Lk);
  const int64_t n = (int64_t)B * (Lkp / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(key_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, mask, msb, B, Lk, Lkp,
                     kbias, kfull);
  return hipGetLastError();
}

hipError_t launch_prep_copies(const bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                              bf16* xr, bf16* xt, hipStream_t stream, uint32_t* rowmax2, const float* cos_t,
                              const float* sin_t, int64_t tsb) {
  const int Lp = transpose_padded_len(L);
  if ((int64_t)B * H == 0 || Lp == 0 || (!xr && !xt)) return hipSuccess;
  const int64_t blocks = (int64_t)(Lp / 64) * B * H;
  if (blocks > 2147483647) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks);
  if (D == 128)
    hipLaunchKernelGGL(prep_copies_kernel<128>, grid, dim3(256), 0, stream, x, sb, sh, sl, H, L, Lp, xr, xt, rowmax2,
                       cos_t, sin_t, tsb);
  else
    hipLaunchKernelGGL(prep_copies_kernel<64>, grid, dim3(256), 0, stream, x, sb, sh, sl, H, L, Lp, xr, xt, rowmax2,
                       cos_t, sin_t, tsb);
  return hipGetLastError();
}

// dq = transposed rotation of bf16(acc): the ring's fp32 dq sum cast to the
// input dtype (torch/.../_context_parallel/_attention.py:636) followed by the
// rotation's backward (src/avgen/models/rope.py:332-338 through autograd),
// in one pass.  One thread per 8 channels of a row.
__global__ __launch_bounds__(256) void dq_finish_kernel(const float* __restrict__ acc, int64_t asb, int64_t ash,
                                                        int64_t asl, int H, int L, int D, const float* __restrict__ ct,
                                                        const float* __restrict__ st, int64_t tsb,
                                                        bf16* __restrict__ dq, int64_t dsb, int64_t dsh, int64_t dsl,
                                                        int64_t units) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const int cpr = D / 8;
  const int c = (int)(u % cpr);
  const int64_t row = u / cpr;
  const int i = (int)(row % L);
  const int h = (int)((row / L) % H);
  const int b = (int)(row / ((int64_t)L * H));
  const float* ap = acc + b * asb + h * ash + (int64_t)i * asl + 8 * c;
  const f32x4 lo = *reinterpret_cast<const f32x4*>(ap);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(ap + 4);
  u32x4 w = {pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]), pack_bf16x2(hi[0], hi[1]),
             pack_bf16x2(hi[2], hi[3])};
  if (ct) {
    const int64_t t = b * tsb + (int64_t)i * (D / 2) + 4 * c;
    w = rotate8(w, *reinterpret_cast<const f32x4*>(ct + t), *reinterpret_cast<const f32x4*>(st + t), true);
  }
  *reinterpret_cast<u32x4*>(dq + b * dsb + h * dsh + (int64_t)i * dsl + 8 * c) = w;
}

hipError_t launch_dq_finish(const float* acc, int64_t asb, int64_t ash, int64_t asl, int B, int H, int L, int D,
                            const float* cos_t, const float* sin_t, int64_t tsb, bf16* dq, int64_t dsb, int64_t dsh,
                            int64_t dsl, hipStream_t stream) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  if (units == 0) return hipSuccess;
  const int64_t blocks = (units + 255) / 256;
  if (blocks > 2147483647) return hipErrorInvalidValue;
  LaunchTimer timer(kKidDqFinish, stream);
  hipLaunchKernelGGL(dq_finish_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, acc, asb, ash, asl, H, L, D,
                     cos_t, sin_t, tsb, dq, dsb, dsh, dsl, units);
  return hipGetLastError();
}

}  // namespace avattn
