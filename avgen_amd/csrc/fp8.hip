// fp8 (OCP e4m3) operand preparation for the fp8-QK^T forward.
//
// Per-head absmax scaling: scale[h] = max |x[b, h, i, d]| / 448 over every
// batch, position and channel of head h (1 for an all-zero head), so that
// x / scale[h] spans [-448, 448], the finite range of e4m3; a value is
// quantized as e4m3(x * (1 / scale[h])) with one fp32 multiply by the
// correctly rounded fp32 reciprocal and round-to-nearest-even conversion, and
// dequantized by multiplying with scale[h].  The scores then come out as
// (q8 . k8) * q_scale[h] * k_scale[hk].
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

constexpr float kE4m3Max = 448.f;

// Bit patterns of non-negative floats order like the floats, so the running
// per-head maximum is kept as an unsigned atomic max on the bits.
__global__ __launch_bounds__(256) void absmax_clear_kernel(uint32_t* bits, int H) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < H) bits[i] = 0u;
}

// Grid (blocks, H): each workgroup folds a strided share of head h's
// 16-byte chunks (8 bf16) into one maximum.
__global__ __launch_bounds__(256) void absmax_kernel(const bf16* __restrict__ x, int64_t sb, int64_t sh, int64_t sl,
                                                     int B, int L, int D, uint32_t* __restrict__ bits) {
  const int h = blockIdx.y;
  const int cpr = D / 8;
  const int64_t units = (int64_t)B * L * cpr;
  float m = 0.f;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % cpr);
    const int64_t r = u / cpr;
    const int i = (int)(r % L), b = (int)(r / L);
    const u32x4 w = *reinterpret_cast<const u32x4*>(x + b * sb + h * sh + (int64_t)i * sl + 8 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16_lo(w[j])), fabsf(bf16_hi(w[j]))));
  }
  // Wave maximum, then one atomic per wave.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) atomicMax(bits + h, __float_as_uint(m));
}

__global__ __launch_bounds__(256) void absmax_finish_kernel(const uint32_t* bits, float* scale, int H) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < H) {
    const float m = __uint_as_float(bits[i]);
    scale[i] = m > 0.f ? m / kE4m3Max : 1.f;
  }
}

// Row-major e4m3 copy of x (B, H, L, D) strided, zero rows past L:
// out[((b*H + h)*Lp + i)*D + d] = e4m3(x[b, h, i, d] * (1 / scale[h])).
// One workgroup per 64 rows of one (b, h), one thread per 16 channels of a
// row (32 bytes in, 16 bytes out).  With rowmax2 set it also writes the
// largest squared norm of its tile's quantized rows (in e4m3 units, summed
// in fp32) to rowmax2[(b*H + h)*(Lp/64) + tile] as float bits: the key-side
// factor of the score bound the fp8 forward uses.
template <int D>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const bf16* __restrict__ x, int64_t sb, int64_t sh,
                                                            int64_t sl, int H, int L, int Lp,
                                                            const float* __restrict__ scale,
                                                            uint8_t* __restrict__ out,
                                                            uint32_t* __restrict__ rowmax2) {
  constexpr int CPR = D / 16;     // threads per row
  constexpr int RPP = 256 / CPR;  // rows per pass
  __shared__ float wmax[4];
  const int ntiles = Lp / 64;
  const int tile = blockIdx.x % ntiles;
  const int bh = blockIdx.x / ntiles;
  const int h = bh % H, b = bh / H;
  const int c = threadIdx.x % CPR;
  const float inv = 1.f / scale[h];
  float nmax = 0.f;
#pragma unroll
  for (int r0 = 0; r0 < 64; r0 += RPP) {
    const int i = tile * 64 + r0 + threadIdx.x / CPR;
    u32x4 o = {0u, 0u, 0u, 0u};
    if (i < L) {
      const bf16* src = x + b * sb + h * sh + (int64_t)i * sl + 16 * c;
      const u32x4 w0 = *reinterpret_cast<const u32x4*>(src);
      const u32x4 w1 = *reinterpret_cast<const u32x4*>(src + 8);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        o[j] = pack_fp8x4(bf16_lo(w0[2 * j]) * inv, bf16_hi(w0[2 * j]) * inv, bf16_lo(w0[2 * j + 1]) * inv,
                          bf16_hi(w0[2 * j + 1]) * inv);
        o[2 + j] = pack_fp8x4(bf16_lo(w1[2 * j]) * inv, bf16_hi(w1[2 * j]) * inv, bf16_lo(w1[2 * j + 1]) * inv,
                              bf16_hi(w1[2 * j + 1]) * inv);
      }
    }
    *reinterpret_cast<u32x4*>(out + ((int64_t)bh * Lp + i) * D + 16 * c) = o;
    if (rowmax2) {
      float s2 = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v0 = __builtin_amdgcn_cvt_f32_fp8((int)o[j], 0);
        const float v1 = __builtin_amdgcn_cvt_f32_fp8((int)o[j], 1);
        const float v2 = __builtin_amdgcn_cvt_f32_fp8((int)o[j], 2);
        const float v3 = __builtin_amdgcn_cvt_f32_fp8((int)o[j], 3);
        s2 = fmaf(v0, v0, s2);
        s2 = fmaf(v1, v1, s2);
        s2 = fmaf(v2, v2, s2);
        s2 = fmaf(v3, v3, s2);
      }
#pragma unroll
      for (int off = CPR / 2; off > 0; off >>= 1) s2 += __shfl_xor(s2, off, CPR);
      nmax = fmaxf(nmax, s2);
    }
  }
  if (rowmax2) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) nmax = fmaxf(nmax, __shfl_xor(nmax, off));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = nmax;
    __syncthreads();
    if (threadIdx.x == 0) rowmax2[blockIdx.x] = __float_as_uint(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
  }
}

hipError_t launch_absmax_scales(const bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                                float* scale, uint32_t* bits, hipStream_t stream) {
  if (H == 0) return hipSuccess;
  LaunchTimer timer(kKidAbsmax, stream);
  const unsigned hb = (unsigned)((H + 255) / 256);
  hipLaunchKernelGGL(absmax_clear_kernel, dim3(hb), dim3(256), 0, stream, bits, H);
  const int64_t units = (int64_t)B * L * (D / 8);
  if (units > 0) {
    // About 2048 workgroups in all: enough to fill the chip, few atomics.
    int64_t per = (2048 + H - 1) / H;
    const int64_t need = (units + 255) / 256;
    if (per > need) per = need;
    if (per > 65535) per = 65535;
    hipLaunchKernelGGL(absmax_kernel, dim3((unsigned)per, (unsigned)H), dim3(256), 0, stream, x, sb, sh, sl, B, L, D,
                       bits);
  }
  hipLaunchKernelGGL(absmax_finish_kernel, dim3(hb), dim3(256), 0, stream, bits, scale, H);
  return hipGetLastError();
}

hipError_t launch_quantize_rows(const bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                                const float* scale, uint8_t* out, uint32_t* rowmax2, hipStream_t stream) {
  const int Lp = transpose_padded_len(L);
  const int64_t blocks = (int64_t)B * H * (Lp / 64);
  if (blocks == 0) return hipSuccess;
  if (D == 128)
    hipLaunchKernelGGL(quantize_rows_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, stream, x, sb, sh, sl, H, L,
                       Lp, scale, out, rowmax2);
  else
    hipLaunchKernelGGL(quantize_rows_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, stream, x, sb, sh, sl, H, L, Lp,
                       scale, out, rowmax2);
  return hipGetLastError();
}

}  // namespace avattn
