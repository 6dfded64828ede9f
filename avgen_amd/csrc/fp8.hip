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
// One thread per 16 channels (32 bytes in, 16 bytes out).
template <int D>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const bf16* __restrict__ x, int64_t sb, int64_t sh,
                                                            int64_t sl, int B, int H, int L, int Lp,
                                                            const float* __restrict__ scale,
                                                            uint8_t* __restrict__ out) {
  constexpr int CPR = D / 16;
  const int64_t units = (int64_t)B * H * Lp * CPR;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % CPR);
    const int64_t row = u / CPR;
    const int i = (int)(row % Lp);
    const int bh = (int)(row / Lp);
    const int h = bh % H, b = bh / H;
    u32x4 o = {0u, 0u, 0u, 0u};
    if (i < L) {
      const float inv = 1.f / scale[h];
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
    *reinterpret_cast<u32x4*>(out + row * D + 16 * c) = o;
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
                                const float* scale, uint8_t* out, hipStream_t stream) {
  const int Lp = transpose_padded_len(L);
  const int64_t units = (int64_t)B * H * Lp * (D / 16);
  if (units == 0) return hipSuccess;
  int64_t blocks = (units + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (D == 128)
    hipLaunchKernelGGL(quantize_rows_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, stream, x, sb, sh, sl, B, H, L,
                       Lp, scale, out);
  else
    hipLaunchKernelGGL(quantize_rows_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, stream, x, sb, sh, sl, B, H, L,
                       Lp, scale, out);
  return hipGetLastError();
}

}  // namespace avattn
