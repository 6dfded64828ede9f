// Online-softmax merge of a chunk's (out, lse) into the running accumulator,
// the ring-attention merge step of torch/.../_context_parallel/_attention.py
// :182-183, in fp32:
//   out <- out - sigmoid(lse_b - lse) * (out - out_b)
//   lse <- lse - logsigmoid(lse - lse_b)
// sigmoid and logsigmoid use the same closed forms as PyTorch's elementwise
// kernels: 1 / (1 + exp(-x)) and min(x, 0) - log1p(exp(-|x|)).
// An LSE of -inf (a row with every key masked) is the identity element; a NaN
// LSE (a row whose scores held a NaN) merges through the formula and stays
// NaN (lse_merge_coeffs).
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

template <int D, bool BLK_BF16>
__global__ __launch_bounds__(256) void lse_merge_kernel(float* __restrict__ out, float* __restrict__ lse,
                                                        const void* __restrict__ out_b_raw,
                                                        const float* __restrict__ lse_b, int64_t rows) {
  constexpr int TPR = D / 8;  // 8 channels per thread
  constexpr int RPB = 256 / TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int c = threadIdx.x % TPR;
  if (row >= rows) return;
  const float la = lse[row];
  const float lb = lse_b[row];
  float o[8], ob[8];
  float* op = out + row * D + 8 * c;
  *reinterpret_cast<f32x4*>(&o[0]) = *reinterpret_cast<const f32x4*>(op);
  *reinterpret_cast<f32x4*>(&o[4]) = *reinterpret_cast<const f32x4*>(op + 4);
  if constexpr (BLK_BF16) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const bf16*>(out_b_raw) + row * D + 8 * c);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      ob[2 * w] = __uint_as_float(v[w] << 16);
      ob[2 * w + 1] = __uint_as_float(v[w] & 0xffff0000u);
    }
  } else {
    const float* bp = reinterpret_cast<const float*>(out_b_raw) + row * D + 8 * c;
    *reinterpret_cast<f32x4*>(&ob[0]) = *reinterpret_cast<const f32x4*>(bp);
    *reinterpret_cast<f32x4*>(&ob[4]) = *reinterpret_cast<const f32x4*>(bp + 4);
  }
  int mode;
  float w;
  const float nl = lse_merge_coeffs(la, lb, mode, w);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = lse_merge_elem(o[j], ob[j], mode, w);
  *reinterpret_cast<f32x4*>(op) = *reinterpret_cast<const f32x4*>(&o[0]);
  *reinterpret_cast<f32x4*>(op + 4) = *reinterpret_cast<const f32x4*>(&o[4]);
  // Every thread of the row has read lse[row] above (same wave, program
  // order), so the write cannot race with those reads.
  if (c == 0) lse[row] = nl;
}

template <int D>
static void launch_merge_d(float* out, float* lse, const void* ob, const float* lb, int64_t rows, bool bf,
                           hipStream_t stream) {
  constexpr int RPB = 256 / (D / 8);
  const dim3 grid((unsigned)((rows + RPB - 1) / RPB));
  LaunchTimer timer(kKidMerge, stream);
  if (bf)
    hipLaunchKernelGGL((lse_merge_kernel<D, true>), grid, dim3(256), 0, stream, out, lse, ob, lb, rows);
  else
    hipLaunchKernelGGL((lse_merge_kernel<D, false>), grid, dim3(256), 0, stream, out, lse, ob, lb, rows);
}

hipError_t launch_lse_merge(float* out_acc, float* lse_acc, const void* out_blk, const float* lse_blk, int64_t rows,
                            int D, bool blk_bf16, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (D == 128)
    launch_merge_d<128>(out_acc, lse_acc, out_blk, lse_blk, rows, blk_bf16, stream);
  else
    launch_merge_d<64>(out_acc, lse_acc, out_blk, lse_blk, rows, blk_bf16, stream);
  return hipGetLastError();
}

}  // namespace avattn
