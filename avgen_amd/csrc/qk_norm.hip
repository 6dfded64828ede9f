// Per-head RMSNorm of q or k rows fused with the interleaved-pair rotation:
// the steps between the q/k projections and the attention kernel
// (src/avgen/models/layers.py:530-536: q_norm/k_norm, then apply_rotary),
// and their backward.
//
// Forward, per row of head_dim values (torch's F.rms_norm with a bf16 gain,
// src/avgen/models/layers.py:106-118, then src/avgen/models/rope.py:297-338):
//   rstd = 1/sqrt(mean(x^2) + eps)            (fp32)
//   n    = bf16((x * rstd) * w)               (the norm's bf16 output)
//   y    = bf16(rotate(n, cos, sin))          (fp32 rotation, as rotate8)
// Backward, given dy:
//   g    = bf16(rotate^T(dy))                 (the rotation's autograd grad)
//   xh   = x * rstd,  wg = w * g
//   dx   = bf16(rstd * (wg - xh * mean(wg * xh)))
//   dw   = sum over rows of g * xh            (fp32, per-block partials then
//                                              one reduction: deterministic)
// One row is D/8 lanes holding 16 bytes each, so every access is a full
// 128-bit load or store; a wave takes one token and its heads, so the
// token's rotation tables are read once, not once per head.  HBM-bound: one
// read and one write of the rows (two reads in the backward).
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

namespace {

constexpr int kNormThreads = 64;      // one wave per token: D/8 lanes per head row, 64/(D/8) heads at a time
constexpr int kNormBwdBlocks = 4096;  // fixed grid of the backward: dW partials per block

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f[2 * p] = __uint_as_float(v[p] << 16);
    f[2 * p + 1] = __uint_as_float(v[p] & 0xffff0000u);
  }
}

// Sum over the R lanes of one row (consecutive lanes, R a power of two).
template <int R>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int off = R / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ void load_gain(const bf16* w, int c, float* out) {
  if (w) {
    unpack8(*reinterpret_cast<const u32x4*>(w + 8 * c), out);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = 1.f;
  }
}

}  // namespace

// Token-major: a wave takes token (b, i), loads this lane's 4 cos / 4 sin
// values once, and normalises the token's rows head by head (64/(D/8)
// heads per pass; for a (batch, seq, heads, dim) layout those rows are one
// contiguous run).
template <int D>
__global__ __launch_bounds__(kNormThreads) void qk_norm_fwd_kernel(QkNormArgs a) {
#pragma clang fp contract(off)
  constexpr int R = D / 8;
  constexpr int HPW = kNormThreads / R;
  const int c = threadIdx.x % R, hg = threadIdx.x / R;
  float w[8];
  load_gain(a.w, c, w);
  const int64_t ntok = (int64_t)a.B * a.L;
  for (int64_t tok = blockIdx.x; tok < ntok; tok += gridDim.x) {
    const int b = (int)(tok / a.L), i = (int)(tok % a.L);
    f32x4 cs, sn;
    if (a.ct) {
      const int64_t t = b * a.tsb + (int64_t)i * (D / 2) + 4 * c;
      cs = *reinterpret_cast<const f32x4*>(a.ct + t);
      sn = *reinterpret_cast<const f32x4*>(a.st + t);
    }
    // The next pass's row is loaded before this pass's arithmetic.
    const bf16* xrow = a.x + b * a.xsb + (int64_t)i * a.xsl + 8 * c;
    u32x4 xn{};
    if (hg < a.H) xn = *reinterpret_cast<const u32x4*>(xrow + hg * a.xsh);
    for (int h = hg; h < a.H; h += HPW) {  // uniform over the row's lanes
      const u32x4 xv = xn;
      if (h + HPW < a.H) xn = *reinterpret_cast<const u32x4*>(xrow + (h + HPW) * a.xsh);
      float x[8];
      unpack8(xv, x);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
      ss = row_sum<R>(ss);
      const float rstd = 1.f / __builtin_sqrtf(ss / (float)D + a.eps);
      u32x4 n;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float t0 = x[2 * p] * rstd, t1 = x[2 * p + 1] * rstd;
        n[p] = pack_bf16x2(t0 * w[2 * p], t1 * w[2 * p + 1]);
      }
      if (a.ct) n = rotate8(n, cs, sn, false);
      *reinterpret_cast<u32x4*>(a.out + b * a.osb + h * a.osh + (int64_t)i * a.osl + 8 * c) = n;
    }
  }
}

template <int D>
__global__ __launch_bounds__(kNormThreads) void qk_norm_bwd_kernel(QkNormArgs a) {
#pragma clang fp contract(off)
  constexpr int R = D / 8;
  constexpr int HPW = kNormThreads / R;
  __shared__ float red[HPW][D];
  const int c = threadIdx.x % R, hg = threadIdx.x / R;
  float w[8], dw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) dw[j] = 0.f;
  load_gain(a.w, c, w);
  const int64_t ntok = (int64_t)a.B * a.L;
  for (int64_t tok = blockIdx.x; tok < ntok; tok += gridDim.x) {
    const int b = (int)(tok / a.L), i = (int)(tok % a.L);
    f32x4 cs, sn;
    if (a.ct) {
      const int64_t t = b * a.tsb + (int64_t)i * (D / 2) + 4 * c;
      cs = *reinterpret_cast<const f32x4*>(a.ct + t);
      sn = *reinterpret_cast<const f32x4*>(a.st + t);
    }
    // The next pass's rows are loaded before this pass's arithmetic.
    const bf16* xrow = a.x + b * a.xsb + (int64_t)i * a.xsl + 8 * c;
    const bf16* grow = a.dy + b * a.dsb + (int64_t)i * a.dsl + 8 * c;
    u32x4 xn{}, gn{};
    if (hg < a.H) {
      xn = *reinterpret_cast<const u32x4*>(xrow + hg * a.xsh);
      gn = *reinterpret_cast<const u32x4*>(grow + hg * a.dsh);
    }
    for (int h = hg; h < a.H; h += HPW) {
      float x[8], g[8];
      const u32x4 xv = xn;
      u32x4 gv = gn;
      if (h + HPW < a.H) {
        xn = *reinterpret_cast<const u32x4*>(xrow + (h + HPW) * a.xsh);
        gn = *reinterpret_cast<const u32x4*>(grow + (h + HPW) * a.dsh);
      }
      unpack8(xv, x);
      if (a.ct) gv = rotate8(gv, cs, sn, true);
      unpack8(gv, g);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
      ss = row_sum<R>(ss);
      const float rstd = 1.f / __builtin_sqrtf(ss / (float)D + a.eps);
      float xh[8], wg[8], dot = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xh[j] = x[j] * rstd;
        wg[j] = w[j] * g[j];
        dot += wg[j] * xh[j];
        dw[j] += g[j] * xh[j];
      }
      const float m = row_sum<R>(dot) / (float)D;
      u32x4 dx;
#pragma unroll
      for (int p = 0; p < 4; ++p)
        dx[p] = pack_bf16x2(rstd * (wg[2 * p] - xh[2 * p] * m), rstd * (wg[2 * p + 1] - xh[2 * p + 1] * m));
      *reinterpret_cast<u32x4*>(a.dx + b * a.xgb + h * a.xgh + (int64_t)i * a.xgl + 8 * c) = dx;
    }
  }
  if (!a.wpart) return;  // uniform: no gain, no dW
#pragma unroll
  for (int j = 0; j < 8; ++j) red[hg][8 * c + j] = dw[j];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kNormThreads) {
    float s = 0.f;
    for (int r = 0; r < HPW; ++r) s += red[r][d];
    a.wpart[(int64_t)blockIdx.x * D + d] = s;
  }
}

// dw[d] = sum over the backward's blocks of their partials: one workgroup
// per d, each thread a strided share of the partials, then a tree over the
// threads (a fixed order, so the result is the same on every run).
__global__ __launch_bounds__(256) void qk_norm_dw_kernel(const float* __restrict__ part, int nblocks, int D,
                                                         float* __restrict__ dw) {
  __shared__ float red[256];
  const int d = blockIdx.x;
  float s = 0.f;
  for (int k = threadIdx.x; k < nblocks; k += 256) s += part[(int64_t)k * D + d];
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) dw[d] = red[0];
}

__global__ __launch_bounds__(128) void qk_norm_dw_zero_kernel(int D, float* __restrict__ dw) {
  if ((int)threadIdx.x < D) dw[threadIdx.x] = 0.f;
}

hipError_t launch_qk_norm_dw_zero(float* dw, int D, hipStream_t stream) {
  hipLaunchKernelGGL(qk_norm_dw_zero_kernel, dim3(1), dim3(128), 0, stream, D, dw);
  return hipGetLastError();
}

size_t qk_norm_bwd_workspace_bytes(int D) { return (size_t)kNormBwdBlocks * D * sizeof(float); }

static int norm_grid(int64_t tokens, int cap) {
  return (int)(tokens < 1 ? 1 : (tokens > cap ? cap : tokens));
}

hipError_t launch_qk_norm(const QkNormArgs& a, int D, hipStream_t stream) {
  const int64_t tokens = (int64_t)a.B * a.L;
  if (tokens == 0 || a.H == 0) return hipSuccess;
  LaunchTimer timer(kKidQkNorm, stream);
  const dim3 grid(norm_grid(tokens, 1 << 20)), block(kNormThreads);
  if (D == 128)
    hipLaunchKernelGGL(qk_norm_fwd_kernel<128>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(qk_norm_fwd_kernel<64>, grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_qk_norm_bwd(const QkNormArgs& a, int D, float* dw, hipStream_t stream) {
  const int64_t tokens = (int64_t)a.B * a.L;
  if (tokens == 0 || a.H == 0) return hipSuccess;
  const int nb = norm_grid(tokens, kNormBwdBlocks);
  {
    LaunchTimer timer(kKidQkNormBwd, stream);
    if (D == 128)
      hipLaunchKernelGGL(qk_norm_bwd_kernel<128>, dim3(nb), dim3(kNormThreads), 0, stream, a);
    else
      hipLaunchKernelGGL(qk_norm_bwd_kernel<64>, dim3(nb), dim3(kNormThreads), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (!a.wpart) return hipSuccess;
  hipLaunchKernelGGL(qk_norm_dw_kernel, dim3(D), dim3(256), 0, stream, a.wpart, nb, D, dw);
  return hipGetLastError();
}

}  // namespace avattn
