// 3D rotary embedding kernels: table construction from physical coordinates
// (src/avgen/models/rope.py:218-294) and the interleaved-pair rotation
// (src/avgen/models/rope.py:297-338) with its autograd transpose.  Both are
// HBM-bound elementwise passes; each thread handles 8 channels (16 bytes of
// bf16) so loads and stores are full 128-bit accesses.
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

struct RopeTableArgs {
  const float* coords;
  int64_t csb, csr;
  int B, L, P;
  float inv_freq[64];
  int axis[64];
  int apply_mul[3];
  float pos_mul[3];
  int apply_div[3];
  float pos_div[3];
  float* cos_out;
  float* sin_out;
};

// One thread per (b, i, pair).  The position goes through the same fp32
// operations, in the same order, as the reference: optional multiply by
// time_scale, optional division by the linear factor, then one product
// with the pair's inverse frequency.
__global__ __launch_bounds__(256) void rope_tables_kernel(RopeTableArgs a) {
  const int64_t n = (int64_t)a.B * a.L * a.P;
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < n; u += (int64_t)gridDim.x * blockDim.x) {
    const int p = (int)(u % a.P);
    const int64_t bi = u / a.P;
    const int i = (int)(bi % a.L);
    const int b = (int)(bi / a.L);
    const int ax = a.axis[p];
    float pos = a.coords[b * a.csb + (int64_t)i * a.csr + ax];
    if (a.apply_mul[ax]) pos = __fmul_rn(pos, a.pos_mul[ax]);
    if (a.apply_div[ax]) pos = __fdiv_rn(pos, a.pos_div[ax]);
    const float ang = __fmul_rn(pos, a.inv_freq[p]);
    a.cos_out[u] = cosf(ang);
    a.sin_out[u] = sinf(ang);
  }
}

__global__ __launch_bounds__(256) void rope_apply_kernel(const bf16* __restrict__ x, int64_t xsb, int64_t xsh,
                                                         int64_t xsl, int B, int H, int L, int D,
                                                         const float* __restrict__ ct, const float* __restrict__ st,
                                                         int64_t tsb, int inverse, bf16* __restrict__ out,
                                                         int64_t osb, int64_t osh, int64_t osl) {
  const int cpr = D / 8;  // 16-byte chunks per row
  const int64_t n = (int64_t)B * H * L * cpr;
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < n; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % cpr);
    const int64_t row = u / cpr;
    const int i = (int)(row % L);
    const int h = (int)((row / L) % H);
    const int b = (int)(row / ((int64_t)L * H));
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + b * xsb + h * xsh + (int64_t)i * xsl + 8 * c);
    const int64_t t = b * tsb + (int64_t)i * (D / 2) + 4 * c;
    const f32x4 cs = *reinterpret_cast<const f32x4*>(ct + t);
    const f32x4 sn = *reinterpret_cast<const f32x4*>(st + t);
    *reinterpret_cast<u32x4*>(out + b * osb + h * osh + (int64_t)i * osl + 8 * c) = rotate8(v, cs, sn, inverse != 0);
  }
}

static int grid_for(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return (int)(blocks < 1 ? 1 : (blocks > 16384 ? 16384 : blocks));
}

hipError_t launch_rope_tables(const float* coords, int64_t csb, int64_t csr, int B, int L, int P,
                              const float* inv_freq, const int32_t* axis_of_pair, const int32_t* apply_mul,
                              const float* pos_mul, const int32_t* apply_div, const float* pos_div, float* cos_out,
                              float* sin_out, hipStream_t stream) {
  RopeTableArgs a;
  a.coords = coords;
  a.csb = csb;
  a.csr = csr;
  a.B = B;
  a.L = L;
  a.P = P;
  for (int p = 0; p < 64; ++p) {
    a.inv_freq[p] = p < P ? inv_freq[p] : 0.f;
    a.axis[p] = p < P ? axis_of_pair[p] : 0;
  }
  for (int ax = 0; ax < 3; ++ax) {
    a.apply_mul[ax] = apply_mul[ax];
    a.pos_mul[ax] = pos_mul[ax];
    a.apply_div[ax] = apply_div[ax];
    a.pos_div[ax] = pos_div[ax];
  }
  a.cos_out = cos_out;
  a.sin_out = sin_out;
  const int64_t n = (int64_t)B * L * P;
  if (n == 0) return hipSuccess;
  LaunchTimer timer(kKidRopeTables, stream);
  hipLaunchKernelGGL(rope_tables_kernel, dim3(grid_for(n)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_rope_apply(const bf16* x, int64_t xsb, int64_t xsh, int64_t xsl, int B, int H, int L, int D,
                             const float* cos_tab, const float* sin_tab, int64_t tsb, bool inverse, bf16* out,
                             int64_t osb, int64_t osh, int64_t osl, hipStream_t stream) {
  const int64_t n = (int64_t)B * H * L * (D / 8);
  if (n == 0) return hipSuccess;
  LaunchTimer timer(kKidRopeApply, stream);
  hipLaunchKernelGGL(rope_apply_kernel, dim3(grid_for(n)), dim3(256), 0, stream, x, xsb, xsh, xsl, B, H, L, D,
                     cos_tab, sin_tab, tsb, inverse ? 1 : 0, out, osb, osh, osl);
  return hipGetLastError();
}

}  // namespace avattn
