// Diagnostic: the dQ accumulation a backward without staged dS would need.
//
// A dK/dV workgroup owns one 128-key block and visits every 64-row query
// tile; without staging dS, its contribution to dQ is one 64 x D fp32
// partial tile per (key block, query tile), to be summed over the key
// blocks.  This kernel replays exactly that traffic pattern with synthetic
// partials (every value 1.0) and nothing else, so its time is what the
// accumulation alone costs: either with fp32 vector atomics into one
// (heads, tiles, 64, D) accumulator (what a fused backward would issue), or
// as plain stores of the same bytes (the rate the memory system gives
// without read-modify-write).  Launch shape of the dK/dV kernel: one
// 512-thread workgroup per (head, key block), mapped so that consecutive
// key blocks of a head share an XCD; block kb starts at query tile 2*kb
// (mod tiles) so concurrently running workgroups hit different tiles.
#include "avattn.h"
#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {
namespace {

template <int D, bool ATOMIC>
__global__ __launch_bounds__(512) void diag_dq_partials_kernel(float* __restrict__ acc, int heads, int key_blocks,
                                                               int tiles, int tiles_per_block) {
  constexpr int TILE = 64 * D;  // floats per partial tile
  const int total = heads * key_blocks;
  const int bid = xcd_remap(blockIdx.x, total);
  const int h = bid / key_blocks, kb = bid % key_blocks;
  for (int i = 0; i < tiles_per_block; ++i) {
    const int t = (i + 2 * kb) % tiles;
    float* p = acc + ((int64_t)h * tiles + t) * TILE + threadIdx.x;
#pragma unroll
    for (int j = 0; j < TILE / 512; ++j) {
      if constexpr (ATOMIC)
        __hip_atomic_fetch_add(p + 512 * j, 1.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        p[512 * j] = 1.f;
    }
  }
}

}  // namespace
}  // namespace avattn

using namespace avattn;

extern "C" int avattn_diag_dq_partials(float* acc, int32_t heads, int32_t key_blocks, int32_t query_tiles,
                                       int32_t tiles_per_block, int32_t head_dim, int32_t atomic,
                                       avattn_stream_t stream) {
  if (!acc) return AVATTN_ERR_NULL_POINTER;
  if (heads <= 0 || key_blocks <= 0 || query_tiles <= 0 || tiles_per_block <= 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim != 64 && head_dim != 128) return AVATTN_ERR_HEAD_DIM;
  if (tiles_per_block > query_tiles) return AVATTN_ERR_ARGUMENT;
  if ((int64_t)heads * key_blocks > (1 << 30)) return AVATTN_ERR_TOO_LARGE;
  if (reinterpret_cast<uintptr_t>(acc) & 15u) return AVATTN_ERR_LAYOUT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(heads * key_blocks)), block(512);
  LaunchTimer timer(kKidDiag, s);
  if (head_dim == 128) {
    if (atomic)
      hipLaunchKernelGGL((diag_dq_partials_kernel<128, true>), grid, block, 0, s, acc, heads, key_blocks, query_tiles,
                         tiles_per_block);
    else
      hipLaunchKernelGGL((diag_dq_partials_kernel<128, false>), grid, block, 0, s, acc, heads, key_blocks,
                         query_tiles, tiles_per_block);
  } else {
    if (atomic)
      hipLaunchKernelGGL((diag_dq_partials_kernel<64, true>), grid, block, 0, s, acc, heads, key_blocks, query_tiles,
                         tiles_per_block);
    else
      hipLaunchKernelGGL((diag_dq_partials_kernel<64, false>), grid, block, 0, s, acc, heads, key_blocks,
                         query_tiles, tiles_per_block);
  }
  return hipGetLastError() == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH;
}
