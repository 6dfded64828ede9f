// C ABI entry points (include/avattn.h): argument validation, then kernel
// launches on the caller's stream.  Validation happens before any HIP call, so
// a rejected call touches no device state.
#include "avattn.h"

#include <math.h>

#include <mutex>

#include "avattn_kernels.h"

using namespace avattn;

namespace {

constexpr int64_t kMaxI32 = 2147483647;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Row starts must stay 16-byte aligned: every stride a multiple of 8 bf16
// (or 4 floats for an fp32 tensor).
bool strides_ok(const int64_t* s) { return s && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }
bool strides_ok_f32(const int64_t* s) { return s && s[0] % 4 == 0 && s[1] % 4 == 0 && s[2] % 4 == 0; }

int check_dims(int32_t B, int32_t Hq, int32_t Hkv, int32_t Lq, int32_t Lk, int32_t D) {
  if (B < 0 || Hq < 0 || Hkv < 0 || Lq < 0 || Lk < 0) return AVATTN_ERR_BAD_SHAPE;
  if (D != 64 && D != 128) return AVATTN_ERR_HEAD_DIM;
  if (Hkv == 0 || Hq == 0) return (B == 0) ? AVATTN_OK : AVATTN_ERR_GQA;
  if (Hq % Hkv != 0) return AVATTN_ERR_GQA;
  // Grid sizes and per-(b,h) row indices are 32-bit.
  const int64_t qtiles = ((int64_t)Lq + 127) / 128;
  const int64_t ktiles = ((int64_t)Lk + 127) / 128;
  if (qtiles * B * Hq > kMaxI32 || ktiles * B * Hkv > kMaxI32) return AVATTN_ERR_TOO_LARGE;
  if ((int64_t)B * Hq * Lq > ((int64_t)1 << 40)) return AVATTN_ERR_TOO_LARGE;
  // Every kernel addresses one (batch, kv head) slice of a padded key copy
  // through a 32-bit buffer range: Lkp * D bf16 must stay below 2^32 bytes.
  const int64_t Lkp = transpose_padded_len(Lk);
  if (Lkp * D * 2 >= ((int64_t)1 << 32)) return AVATTN_ERR_TOO_LARGE;
  return AVATTN_OK;
}

// check_dims, plus the backward's own range: its dK/dV kernel stages the
// padded q and dout rows of all query heads of one group through one 32-bit
// buffer range each (group * Lqp * D bf16 below 2^32 bytes).  The forward
// builds no range over q, so long grouped-query shapes stay valid there.
int check_bwd_dims(int32_t B, int32_t Hq, int32_t Hkv, int32_t Lq, int32_t Lk, int32_t D) {
  const int st = check_dims(B, Hq, Hkv, Lq, Lk, D);
  if (st != AVATTN_OK || Hkv == 0 || Hq == 0) return st;
  const int64_t Lqp = transpose_padded_len(Lq);
  if ((int64_t)(Hq / Hkv) * Lqp * D * 2 >= ((int64_t)1 << 32)) return AVATTN_ERR_TOO_LARGE;
  return AVATTN_OK;
}

int launch_status(hipError_t e) { return e == hipSuccess ? AVATTN_OK : AVATTN_ERR_LAUNCH; }

size_t round256(size_t x) { return (x + 255) / 256 * 256; }

// Fused ring-step extras (avattn_ring_fwd_step / avattn_ring_bwd_step).
struct RingOpts {
  const float* cos_q = nullptr;  // RoPE of the (unrotated) query shard
  const float* sin_q = nullptr;
  int64_t rqsb = 0;
  const float* cos_k = nullptr;  // RoPE of the (unrotated) key chunk
  const float* sin_k = nullptr;
  int64_t rksb = 0;
  float* o_acc = nullptr;  // forward: running fp32 merge
  float* lse_acc = nullptr;
  bool first = false, last = false;
};

// Rotation tables: both or neither, 16-byte aligned, batch stride a multiple
// of 4 floats.
int check_tables(const float* c, const float* s, int64_t batch_stride) {
  if (!c && !s) return AVATTN_OK;
  if (!c || !s) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(c) || !aligned16(s) || batch_stride % 4 != 0 || batch_stride < 0) return AVATTN_ERR_LAYOUT;
  return AVATTN_OK;
}

// Key bias (B, Lkp) floats and per-32-key-tile flags (B, Lkp/32) ints, each
// with a 64-entry tail pad (tile loads read 64 entries from a tile start).
size_t kbias_bytes(int32_t B, size_t Lkp) { return round256(((size_t)B * Lkp + 64) * sizeof(float)); }
size_t kfull_bytes(int32_t B, size_t Lkp) { return round256(((size_t)B * (Lkp / 32) + 64) * sizeof(int)); }

// Forward workspace: [k rows | v^T | key bias | key tile flags | max squared
// k row norm per (b, kv head, 64-key tile)], each region 256-byte aligned.
struct FwdWorkspace {
  size_t kr, vt, kbias, kfull, kmax2, total;
};

// The fp8 forward has the e4m3 k rows (one byte per element) in place of
// the bf16 ones.
FwdWorkspace fwd_workspace(int32_t B, int32_t Hkv, int32_t Lk, int32_t D, bool fp8 = false) {
  FwdWorkspace w{};
  const size_t Lkp = transpose_padded_len(Lk);
  const size_t kcopy = round256((size_t)B * Hkv * D * Lkp * sizeof(bf16));
  w.kr = 0;
  w.vt = w.kr + (fp8 ? round256((size_t)B * Hkv * D * Lkp) : kcopy);
  w.kbias = w.vt + kcopy;
  w.kfull = w.kbias + kbias_bytes(B, Lkp);
  w.kmax2 = w.kfull + kfull_bytes(B, Lkp);
  w.total = w.kmax2 + round256((size_t)B * Hkv * (Lkp / 64) * sizeof(uint32_t));
  return w;
}

// Backward workspace: [lse2 | ndelta | q rows | dout rows |
// k rows | v rows | k^T | key bias | key tile flags | dK/dV tail-split
// partials (problems of more than 256 key blocks)], each region 256-byte
// aligned.
struct BwdWorkspace {
  size_t lse2, ndelta, qr, dor, kr, vr, kt, kbias, kfull, split, total;
};

BwdWorkspace bwd_workspace(int32_t B, int32_t Hq, int32_t Hkv, int32_t Lq, int32_t Lk, int32_t D) {
  BwdWorkspace w{};
  const size_t Lqp = transpose_padded_len(Lq), Lkp = transpose_padded_len(Lk);
  const size_t stats = round256((size_t)B * Hq * Lqp * sizeof(float));
  const size_t qcopy = round256((size_t)B * Hq * D * Lqp * sizeof(bf16));
  const size_t kcopy = round256((size_t)B * Hkv * D * Lkp * sizeof(bf16));
  w.lse2 = 0;
  w.ndelta = w.lse2 + stats;
  w.qr = w.ndelta + stats;
  w.dor = w.qr + qcopy;
  w.kr = w.dor + qcopy;
  w.vr = w.kr + kcopy;
  w.kt = w.vr + kcopy;
  w.kbias = w.kt + kcopy;
  w.kfull = w.kbias + kbias_bytes(B, Lkp);
  w.split = w.kfull + kfull_bytes(B, Lkp);
  w.total = w.split + split_part_bytes((int64_t)B * Hkv * ((Lk + 127) / 128), D);
  return w;
}

// Key windows: both arrays or neither, 4-byte aligned, batch stride 0
// (shared) or >= len_q; not with the fused RoPE or fp8 variants.
int check_windows(const int32_t* lo, const int32_t* hi, int64_t batch_stride, int32_t len_q, bool excluded) {
  if (!lo && !hi) return AVATTN_OK;
  if (!lo || !hi) return AVATTN_ERR_NULL_POINTER;
  if (excluded) return AVATTN_ERR_ARGUMENT;
  if (((reinterpret_cast<uintptr_t>(lo) | reinterpret_cast<uintptr_t>(hi)) & 3u) != 0) return AVATTN_ERR_LAYOUT;
  if (batch_stride != 0 && batch_stride < len_q) return AVATTN_ERR_ARGUMENT;
  return AVATTN_OK;
}

int check_qk_norm(const void* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                  int32_t head_dim, const void* weight, float eps, const float* cos_tab, const float* sin_tab,
                  int64_t table_batch_stride) {
  if (batch < 0 || heads < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim != 64 && head_dim != 128) return AVATTN_ERR_HEAD_DIM;
  if (!x_strides) return AVATTN_ERR_NULL_POINTER;
  if (!(eps >= 0.f) || !isfinite(eps)) return AVATTN_ERR_ARGUMENT;
  if (!cos_tab != !sin_tab) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!x) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(x) || !strides_ok(x_strides) || (weight && !aligned16(weight))) return AVATTN_ERR_LAYOUT;
  if (cos_tab && (!aligned16(cos_tab) || !aligned16(sin_tab) || table_batch_stride % 4 != 0))
    return AVATTN_ERR_LAYOUT;
  if ((int64_t)batch * heads > kMaxI32 || len > kMaxI32) return AVATTN_ERR_TOO_LARGE;
  return AVATTN_OK;
}

QkNormArgs qk_norm_args(const void* x, const int64_t* xs, int32_t batch, int32_t heads, int32_t len,
                        const void* weight, float eps, const float* cos_tab, const float* sin_tab, int64_t tsb) {
  QkNormArgs a{};
  a.x = static_cast<const bf16*>(x);
  a.xsb = xs[0]; a.xsh = xs[1]; a.xsl = xs[2];
  a.B = batch; a.H = heads; a.L = len;
  a.w = static_cast<const bf16*>(weight);
  a.eps = eps;
  a.ct = cos_tab; a.st = sin_tab; a.tsb = tsb;
  return a;
}

// The staged dS region starts on a 4 KB boundary after the base workspace.
size_t staged_ds_offset(const BwdWorkspace& w) { return (w.total + 4095) / 4096 * 4096; }

}  // namespace

extern "C" {

const char* avattn_strerror(int status) {
  switch (status) {
    case AVATTN_OK: return "success";
    case AVATTN_ERR_NULL_POINTER: return "a required pointer argument is NULL";
    case AVATTN_ERR_BAD_SHAPE: return "invalid (negative) size";
    case AVATTN_ERR_HEAD_DIM: return "unsupported head_dim (supported: 64, 128)";
    case AVATTN_ERR_GQA: return "heads_q must be a positive multiple of heads_kv";
    case AVATTN_ERR_LAYOUT:
      return "misaligned tensor: pointers must be 16-byte aligned, head_dim contiguous and "
             "batch/head/seq strides multiples of 8 elements";
    case AVATTN_ERR_WORKSPACE:
      return "workspace missing, misaligned or smaller than avattn_fwd_workspace_size() / "
             "avattn_bwd_workspace_size()";
    case AVATTN_ERR_LAUNCH: return "HIP kernel launch failed";
    case AVATTN_ERR_TOO_LARGE: return "problem size exceeds the 32-bit grid/index range";
    case AVATTN_ERR_ARGUMENT: return "invalid argument";
    case AVATTN_ERR_SCRATCH:
      return "problem needs more device scratch than avattn_fwd_noalloc's fixed array "
             "(AVATTN_FWD_NOALLOC_SCRATCH = 64 MiB); use avattn_fwd with a workspace";
    default: return "unknown avattn status";
  }
}

int avattn_abi_version(void) { return 14; }

}  // extern "C"

namespace {

// avattn_fwd and avattn_fwd_fp8 (q_scale/k_scale non-null selects fp8).
int fwd_impl(const void* q, const void* k, const void* v, const int64_t* q_strides, const int64_t* k_strides,
             const int64_t* v_strides, int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q,
             int32_t len_k, int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
             const float* rope_cos_q, const float* rope_sin_q, int64_t rope_batch_stride, bool fp8,
             const float* q_scale, const float* k_scale, float scale, void* out, const int64_t* out_strides,
             float* lse, void* workspace, size_t workspace_bytes, avattn_stream_t stream,
             const int32_t* window_lo = nullptr, const int32_t* window_hi = nullptr, int64_t window_batch_stride = 0,
             const RingOpts* ring = nullptr) {
  int st = check_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (st != AVATTN_OK) return st;
  if (!q_strides || !k_strides || !v_strides || !out_strides) return AVATTN_ERR_NULL_POINTER;
  if (!(scale > 0.f) || !isfinite(scale)) return AVATTN_ERR_ARGUMENT;
  if ((rope_cos_q == nullptr) != (rope_sin_q == nullptr)) return AVATTN_ERR_ARGUMENT;
  const int64_t rows = (int64_t)batch * heads_q * len_q;
  if (rows == 0) return AVATTN_OK;
  if (!q || !out || !lse) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(q) || !aligned16(out) || !strides_ok(q_strides) || !strides_ok(out_strides))
    return AVATTN_ERR_LAYOUT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (len_k == 0)
    return launch_status(launch_empty(static_cast<bf16*>(out), out_strides[0], out_strides[1], out_strides[2], batch,
                                      heads_q, len_q, head_dim, lse, s));
  if (!k || !v) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(k) || !aligned16(v) || !strides_ok(k_strides) || !strides_ok(v_strides)) return AVATTN_ERR_LAYOUT;
  if (rope_cos_q && (!aligned16(rope_cos_q) || !aligned16(rope_sin_q) || rope_batch_stride % 4 != 0))
    return AVATTN_ERR_LAYOUT;
  if (key_mask && key_mask_batch_stride != 0 && key_mask_batch_stride < len_k) return AVATTN_ERR_ARGUMENT;
  if (fp8 && (!q_scale || !k_scale)) return AVATTN_ERR_NULL_POINTER;
  if (fp8 && ((reinterpret_cast<uintptr_t>(q_scale) | reinterpret_cast<uintptr_t>(k_scale)) & 3u))
    return AVATTN_ERR_LAYOUT;
  st = check_windows(window_lo, window_hi, window_batch_stride, len_q, fp8 || rope_cos_q != nullptr);
  if (st != AVATTN_OK) return st;
  const FwdWorkspace wl = fwd_workspace(batch, heads_kv, len_k, head_dim, fp8);
  if (!workspace || workspace_bytes < wl.total || !aligned16(workspace)) return AVATTN_ERR_WORKSPACE;

  FwdArgs a{};
  a.q = static_cast<const bf16*>(q);
  a.k = static_cast<const bf16*>(k);
  a.v = static_cast<const bf16*>(v);
  a.qsb = q_strides[0]; a.qsh = q_strides[1]; a.qsl = q_strides[2];
  a.ksb = k_strides[0]; a.ksh = k_strides[1]; a.ksl = k_strides[2];
  a.vsb = v_strides[0]; a.vsh = v_strides[1]; a.vsl = v_strides[2];
  a.B = batch; a.Hq = heads_q; a.Hkv = heads_kv; a.Lq = len_q; a.Lk = len_k;
  a.mask = key_mask;
  a.msb = key_mask_batch_stride;
  a.cos_q = rope_cos_q;
  a.sin_q = rope_sin_q;
  a.rsb = rope_batch_stride;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.o = static_cast<bf16*>(out);
  a.osb = out_strides[0]; a.osh = out_strides[1]; a.osl = out_strides[2];
  a.lse = lse;
  char* ws = static_cast<char*>(workspace);
  a.kr = fp8 ? nullptr : reinterpret_cast<bf16*>(ws + wl.kr);
  a.k8 = fp8 ? reinterpret_cast<uint8_t*>(ws + wl.kr) : nullptr;
  a.q_scale = fp8 ? q_scale : nullptr;
  a.k_scale = fp8 ? k_scale : nullptr;
  a.vt = reinterpret_cast<bf16*>(ws + wl.vt);
  a.kbias = reinterpret_cast<float*>(ws + wl.kbias);
  a.kfull = reinterpret_cast<int*>(ws + wl.kfull);
  a.kmax2 = reinterpret_cast<uint32_t*>(ws + wl.kmax2);
  a.Lkp = transpose_padded_len(len_k);
  a.wlo = window_lo;
  a.whi = window_hi;
  a.wsb = window_batch_stride;
  if (ring) {
    a.cos_k = ring->cos_k;
    a.sin_k = ring->sin_k;
    a.rksb = ring->rksb;
    a.o_acc = ring->o_acc;
    a.lse_acc = ring->lse_acc;
    a.acc_first = ring->first;
    a.acc_final = ring->last;
  }
  return launch_status(launch_fwd(a, head_dim, s));
}

}  // namespace

extern "C" {

int avattn_fwd(const void* q, const void* k, const void* v, const int64_t* q_strides, const int64_t* k_strides,
               const int64_t* v_strides, int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q,
               int32_t len_k, int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
               const float* rope_cos_q, const float* rope_sin_q, int64_t rope_batch_stride, float scale, void* out,
               const int64_t* out_strides, float* lse, void* workspace, size_t workspace_bytes,
               avattn_stream_t stream) {
  return fwd_impl(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                  key_mask, key_mask_batch_stride, rope_cos_q, rope_sin_q, rope_batch_stride, false, nullptr,
                  nullptr, scale, out, out_strides, lse, workspace, workspace_bytes, stream);
}

int avattn_fwd_fp8(const void* q, const void* k, const void* v, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q,
                   int32_t len_k, int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
                   const float* q_scale, const float* k_scale, float scale, void* out, const int64_t* out_strides,
                   float* lse, void* workspace, size_t workspace_bytes, avattn_stream_t stream) {
  return fwd_impl(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                  key_mask, key_mask_batch_stride, nullptr, nullptr, 0, true, q_scale, k_scale, scale, out,
                  out_strides, lse, workspace, workspace_bytes, stream);
}

int avattn_fwd_windowed(const void* q, const void* k, const void* v, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides, int32_t batch, int32_t heads_q,
                        int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
                        int64_t key_mask_batch_stride, const int32_t* window_lo, const int32_t* window_hi,
                        int64_t window_batch_stride, float scale, void* out, const int64_t* out_strides, float* lse,
                        void* workspace, size_t workspace_bytes, avattn_stream_t stream) {
  if (!window_lo || !window_hi) return AVATTN_ERR_NULL_POINTER;
  return fwd_impl(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                  key_mask, key_mask_batch_stride, nullptr, nullptr, 0, false, nullptr, nullptr, scale, out,
                  out_strides, lse, workspace, workspace_bytes, stream, window_lo, window_hi, window_batch_stride);
}

size_t avattn_fwd_fp8_workspace_size(int32_t batch, int32_t heads_kv, int32_t len_k, int32_t head_dim) {
  if (batch <= 0 || heads_kv <= 0 || len_k <= 0 || head_dim <= 0) return 0;
  return fwd_workspace(batch, heads_kv, len_k, head_dim, true).total;
}

int avattn_fp8_absmax_scales(const void* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                             int32_t head_dim, float* scale_out, avattn_stream_t stream) {
  if (batch < 0 || heads < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim != 64 && head_dim != 128) return AVATTN_ERR_HEAD_DIM;
  if (!x_strides) return AVATTN_ERR_NULL_POINTER;
  if (heads == 0) return AVATTN_OK;
  if (heads > 65535) return AVATTN_ERR_TOO_LARGE;
  if ((int64_t)batch * len * (head_dim / 8) > ((int64_t)1 << 40)) return AVATTN_ERR_TOO_LARGE;
  if (!scale_out || ((int64_t)batch * len > 0 && !x)) return AVATTN_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(scale_out) & 3u) != 0) return AVATTN_ERR_LAYOUT;
  if ((int64_t)batch * len > 0 && (!aligned16(x) || !strides_ok(x_strides))) return AVATTN_ERR_LAYOUT;
  return launch_status(launch_absmax_scales(static_cast<const bf16*>(x), x_strides[0], x_strides[1], x_strides[2],
                                            batch, heads, len, head_dim, scale_out,
                                            reinterpret_cast<uint32_t*>(scale_out),
                                            reinterpret_cast<hipStream_t>(stream)));
}

size_t avattn_fwd_workspace_size(int32_t batch, int32_t heads_kv, int32_t len_k, int32_t head_dim) {
  if (batch <= 0 || heads_kv <= 0 || len_k <= 0 || head_dim <= 0) return 0;
  return fwd_workspace(batch, heads_kv, len_k, head_dim).total;
}

size_t avattn_bwd_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                                 int32_t head_dim) {
  if (batch <= 0 || heads_q <= 0 || heads_kv <= 0 || len_q <= 0 || len_k <= 0 || head_dim <= 0) return 0;
  return bwd_workspace(batch, heads_q, heads_kv, len_q, len_k, head_dim).total;
}

size_t avattn_bwd_staged_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q,
                                        int32_t len_k, int32_t head_dim, int32_t kv_pairs_per_pass) {
  if (batch <= 0 || heads_q <= 0 || heads_kv <= 0 || len_q <= 0 || len_k <= 0 || head_dim <= 0 ||
      kv_pairs_per_pass <= 0 || heads_q % heads_kv != 0)
    return 0;
  const BwdWorkspace wl = bwd_workspace(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  const int64_t pairs = (int64_t)batch * heads_kv;
  const int64_t n = kv_pairs_per_pass < pairs ? kv_pairs_per_pass : pairs;
  return staged_ds_offset(wl) + (size_t)n * ds_bytes_per_kv(heads_q / heads_kv, len_q, len_k);
}

// Compact staged-dS layout of a windowed backward (BwdArgs::ds_tab).
struct CompactDs {
  const int32_t* table = nullptr;
  int64_t table_batch_stride = 0;  // in tiles
  int64_t units_per_head = 0;
};

size_t avattn_bwd_compact_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q,
                                         int32_t len_k, int32_t head_dim, int32_t pairs_per_pass,
                                         int64_t ds_units_per_head) {
  if (check_bwd_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim) != AVATTN_OK) return 0;
  if ((int64_t)batch * heads_q == 0 || len_q == 0 || len_k == 0 || pairs_per_pass <= 0 || ds_units_per_head < 1)
    return 0;
  const BwdWorkspace wl = bwd_workspace(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  const int64_t n = pairs_per_pass < (int64_t)batch * heads_kv ? pairs_per_pass : (int64_t)batch * heads_kv;
  return staged_ds_offset(wl) + (size_t)n * ds_bytes_per_kv(heads_q / heads_kv, len_q, len_k, ds_units_per_head);
}

static int bwd_impl(const void* dout, const void* q, const void* k, const void* v, const void* out, const float* lse,
                    const int64_t* dout_strides, const int64_t* q_strides, const int64_t* k_strides,
                    const int64_t* v_strides, const int64_t* out_strides, int32_t batch, int32_t heads_q,
                    int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
                    int64_t key_mask_batch_stride, float scale, void* dq, const int64_t* dq_strides, void* dk,
                    const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* workspace,
                    size_t workspace_bytes, uint32_t flags, avattn_stream_t stream, const int32_t* window_lo,
                    const int32_t* window_hi, int64_t window_batch_stride, const RingOpts* ring = nullptr,
                    const CompactDs* compact = nullptr) {
  int st = check_bwd_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (flags & ~(AVATTN_BWD_REUSE_QUERY_SIDE | AVATTN_BWD_DQ_ACCUMULATE_F32 | AVATTN_BWD_STAGE_DS |
                AVATTN_BWD_DEFER_DQ))
    return AVATTN_ERR_ARGUMENT;
  const bool defer = (flags & AVATTN_BWD_DEFER_DQ) != 0;
  if (defer && !(flags & AVATTN_BWD_STAGE_DS)) return AVATTN_ERR_ARGUMENT;
  const bool dq_f32 = (flags & AVATTN_BWD_DQ_ACCUMULATE_F32) != 0;
  if (st != AVATTN_OK) return st;
  if (!dout_strides || !q_strides || !k_strides || !v_strides || !out_strides || !dq_strides || !dk_strides ||
      !dv_strides)
    return AVATTN_ERR_NULL_POINTER;
  if (!(scale > 0.f) || !isfinite(scale)) return AVATTN_ERR_ARGUMENT;
  if ((int64_t)batch * heads_q == 0) return AVATTN_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool have_q = len_q > 0, have_k = len_k > 0;
  if (have_q && !defer &&
      (!dq || !aligned16(dq) || !(dq_f32 ? strides_ok_f32(dq_strides) : strides_ok(dq_strides))))
    return !dq ? AVATTN_ERR_NULL_POINTER : AVATTN_ERR_LAYOUT;
  if (have_k && (!dk || !dv)) return AVATTN_ERR_NULL_POINTER;
  if (have_k && (!aligned16(dk) || !aligned16(dv) || !strides_ok(dk_strides) || !strides_ok(dv_strides)))
    return AVATTN_ERR_LAYOUT;
  if (!have_q || !have_k) {
    // Empty attention: every gradient is zero.
    hipError_t e = hipSuccess;
    if (have_q && !dq_f32 && !defer)  // an fp32 accumulator gets nothing added; a deferred dq is zeroed later
      e = launch_zero_rows(static_cast<bf16*>(dq), dq_strides[0], dq_strides[1], dq_strides[2], batch, heads_q, len_q,
                           head_dim, s);
    if (e == hipSuccess && have_k)
      e = launch_zero_rows(static_cast<bf16*>(dk), dk_strides[0], dk_strides[1], dk_strides[2], batch, heads_kv,
                           len_k, head_dim, s);
    if (e == hipSuccess && have_k)
      e = launch_zero_rows(static_cast<bf16*>(dv), dv_strides[0], dv_strides[1], dv_strides[2], batch, heads_kv,
                           len_k, head_dim, s);
    return launch_status(e);
  }
  if (!dout || !q || !k || !v || !out || !lse) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(dout) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) ||
      !strides_ok(dout_strides) || !strides_ok(q_strides) || !strides_ok(k_strides) || !strides_ok(v_strides) ||
      !strides_ok(out_strides))
    return AVATTN_ERR_LAYOUT;
  if (key_mask && key_mask_batch_stride != 0 && key_mask_batch_stride < len_k) return AVATTN_ERR_ARGUMENT;
  st = check_windows(window_lo, window_hi, window_batch_stride, len_q, false);
  if (st != AVATTN_OK) return st;
  // Windows run on the staged-dS path only, and dq is not deferred.
  if (window_lo && (!(flags & AVATTN_BWD_STAGE_DS) || (flags & AVATTN_BWD_DEFER_DQ))) return AVATTN_ERR_ARGUMENT;
  const int64_t ntiles = transpose_padded_len(len_q) / 64;
  if (compact) {
    // A table for every batch row (or one shared), 16-byte aligned; the
    // units of one query head addressable through a 32-bit buffer range.
    if (!window_lo || !compact->table) return AVATTN_ERR_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(compact->table) & 15u) return AVATTN_ERR_LAYOUT;
    if (compact->table_batch_stride != 0 && compact->table_batch_stride < ntiles) return AVATTN_ERR_ARGUMENT;
    if (compact->units_per_head < 1 || compact->units_per_head * 8192 >= ((int64_t)1 << 32))
      return AVATTN_ERR_ARGUMENT;
  }
  const int64_t ds_units = compact ? compact->units_per_head : 0;
  const BwdWorkspace wl = bwd_workspace(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (!workspace || workspace_bytes < wl.total || !aligned16(workspace)) return AVATTN_ERR_WORKSPACE;

  BwdArgs a{};
  a.dout = static_cast<const bf16*>(dout);
  a.q = static_cast<const bf16*>(q);
  a.k = static_cast<const bf16*>(k);
  a.v = static_cast<const bf16*>(v);
  a.out = static_cast<const bf16*>(out);
  a.lse = lse;
  a.dosb = dout_strides[0]; a.dosh = dout_strides[1]; a.dosl = dout_strides[2];
  a.qsb = q_strides[0]; a.qsh = q_strides[1]; a.qsl = q_strides[2];
  a.ksb = k_strides[0]; a.ksh = k_strides[1]; a.ksl = k_strides[2];
  a.vsb = v_strides[0]; a.vsh = v_strides[1]; a.vsl = v_strides[2];
  a.osb = out_strides[0]; a.osh = out_strides[1]; a.osl = out_strides[2];
  a.B = batch; a.Hq = heads_q; a.Hkv = heads_kv; a.Lq = len_q; a.Lk = len_k;
  a.mask = key_mask;
  a.msb = key_mask_batch_stride;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.dq = dq_f32 ? nullptr : static_cast<bf16*>(dq);
  a.dq_acc = dq_f32 ? static_cast<float*>(dq) : nullptr;
  a.reuse_q = (flags & AVATTN_BWD_REUSE_QUERY_SIDE) != 0;
  a.dqsb = dq_strides[0]; a.dqsh = dq_strides[1]; a.dqsl = dq_strides[2];
  a.dk = static_cast<bf16*>(dk);
  a.dksb = dk_strides[0]; a.dksh = dk_strides[1]; a.dksl = dk_strides[2];
  a.dv = static_cast<bf16*>(dv);
  a.dvsb = dv_strides[0]; a.dvsh = dv_strides[1]; a.dvsl = dv_strides[2];
  char* ws = static_cast<char*>(workspace);
  a.lse2 = reinterpret_cast<float*>(ws + wl.lse2);
  a.ndelta = reinterpret_cast<float*>(ws + wl.ndelta);
  a.qr = reinterpret_cast<bf16*>(ws + wl.qr);
  a.dor = reinterpret_cast<bf16*>(ws + wl.dor);
  a.kr = reinterpret_cast<bf16*>(ws + wl.kr);
  a.vr = reinterpret_cast<bf16*>(ws + wl.vr);
  a.kt = reinterpret_cast<bf16*>(ws + wl.kt);
  a.kbias = reinterpret_cast<float*>(ws + wl.kbias);
  a.kfull = reinterpret_cast<int*>(ws + wl.kfull);
  a.split_part = wl.total > wl.split ? reinterpret_cast<float*>(ws + wl.split) : nullptr;
  a.Lqp = transpose_padded_len(len_q);
  a.Lkp = transpose_padded_len(len_k);
  a.kv0 = 0;
  a.nkv = batch * heads_kv;
  a.ds = nullptr;
  a.defer_dq = defer;
  a.wlo = window_lo;
  a.whi = window_hi;
  a.wsb = window_batch_stride;
  if (compact) {
    a.ds_tab = compact->table;
    a.ds_tsb = compact->table_batch_stride;
    a.ds_units = compact->units_per_head;
  }
  if (ring) {
    a.cos_q = ring->cos_q;
    a.sin_q = ring->sin_q;
    a.rqsb = ring->rqsb;
    a.cos_k = ring->cos_k;
    a.sin_k = ring->sin_k;
    a.rksb = ring->rksb;
  }
  int kv_per_pass = 0;
  if (flags & AVATTN_BWD_STAGE_DS) {
    const size_t off = staged_ds_offset(wl);
    const size_t per = ds_bytes_per_kv(heads_q / heads_kv, len_q, len_k, ds_units);
    // A deferred dq needs every pair's dS at once.
    const size_t need = off + (defer ? (size_t)a.nkv * per : per);
    if (workspace_bytes < need) return AVATTN_ERR_WORKSPACE;
    const size_t fit = (workspace_bytes - off) / per;
    // Passes of equal size (the fewest that fit): a short last pass would
    // leave most of the chip idle for its whole launch.
    const size_t npass = ((size_t)a.nkv + fit - 1) / fit;
    kv_per_pass = (int)(((size_t)a.nkv + npass - 1) / npass);
    a.ds = reinterpret_cast<bf16*>(ws + off);
  }
  return launch_status(launch_bwd(a, head_dim, kv_per_pass, s));
}

int avattn_bwd(const void* dout, const void* q, const void* k, const void* v, const void* out, const float* lse,
               const int64_t* dout_strides, const int64_t* q_strides, const int64_t* k_strides,
               const int64_t* v_strides, const int64_t* out_strides, int32_t batch, int32_t heads_q,
               int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
               int64_t key_mask_batch_stride, float scale, void* dq, const int64_t* dq_strides, void* dk,
               const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* workspace,
               size_t workspace_bytes, uint32_t flags, avattn_stream_t stream) {
  return bwd_impl(dout, q, k, v, out, lse, dout_strides, q_strides, k_strides, v_strides, out_strides, batch, heads_q,
                  heads_kv, len_q, len_k, head_dim, key_mask, key_mask_batch_stride, scale, dq, dq_strides, dk,
                  dk_strides, dv, dv_strides, workspace, workspace_bytes, flags, stream, nullptr, nullptr, 0);
}

int avattn_bwd_windowed(const void* dout, const void* q, const void* k, const void* v, const void* out,
                        const float* lse, const int64_t* dout_strides, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                        int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                        int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
                        const int32_t* window_lo, const int32_t* window_hi, int64_t window_batch_stride, float scale,
                        void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                        const int64_t* dv_strides, void* workspace, size_t workspace_bytes, uint32_t flags,
                        avattn_stream_t stream) {
  if (!window_lo || !window_hi) return AVATTN_ERR_NULL_POINTER;
  return bwd_impl(dout, q, k, v, out, lse, dout_strides, q_strides, k_strides, v_strides, out_strides, batch, heads_q,
                  heads_kv, len_q, len_k, head_dim, key_mask, key_mask_batch_stride, scale, dq, dq_strides, dk,
                  dk_strides, dv, dv_strides, workspace, workspace_bytes, flags, stream, window_lo, window_hi,
                  window_batch_stride);
}

int avattn_bwd_windowed_compact(const void* dout, const void* q, const void* k, const void* v, const void* out,
                                const float* lse, const int64_t* dout_strides, const int64_t* q_strides,
                                const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                                int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                                int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
                                const int32_t* window_lo, const int32_t* window_hi, int64_t window_batch_stride,
                                const int32_t* ds_table, int64_t ds_table_batch_stride, int64_t ds_units_per_head,
                                float scale, void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides,
                                void* dv, const int64_t* dv_strides, void* workspace, size_t workspace_bytes,
                                uint32_t flags, avattn_stream_t stream) {
  if (!window_lo || !window_hi || !ds_table) return AVATTN_ERR_NULL_POINTER;
  CompactDs c;
  c.table = ds_table;
  c.table_batch_stride = ds_table_batch_stride;
  c.units_per_head = ds_units_per_head;
  return bwd_impl(dout, q, k, v, out, lse, dout_strides, q_strides, k_strides, v_strides, out_strides, batch, heads_q,
                  heads_kv, len_q, len_k, head_dim, key_mask, key_mask_batch_stride, scale, dq, dq_strides, dk,
                  dk_strides, dv, dv_strides, workspace, workspace_bytes, flags, stream, window_lo, window_hi,
                  window_batch_stride, nullptr, &c);
}

int avattn_bwd_dq_staged(int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                         int32_t head_dim, float scale, void* dq, const int64_t* dq_strides, void* workspace,
                         size_t workspace_bytes, uint32_t flags, avattn_stream_t stream) {
  int st = check_bwd_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (st != AVATTN_OK) return st;
  if (flags & ~AVATTN_BWD_DQ_ACCUMULATE_F32) return AVATTN_ERR_ARGUMENT;
  const bool dq_f32 = (flags & AVATTN_BWD_DQ_ACCUMULATE_F32) != 0;
  if (!(scale > 0.f) || !isfinite(scale)) return AVATTN_ERR_ARGUMENT;
  if ((int64_t)batch * heads_q == 0 || len_q == 0) return AVATTN_OK;
  if (!dq || !dq_strides) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(dq) || !(dq_f32 ? strides_ok_f32(dq_strides) : strides_ok(dq_strides))) return AVATTN_ERR_LAYOUT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (len_k == 0) {
    if (dq_f32) return AVATTN_OK;
    return launch_status(launch_zero_rows(static_cast<bf16*>(dq), dq_strides[0], dq_strides[1], dq_strides[2], batch,
                                          heads_q, len_q, head_dim, s));
  }
  const BwdWorkspace wl = bwd_workspace(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  const size_t off = staged_ds_offset(wl);
  const size_t all = (size_t)batch * heads_kv * ds_bytes_per_kv(heads_q / heads_kv, len_q, len_k);
  if (!workspace || !aligned16(workspace) || workspace_bytes < off + all) return AVATTN_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  BwdArgs a{};
  a.B = batch; a.Hq = heads_q; a.Hkv = heads_kv; a.Lq = len_q; a.Lk = len_k;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.dq = dq_f32 ? nullptr : static_cast<bf16*>(dq);
  a.dq_acc = dq_f32 ? static_cast<float*>(dq) : nullptr;
  a.dqsb = dq_strides[0]; a.dqsh = dq_strides[1]; a.dqsl = dq_strides[2];
  a.kt = reinterpret_cast<bf16*>(ws + wl.kt);
  a.Lqp = transpose_padded_len(len_q);
  a.Lkp = transpose_padded_len(len_k);
  a.kv0 = 0;
  a.nkv = batch * heads_kv;
  a.ds = reinterpret_cast<bf16*>(ws + off);
  return launch_status(launch_bwd_dq_staged(a, head_dim, s));
}

int avattn_lse_merge(float* out_acc, float* lse_acc, const void* out_blk, const float* lse_blk, int64_t n_rows,
                     int32_t head_dim, int32_t blk_is_bf16, avattn_stream_t stream) {
  if (n_rows < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim != 64 && head_dim != 128) return AVATTN_ERR_HEAD_DIM;
  if (n_rows == 0) return AVATTN_OK;
  if (!out_acc || !lse_acc || !out_blk || !lse_blk) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(out_acc) || !aligned16(out_blk)) return AVATTN_ERR_LAYOUT;
  if (n_rows > ((int64_t)1 << 40)) return AVATTN_ERR_TOO_LARGE;
  return launch_status(launch_lse_merge(out_acc, lse_acc, out_blk, lse_blk, n_rows, head_dim, blk_is_bf16 != 0,
                                        reinterpret_cast<hipStream_t>(stream)));
}

int avattn_rope_tables(const float* coords, int64_t coords_batch_stride, int64_t coords_row_stride, int32_t batch,
                       int32_t len, int32_t pairs, const float* inv_freq, const int32_t* axis_of_pair,
                       const int32_t* apply_mul, const float* pos_mul, const int32_t* apply_div,
                       const float* pos_div, float* cos_out, float* sin_out, avattn_stream_t stream) {
  if (batch < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (pairs < 3 || pairs > 64) return AVATTN_ERR_HEAD_DIM;
  if (!inv_freq || !axis_of_pair || !apply_mul || !pos_mul || !apply_div || !pos_div) return AVATTN_ERR_NULL_POINTER;
  for (int p = 0; p < pairs; ++p)
    if (axis_of_pair[p] < 0 || axis_of_pair[p] > 2) return AVATTN_ERR_ARGUMENT;
  if ((int64_t)batch * len == 0) return AVATTN_OK;
  if (!coords || !cos_out || !sin_out) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * len > kMaxI32) return AVATTN_ERR_TOO_LARGE;
  return launch_status(launch_rope_tables(coords, coords_batch_stride, coords_row_stride, batch, len, pairs, inv_freq,
                                          axis_of_pair, apply_mul, pos_mul, apply_div, pos_div, cos_out, sin_out,
                                          reinterpret_cast<hipStream_t>(stream)));
}

int avattn_rope_apply(const void* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                      int32_t head_dim, const float* cos_tab, const float* sin_tab, int64_t table_batch_stride,
                      int32_t inverse, void* out, const int64_t* out_strides, avattn_stream_t stream) {
  if (batch < 0 || heads < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim < 8 || head_dim > 128 || head_dim % 8 != 0) return AVATTN_ERR_HEAD_DIM;
  if (!x_strides || !out_strides) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!x || !out || !cos_tab || !sin_tab) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(x) || !aligned16(out) || !aligned16(cos_tab) || !aligned16(sin_tab) || !strides_ok(x_strides) ||
      !strides_ok(out_strides) || table_batch_stride % 4 != 0)
    return AVATTN_ERR_LAYOUT;
  if ((int64_t)batch * heads > kMaxI32 || len > kMaxI32) return AVATTN_ERR_TOO_LARGE;
  return launch_status(launch_rope_apply(static_cast<const bf16*>(x), x_strides[0], x_strides[1], x_strides[2], batch,
                                         heads, len, head_dim, cos_tab, sin_tab, table_batch_stride, inverse != 0,
                                         static_cast<bf16*>(out), out_strides[0], out_strides[1], out_strides[2],
                                         reinterpret_cast<hipStream_t>(stream)));
}

size_t avattn_qk_norm_rope_bwd_workspace_size(int32_t head_dim) {
  if (head_dim != 64 && head_dim != 128) return 0;
  return qk_norm_bwd_workspace_bytes(head_dim);
}

int avattn_qk_norm_rope(const void* x, const int64_t* x_strides, int32_t batch, int32_t heads, int32_t len,
                        int32_t head_dim, const void* weight, float eps, const float* cos_tab, const float* sin_tab,
                        int64_t table_batch_stride, void* out, const int64_t* out_strides, avattn_stream_t stream) {
  int st = check_qk_norm(x, x_strides, batch, heads, len, head_dim, weight, eps, cos_tab, sin_tab,
                         table_batch_stride);
  if (st != AVATTN_OK) return st;
  if (!out_strides) return AVATTN_ERR_NULL_POINTER;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!out) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(out) || !strides_ok(out_strides)) return AVATTN_ERR_LAYOUT;
  QkNormArgs a = qk_norm_args(x, x_strides, batch, heads, len, weight, eps, cos_tab, sin_tab, table_batch_stride);
  a.out = static_cast<bf16*>(out);
  a.osb = out_strides[0]; a.osh = out_strides[1]; a.osl = out_strides[2];
  return launch_status(launch_qk_norm(a, head_dim, reinterpret_cast<hipStream_t>(stream)));
}

int avattn_qk_norm_rope_bwd(const void* x, const int64_t* x_strides, const void* dy, const int64_t* dy_strides,
                            int32_t batch, int32_t heads, int32_t len, int32_t head_dim, const void* weight, float eps,
                            const float* cos_tab, const float* sin_tab, int64_t table_batch_stride, void* dx,
                            const int64_t* dx_strides, float* dweight, void* workspace, size_t workspace_bytes,
                            avattn_stream_t stream) {
  int st = check_qk_norm(x, x_strides, batch, heads, len, head_dim, weight, eps, cos_tab, sin_tab,
                         table_batch_stride);
  if (st != AVATTN_OK) return st;
  if (!dy_strides || !dx_strides) return AVATTN_ERR_NULL_POINTER;
  if (weight && !dweight) return AVATTN_ERR_NULL_POINTER;
  if (weight && (!workspace || workspace_bytes < qk_norm_bwd_workspace_bytes(head_dim) || !aligned16(workspace)))
    return AVATTN_ERR_WORKSPACE;
  if ((int64_t)batch * heads * len == 0) {
    if (!weight) return AVATTN_OK;
    // No rows: the gain's gradient is zero (the reduction over no blocks).
    return launch_status(launch_qk_norm_dw_zero(dweight, head_dim, reinterpret_cast<hipStream_t>(stream)));
  }
  if (!dy || !dx) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(dy) || !aligned16(dx) || !strides_ok(dy_strides) || !strides_ok(dx_strides))
    return AVATTN_ERR_LAYOUT;
  QkNormArgs a = qk_norm_args(x, x_strides, batch, heads, len, weight, eps, cos_tab, sin_tab, table_batch_stride);
  a.dy = static_cast<const bf16*>(dy);
  a.dsb = dy_strides[0]; a.dsh = dy_strides[1]; a.dsl = dy_strides[2];
  a.dx = static_cast<bf16*>(dx);
  a.xgb = dx_strides[0]; a.xgh = dx_strides[1]; a.xgl = dx_strides[2];
  a.wpart = weight ? static_cast<float*>(workspace) : nullptr;
  return launch_status(launch_qk_norm_bwd(a, head_dim, dweight, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Fused ring steps
// ---------------------------------------------------------------------------
extern "C" {

int avattn_ring_fwd_step(const void* q, const void* k, const void* v, const int64_t* q_strides,
                         const int64_t* k_strides, const int64_t* v_strides, int32_t batch, int32_t heads_q,
                         int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim, const uint8_t* key_mask,
                         int64_t key_mask_batch_stride, const float* rope_cos_q, const float* rope_sin_q,
                         int64_t rope_q_batch_stride, const float* rope_cos_k, const float* rope_sin_k,
                         int64_t rope_k_batch_stride, float scale, float* out_acc, float* lse_acc, void* out,
                         const int64_t* out_strides, uint32_t flags, void* workspace, size_t workspace_bytes,
                         avattn_stream_t stream) {
  if (flags & ~(AVATTN_RING_FIRST | AVATTN_RING_LAST)) return AVATTN_ERR_ARGUMENT;
  int st = check_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (st != AVATTN_OK) return st;
  if ((int64_t)batch * heads_q * len_q == 0) return AVATTN_OK;
  if (len_k == 0) return AVATTN_ERR_BAD_SHAPE;  // a ring chunk holds at least one key
  if (!out_acc || !lse_acc) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(out_acc) || (reinterpret_cast<uintptr_t>(lse_acc) & 3u)) return AVATTN_ERR_LAYOUT;
  st = check_tables(rope_cos_q, rope_sin_q, rope_q_batch_stride);
  if (st == AVATTN_OK) st = check_tables(rope_cos_k, rope_sin_k, rope_k_batch_stride);
  if (st != AVATTN_OK) return st;
  // Without AVATTN_RING_LAST the bf16 output is not written: out may be
  // NULL; fwd_impl's layout checks then run on the accumulator instead.
  const bool last = (flags & AVATTN_RING_LAST) != 0;
  if (last && (!out || !out_strides)) return AVATTN_ERR_NULL_POINTER;
  static const int64_t kNoStrides[3] = {0, 0, 0};
  RingOpts ring;
  ring.cos_k = rope_cos_k;
  ring.sin_k = rope_sin_k;
  ring.rksb = rope_k_batch_stride;
  ring.o_acc = out_acc;
  ring.lse_acc = lse_acc;
  ring.first = (flags & AVATTN_RING_FIRST) != 0;
  ring.last = last;
  return fwd_impl(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                  key_mask, key_mask_batch_stride, rope_cos_q, rope_sin_q, rope_q_batch_stride, false, nullptr,
                  nullptr, scale, last ? out : out_acc, last ? out_strides : kNoStrides, lse_acc, workspace,
                  workspace_bytes, stream, nullptr, nullptr, 0, &ring);
}

int avattn_ring_bwd_step(const void* dout, const void* q, const void* k, const void* v, const void* out,
                         const float* lse, const int64_t* dout_strides, const int64_t* q_strides,
                         const int64_t* k_strides, const int64_t* v_strides, const int64_t* out_strides,
                         int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t len_q, int32_t len_k,
                         int32_t head_dim, const uint8_t* key_mask, int64_t key_mask_batch_stride,
                         const float* rope_cos_q, const float* rope_sin_q, int64_t rope_q_batch_stride,
                         const float* rope_cos_k, const float* rope_sin_k, int64_t rope_k_batch_stride, float scale,
                         float* dq_acc, const int64_t* dq_acc_strides, void* dk, const int64_t* dk_strides, void* dv,
                         const int64_t* dv_strides, void* workspace, size_t workspace_bytes, uint32_t flags,
                         avattn_stream_t stream) {
  if (flags & ~(AVATTN_BWD_REUSE_QUERY_SIDE | AVATTN_BWD_STAGE_DS)) return AVATTN_ERR_ARGUMENT;
  int st = check_tables(rope_cos_q, rope_sin_q, rope_q_batch_stride);
  if (st == AVATTN_OK) st = check_tables(rope_cos_k, rope_sin_k, rope_k_batch_stride);
  if (st != AVATTN_OK) return st;
  RingOpts ring;
  ring.cos_q = rope_cos_q;
  ring.sin_q = rope_sin_q;
  ring.rqsb = rope_q_batch_stride;
  ring.cos_k = rope_cos_k;
  ring.sin_k = rope_sin_k;
  ring.rksb = rope_k_batch_stride;
  return bwd_impl(dout, q, k, v, out, lse, dout_strides, q_strides, k_strides, v_strides, out_strides, batch, heads_q,
                  heads_kv, len_q, len_k, head_dim, key_mask, key_mask_batch_stride, scale, dq_acc, dq_acc_strides, dk,
                  dk_strides, dv, dv_strides, workspace, workspace_bytes, flags | AVATTN_BWD_DQ_ACCUMULATE_F32,
                  stream, nullptr, nullptr, 0, &ring);
}

int avattn_ring_dq_finish(const float* dq_acc, const int64_t* dq_acc_strides, int32_t batch, int32_t heads,
                          int32_t len, int32_t head_dim, const float* rope_cos, const float* rope_sin,
                          int64_t rope_batch_stride, void* dq, const int64_t* dq_strides, avattn_stream_t stream) {
  if (batch < 0 || heads < 0 || len < 0) return AVATTN_ERR_BAD_SHAPE;
  if (head_dim != 64 && head_dim != 128) return AVATTN_ERR_HEAD_DIM;
  if (!dq_acc_strides || !dq_strides) return AVATTN_ERR_NULL_POINTER;
  int st = check_tables(rope_cos, rope_sin, rope_batch_stride);
  if (st != AVATTN_OK) return st;
  if ((int64_t)batch * heads * len == 0) return AVATTN_OK;
  if (!dq_acc || !dq) return AVATTN_ERR_NULL_POINTER;
  if (!aligned16(dq_acc) || !aligned16(dq) || !strides_ok_f32(dq_acc_strides) || !strides_ok(dq_strides))
    return AVATTN_ERR_LAYOUT;
  if ((int64_t)batch * heads * len > ((int64_t)1 << 40)) return AVATTN_ERR_TOO_LARGE;
  return launch_status(launch_dq_finish(dq_acc, dq_acc_strides[0], dq_acc_strides[1], dq_acc_strides[2], batch, heads,
                                        len, head_dim, rope_cos, rope_sin, rope_batch_stride, static_cast<bf16*>(dq),
                                        dq_strides[0], dq_strides[1], dq_strides[2],
                                        reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free forward
// ---------------------------------------------------------------------------
// The forward's workspace (padded k/v copies, key bias and flags, k row-norm
// maxima) lives in this array instead of a caller buffer.  Each GPU the
// library runs on holds its own copy, at its own address, until the process
// ends.  Nothing in it needs clearing between calls: every region the
// kernels read is fully written by the same call first (the copies, bias and
// flags of every padded key, one norm maximum per 64-key tile).  In host code
// `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[AVATTN_FWD_NOALLOC_SCRATCH];

namespace {

constexpr int kMaxScratchDevices = 128;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device, with that device current).
int scratch_on_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return AVATTN_ERR_LAUNCH;
  if (dev >= kMaxScratchDevices) return AVATTN_ERR_ARGUMENT;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return AVATTN_ERR_LAUNCH;
    if (sdev != dev) return AVATTN_ERR_ARGUMENT;  // the array of another GPU
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) return AVATTN_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AVATTN_OK;
}

}  // namespace

extern "C" int avattn_fwd_noalloc(const void* q, const void* k, const void* v, const int64_t* q_strides,
                                  const int64_t* k_strides, const int64_t* v_strides, int32_t batch, int32_t heads_q,
                                  int32_t heads_kv, int32_t len_q, int32_t len_k, int32_t head_dim,
                                  const uint8_t* key_mask, int64_t key_mask_batch_stride, const float* rope_cos_q,
                                  const float* rope_sin_q, int64_t rope_batch_stride, float scale, void* out,
                                  const int64_t* out_strides, float* lse, avattn_stream_t stream) {
  // Size checks first (no HIP call on a rejected problem); fwd_impl repeats
  // the rest of the validation before it launches anything.
  const int st = check_dims(batch, heads_q, heads_kv, len_q, len_k, head_dim);
  if (st != AVATTN_OK) return st;
  const size_t need = avattn_fwd_workspace_size(batch, heads_kv, len_k, head_dim);
  if (need > AVATTN_FWD_NOALLOC_SCRATCH) return AVATTN_ERR_SCRATCH;
  void* ws = nullptr;
  if (need > 0 && (int64_t)batch * heads_q * len_q > 0) {
    const int s = scratch_on_current_device(reinterpret_cast<hipStream_t>(stream), &ws);
    if (s != AVATTN_OK) return s;
  }
  return fwd_impl(q, k, v, q_strides, k_strides, v_strides, batch, heads_q, heads_kv, len_q, len_k, head_dim,
                  key_mask, key_mask_batch_stride, rope_cos_q, rope_sin_q, rope_batch_stride, false, nullptr,
                  nullptr, scale, out, out_strides, lse, ws, ws ? AVATTN_FWD_NOALLOC_SCRATCH : 0, stream);
}
