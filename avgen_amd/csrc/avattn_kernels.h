// Kernel argument blocks and launchers shared between the kernel files and
// the C-ABI layer.  All strides are in elements; head_dim is contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "avattn_device.h"

namespace avattn {

struct FwdArgs {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  int64_t qsb, qsh, qsl;
  int64_t ksb, ksh, ksl;
  int64_t vsb, vsh, vsl;
  int B, Hq, Hkv, Lq, Lk;
  const uint8_t* mask;
  int64_t msb;
  const float* cos_q;
  const float* sin_q;
  int64_t rsb;
  float scale;       // softmax scale applied to q.k
  float scale_log2;  // scale * log2(e)
  bf16* o;
  int64_t osb, osh, osl;
  float* lse;
  // Padded copies (prep.hip), written by the launcher: k rows, element
  // (b, h, j, d) at ((b*Hkv + h)*Lkp + j)*D + d; v head_dim-major, element
  // (b, h, d, j) at ((b*Hkv + h)*D + d)*Lkp + j.
  bf16* kr;
  bf16* vt;
  float* kbias;  // (B, Lkp): 0 attended / -inf
  int* kfull;    // (B, Lkp/32): 1 if every key of the 32-key tile is attended
  int Lkp;
  // fp8 variant only (null otherwise): per-head scales and the e4m3
  // row-major k copy k8 = e4m3(k / k_scale[hk]), element (b, h, j, d) at byte
  // ((b*Hkv + h)*Lkp + j)*D + d.  q is quantized against the softmax
  // constant and k's scale (attn_fwd.hip); q_scale[h] only bounds |q| / 448.
  const float* q_scale;
  const float* k_scale;
  uint8_t* k8;
  // Largest squared row norm of k (bf16 path) or of k8 in e4m3 units (fp8)
  // per 64-key tile, (b, kv head, tile) at ((b*Hkv + h)*(Lkp/64) + tile),
  // float bits (written by the k copy): the largest over a head bounds every
  // score of a query row by |q_row| * sqrt(max).
  uint32_t* kmax2;
  // Key windows (null: every key): query row i of batch b attends to keys
  // [wlo[b*wsb + i], whi[b*wsb + i]) (and the key mask), shared by all heads.
  const int* wlo;
  const int* whi;
  int64_t wsb;
  // K rotation (null: k is used as given): the k copy rotates row j of batch
  // b with the tables (b, 0, j, pair) at b*rksb + j*(D/2) + pair, as q is
  // rotated on load with cos_q/sin_q.
  const float* cos_k;
  const float* sin_k;
  int64_t rksb;
  // Ring step (null o_acc: a plain forward writing o and lse): this chunk's
  // (bf16-rounded output, lse) is merged into the running fp32 accumulator
  // o_acc (B, Hq, Lq, D) contiguous and lse_acc (B, Hq, Lq) with the ring
  // merge (lse_merge_coeffs); acc_first: the accumulator holds nothing yet
  // and takes this chunk's result; acc_final: also write bf16(merged) to o.
  float* o_acc;
  float* lse_acc;
  bool acc_first;
  bool acc_final;
};

struct BwdArgs {
  const bf16* dout;
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* out;
  const float* lse;
  int64_t dosb, dosh, dosl;
  int64_t qsb, qsh, qsl;
  int64_t ksb, ksh, ksl;
  int64_t vsb, vsh, vsl;
  int64_t osb, osh, osl;
  int B, Hq, Hkv, Lq, Lk;
  const uint8_t* mask;
  int64_t msb;
  float scale;
  float scale_log2;
  bf16* dq;
  int64_t dqsb, dqsh, dqsl;
  bf16* dk;
  int64_t dksb, dksh, dksl;
  bf16* dv;
  int64_t dvsb, dvsh, dvsl;
  // Workspace (written by the launcher's first kernels).
  // Per query row (b, hq, i) at index (b*Hq + hq)*Lqp + i, i < Lqp:
  float* ndelta;  // -rowsum(dout * out); 0 for padded rows
  float* lse2;    // lse * log2(e); +inf for rows with lse == -inf and padded rows
  // Padded copies (prep.hip) with H/Lp = Hq/Lqp (q, dout) or Hkv/Lkp
  // (k, v): row copies (*r) hold element (b, h, j, d) at ((b*H + h)*Lp + j)*D
  // + d, head_dim-major copies (*t) at ((b*H + h)*D + d)*Lp + j.
  bf16* qr;
  bf16* dor;
  bf16* kr;
  bf16* vr;
  bf16* kt;
  float* kbias;  // (B, Lkp): 0 attended / -inf
  int* kfull;    // (B, Lkp/32): 1 if every key of the 32-key tile is attended
  int Lqp, Lkp;
  // dq as an fp32 accumulator (dq_acc += this chunk's dq; dq is then null),
  // strides dqsb/dqsh/dqsl in floats.
  float* dq_acc;
  // The query-side preparation (q/dout copies, lse2, ndelta) is already in
  // the workspace: skip it.
  bool reuse_q;
  // Pass over the flattened (b, kv head) pairs kv0 .. kv0 + nkv - 1 (b*Hkv +
  // hk); the whole problem unless dS is staged in several passes.
  int kv0, nkv;
  // Staged dS (null: the dQ kernel recomputes S and dP from q, k, v, dout).
  // The dK/dV kernel stores dS = P * (dP - delta) in bf16 for every query
  // head of its pass (masked keys and keys past the end as 0) and the dQ
  // kernel contracts it with K^T.  Unit (bq, qg, kt), bq = b*Hq + hq -
  // kv0*group, qg = 32-row query group (Lqp/32 of them), kt = 128-key block
  // (ceil(Lk/128) of them), is 8 KB at byte ((bq*(Lqp/32) + qg)*nkt + kt) *
  // 8192, ordered [k2 (2)][128 keys][16 rows]: row 16*k2 + r of key j at
  // bf16 (k2*128 + j)*16 + r, so a dS wave stores 8 consecutive rows of its
  // key as 16 bytes (1 KB per instruction) and the dQ kernel reads 8
  // consecutive keys of a row with two transposed LDS reads.
  bf16* ds;
  // With ds: leave dq to launch_bwd_dq_staged (a later call on the same
  // workspace, possibly on another stream).
  bool defer_dq;
  // Key windows as in FwdArgs (null: every key); non-decreasing in the row
  // (lo and hi), staged dS only.
  const int* wlo;
  const int* whi;
  int64_t wsb;
  // Compact dS layout for key windows (null: the dense unit layout above).
  // Per 64-row query tile T of batch b, four ints at ds_tab + (b*ds_tsb +
  // T)*4: the first 128-key block the tile's rows admit (kb_lo), the number
  // of blocks (nblk; the dK/dV kernel visits tile T from block kt iff kb_lo
  // <= kt < kb_lo + nblk), the unit index of the tile's first 32-row group
  // within its query head's units (gbase), unused.  Group 2T + h, block kt is
  // unit bq*ds_units + gbase + h*nblk + (kt - kb_lo); each query head of a
  // pass owns ds_units units (at least twice the sum of nblk over its tiles).
  const int* ds_tab;
  int64_t ds_tsb;
  int64_t ds_units;
  // RoPE fused into the backward (null: q and k are used as given): q and k
  // are the unrotated inputs; the query-side copies and the recomputing dQ
  // kernel rotate q with cos_q/sin_q (b*rqsb + i*(D/2) + pair), the k copies
  // and the dK/dV kernel's own key rows rotate k with cos_k/sin_k, and dk is
  // written as the transposed rotation of the rotated key's gradient
  // (rounded to bf16 first).  dq stays the rotated query's gradient (the
  // ring finishes it once over all chunks, avattn_ring_dq_finish).
  const float* cos_q;
  const float* sin_q;
  int64_t rqsb;
  const float* cos_k;
  const float* sin_k;
  int64_t rksb;
  // Split of the dK/dV grid's partial last round (null: no split; see
  // plan_tail_split): the last nsplit 128-key blocks of a pass each go to
  // nparts workgroups, one per range of query tiles, which store fp32
  // partial sums in slot (block - first split block) * nparts + part of
  // 256 x D floats (dv rows, then dk rows); a reduction kernel adds the
  // parts in order and writes dk and dv.
  float* split_part;
  int nsplit, nparts;
};

// Partial-sum slots of the dK/dV tail split, 256 x D floats each; the
// region is there when the grid (one workgroup per 128-key block) has more
// workgroups than a 256-CU device runs at once.
constexpr int kSplitSlots = 512;
inline size_t split_part_bytes(int64_t dkv_blocks, int D) {
  return dkv_blocks > 256 ? (size_t)kSplitSlots * 256 * D * sizeof(float) : 0;
}

// Split of a grid's partial last round.  A grid of `total` equal workgroups,
// one per CU at a time on `cus` CUs, leaves r = total % cus of them alone in
// its last round; giving each of those r to p workgroups of 1/p the work
// makes that round ceil(r p / cus) / p as long.  Returns the p in 2..8 (r p
// within max_slots) that makes it shortest, the smaller on ties, or no split
// ({0, 0}) when none is shorter or the grid fits in one round.
struct TailSplit {
  int nsplit, nparts;
};
inline TailSplit plan_tail_split(int64_t total, int cus, int max_slots) {
  TailSplit t{0, 0};
  if (cus <= 0 || total <= cus) return t;
  const int r = (int)(total % cus);
  if (r == 0) return t;
  int best_num = 1, best_den = 1;  // round length best_num / best_den
  for (int p = 2; p <= 8 && r * p <= max_slots; ++p) {
    const int num = (r * p + cus - 1) / cus;
    if (num * best_den < best_num * p) {
      best_num = num;
      best_den = p;
      t = TailSplit{r, p};
    }
  }
  return t;
}

// Bytes of staged dS per (b, kv head) pair: dense, or the compact layout's
// units_per_head units per query head.
inline size_t ds_bytes_per_kv(int group, int Lq, int Lk, int64_t units_per_head = 0) {
  if (units_per_head > 0) return (size_t)group * (size_t)units_per_head * 8192;
  const size_t Lqp = (size_t)(Lq + 63) / 64 * 64;
  return (size_t)group * (Lqp / 32) * (size_t)((Lk + 127) / 128) * 8192;
}

// Kernel ids of the opt-in launch timer (avattn_timing_* in include/avattn.h).
enum KernelId : int {
  kKidFwd = 0,
  kKidBwdPre = 1,
  kKidBwdDkdv = 2,
  kKidBwdDq = 3,
  kKidMerge = 4,
  kKidRopeApply = 5,
  kKidRopeTables = 6,
  kKidTranspose = 7,
  kKidFwdFp8 = 8,
  kKidAbsmax = 9,
  kKidBwdDqDs = 10,
  kKidQkNorm = 11,
  kKidQkNormBwd = 12,
  kKidDqFinish = 13,
  kKidDkdvReduce = 14,
  kKidDiag = 15,
};

// Records HIP events around one launch on `stream` while timing is enabled.
class LaunchTimer {
 public:
  LaunchTimer(int kernel_id, hipStream_t stream);
  ~LaunchTimer();
  LaunchTimer(const LaunchTimer&) = delete;
  LaunchTimer& operator=(const LaunchTimer&) = delete;

 private:
  int slot_;
  hipStream_t stream_;
};

// Sequence length of a padded copy (prep.hip): whole 64-row tiles.  In 64
// bits, so that the validation of a length near INT32_MAX sees the true
// padded length; validated problems fit in int.
inline int64_t transpose_padded_len(int64_t L) { return (L + 63) / 64 * 64; }

// Padded key bias (B, Lkp) floats (0 attended / -inf) and per-32-key-tile
// "all attended" flags (B, Lkp/32); mask may be null (only the tail is masked).
hipError_t launch_key_prep(const uint8_t* mask, int64_t msb, int B, int Lk, float* kbias, int* kfull,
                           hipStream_t stream);

// x (B, H, L, D) strided -> xr (B*H, Lp, D) and/or xt (B*H, D, Lp), contiguous,
// zero padded to Lp = transpose_padded_len(L); either output may be null.
// With rowmax2 set (B*H*(Lp/64) words), also the largest squared row norm of
// each 64-row tile of each (b, h) slice, as float bits.
// With cos/sin tables (b, 0, i, pair) at b*tsb + i*(D/2) + pair, rows are
// rotated (rotate8) before they are copied.
hipError_t launch_prep_copies(const bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                              bf16* xr, bf16* xt, hipStream_t stream, uint32_t* rowmax2 = nullptr,
                              const float* cos_t = nullptr, const float* sin_t = nullptr, int64_t tsb = 0);

// dq (bf16, strided) = transposed rotation of bf16(dq_acc) (fp32, strided);
// a plain cast when cos_t is null.
hipError_t launch_dq_finish(const float* acc, int64_t asb, int64_t ash, int64_t asl, int B, int H, int L, int D,
                            const float* cos_t, const float* sin_t, int64_t tsb, bf16* dq, int64_t dsb, int64_t dsh,
                            int64_t dsl, hipStream_t stream);

// Per-head e4m3 scales of x (B, H, L, D) strided: scale[h] = max|x[:, h]| / 448
// (1 for an all-zero head).  `bits` (H words) holds the running maxima; it
// may alias `scale`.
hipError_t launch_absmax_scales(const bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                                float* scale, uint32_t* bits, hipStream_t stream);

// x (B, H, L, D) strided -> e4m3 row-major copy (B*H, Lp, D) bytes of
// x * (1 / scale[h]), zero padded to Lp = transpose_padded_len(L); with
// rowmax2 set, also the largest squared norm of the quantized rows of each
// 64-row tile, rowmax2[(b*H + h)*(Lp/64) + tile] (float bits).
hipError_t launch_quantize_rows(const bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                                const float* scale, uint8_t* out, uint32_t* rowmax2, hipStream_t stream);

// Forward; the fp8 q k^T variant when a.k8 is set (a.q_scale, a.k_scale too).
hipError_t launch_fwd(const FwdArgs& a, int head_dim, hipStream_t stream);
hipError_t launch_empty(bf16* o, int64_t osb, int64_t osh, int64_t osl, int B, int H, int L, int D, float* lse,
                        hipStream_t stream);
// Backward.  With a.ds set, the (b, kv head) pairs go in passes of
// kv_per_pass, each staging its dS in a.ds (ds_bytes_per_kv bytes per pair).
hipError_t launch_bwd(const BwdArgs& a, int head_dim, int kv_per_pass, hipStream_t stream);
// dQ from the dS and K^T copy a deferred launch_bwd left in the workspace
// (every (b, kv head) pair in one pass).
hipError_t launch_bwd_dq_staged(const BwdArgs& a, int head_dim, hipStream_t stream);
// Fused q/k RMSNorm + rotation (qk_norm.hip).  Rows (b, h, i) of x, dy,
// out and dx at b*sb + h*sh + i*sl (elements), head_dim contiguous.
struct QkNormArgs {
  const bf16* x;
  int64_t xsb, xsh, xsl;
  int B, H, L;
  const bf16* w;     // (head_dim) gain, or null for none
  float eps;
  const float* ct;   // rotation tables (b, 0, i, pair) at b*tsb + i*head_dim/2 + pair; null: no rotation
  const float* st;
  int64_t tsb;
  bf16* out;         // forward output
  int64_t osb, osh, osl;
  const bf16* dy;    // backward: gradient of the output
  int64_t dsb, dsh, dsl;
  bf16* dx;          // backward: gradient of x
  int64_t xgb, xgh, xgl;
  float* wpart;      // backward: per-block dW partials (qk_norm_bwd_workspace_bytes), null without a gain
};
size_t qk_norm_bwd_workspace_bytes(int head_dim);
hipError_t launch_qk_norm(const QkNormArgs& a, int head_dim, hipStream_t stream);
// Backward; with a.wpart also dw (head_dim floats) = the gain's gradient.
hipError_t launch_qk_norm_bwd(const QkNormArgs& a, int head_dim, float* dw, hipStream_t stream);
// dw[0 .. head_dim) = 0 (the gain gradient of an empty input).
hipError_t launch_qk_norm_dw_zero(float* dw, int head_dim, hipStream_t stream);

hipError_t launch_zero_rows(bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                            hipStream_t stream);
hipError_t launch_lse_merge(float* out_acc, float* lse_acc, const void* out_blk, const float* lse_blk, int64_t rows,
                            int D, bool blk_bf16, hipStream_t stream);
hipError_t launch_rope_tables(const float* coords, int64_t csb, int64_t csr, int B, int L, int P,
                              const float* inv_freq, const int32_t* axis_of_pair, const int32_t* apply_mul,
                              const float* pos_mul, const int32_t* apply_div, const float* pos_div, float* cos_out,
                              float* sin_out, hipStream_t stream);
hipError_t launch_rope_apply(const bf16* x, int64_t xsb, int64_t xsh, int64_t xsl, int B, int H, int L, int D,
                             const float* cos_tab, const float* sin_tab, int64_t tsb, bool inverse, bf16* out,
                             int64_t osb, int64_t osh, int64_t osl, hipStream_t stream);

}  // namespace avattn
