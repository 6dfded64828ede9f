/*
 * avattn.h — C ABI of the MI355X (gfx950) video-DiT attention hot path.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * launches on the caller's HIP stream, never allocates and never frees, and
 * returns an AVATTN_* status code (0 = success).  No call synchronises the
 * device.  Inputs are read-only.
 *
 * Tensor conventions (matching the reference's Python boundary):
 *   q, k, v, out, dq, dk, dv : bf16, logical shape (batch, heads, seq, head_dim),
 *                              arbitrary batch/head/seq strides (in elements),
 *                              head_dim contiguous, 16-byte aligned rows.
 *   lse                      : float32, contiguous (batch, heads_q, len_q),
 *                              natural log; -inf for a query whose keys are all
 *                              masked (its output row is 0).
 *   key_mask                 : uint8/bool (batch, len_k), nonzero = attend;
 *                              NULL = every key valid.
 *   rope cos/sin tables      : float32 (batch, 1, seq, head_dim/2).
 *
 * Reference interfaces replaced (paths relative to the avgen source tree,
 * torch/... = the installed PyTorch):
 *   avattn_fwd          src/avgen/models/attention.py:227-273 (attention ->
 *                       F.scaled_dot_product_attention) and the ring local
 *                       step torch/.../_context_parallel/_attention.py:468-474
 *                       (aten::_scaled_dot_product_flash_attention -> out, lse)
 *   avattn_bwd          torch/.../_context_parallel/_attention.py:567-575
 *                       (aten::_scaled_dot_product_flash_attention_backward)
 *   avattn_lse_merge    torch/.../_context_parallel/_attention.py:138-223
 *                       (_SDPAMerger._merge_one, formula :182-183)
 *   avattn_rope_tables  src/avgen/models/rope.py:218-294 (build_rotary_tables)
 *   avattn_rope_apply   src/avgen/models/rope.py:297-338 (apply_rotary) and
 *                       its autograd backward
 *   avattn_fwd_fp8,     no counterpart in the reference (its attention is
 *   avattn_fp8_absmax_scales   bf16 SDPA only): the fp8 (e4m3) q k^T forward
 *                       of the sampling-time CFG configuration, a drop-in for
 *                       attention() (src/avgen/models/attention.py:227-273)
 *                       where fp8 scores are acceptable
 *   avattn_fwd_windowed, src/avgen/models/blocks.py:54-104 (the dense
 *   avattn_bwd_windowed  temporal_neighbour_mask fed to attention) and
 *                       src/avgen/data/packing.py:181-200 (the packed
 *                       block-diagonal mask) as per-row key windows
 *   avattn_qk_norm_rope, src/avgen/models/layers.py:530-536 (q_norm/k_norm
 *   avattn_qk_norm_rope_bwd  then apply_rotary) and their autograd backward
 *   avattn_fwd_f32,     the same interfaces as avattn_fwd / avattn_bwd /
 *   avattn_bwd_f32,     avattn_rope_apply / avattn_fwd_windowed /
 *   avattn_fwd_windowed_f32,  avattn_bwd_windowed for float32 tensors (the
 *   avattn_bwd_windowed_f32,  reference's attention and rotation run in
 *   avattn_bwd_f32_staged_workspace_size,  the caller's dtype; its CPU
 *   avattn_rope_apply_f32,  tests and config c1 are float32)
 *   avattn_qk_norm_rope_f32,  avattn_qk_norm_rope(_bwd) for float32 rows
 *   avattn_qk_norm_rope_bwd_f32  (a float32 model's q_norm/k_norm, with
 *                       the gain in fp32, then apply_rotary)
 */
#ifndef AVATTN_H
#define AVATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque HIP stream handle (hipStream_t); NULL = the default stream. */
typedef void* avattn_stream_t;

/* Status codes. */
#define AVATTN_OK                   0
#define AVATTN_ERR_NULL_POINTER     1  /* a required pointer is NULL               */
#define AVATTN_ERR_BAD_SHAPE        2  /* negative/zero size where not allowed     */
#define AVATTN_ERR_HEAD_DIM         3  /* head_dim not supported (64 or 128)       */
#define AVATTN_ERR_GQA              4  /* heads_q not a multiple of heads_kv       */
#define AVATTN_ERR_LAYOUT           5  /* misaligned pointer / row stride          */
#define AVATTN_ERR_WORKSPACE        6  /* workspace missing or too small           */
#define AVATTN_ERR_LAUNCH           7  /* HIP reported an error at launch          */
#define AVATTN_ERR_TOO_LARGE        8  /* a size exceeds the 32-bit index range    */
#define AVATTN_ERR_ARGUMENT         9  /* other invalid argument                   */
#define AVATTN_ERR_SCRATCH         10  /* avattn_fwd_noalloc: problem exceeds its  */
                                       /* fixed device scratch                     */

/* Human-readable text for a status code (static storage, never NULL). */
const char* avattn_strerror(int status);

/* ABI version; bumped on any signature change. */
int avattn_abi_version(void);

/*
 * Forward: out = softmax(scale * q k^T + mask_bias) v, lse = logsumexp rows.
 * Replaces attention() (src/avgen/models/attention.py:227-273) and the ring
 * local step op (torch/.../_context_parallel/_attention.py:468-474).
 *
 * q_strides/k_strides/v_strides/out_strides: 3 entries each (batch, head, seq),
 * in elements.  heads_kv must divide heads_q (grouped-query attention).
 * key_mask may be NULL; otherwise key_mask[b * key_mask_batch_stride + j].
 * rope_cos_q/rope_sin_q may be NULL; when given, q is rotated on load with the
 * interleaved-pair rotation of src/avgen/models/rope.py:332-338 (fp32 math,
 * bf16 round) before q k^T — table element (b, 0, i, p) at
 * b * rope_batch_stride + i * (head_dim/2) + p.
 * A zero len_q or len_k writes zeros to out (and -inf to lse) without a
 * compute launch (src/avgen/models/attention.py:261-262).
 * workspace must hold avattn_fwd_workspace_size() bytes (16-byte aligned);
 * it is scratch for this call only (padded copies of k and v, key bias).
 */
int avattn_fwd(const void* q, const void* k, const void* v,
               const int64_t* q_strides, const int64_t* k_strides,
               const int64_t* v_strides,
               int32_t batch, int32_t heads_q, int32_t heads_kv,
               int32_t len_q, int32_t len_k, int32_t head_dim,
               const uint8_t* key_mask, int64_t key_mask_batch_stride,
               const float* rope_cos_q, const float* rope_sin_q,
               int64_t rope_batch_stride,
               float scale,
               void* out, const int64_t* out_strides,
               float* lse,
               void* workspace, size_t workspace_bytes,
               avattn_stream_t stream);

/*
 * avattn_fwd without a workspace argument and without any allocation: no
 * counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The operand copies and key statistics avattn_fwd keeps
 * in its workspace go to a fixed device array of AVATTN_FWD_NOALLOC_SCRATCH
 * bytes that the library holds on each GPU it runs on until the process
 * ends; a problem whose avattn_fwd_workspace_size() exceeds it returns
 * AVATTN_ERR_SCRATCH (nothing launched).  The caller still provides q, k, v,
 * out and lse.  The stream must belong to the current device.  Calls that
 * overlap on one GPU (concurrent streams, threads) share the array and race:
 * order them.  The first call on a device looks the array up
 * (hipGetSymbolAddress) and may return AVATTN_ERR_LAUNCH if that fails.
 * Every other argument and result is that of avattn_fwd, bit for bit.
 */
#define AVATTN_FWD_NOALLOC_SCRATCH ((size_t)64 << 20)
int avattn_fwd_noalloc(const void* q, const void* k, const void* v,
                       const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides,
                       int32_t batch, int32_t heads_q, int32_t heads_kv,
                       int32_t len_q, int32_t len_k, int32_t head_dim,
                       const uint8_t* key_mask, int64_t key_mask_batch_stride,
                       const float* rope_cos_q, const float* rope_sin_q,
                       int64_t rope_batch_stride,
                       float scale,
                       void* out, const int64_t* out_strides,
                       float* lse,
                       avattn_stream_t stream);

/*
 * Workspace bytes avattn_fwd needs for these sizes: a row-major copy of k and
 * a head_dim-major copy of v, sequences padded to a multiple of 64, plus the
 * padded per-key bias and per-32-key flags (0 when there is nothing to do).
 */
size_t avattn_fwd_workspace_size(int32_t batch, int32_t heads_kv, int32_t len_k, int32_t head_dim);

/*
 * Workspace bytes avattn_bwd needs for these sizes: two floats per query row
 * (softmax statistics), row-major copies of q and dout,
 * row-major copies of k and v and a head_dim-major copy of k (sequences
 * padded to multiples of 64), plus the padded per-key bias and per-32-key
 * flags, plus, when batch * heads_kv * ceil(len_k / 128) (dK/dV
 * workgroups) exceeds 256, 512 * 256 * head_dim floats of partial sums for
 * the workgroups that share the dK/dV grid's last round (0 when there is
 * nothing to do).
 */
size_t avattn_bwd_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                 int32_t len_q, int32_t len_k, int32_t head_dim);

/*
 * Workspace bytes avattn_bwd needs with AVATTN_BWD_STAGE_DS when
 * kv_pairs_per_pass (batch, kv head) pairs are done per pass: the
 * avattn_bwd_workspace_size() part, rounded up to 4 KB, plus the staged dS of
 * that many pairs, 2 bytes per (query head of the pair, query row, key) with
 * rows padded to 64 and keys to 128 (capped at batch*heads_kv pairs; 0 for
 * empty or invalid sizes).  No counterpart in the reference (torch's flash
 * backward keeps dS on chip and sums dQ with atomics).
 */
size_t avattn_bwd_staged_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                        int32_t len_q, int32_t len_k, int32_t head_dim,
                                        int32_t kv_pairs_per_pass);

/*
 * Forward with q k^T on fp8 (OCP e4m3) operands: per-head scales
 * q_scale[heads_q], k_scale[heads_kv] (device float32, e.g. from
 * avattn_fp8_absmax_scales).  k8 = e4m3(k * (1/k_scale[hk])) (fp32 multiply
 * by the correctly rounded reciprocal); q is quantized against the softmax
 * constant and k's scale, q8 = e4m3(q * (g * 2^-eq)) with
 * g = (scale * log2 e) * k_scale[hk] and 2^eq the smallest power of two
 * >= g * q_scale[h] (fp32 products, eq clamped to [-126, 127]); scores =
 * 2^eq * (q8 . k8) * ln 2 (~ scale * q.k).  Round to nearest even, no
 * saturation: |q / q_scale| and |k / k_scale| must stay below 448 (464
 * for k).  P, V and the output
 * accumulation are as in avattn_fwd (bf16 P, fp32 accumulate), and so are
 * the arguments, masks, GQA, lse and zero-length behaviour; there is no RoPE
 * argument (pass rotated q and k).  workspace must hold
 * avattn_fwd_fp8_workspace_size() bytes (an e4m3 copy of k, a head_dim-major
 * copy of v, key bias and flags).  Forward only (no backward).
 */
int avattn_fwd_fp8(const void* q, const void* k, const void* v,
                   const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides,
                   int32_t batch, int32_t heads_q, int32_t heads_kv,
                   int32_t len_q, int32_t len_k, int32_t head_dim,
                   const uint8_t* key_mask, int64_t key_mask_batch_stride,
                   const float* q_scale, const float* k_scale,
                   float scale,
                   void* out, const int64_t* out_strides,
                   float* lse,
                   void* workspace, size_t workspace_bytes,
                   avattn_stream_t stream);

/* Workspace bytes avattn_fwd_fp8 needs (0 when there is nothing to do). */
size_t avattn_fwd_fp8_workspace_size(int32_t batch, int32_t heads_kv, int32_t len_k, int32_t head_dim);

/*
 * Per-head e4m3 scales of x (batch, heads, len, head_dim) bf16 (strides as
 * for q): scale_out[h] = max |x[:, h, :, :]| / 448 over every batch, position
 * and channel of head h, in fp32 (correctly rounded division), or 1 for an
 * all-zero head; x must be finite.  scale_out: device float32[heads], also
 * used as the scratch of the running maxima (no workspace).
 */
int avattn_fp8_absmax_scales(const void* x, const int64_t* x_strides,
                             int32_t batch, int32_t heads, int32_t len,
                             int32_t head_dim, float* scale_out,
                             avattn_stream_t stream);

/*
 * Backward of avattn_fwd with recomputation of the probabilities from
 * (q, k, lse): given dout, returns dq, dk, dv.  Replaces
 * aten::_scaled_dot_product_flash_attention_backward as called by the ring
 * (torch/.../_context_parallel/_attention.py:567-575): out/lse may be the
 * *merged* output and LSE of all KV chunks, in which case dq/dk/dv are this
 * chunk's contributions.  dk/dv of a masked key are exactly 0.  With
 * heads_kv < heads_q, dk/dv sum over the query heads of each group.
 * workspace must hold avattn_bwd_workspace_size() bytes; its query-side part
 * (statistics and the q/dout copies, at offsets that depend only on batch,
 * heads_q, len_q and head_dim) may be kept between calls, everything else is
 * scratch for this call.
 * flags (bitwise or, 0 = neither):
 *   AVATTN_BWD_REUSE_QUERY_SIDE  the workspace already holds the query-side
 *       preparation of a previous avattn_bwd call with the same dout, q, out,
 *       lse, scale, batch, heads_q, len_q and head_dim (e.g. the previous KV
 *       chunk of one ring step); it is not recomputed.  The caller asserts
 *       this; stale contents give wrong gradients.
 *   AVATTN_BWD_DQ_ACCUMULATE_F32 dq is float32 (strides in float elements,
 *       multiples of 4, 16-byte aligned) and this chunk's dq is added to it
 *       in fp32 (before any rounding) instead of being written as bf16: the
 *       fp32 dq sum over KV chunks of the ring backward
 *       (torch/.../_context_parallel/_attention.py:505-506, 623, 636) without a
 *       separate add per chunk.
 *   AVATTN_BWD_STAGE_DS           the dK/dV kernel stores dS in the workspace
 *       and dq is one product of dS with k, instead of a second kernel that
 *       recomputes the scores and dP (two of its three products).  The
 *       workspace must hold avattn_bwd_staged_workspace_size() bytes for at
 *       least one pair per pass; the pairs go in passes of as many as fit.
 *       Same results to rounding (dq sums dS rounded to bf16, as the
 *       recomputing kernel does).
 *   AVATTN_BWD_DEFER_DQ           with AVATTN_BWD_STAGE_DS and a workspace
 *       holding every pair's dS: compute dk and dv only (dq / dq_strides are
 *       not used); avattn_bwd_dq_staged on the same workspace then computes
 *       dq, e.g. on another stream while the next KV chunk's dk/dv run.
 */
#define AVATTN_BWD_REUSE_QUERY_SIDE  1u
#define AVATTN_BWD_DQ_ACCUMULATE_F32 2u
#define AVATTN_BWD_STAGE_DS          4u
#define AVATTN_BWD_DEFER_DQ          8u
int avattn_bwd(const void* dout, const void* q, const void* k, const void* v,
               const void* out, const float* lse,
               const int64_t* dout_strides, const int64_t* q_strides,
               const int64_t* k_strides, const int64_t* v_strides,
               const int64_t* out_strides,
               int32_t batch, int32_t heads_q, int32_t heads_kv,
               int32_t len_q, int32_t len_k, int32_t head_dim,
               const uint8_t* key_mask, int64_t key_mask_batch_stride,
               float scale,
               void* dq, const int64_t* dq_strides,
               void* dk, const int64_t* dk_strides,
               void* dv, const int64_t* dv_strides,
               void* workspace, size_t workspace_bytes,
               uint32_t flags,
               avattn_stream_t stream);

/*
 * dq of a backward that avattn_bwd ran with AVATTN_BWD_STAGE_DS |
 * AVATTN_BWD_DEFER_DQ on this workspace and these sizes: dq = scale * dS k
 * from the staged dS and the copy of k in the workspace (the workspace must
 * not be reused in between; order this call after that one, e.g. by an
 * event when it runs on another stream).  flags: 0 (dq bf16, written) or
 * AVATTN_BWD_DQ_ACCUMULATE_F32 (dq fp32, added to), as for avattn_bwd.  No
 * counterpart in the reference (its flash backward returns dq with dk/dv).
 */
int avattn_bwd_dq_staged(int32_t batch, int32_t heads_q, int32_t heads_kv,
                         int32_t len_q, int32_t len_k, int32_t head_dim,
                         float scale, void* dq, const int64_t* dq_strides,
                         void* workspace, size_t workspace_bytes,
                         uint32_t flags, avattn_stream_t stream);

/*
 * Attention with per-query-row key windows: row i of batch b attends to the
 * keys j with window_lo[b*wsb + i] <= j < window_hi[b*wsb + i] (and, if
 * given, key_mask[b, j]), the same for every head; wsb = window_batch_stride
 * (0: one window array for every batch).  int32 device arrays of len_q
 * entries per batch, values clamped into 0 <= lo <= hi <= len_k; a row with
 * an empty window gets out = 0 and lse = -inf.  The forward visits only the
 * 64-key tiles that meet its rows' windows.  The backward (staged dS only:
 * flags must include AVATTN_BWD_STAGE_DS and not AVATTN_BWD_DEFER_DQ)
 * requires lo and hi non-decreasing in the row (sorted time coordinates,
 * packed sequences); it then visits only the query and key tiles that meet.
 * Every other argument, the workspace sizes and the error codes are those of
 * avattn_fwd / avattn_bwd (no RoPE argument: pass rotated q and k).
 * Replaces the dense (B, 1, Lq, Lk) masks of
 * src/avgen/models/blocks.py:54-104 (temporal_neighbour_mask, with sorted
 * time coordinates) and src/avgen/data/packing.py:185-200 (the block-diagonal
 * attention_mask of a packed layout; windows from cu_seqlens, :164-183).
 */
int avattn_fwd_windowed(const void* q, const void* k, const void* v,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides,
                        int32_t batch, int32_t heads_q, int32_t heads_kv,
                        int32_t len_q, int32_t len_k, int32_t head_dim,
                        const uint8_t* key_mask, int64_t key_mask_batch_stride,
                        const int32_t* window_lo, const int32_t* window_hi,
                        int64_t window_batch_stride,
                        float scale,
                        void* out, const int64_t* out_strides,
                        float* lse,
                        void* workspace, size_t workspace_bytes,
                        avattn_stream_t stream);
int avattn_bwd_windowed(const void* dout, const void* q, const void* k, const void* v,
                        const void* out, const float* lse,
                        const int64_t* dout_strides, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides,
                        const int64_t* out_strides,
                        int32_t batch, int32_t heads_q, int32_t heads_kv,
                        int32_t len_q, int32_t len_k, int32_t head_dim,
                        const uint8_t* key_mask, int64_t key_mask_batch_stride,
                        const int32_t* window_lo, const int32_t* window_hi,
                        int64_t window_batch_stride,
                        float scale,
                        void* dq, const int64_t* dq_strides,
                        void* dk, const int64_t* dk_strides,
                        void* dv, const int64_t* dv_strides,
                        void* workspace, size_t workspace_bytes,
                        uint32_t flags,
                        avattn_stream_t stream);

/*
 * avattn_bwd_windowed with the staged dS stored compactly: only the 128-key
 * blocks each 64-row query tile's windows admit, so the workspace (and the
 * number of passes) scales with the admitted (query, key) pairs instead of
 * len_q * len_k.  ds_table (int32 device memory, 16-byte aligned) holds four
 * ints per 64-row tile T = 0 .. ceil(len_q/64)-1 of batch row b at
 * (b * ds_table_batch_stride + T) * 4 (stride 0: one table for every batch
 * row; else at least ceil(len_q/64)):
 *   [0] kb_lo  first 128-key block a row of the tile admits, floor(lo0/128)
 *              with lo0 = clamp(window_lo[first row], 0, len_k);
 *   [1] nblk   blocks kb_lo .. kb_lo+nblk-1: the blocks kt with
 *              lo0 < min(128*(kt+1), len_k) and hi1 > 128*kt, where hi1 =
 *              clamp(window_hi[last valid row], lo1, len_k) and lo1 the
 *              clamped window_lo of that row (0 when lo0 == len_k);
 *   [2] gbase  sum of 2*nblk over the tiles before T (the tile's first unit);
 *   [3] unused.
 * ds_units_per_head: at least 2 * (sum of nblk over a batch row's tiles) for
 * every batch row, below 2^19.  Size the workspace with
 * avattn_bwd_compact_workspace_size().  The results are those of
 * avattn_bwd_windowed, bit for bit.  The table follows from the windows
 * alone; a table that disagrees with them makes results wrong but writes no
 * memory outside the workspace.  No counterpart in the reference (its dense
 * masks have no staged dS).
 */
int avattn_bwd_windowed_compact(const void* dout, const void* q, const void* k, const void* v,
                                const void* out, const float* lse,
                                const int64_t* dout_strides, const int64_t* q_strides,
                                const int64_t* k_strides, const int64_t* v_strides,
                                const int64_t* out_strides,
                                int32_t batch, int32_t heads_q, int32_t heads_kv,
                                int32_t len_q, int32_t len_k, int32_t head_dim,
                                const uint8_t* key_mask, int64_t key_mask_batch_stride,
                                const int32_t* window_lo, const int32_t* window_hi,
                                int64_t window_batch_stride,
                                const int32_t* ds_table, int64_t ds_table_batch_stride,
                                int64_t ds_units_per_head,
                                float scale,
                                void* dq, const int64_t* dq_strides,
                                void* dk, const int64_t* dk_strides,
                                void* dv, const int64_t* dv_strides,
                                void* workspace, size_t workspace_bytes,
                                uint32_t flags,
                                avattn_stream_t stream);

/* Workspace of avattn_bwd_windowed_compact staging the dS of
 * pairs_per_pass (batch, kv head) pairs at once (0 for an empty problem). */
size_t avattn_bwd_compact_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                         int32_t len_q, int32_t len_k, int32_t head_dim,
                                         int32_t pairs_per_pass, int64_t ds_units_per_head);

/*
 * Online-softmax merge of one chunk's (out_blk, lse_blk) into the running
 * (out_acc, lse_acc), in place, in fp32:
 *   out_acc <- out_acc - sigmoid(lse_blk - lse_acc) * (out_acc - out_blk)
 *   lse_acc <- lse_acc - logsigmoid(lse_acc - lse_blk)
 * (torch/.../_context_parallel/_attention.py:182-183).  Rows are
 * (batch*heads*len_q) contiguous rows of head_dim.  out_blk is bf16 when
 * blk_is_bf16 != 0, else fp32.  -inf LSEs (fully masked rows) merge as the
 * identity element: a -inf block leaves the accumulator unchanged and a -inf
 * accumulator takes the block (torch's formula returns NaN there).
 */
int avattn_lse_merge(float* out_acc, float* lse_acc,
                     const void* out_blk, const float* lse_blk,
                     int64_t n_rows, int32_t head_dim, int32_t blk_is_bf16,
                     avattn_stream_t stream);

/*
 * One step of the non-causal ring forward with the rotation and the merge
 * fused in: replaces, per KV chunk, apply_rotary on the query shard and on
 * the chunk's keys (src/avgen/models/rope.py:297-338, called at
 * src/avgen/models/layers.py:535-536), the ring's local attention op
 * (torch/.../_context_parallel/_attention.py:468-474) and
 * _SDPAMerger.step (:182-183; with convert_to_f32, :209-211), and on the last
 * chunk _SDPAMerger.results() (:215-223).
 * q and k are UNROTATED; rope_cos_q/rope_sin_q (tables of the query shard's
 * positions) rotate q on load and rope_cos_k/rope_sin_k (tables of this
 * chunk's positions) rotate k in its operand copy; either pair may be NULL
 * (no rotation).  Tables as for avattn_fwd: element (b, 0, i, p) at
 * b * batch_stride + i * (head_dim/2) + p.
 * out_acc (float32, contiguous (batch, heads_q, len_q, head_dim)) and lse_acc
 * (float32, contiguous (batch, heads_q, len_q)) hold the running merge:
 * this chunk's output, rounded to bf16 as the ring's op returns it, and its
 * LSE are merged into them in fp32 with the formula of avattn_lse_merge
 * (bit-identical to a separate avattn_lse_merge call).  flags:
 *   AVATTN_RING_FIRST  out_acc/lse_acc hold nothing yet (not read): they take
 *                      this chunk's result.
 *   AVATTN_RING_LAST   also write the merged output, cast to bf16, to out
 *                      (out_strides as for avattn_fwd); without it out and
 *                      out_strides are not used and may be NULL.
 * After the last step lse_acc is the ring's LSE.  len_k must be positive.
 * Every other argument, the workspace (avattn_fwd_workspace_size) and the
 * error codes are those of avattn_fwd.
 */
#define AVATTN_RING_FIRST 1u
#define AVATTN_RING_LAST  2u
int avattn_ring_fwd_step(const void* q, const void* k, const void* v,
                         const int64_t* q_strides, const int64_t* k_strides,
                         const int64_t* v_strides,
                         int32_t batch, int32_t heads_q, int32_t heads_kv,
                         int32_t len_q, int32_t len_k, int32_t head_dim,
                         const uint8_t* key_mask, int64_t key_mask_batch_stride,
                         const float* rope_cos_q, const float* rope_sin_q,
                         int64_t rope_q_batch_stride,
                         const float* rope_cos_k, const float* rope_sin_k,
                         int64_t rope_k_batch_stride,
                         float scale,
                         float* out_acc, float* lse_acc,
                         void* out, const int64_t* out_strides,
                         uint32_t flags,
                         void* workspace, size_t workspace_bytes,
                         avattn_stream_t stream);

/*
 * One step of the non-causal ring backward with the rotation fused in:
 * replaces, per KV chunk, the ring's local backward op
 * (torch/.../_context_parallel/_attention.py:567-575) with its fp32 dq sum
 * (:505-506, 623), and the rotation's backward for this chunk's keys
 * (src/avgen/models/rope.py:332-338 through autograd).  q and k are
 * UNROTATED with their tables as in avattn_ring_fwd_step; out/lse are the
 * ring's merged output and LSE.  dq_acc (float32, strides in floats,
 * multiples of 4) gets this chunk's gradient of the ROTATED query added in
 * fp32; avattn_ring_dq_finish turns the sum into dq once all chunks are in.
 * dk is the gradient of the unrotated keys: the rotated keys' gradient
 * rounded to bf16, then the transposed rotation, rounded again (the
 * reference's autograd order); dv as avattn_bwd.  flags: any of
 * AVATTN_BWD_REUSE_QUERY_SIDE and AVATTN_BWD_STAGE_DS (the query-side copies
 * kept in the workspace are the rotated ones); dq accumulation is implied.
 * Every other argument, the workspace sizes and the error codes are those of
 * avattn_bwd.
 */
int avattn_ring_bwd_step(const void* dout, const void* q, const void* k, const void* v,
                         const void* out, const float* lse,
                         const int64_t* dout_strides, const int64_t* q_strides,
                         const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* out_strides,
                         int32_t batch, int32_t heads_q, int32_t heads_kv,
                         int32_t len_q, int32_t len_k, int32_t head_dim,
                         const uint8_t* key_mask, int64_t key_mask_batch_stride,
                         const float* rope_cos_q, const float* rope_sin_q,
                         int64_t rope_q_batch_stride,
                         const float* rope_cos_k, const float* rope_sin_k,
                         int64_t rope_k_batch_stride,
                         float scale,
                         float* dq_acc, const int64_t* dq_acc_strides,
                         void* dk, const int64_t* dk_strides,
                         void* dv, const int64_t* dv_strides,
                         void* workspace, size_t workspace_bytes,
                         uint32_t flags,
                         avattn_stream_t stream);

/*
 * The ring backward's last step for the query shard: dq (bf16) = transposed
 * rotation of bf16(dq_acc), i.e. the fp32 dq sum cast to the input dtype
 * (torch/.../_context_parallel/_attention.py:636) followed by the rotation's
 * backward (src/avgen/models/rope.py:332-338 through autograd); a plain cast
 * when rope_cos/rope_sin are NULL.  Strides: 3 entries (batch, head, seq),
 * head_dim contiguous (floats for dq_acc, bf16 elements for dq).
 */
int avattn_ring_dq_finish(const float* dq_acc, const int64_t* dq_acc_strides,
                          int32_t batch, int32_t heads, int32_t len, int32_t head_dim,
                          const float* rope_cos, const float* rope_sin,
                          int64_t rope_batch_stride,
                          void* dq, const int64_t* dq_strides,
                          avattn_stream_t stream);

/*
 * Rotary tables from physical coordinates (src/avgen/models/rope.py:218-294).
 * coords: float32, element (b, i, a) at b*coords_batch_stride +
 * i*coords_row_stride + a.  inv_freq[p] and axis_of_pair[p] (0=time,
 * 1=height, 2=width) give each pair's inverse frequency and axis; for each
 * axis a, the position is coords[..., a], then multiplied by pos_mul[a] if
 * apply_mul[a] != 0, then divided by pos_div[a] if apply_div[a] != 0 (the
 * time_scale and linear-scaling steps of rope.py:270-277, in that order).
 * inv_freq, axis_of_pair, apply_mul, pos_mul, apply_div and pos_div are HOST
 * pointers (pairs <= 64 entries, or 3 per-axis entries); their values are
 * copied into the launch.  coords, cos_out and sin_out are device pointers.
 * Writes contiguous cos/sin of shape (batch, 1, len, pairs).
 */
int avattn_rope_tables(const float* coords, int64_t coords_batch_stride,
                       int64_t coords_row_stride,
                       int32_t batch, int32_t len, int32_t pairs,
                       const float* inv_freq, const int32_t* axis_of_pair,
                       const int32_t* apply_mul, const float* pos_mul,
                       const int32_t* apply_div, const float* pos_div,
                       float* cos_out, float* sin_out,
                       avattn_stream_t stream);

/*
 * Interleaved-pair rotation of x (src/avgen/models/rope.py:297-338), fp32
 * math with each product rounded separately, result rounded to bf16.
 * inverse == 0: forward rotation (e*c - o*s, e*s + o*c).
 * inverse != 0: the transpose (e*c + o*s, o*c - e*s), i.e. the gradient of the
 * forward rotation as torch autograd evaluates it.
 * x/out strides: 3 entries (batch, head, seq), head_dim contiguous.  The
 * tables are indexed (b, 0, i, p) at b*table_batch_stride + i*pairs + p.
 */
int avattn_rope_apply(const void* x, const int64_t* x_strides,
                      int32_t batch, int32_t heads, int32_t len,
                      int32_t head_dim,
                      const float* cos_tab, const float* sin_tab,
                      int64_t table_batch_stride, int32_t inverse,
                      void* out, const int64_t* out_strides,
                      avattn_stream_t stream);

/*
 * Per-head RMSNorm of q or k rows fused with the rotation: replaces the
 * q_norm / k_norm step and the apply_rotary call that follows it
 * (src/avgen/models/layers.py:530-536; the norm is F.rms_norm with the gain
 * cast to bf16, src/avgen/models/layers.py:106-118; the rotation
 * src/avgen/models/rope.py:297-338).  Per row of head_dim values:
 * rstd = 1/sqrt(mean(x^2) + eps); n = bf16((x*rstd)*weight) (fp32 math);
 * out = bf16 rotation of n as in avattn_rope_apply (inverse 0), or out = n
 * when cos_tab is NULL.  weight: bf16 (head_dim), NULL = no gain.
 * x/out strides: 3 entries (batch, head, seq), head_dim contiguous; a
 * (batch, seq, heads, head_dim) projection output passes as a strided view.
 * head_dim 64 or 128.  Tables as for avattn_rope_apply.
 */
int avattn_qk_norm_rope(const void* x, const int64_t* x_strides,
                        int32_t batch, int32_t heads, int32_t len,
                        int32_t head_dim, const void* weight, float eps,
                        const float* cos_tab, const float* sin_tab,
                        int64_t table_batch_stride,
                        void* out, const int64_t* out_strides,
                        avattn_stream_t stream);

/* Device workspace bytes avattn_qk_norm_rope_bwd needs (dW partials). */
size_t avattn_qk_norm_rope_bwd_workspace_size(int32_t head_dim);

/*
 * Backward of avattn_qk_norm_rope given dy (the gradient of out):
 * g = bf16 transposed rotation of dy (avattn_rope_apply, inverse 1), then the
 * RMSNorm gradient dx = bf16(rstd*(w*g - xh*mean(w*g*xh))), xh = x*rstd,
 * and, when weight is not NULL, dweight (head_dim floats, fp32) = sum over
 * all rows of g*xh, reduced in a fixed order (deterministic).  dy/dx
 * strides as x.  The workspace is used only with a weight.
 */
int avattn_qk_norm_rope_bwd(const void* x, const int64_t* x_strides,
                            const void* dy, const int64_t* dy_strides,
                            int32_t batch, int32_t heads, int32_t len,
                            int32_t head_dim, const void* weight, float eps,
                            const float* cos_tab, const float* sin_tab,
                            int64_t table_batch_stride,
                            void* dx, const int64_t* dx_strides,
                            float* dweight, void* workspace,
                            size_t workspace_bytes, avattn_stream_t stream);

/*
 * Launch timing (diagnostics; no counterpart in the reference, whose kernels
 * are PyTorch's).  While enabled, every kernel launch of this library
 * records a pair of HIP events on its launch stream; avattn_timing_read sums
 * the elapsed times of one kernel kind (it synchronizes on the recorded
 * events).  Kernel ids: 0 forward, 1 backward preprocess, 2 backward dK/dV,
 * 3 backward dQ, 4 LSE merge, 5 rotary apply, 6 rotary tables,
 * 7 operand copies (forward and backward operand preparation, including the
 * fp8 forward's e4m3 k copy), 8 fp8 forward, 9 fp8 absmax scales,
 * 10 dQ from staged dS, 11 q/k norm + rotation, 12 its backward,
 * 13 the ring dq finish (avattn_ring_dq_finish), 14 the sum of the
 * partial results of split dK/dV workgroups, 15 avattn_diag_dq_partials.
 * avattn_timing_begin creates `capacity` event pairs (call it outside any
 * timed or captured region); launches beyond capacity are not recorded and
 * make avattn_timing_read return AVATTN_ERR_WORKSPACE.
 */
int avattn_timing_begin(int32_t capacity);
int avattn_timing_end(void);
int avattn_timing_read(int32_t kernel_id, double* total_ms, int32_t* launches);
int avattn_timing_reset(void);

/*
 * Diagnostic (no counterpart in the reference): replays the dQ accumulation
 * a backward without staged dS would issue, with synthetic partials of 1.0
 * and no other work.  One 512-thread workgroup per (head, 128-key block)
 * adds (atomic != 0: fp32 vector atomics, agent scope) or stores
 * (atomic == 0) one 64 x head_dim fp32 tile for each of tiles_per_block
 * query tiles, starting at tile 2*key_block (mod query_tiles), into
 * acc[heads][query_tiles][64][head_dim] (device float32, 16-byte aligned;
 * the caller's allocation must hold that many floats).  With atomics every
 * element ends up incremented by the number of key blocks that visited its
 * tile.  Time it with the avattn_timing_* diagnostics (kernel id 15).
 */
int avattn_diag_dq_partials(float* acc, int32_t heads, int32_t key_blocks,
                            int32_t query_tiles, int32_t tiles_per_block,
                            int32_t head_dim, int32_t atomic,
                            avattn_stream_t stream);

/*
 * float32 attention: the same contract as avattn_fwd / avattn_bwd /
 * avattn_rope_apply with every tensor (q, k, v, out, dout, dq, dk, dv, x)
 * float32 instead of bf16 and every product computed in fp32, for callers
 * whose tensors are float32 — the reference's attention() runs in the
 * caller's dtype (src/avgen/models/attention.py:227-273 ->
 * F.scaled_dot_product_attention), its rotation in fp32
 * (src/avgen/models/rope.py:332-338), and BASELINE config c1 is float32.
 * Strides are in elements, multiples of 4 (16-byte aligned rows); head_dim
 * 64 or 128 (rotation: any multiple of 4 up to 128).  No rotation is fused
 * into the attention calls: rotate with avattn_rope_apply_f32 first.
 * lse, the key mask and the row states (no valid key: out 0, lse -inf; a
 * NaN or +inf score: NaN) are as for avattn_fwd.  The backward needs
 * avattn_bwd_f32_workspace_size() bytes of workspace (256-byte aligned:
 * the row statistics), uses no atomics and is bitwise reproducible; a
 * masked key's dk and dv are exactly 0.  With a workspace of at least
 * avattn_bwd_f32_staged_workspace_size(..., 1) bytes the dK/dV kernel also
 * stores dS (fp32) past the statistics and dq is one product of dS with k,
 * in equal passes of as many (batch, kv head) pairs as the workspace holds
 * (the same results to rounding as recomputing dq, bitwise independent of
 * the pass size); a smaller workspace recomputes S and dP for dq.
 * Rotation: each product and sum
 * rounded on its own, no final rounding (the output is fp32), so it equals
 * torch's fp32 ops bit for bit.
 */
int avattn_fwd_f32(const float* q, const float* k, const float* v,
                   const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides,
                   int32_t batch, int32_t heads_q, int32_t heads_kv,
                   int32_t len_q, int32_t len_k, int32_t head_dim,
                   const uint8_t* key_mask, int64_t key_mask_batch_stride,
                   float scale,
                   float* out, const int64_t* out_strides,
                   float* lse,
                   avattn_stream_t stream);

size_t avattn_bwd_f32_workspace_size(int32_t batch, int32_t heads_q, int32_t len_q);

/* Workspace bytes for avattn_bwd_f32 staging the dS of kv_pairs_per_pass
 * (batch, kv head) pairs per pass: the statistics rounded up to 4 KB, plus
 * per pair 4 * (heads_q/heads_kv) * roundup(len_q, 32) * roundup(len_k, 128)
 * bytes. */
size_t avattn_bwd_f32_staged_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                            int32_t len_q, int32_t len_k,
                                            int32_t kv_pairs_per_pass);

int avattn_bwd_f32(const float* dout, const float* q, const float* k, const float* v,
                   const float* out, const float* lse,
                   const int64_t* dout_strides, const int64_t* q_strides,
                   const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* out_strides,
                   int32_t batch, int32_t heads_q, int32_t heads_kv,
                   int32_t len_q, int32_t len_k, int32_t head_dim,
                   const uint8_t* key_mask, int64_t key_mask_batch_stride,
                   float scale,
                   float* dq, const int64_t* dq_strides,
                   float* dk, const int64_t* dk_strides,
                   float* dv, const int64_t* dv_strides,
                   void* workspace, size_t workspace_bytes,
                   avattn_stream_t stream);

/*
 * avattn_fwd_f32 / avattn_bwd_f32 with per-query-row key windows, as
 * avattn_fwd_windowed / avattn_bwd_windowed (src/avgen/models/blocks.py:
 * 54-104, the temporal neighbour mask with sorted time coordinates;
 * src/avgen/data/packing.py:181-200, the packed block-diagonal mask): row i
 * of batch b attends the keys j with window_lo[b*wsb + i] <= j <
 * window_hi[b*wsb + i] (and key_mask), values clamped into 0 <= lo <= hi <=
 * len_k; a row with an empty window gets out 0 and lse -inf.  The forward
 * visits only the key tiles meeting its rows' windows.  The backward
 * requires lo and hi non-decreasing in the row; it then visits only the
 * query tiles whose rows meet each key block and, with staged dS, multiplies
 * only the (rows, key block) pairs the dK/dV kernel wrote.  Workspace and
 * errors as avattn_bwd_f32 (staged dS with the staged size).
 */
int avattn_fwd_windowed_f32(const float* q, const float* k, const float* v,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides,
                            int32_t batch, int32_t heads_q, int32_t heads_kv,
                            int32_t len_q, int32_t len_k, int32_t head_dim,
                            const uint8_t* key_mask, int64_t key_mask_batch_stride,
                            const int32_t* window_lo, const int32_t* window_hi,
                            int64_t window_batch_stride,
                            float scale,
                            float* out, const int64_t* out_strides,
                            float* lse,
                            avattn_stream_t stream);

int avattn_bwd_windowed_f32(const float* dout, const float* q, const float* k, const float* v,
                            const float* out, const float* lse,
                            const int64_t* dout_strides, const int64_t* q_strides,
                            const int64_t* k_strides, const int64_t* v_strides,
                            const int64_t* out_strides,
                            int32_t batch, int32_t heads_q, int32_t heads_kv,
                            int32_t len_q, int32_t len_k, int32_t head_dim,
                            const uint8_t* key_mask, int64_t key_mask_batch_stride,
                            const int32_t* window_lo, const int32_t* window_hi,
                            int64_t window_batch_stride,
                            float scale,
                            float* dq, const int64_t* dq_strides,
                            float* dk, const int64_t* dk_strides,
                            float* dv, const int64_t* dv_strides,
                            void* workspace, size_t workspace_bytes,
                            avattn_stream_t stream);

/*
 * avattn_qk_norm_rope / avattn_qk_norm_rope_bwd on float32 rows with a
 * float32 gain (src/avgen/models/layers.py:106-118: outside autocast the
 * gain stays in the activation's dtype, fp32): n = (x*rstd)*w and its
 * rotation in fp32 (each product and sum rounded on its own), no final
 * rounding; backward as the bf16 one in fp32 (dx, and dweight summed in a
 * fixed order).  Arguments, layouts and errors as the bf16 functions
 * (float* instead of void*); the backward workspace is
 * avattn_qk_norm_rope_bwd_workspace_size(head_dim) bytes, used with a gain.
 */
int avattn_qk_norm_rope_f32(const float* x, const int64_t* x_strides,
                            int32_t batch, int32_t heads, int32_t len,
                            int32_t head_dim, const float* weight, float eps,
                            const float* cos_tab, const float* sin_tab,
                            int64_t table_batch_stride,
                            float* out, const int64_t* out_strides,
                            avattn_stream_t stream);

int avattn_qk_norm_rope_bwd_f32(const float* x, const int64_t* x_strides,
                                const float* dy, const int64_t* dy_strides,
                                int32_t batch, int32_t heads, int32_t len,
                                int32_t head_dim, const float* weight, float eps,
                                const float* cos_tab, const float* sin_tab,
                                int64_t table_batch_stride,
                                float* dx, const int64_t* dx_strides,
                                float* dweight,
                                void* workspace, size_t workspace_bytes,
                                avattn_stream_t stream);

int avattn_rope_apply_f32(const float* x, const int64_t* x_strides,
                          int32_t batch, int32_t heads, int32_t len,
                          int32_t head_dim,
                          const float* cos_tab, const float* sin_tab,
                          int64_t table_batch_stride, int32_t inverse,
                          float* out, const int64_t* out_strides,
                          avattn_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* AVATTN_H */
