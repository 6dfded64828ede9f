// Attention backward for gfx950, recomputing the probabilities from (q, k,
// lse) instead of storing them.  No atomics (bitwise reproducible):
//   1. preprocess: per query row, lse2 = lse * log2(e) and
//      ndelta = -rowsum(dout * out) (the `D` term of dS = P * (dP - D)), in
//      arrays padded to whole 64-row tiles (+inf / 0 past the end so padded
//      rows get P = 0); plus the padded operand copies (prep.hip): row-major
//      q and dout, head_dim-major k (and row-major k, v for 3'');
//   2. dK/dV: one workgroup per 128 keys (32 per wave, kept in registers as
//      MFMA operands); loops over 64-row query tiles of every query head
//      that reads this KV head; with staged dS it also stores dS (bf16) to
//      the workspace;
//   3. dQ, either
//      3'. from the staged dS: dQ = scale * dS K, one product, one workgroup
//          per 256 query rows streaming the dS once (bwd_dq_ds_kernel), or
//      3''. recomputing S and dP: one workgroup per 256 query rows (32 per
//          wave), 32-key tiles (bwd_dq_kernel).
// Every MFMA operand read from LDS is one 16-byte chunk of a tile row or two
// 8-byte transposed reads (ds_read_b64_tr_b16) of a row-major tile: the
// products contracting over the sequence read their operands across the
// rows, and the rows feeding the first product are read in perm23 order so
// that their C layout lines up with those eight consecutive rows.
// With out/lse the merged result over all KV chunks, the outputs are one
// chunk's contributions, which is how the ring backward calls the op
// (torch/.../_context_parallel/_attention.py:567-575).
#include <type_traits>

#include "avattn_device.h"
#include "avattn_kernels.h"

namespace avattn {

// ---------------------------------------------------------------------------
// 1. lse2 / ndelta
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdArgs a) {
  constexpr int TPR = D / 8;  // threads per row
  constexpr int RPB = 256 / TPR;
  const int64_t rows = (int64_t)a.B * a.Hq * a.Lqp;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int c = threadIdx.x % TPR;
  const int i = (int)(row % a.Lqp);
  const int64_t bh = row / a.Lqp;
  const bool valid = row < rows && i < a.Lq;
  float acc = 0.f;
  if (valid) {
    const int h = (int)(bh % a.Hq);
    const int b = (int)(bh / a.Hq);
    const u32x4 x = *reinterpret_cast<const u32x4*>(a.dout + b * a.dosb + h * a.dosh + (int64_t)i * a.dosl + 8 * c);
    const u32x4 y = *reinterpret_cast<const u32x4*>(a.out + b * a.osb + h * a.osh + (int64_t)i * a.osl + 8 * c);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      acc = fmaf(__uint_as_float(x[w] << 16), __uint_as_float(y[w] << 16), acc);
      acc = fmaf(__uint_as_float(x[w] & 0xffff0000u), __uint_as_float(y[w] & 0xffff0000u), acc);
    }
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, TPR);
  if (row < rows && c == 0) {
    a.ndelta[row] = -acc;
    if (valid) {
      const float l = a.lse[bh * a.Lq + i];
      a.lse2[row] = (l == kNegInf) ? kPosInf : l * kLog2e;
    } else {
      a.lse2[row] = kPosInf;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. dK / dV
// ---------------------------------------------------------------------------
// One workgroup = 128 keys and 8 waves in two roles; waves w and w+4 own the
// same 32 keys (lane % 32 owns key column kt*128 + 32*(w%4) + lane % 32) and
// run on the same SIMD.  For each 32-row half `sub` of a 64-row query tile
// (lane l supplies query row 32*sub + perm23(l % 32) to the first products):
//   P waves (w < 4):   S  = Q K^T      A = Q rows (LDS)   B = K^T (registers)
//                      P  = exp2(S*c - lse2[q])   -> bf16, handed to the partner
//                      dV^T += dO^T P  A = dO^T (LDS, transposed reads), B = P
//   dS waves (w >= 4): dP = dO V^T     A = dO rows (LDS)  B = V^T (registers)
//                      dS = P * (dP + ndelta[q])  (P from the partner)
//                      dK^T += Q^T dS  A = Q^T (LDS, transposed reads), B = dS
// C-layout register 8*k2 + e of lane l holds query 32*sub + 16*k2 + 8*(l/32)
// + e, so the A operands of the last products are two transposed reads of
// the row tiles (rows +0..3, +4..7), the row statistics 16-byte LDS reads,
// and P travels between the partners as each lane's own registers (one
// 16-byte LDS write and read per 16 rows).
//
// One barrier per tile (T: tile staged).  The dS waves run their dS phase one
// tile behind, so the P they need was written before the last barrier: in
// iteration t a P wave runs QK^T and the softmax of tile t, then dV; its
// partner runs dO V^T of tile t (low priority, MFMAs only), then dS and dK of
// tile t - 1 (high priority), so one wave's VALU work always has the other's
// MFMAs to hide behind.  Keys that are masked (or past the end) are
// not special-cased in the loop: each key's dK/dV column depends only on that
// key, and those columns are written as zeros (or not at all) at the end.
// With STAGE the dS waves also store their dS tiles (BwdArgs::ds).  With WIN
// (key windows non-decreasing in the row, BwdArgs::wlo/whi; staged dS only)
// the workgroup visits only the 64-row tiles whose rows' window union meets
// its keys, and the P waves set the scores outside a row's window to -inf
// in tiles not inside every window (so P and dS are 0 there).
template <int D, bool MASK, bool STAGE, bool WIN, bool CT>
__global__ __launch_bounds__(512, 1) void bwd_dkdv_kernel(BwdArgs a) {
  static_assert(!WIN || STAGE, "windows with staged dS only");
  static_assert(!CT || WIN, "the compact dS layout (BwdArgs::ds_tab) is for windows");
  constexpr int BK = 128, BQ = 64, NW = 8;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int TE = BQ * D;
  // Query tiles are staged as Q rows and as dO rows plus the rows'
  // statistics, three slots of each (tile t in slot t % 3).  The first
  // products read the rows; the last two read the same tiles transposed
  // (ds_read_b64_tr_b16), so no head_dim-major copy is staged.  Tile t's Q
  // is read until the end of iteration t + 1 (dK^T), its dO and statistics
  // until the end of iteration t: during iteration t the Q rows of tile t + 1
  // and the rest of tile t + 2 are loaded, into the slots tiles t - 2 and
  // t - 1 used.
  struct RowStage {
    bf16 dout[TE];  // dO rows: TileLayout<D>
    float lse2[BQ];
    float ndl[BQ];  // ndelta: the dP accumulators start from it
    int wlo[WIN ? BQ : 4];  // key windows of the tile's rows (WIN)
    int whi[WIN ? BQ : 4];
  };
  struct Smem {
    bf16 q[3][TE];  // Q rows: TileLayout<D>
    RowStage rs[3];
    // P hand-over, one buffer per slot (tile t's P is written in iteration t
    // and read in iteration t + 1): 1 KB per (key group, sub, k2),
    // lane-major.
    u32x4 xp[3][4 * 2 * 2 * 64];
  };
  __shared__ __attribute__((aligned(16))) Smem sm;
  // Byte strides of the slots (the reads below add them to per-lane bases).
  constexpr uint32_t kQS = TE * 2, kRS = sizeof(RowStage), kXS = sizeof(sm.xp[0]);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int role = wave >> 2, kw = wave & 3;
  const int l32 = lane & 31, hh = lane >> 5;
  const int prow = perm23(l32);

  const int nkt = (a.Lk + BK - 1) / BK;
  const int total = nkt * a.nkv;
  // Key blocks 0 .. nfull-1 take one workgroup each (query tiles all); the
  // last a.nsplit blocks (the grid's partial last round) take a.nparts
  // workgroups each, one per range of query tiles, whose fp32 partial
  // dK/dV dkv_reduce_kernel sums.
  const int nfull = total - a.nsplit;
  int bid, part = -1;
  if ((int)blockIdx.x < nfull) {
    bid = xcd_remap(blockIdx.x, nfull);
  } else {
    const int i = blockIdx.x - nfull;
    bid = nfull + i / a.nparts;
    part = i % a.nparts;
  }
  const int kt = bid % nkt;
  const int bhk = a.kv0 + bid / nkt;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.Hq / a.Hkv;

  const int key = kt * BK + kw * 32 + l32;
  bool kvalid = key < a.Lk;
  if (MASK && kvalid) kvalid = a.mask[b * a.msb + key] != 0;

  // This wave's B operand: K (P waves, rotated when the backward carries the
  // key's rotation) or V (dS waves) of the lane's key, read once from the
  // caller's tensors; zeros past the end.
  bf16x8 kv[KS];
  {
    const bool in = key < a.Lk;
    const bf16* src = role == 0 ? a.k + b * a.ksb + hk * a.ksh + (int64_t)key * a.ksl + 8 * hh
                                : a.v + b * a.vsb + hk * a.vsh + (int64_t)key * a.vsl + 8 * hh;
    const bool rot = role == 0 && a.cos_k != nullptr;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (in) {
        x = *reinterpret_cast<const u32x4*>(src + 16 * ks);
        if (rot) {
          const int64_t t = b * a.rksb + (int64_t)key * (D / 2) + 8 * ks + 4 * hh;
          x = rotate8(x, *reinterpret_cast<const f32x4*>(a.cos_k + t), *reinterpret_cast<const f32x4*>(a.sin_k + t),
                      false);
        }
      }
      kv[ks] = bits_to_bf16x8(x);
    }
  }

  f32x16 acc[DT];  // dV^T (P waves) or dK^T (dS waves)
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = zero16();

  // Loop-invariant per-lane LDS element offsets.
  int ro[KS];  // row tiles: chunk (16*ks + 8*hh) of row perm23(l32)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) ro[ks] = TileLayout<D>::off(prow, 16 * ks + 8 * hh);
  // Transposed reads of the same tiles (A operands of dV^T += dO^T P and
  // dK^T += Q^T dS): channel block dt, rows 16*(2*sub + k2) + 8*hh + 4*h ..
  // +3 for the read h = 0, 1 (tr_read_off).  Rows advance by 16 per
  // (sub, k2), which keeps the row swizzle, so the offsets are
  // loop-invariant.
  int tro[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int h = 0; h < 2; ++h) tro[dt][h] = tr_read_off<D>(lane, dt, h);
  // Per-lane LDS byte addresses in slot 0 (opaque: slot and row-block
  // offsets go into the reads' offset fields).  P waves read Q as rows and
  // dO transposed, dS waves dO as rows and Q transposed.
  uint32_t rb[KS], tb[DT][2];
  {
    const uint32_t q0 = lds_addr(&sm.q[0][0]), d0 = lds_addr(&sm.rs[0].dout[0]);
    const uint32_t rrow = role == 0 ? q0 : d0, rtr = role == 0 ? d0 : q0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) rb[ks] = opaque(rrow + 2 * ro[ks]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int h = 0; h < 2; ++h) tb[dt][h] = opaque(rtr + 2 * tro[dt][h]);
  }
  // Row statistics of the lane's rows 8*hh + ...: lse2 at sb, ndelta and
  // the windows at the offsets below.
  const uint32_t sb = opaque(lds_addr(&sm.rs[0].lse2[0]) + 32 * hh);
  constexpr uint32_t kNdlOff = BQ * 4, kWloOff = 2 * BQ * 4, kWhiOff = kWloOff + sizeof(sm.rs[0].wlo);
  static_assert(offsetof(RowStage, ndl) - offsetof(RowStage, lse2) == kNdlOff &&
                    offsetof(RowStage, wlo) - offsetof(RowStage, lse2) == kWloOff &&
                    offsetof(RowStage, whi) - offsetof(RowStage, lse2) == kWhiOff,
                "row statistics offsets");
  // This lane's 16 bytes of the P hand-over: + kXS*slot + 1024*(2*sub + k2).
  const uint32_t xb = opaque(lds_addr(&sm.xp[0][0]) + 16 * (kw * 4 * 64 + lane));

  const int nqt = a.Lqp / BQ;
  // Query tiles visited: tq0 .. tq0 + ntq - 1 of every query head of the
  // group (all of them without windows).  With monotone windows, tile T
  // meets this block's keys [k0, k1) iff lo(first row of T) < k1 and
  // hi(last row of T) > k0; both conditions hold on a prefix / suffix of the
  // tiles, so their counts give the range.
  int tq0 = 0, ntq = nqt;
  // WIN: tiles [w_ia, w_ib) hold only rows whose windows cover all 32 keys
  // of this wave (hi(first row) >= kk0 + 32 and lo(last row) <= kk0; each
  // condition holds on a suffix / prefix of the tiles); the others mask
  // scores per (row, key).
  int w_ia = 0, w_ib = 0;
  if constexpr (WIN) {
    __shared__ int cred[NW][2];
    const int k0 = kt * BK, k1 = min(k0 + BK, a.Lk);
    const int* lo = a.wlo + b * a.wsb;
    const int* hi = a.whi + b * a.wsb;
    const int nvt = (a.Lq + BQ - 1) / BQ;  // tiles holding valid rows
    int c_lo = 0, c_hi = 0;
    for (int T = tid; T < nvt; T += NW * 64) {
      const int f = T * BQ, l = min(f + BQ - 1, a.Lq - 1);
      const int lof = min(max(lo[f], 0), a.Lk);
      const int lol = min(max(lo[l], 0), a.Lk);
      const int hil = min(max(hi[l], lol), a.Lk);
      c_hi += lof < k1;
      c_lo += hil <= k0;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      c_lo += __shfl_xor(c_lo, off);
      c_hi += __shfl_xor(c_hi, off);
    }
    if (lane == 0) {
      cred[wave][0] = c_lo;
      cred[wave][1] = c_hi;
    }
    __syncthreads();
    int s_lo = 0, s_hi = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      s_lo += cred[w][0];
      s_hi += cred[w][1];
    }
    tq0 = __builtin_amdgcn_readfirstlane(s_lo);
    ntq = __builtin_amdgcn_readfirstlane(max(s_hi - s_lo, 0));
    const int kk0 = kt * BK + kw * 32;
    int c_a = 0, c_b = 0;
    for (int T = lane; T < nvt; T += 64) {
      const int f = T * BQ, l = min(f + BQ - 1, a.Lq - 1);
      c_a += hi[f] < kk0 + 32;
      c_b += lo[l] <= kk0;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      c_a += __shfl_xor(c_a, off);
      c_b += __shfl_xor(c_b, off);
    }
    w_ia = __builtin_amdgcn_readfirstlane(c_a);
    w_ib = __builtin_amdgcn_readfirstlane(c_b);
  }
  if (part >= 0) {  // this part's share of the tiles (possibly none)
    const int p0 = ntq * part / a.nparts, p1 = ntq * (part + 1) / a.nparts;
    tq0 += p0;
    ntq = p1 - p0;
  }
  const int niter = ntq * group;
  auto tile_head = [&](int it) { return it / ntq; };     // query head within the group
  auto tile_idx = [&](int it) { return tq0 + it % ntq; };  // 64-row tile of that head
  // Buffers over the query heads of this KV head's group (b, hk*group ..).
  const int64_t bq0 = (int64_t)(b * a.Hq + hk * group);
  const uint32_t qbytes = (uint32_t)group * a.Lqp * D * 2;
  const u32x4 rq = make_rsrc(a.qr + bq0 * a.Lqp * D, qbytes);
  const u32x4 rdo = make_rsrc(a.dor + bq0 * a.Lqp * D, qbytes);
  const u32x4 rl2 = make_rsrc(a.lse2 + bq0 * a.Lqp, (uint32_t)group * a.Lqp * 4);
  const u32x4 rnd = make_rsrc(a.ndelta + bq0 * a.Lqp, (uint32_t)group * a.Lqp * 4);
  // A tile is loaded in two parts, one load at a time between MFMAs (a burst
  // of them at the start of a phase would hold up the wave's instruction
  // stream): the dS waves load its Q rows (kQOps loads per wave) during their
  // dP phase of the iteration before, the P waves its dO rows and statistics
  // (kROps) during their dV phase of the iteration before that.
  TileStager<BQ, D, 4> rst;  // 64 rows of D channels (row stride D) over 4 waves
  rst.init(D, kw, lane);
  constexpr int kQOps = TileStager<BQ, D, 4>::kPer;
  constexpr int kROps = kQOps + 2 + (WIN ? 2 : 0);
  auto tile_rows = [&](int it) {  // first row of tile `it` in the group's copies
    return (uint32_t)tile_head(it) * a.Lqp + (uint32_t)tile_idx(it) * BQ;
  };
  // Window arrays of this batch (WIN); rows past Lq read as 0 (empty).
  u32x4 rwl = {0u, 0u, 0u, 0u}, rwh = {0u, 0u, 0u, 0u};
  if constexpr (WIN) {
    rwl = make_rsrc(a.wlo + b * a.wsb, (uint32_t)a.Lq * 4);
    rwh = make_rsrc(a.whi + b * a.wsb, (uint32_t)a.Lq * 4);
  }
  // Q load i of tile `it` into Q slot `qd`.
  auto q_op = [&](int it, bf16* qd, int i) { rst.stage_one(qd, rq, tile_rows(it) * D * 2, i); };
  // Row load i of tile `it` into row slot `rsg`.
  auto r_op = [&](int it, RowStage& rsg, int i) {
    const uint32_t row0 = tile_rows(it);
    if (i < kQOps)
      rst.stage_one(rsg.dout, rdo, row0 * D * 2, i);
    else if (i == kQOps)
      dma4(rl2, lds_addr(rsg.lse2), lane * 4, row0 * 4);  // every wave loads the stats: no branch
    else if (i == kQOps + 1)
      dma4(rnd, lds_addr(rsg.ndl), lane * 4, row0 * 4);
    else if (i == kQOps + 2)
      dma4(rwl, lds_addr(rsg.wlo), lane * 4, (uint32_t)tile_idx(it) * BQ * 4);
    else
      dma4(rwh, lds_addr(rsg.whi), lane * 4, (uint32_t)tile_idx(it) * BQ * 4);
  };
  // Vector-memory operations complete in issue order (a load issued behind a
  // store only counts as done once the store has been written).  A P wave
  // issues rows(t + 1) in iteration t - 1 and rows(t + 2) in iteration t, so
  // at tile t + 1's T wait only the kROps loads of rows(t + 2) may still be
  // outstanding.  A dS wave issues Q(t + 1) in iteration t, followed only by
  // the dS stores of tile t - 1 (STAGE, t >= 1): kDsStores of them.
  constexpr int kDsStores = 4;
  // Slots of a phase that issue its `count` loads: every slot from 4 on (the
  // start of a phase is left to its operand and statistics reads); the rest
  // follow the phase's loop.
  constexpr int kLoad0 = 4;
  auto load_slot = [](int j, int nslots, int count) { return j >= kLoad0 && j - kLoad0 < count && j < nslots; };
  auto loads_in_loop = [](int nslots) { return nslots > kLoad0 ? nslots - kLoad0 : 0; };
  // Operand reads in flight ahead of the MFMAs (three measured faster than
  // four or six: fewer LDS requests queued at once).
  constexpr int kRA = 3;

  // dS staging (STAGE): per tile each dS wave stores its 32 keys x 64 rows
  // of dS as four 16-byte stores per lane (group g = 2*sub + k2: the lane's
  // key, its 8 consecutive rows), each instruction 1 KB contiguous in unit
  // `sub`, in the first slot of each group's dK^T MFMAs.
  const uint32_t ds_keep = kvalid ? 0xffffffffu : 0u;  // dS of masked / past-the-end keys is stored as 0
  const uint32_t ds_voff = DsUnit::store_offset(kw * 32 + l32, lane, 0, 0, 0);

  const float c = a.scale_log2;

  // The loop bodies below are explicitly software-pipelined: each "slot" is
  // one MFMA plus the LDS read it needs kRA slots later, at most one load of
  // the next tile, and a share of the VALU work; sched_barrier(0) pins the
  // slot order (the scheduler would otherwise sink each read next to its
  // MFMA and bunch the loads and the VALU work).
  // Iteration `it` of a P wave; uc = it % 3 (compile-time), the slot.
  auto body_p = [&](int it, auto uc) {
    constexpr int u = decltype(uc)::value;
    wait_vmem_n<kROps>();  // this tile's rows landed (for this wave)
    barrier_lds();             // T: ... for every wave; the slots loaded into below are free
    // The wave whose phase ends in VALU-dependent work gets issue priority:
    // P waves up to the end of the softmax (2, then 0 in dV), dS waves in
    // their dS phase (2; 1 in their dP phase, which measured 0.8% faster
    // than 0).
    __builtin_amdgcn_s_setprio(2);
    // Loads during dV: rows of tile it + 2 (the last tiles re-load into
    // slots nothing reads any more).
    const int itr = min(it + 2, niter - 1);
    RowStage& lrs = sm.rs[(u + 2) % 3];

    constexpr int NS = 2 * KS;  // QK^T MFMAs: (sub, ks)
    auto qop = [&](int j) { return lds_ld<bf16x8>(rb[j % KS] + u * kQS + (j / KS) * 64 * D); };
    bf16x8 qa[kRA];
#pragma unroll
    for (int j = 0; j < kRA; ++j) qa[j] = qop(j);
    // lse2 of this lane's 16 rows per sub (8 consecutive rows per k2), read
    // one f32x4 per slot from slot 1 on (the softmax needs them only later;
    // reading them up front delays the first MFMAs' operands).
    f32x4 l2[2][2][2];
    auto l2_read = [&](int q8) {
      l2[q8 >> 2][(q8 >> 1) & 1][q8 & 1] =
          lds_ld<f32x4>(sb + u * kRS + 4 * (32 * (q8 >> 2) + 16 * ((q8 >> 1) & 1) + 4 * (q8 & 1)));
    };
    __builtin_amdgcn_sched_barrier(0);

    f32x16 s[2] = {zero16(), zero16()};
    bf16x8 pb[2][2];
    u32x4 up[2][2];
    // WIN: a tile outside [w_ia, w_ib) masks the scores of a row half per
    // (row, key) before its softmax steps: one wave-uniform branch per half,
    // not taken on the (common) inside tiles.
    bool edge = false;
    if constexpr (WIN) {
      const int T = tile_idx(it);
      edge = T < w_ia || T >= w_ib;
    }
    auto mask_sub = [&](int sub) {
      if constexpr (WIN) {
        if (__builtin_expect(edge, 0)) {
#pragma unroll
          for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
            for (int h4 = 0; h4 < 2; ++h4) {
              // rows 32*sub + 16*k2 + 8*hh + 4*h4 + [0, 4) of the tile
              const uint32_t r0 = sb + u * kRS + 4 * (32 * sub + 16 * k2 + 4 * h4);
              const u32x4 lo = lds_ld<u32x4>(r0 + kWloOff), hi = lds_ld<u32x4>(r0 + kWhiOff);
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (key < (int)lo[r] || key >= (int)hi[r]) s[sub][8 * k2 + 4 * h4 + r] = kNegInf;
            }
        }
      }
    };
    // Softmax step (sub, k2, e2): two probabilities, packed; the last step
    // of a (sub, k2) hands its 16 bytes to the partner wave.
    auto smx = [&](int sub, int k2, int e2) {
      const int e = 2 * e2;
      const f32x4& lv = l2[sub][k2][e >> 2];
      const float s0 = s[sub][8 * k2 + e], s1 = s[sub][8 * k2 + e + 1];
      const float p0 = __builtin_amdgcn_exp2f(fmaf(s0, c, -lv[e & 3]));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(s1, c, -lv[(e & 3) + 1]));
      up[sub][k2][e2] = pack_bf16x2(p0, p1);
      if (e2 == 3) {
        lds_st<u32x4>(xb + u * kXS + 1024 * (2 * sub + k2), up[sub][k2]);
        pb[sub][k2] = bits_to_bf16x8(up[sub][k2]);
      }
    };
    // Softmax steps of sub 0 (8 of them) go into the slots after S(sub 0) is
    // complete (two slots of MFMA latency after its last MFMA).
    constexpr int kLo = KS + 2 < NS ? KS + 2 : NS;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int sub = j / KS, ks = j % KS;
      s[sub] = mfma32(qa[j % kRA], kv[ks], s[sub]);
      if (j + kRA < NS) qa[j % kRA] = qop(j + kRA);
      if (j >= 1 && j <= 8) l2_read(j - 1);
      if (j >= kLo) {
        const int n = NS - kLo;
        if (j == kLo) mask_sub(0);
        for (int st = (j - kLo) * 8 / n; st < (j - kLo + 1) * 8 / n; ++st) smx(0, st >> 2, st & 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q8 = NS - 1; q8 < 8; ++q8) l2_read(q8);  // what the loop had no slot for
    if (kLo >= NS) {
      mask_sub(0);
#pragma unroll
      for (int st = 0; st < 8; ++st) smx(0, st >> 2, st & 3);
    }
    mask_sub(1);
#pragma unroll
    for (int st = 0; st < 8; ++st) smx(1, st >> 2, st & 3);
    // P goes out with the next barrier (T of tile it + 1, where the partner
    // picks it up for its dS phase).
    __builtin_amdgcn_s_setprio(0);

    // dV^T += dO^T P over the (sub, k2, dt) steps, reads kRA steps ahead.
    constexpr int NJ = 4 * DT;
    auto dot_op = [&](int j) {
      const int sk = j / DT, dt = j % DT;  // sk = 2*sub + k2
      const uint32_t off = u * kRS + sk * 32 * D;
      const bf16x4 lo = lds_read_tr16_at(tb[dt][0] + off), hi = lds_read_tr16_at(tb[dt][1] + off);
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    bf16x8 opq[kRA];
#pragma unroll
    for (int j = 0; j < kRA; ++j) opq[j] = dot_op(j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const bf16x8 op = opq[j % kRA];
      if (j + kRA < NJ) opq[j % kRA] = dot_op(j + kRA);
      const int sk = j / DT, dt = j % DT;
      acc[dt] = mfma32(op, pb[sk >> 1][sk & 1], acc[dt]);
      if (load_slot(j, NJ, kROps)) r_op(itr, lrs, j - kLoad0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = loads_in_loop(NJ); i < kROps; ++i) r_op(itr, lrs, i);
  };

  // dS waves, dP phase of the tile in slot uc: dp = dO V^T + ndelta, and the
  // Q loads of tile itq into lq.
  auto dp_phase = [&](auto uc, f32x16(&dp)[2], int itq, bf16* lq) {
    constexpr int u = decltype(uc)::value;
    constexpr int NS = 2 * KS;  // dO V^T MFMAs: (sub, ks)
    auto dop = [&](int j) { return lds_ld<bf16x8>(rb[j % KS] + u * kRS + (j / KS) * 64 * D); };
    bf16x8 da[kRA];
#pragma unroll
    for (int j = 0; j < kRA; ++j) da[j] = dop(j);
    // dP starts at ndelta of its row (registers 8*k2 + e: row 32*sub + 16*k2
    // + 8*hh + e), so the MFMAs deliver dP + ndelta directly.  Sub 0's values
    // are read now, sub 1's in the first slots (its MFMAs start at slot KS).
    auto nd_read = [&](int sub, int q4) {
      const int k2 = q4 >> 1, hf = q4 & 1;
      const f32x4 n4 = lds_ld<f32x4>(sb + u * kRS + kNdlOff + 4 * (32 * sub + 16 * k2 + 4 * hf));
#pragma unroll
      for (int r = 0; r < 4; ++r) dp[sub][8 * k2 + 4 * hf + r] = n4[r];
    };
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) nd_read(0, q4);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int sub = j / KS, ks = j % KS;
      dp[sub] = mfma32(da[j % kRA], kv[ks], dp[sub]);
      if (j + kRA < NS) da[j % kRA] = dop(j + kRA);
      if (j < 4) nd_read(1, j);  // KS >= 4: before sub 1's first MFMA
      if (load_slot(j, NS, kQOps)) q_op(itq, lq, j - kLoad0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = loads_in_loop(NS); i < kQOps; ++i) q_op(itq, lq, i);
  };

  // Where tile `it`'s dS goes (STAGE): a buffer over its two units (query
  // groups 2*tile_idx(it) and +1) and the byte distance between them.
  struct DsDest {
    u32x4 rds;
    uint32_t unit1;
  };
  // Compact layout (WIN with a table): the tile's table entry, read by a
  // scalar load.  Scalar loads return out of order with LDS reads, so while
  // one is outstanding every counted LDS wait would have to become a full
  // one: the entry of the tile whose dS phase comes next is loaded at the
  // end of an iteration (after its last LDS read) and used right after the
  // next barrier, whose wait has drained it.
  struct DsEntry {
    int kb_lo, nblk, gbase;
  };
  auto ds_entry = [&](int it) {
    const int64_t e = ((int64_t)b * a.ds_tsb + tile_idx(it)) * 4;
    return DsEntry{__builtin_amdgcn_readfirstlane(load_const_i32(a.ds_tab, e)),
                   __builtin_amdgcn_readfirstlane(load_const_i32(a.ds_tab, e + 1)),
                   __builtin_amdgcn_readfirstlane(load_const_i32(a.ds_tab, e + 2))};
  };
  auto ds_dest = [&](int it, const DsEntry& en) {
    DsDest d{{0u, 0u, 0u, 0u}, 0u};
    if constexpr (STAGE) {
      const int64_t bq = (int64_t)(bhk - a.kv0) * group + tile_head(it);
      if (CT) {
        // A block outside the entry's range (an inconsistent table) gets an
        // empty buffer, so its stores are dropped; the store offsets are then
        // wholly per-lane (range-checked), see ds_store.
        const bool ok = kt >= en.kb_lo && kt - en.kb_lo < en.nblk && en.gbase >= 0 &&
                        (int64_t)en.gbase + 2 * en.nblk <= a.ds_units;
        const int64_t unit = bq * a.ds_units + (ok ? en.gbase + (kt - en.kb_lo) : 0);
        d.rds = make_rsrc(reinterpret_cast<char*>(a.ds) + unit * 8192, ok ? (uint32_t)(en.nblk + 1) * 8192 : 0u);
        d.unit1 = (uint32_t)en.nblk * 8192;
      } else {
        const int64_t unit = (bq * (2 * nqt) + 2 * tile_idx(it)) * nkt + kt;
        d.rds = make_rsrc(reinterpret_cast<char*>(a.ds) + unit * 8192, (uint32_t)(nkt + 1) * 8192);
        d.unit1 = (uint32_t)nkt * 8192;
      }
    }
    return d;
  };

  // dS waves, dS phase of tile `it` (slot uc), one iteration after its dP
  // phase, so the partner's P has been handed over by the barrier in
  // between: dS = P * dp, dK^T += Q^T dS and, with STAGE, the dS stores
  // (kDsStores per lane) to `dd`.
  auto ds_phase = [&](int it, auto uc, const f32x16(&dp)[2], const DsDest& hoisted) {
    constexpr uint32_t u = decltype(uc)::value;
    // The compact layout's destination was computed at the top of the
    // iteration (see DsEntry); the dense one here, where its few scalar
    // operations schedule best.
    const DsDest dd = (CT) ? hoisted : ds_dest(it, DsEntry{0, 0, 0});
    const u32x4 rds = dd.rds;
    const uint32_t ds_unit1 = dd.unit1;

    // dS for group g = 2*sub + k2 (4 steps of two elements) interleaved with
    // the dK^T MFMAs of group g-1; every LDS read is issued up front or kRA
    // MFMAs ahead.
    u32x4 pv[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) pv[g] = lds_ld<u32x4>(xb + u * kXS + 1024 * g);
    constexpr int NJ = 4 * DT;
    auto qt_op = [&](int j) {
      const int g = j / DT, dt = j % DT;
      const uint32_t off = u * kQS + g * 32 * D;
      const bf16x4 lo = lds_read_tr16_at(tb[dt][0] + off), hi = lds_read_tr16_at(tb[dt][1] + off);
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    bf16x8 opq[kRA];
#pragma unroll
    for (int j = 0; j < kRA; ++j) opq[j] = qt_op(j);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 ud[4];
    auto dstep = [&](int g, int e2) {
      const int sub = g >> 1, k2 = g & 1, e = 2 * e2;
      const float p0 = __uint_as_float(pv[g][e2] << 16), p1 = __uint_as_float(pv[g][e2] & 0xffff0000u);
      ud[g][e2] = pack_bf16x2(p0 * dp[sub][8 * k2 + e], p1 * dp[sub][8 * k2 + e + 1]);
    };
    // Group g's dS: rows 16*k2 + 8*hh .. +7 of unit `sub`, at ((k2*128 +
    // key)*16 + 8*hh) bf16 into the unit.
    auto ds_store = [&](int g) {
      const int sub = g >> 1, k2 = g & 1;
      const u32x4 w = {ud[g][0] & ds_keep, ud[g][1] & ds_keep, ud[g][2] & ds_keep, ud[g][3] & ds_keep};
      const uint32_t unit_off = (sub ? ds_unit1 : 0u) + (uint32_t)k2 * 4096;  // = DsUnit::store_offset
      if (CT)
        store_b128_nt(rds, ds_voff + unit_off, 0u, w);  // the whole offset range-checked
      else
        store_b128_nt(rds, ds_voff, unit_off, w);
    };
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) dstep(0, e2);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int g = j / DT, dt = j % DT;
      const bf16x8 op = opq[j % kRA];
      if (j + kRA < NJ) opq[j % kRA] = qt_op(j + kRA);
      acc[dt] = mfma32(op, bits_to_bf16x8(ud[g]), acc[dt]);
      if (g + 1 < 4) {
        // the next group's 4 steps, spread over this group's DT MFMAs
        for (int st = dt * 4 / DT; st < (dt + 1) * 4 / DT; ++st) dstep(g + 1, st);
      }
      if constexpr (STAGE) {
        if (dt == 0) ds_store(g);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  retire_prologue_loads();
  if (niter > 0 && role == 0) {  // niter is 0 when no window meets this block's keys
#pragma unroll
    for (int i = 0; i < kROps; ++i) r_op(0, sm.rs[0], i);
#pragma unroll
    for (int i = 0; i < kROps; ++i) r_op(min(1, niter - 1), sm.rs[1], i);
  } else if (niter > 0) {
#pragma unroll
    for (int i = 0; i < kQOps; ++i) q_op(0, sm.q[0], i);
  }
  // Tile it lives in slot it % 3 (Q, rows and P hand-over); the loops are
  // unrolled by 3 so that every slot is a compile-time constant.  Every wave
  // passes one barrier per tile (T) and one after the last (F).
  if (niter > 0 && role == 0) {
    for (int it0 = 0;; it0 += 3) {
      const bool more = unrolled_while<3>([&](auto uc) {
        body_p(it0 + uc, uc);
        return it0 + uc + 1 < niter;
      });
      if (!more) break;
    }
    barrier_lds();  // F: the last tile's P handed over
  } else if (niter > 0) {
    // dP of tile it (slot it % 3), kept for the tile's dS phase in the next
    // iteration.
    f32x16 dpb[3][2];
    DsEntry ent{0, 0, 0};  // compact layout: tile it - 1's entry at the top of iteration it
    // Iterations 0 .. niter: iteration niter has only the last tile's dS
    // phase (its barrier pairs with the P waves' F).
    for (int it0 = 0;; it0 += 3) {
      const bool more = unrolled_while<3>([&](auto uc) {
        constexpr int u = decltype(uc)::value, up = (u + 2) % 3;  // slots of tiles it, it - 1
        const int it = it0 + u;
        // Q(it) landed: issued in iteration it - 1, followed there by the dS
        // stores of tile it - 2 if that iteration had a dS phase.
        if (STAGE && it >= 2)
          wait_vmem_n<kDsStores>();
        else
          wait_vmem_n<0>();
        barrier_lds();  // T: tile it staged, tile it - 1's P handed over
        DsDest dd{{0u, 0u, 0u, 0u}, 0u};
        if (CT && it > 0) dd = ds_dest(it - 1, ent);
        if (it < niter) {
          __builtin_amdgcn_s_setprio(1);
          // Loads: Q of tile it + 1 (the last tile re-loads into a slot
          // nothing reads any more).
          dp_phase(uc, dpb[u], min(it + 1, niter - 1), sm.q[(u + 1) % 3]);
        }
        if (it > 0) {
          __builtin_amdgcn_s_setprio(2);
          ds_phase(it - 1, std::integral_constant<int, up>(), dpb[up], dd);
        }
        if (CT && it < niter) ent = ds_entry(it);
        return it < niter;
      });
      if (!more) break;
    }
  }

  if (part >= 0) {
    // Unscaled fp32 partial sums (masked keys and keys past the end as 0);
    // dkv_reduce_kernel scales, rounds and rotates their total.
    float* pp = a.split_part +
                ((((int64_t)(bid - nfull) * a.nparts + part) * 2 + role) * BK + kw * 32 + l32) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 w = {0.f, 0.f, 0.f, 0.f};
        if (kvalid) w = f32x4{acc[dt][4 * g], acc[dt][4 * g + 1], acc[dt][4 * g + 2], acc[dt][4 * g + 3]};
        *reinterpret_cast<f32x4*>(pp + dt * 32 + 8 * g + 4 * hh) = w;
      }
  } else if (key < a.Lk) {
    const float sc = role == 0 ? 1.f : a.scale;
    bf16* op = role == 0 ? a.dv + b * a.dvsb + hk * a.dvsh + (int64_t)key * a.dvsl
                         : a.dk + b * a.dksb + hk * a.dksh + (int64_t)key * a.dksl;
    // dk of an unrotated key: the rotated key's gradient rounded to bf16,
    // then the transposed rotation (what the reference's autograd does
    // through src/avgen/models/rope.py:332-338).
    const bool rot = role == 1 && a.cos_k != nullptr;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w = {0u, 0u};
        if (kvalid) {
          w[0] = pack_bf16x2(acc[dt][4 * g] * sc, acc[dt][4 * g + 1] * sc);
          w[1] = pack_bf16x2(acc[dt][4 * g + 2] * sc, acc[dt][4 * g + 3] * sc);
          if (rot) {
            // channels dt*32 + 8g + 4hh .. +3: pairs (that)/2 and +1
            const int64_t t = b * a.rksb + (int64_t)key * (D / 2) + 16 * dt + 4 * g + 2 * hh;
            const f32x2 c2 = *reinterpret_cast<const f32x2*>(a.cos_k + t);
            const f32x2 s2 = *reinterpret_cast<const f32x2*>(a.sin_k + t);
            w = rotate4(w, c2[0], s2[0], c2[1], s2[1], true);
          }
        }
        *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
      }
  }
}

// dk/dv of the split key blocks: one thread per (block, role, key, 4
// channels) adds the parts' fp32 sums in part order, then scales, rounds to
// bf16 and rotates dk back as the dK/dV kernel's own epilogue does.
template <int D>
__global__ __launch_bounds__(256) void dkv_reduce_kernel(BwdArgs a) {
  constexpr int BK = 128, CQ = D / 4;
  const int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (u >= (int64_t)a.nsplit * 2 * BK * CQ) return;
  const int c = (int)(u % CQ);
  const int r = (int)((u / CQ) % BK);
  const int role = (int)((u / (CQ * BK)) % 2);
  const int s = (int)(u / (CQ * BK * 2));
  const int nkt = (a.Lk + BK - 1) / BK;
  const int bid = nkt * a.nkv - a.nsplit + s;
  const int kt = bid % nkt;
  const int bhk = a.kv0 + bid / nkt;
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int key = kt * BK + r;
  if (key >= a.Lk) return;
  f32x4 t = {0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < a.nparts; ++p)
    t += *reinterpret_cast<const f32x4*>(a.split_part + ((((int64_t)s * a.nparts + p) * 2 + role) * BK + r) * D + 4 * c);
  const float sc = role == 0 ? 1.f : a.scale;
  u32x2 w;
  w[0] = pack_bf16x2(t[0] * sc, t[1] * sc);
  w[1] = pack_bf16x2(t[2] * sc, t[3] * sc);
  if (role == 1 && a.cos_k != nullptr) {
    const int64_t ti = b * a.rksb + (int64_t)key * (D / 2) + 2 * c;  // pairs 2c, 2c + 1
    const f32x2 c2 = *reinterpret_cast<const f32x2*>(a.cos_k + ti);
    const f32x2 s2 = *reinterpret_cast<const f32x2*>(a.sin_k + ti);
    w = rotate4(w, c2[0], s2[0], c2[1], s2[1], true);
  }
  bf16* op = role == 0 ? a.dv + b * a.dvsb + hk * a.dvsh + (int64_t)key * a.dvsl
                       : a.dk + b * a.dksb + hk * a.dksh + (int64_t)key * a.dksl;
  *reinterpret_cast<u32x2*>(op + 4 * c) = w;
}

// ---------------------------------------------------------------------------
// 3. dQ
// ---------------------------------------------------------------------------
// One workgroup = 256 query rows of one (batch, head): 8 waves x 32 rows
// (lane % 32 owns query column q0w + lane % 32), 1 workgroup per CU, so each
// K/V tile is staged once for 256 rows.  For each 32-key tile (lane l supplies
// key row perm23(l % 32) to the first two products):
//   S^T  = K Q^T    A = K rows (LDS)          B = Q^T (registers)
//   dP^T = V dO^T   A = V rows (LDS)          B = dO^T (registers)
//   dS^T = P^T * (dP^T + ndelta[q])           (fp32, key bias masks P^T)
//   dQ^T += K^T dS^T   A = K^T (LDS, head_dim-major)  B = dS^T (C layout reused)
// Ping-pong: waves 0-3 (group A) and 4-7 (group B) share the SIMDs pairwise.
// Group A runs S/dP(t), dS(t), dQ(t) in iteration t; group B is one tile
// behind and runs dS(t-1), dQ(t-1), S/dP(t), carrying S^T/dP^T across the
// barrier.  So while one wave of a SIMD computes dS (VALU), the other issues
// MFMAs, and the per-tile barrier no longer lines both up on the same phase.
// Tiles come from the padded copies through four LDS stages: tile t+2 is
// loaded during iteration t (spread between MFMAs) and tile t-1 stays
// resident for group B.
template <int D>
__global__ __launch_bounds__(512, 1) void bwd_dq_kernel(BwdArgs a) {
  constexpr int NW = 8, BM = 32 * NW, BN = 32;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int TE = BN * D;
  // One LDS object per stage (see bwd_dkdv_kernel).
  struct Stage {
    bf16 k[TE];      // K rows: TileLayout<D>
    bf16 v[TE];      // V rows: TileLayout<D>
    bf16 kt[TE];     // K^T: D rows of BN keys, TileLayout<BN>
    float bias[64];  // key bias (this tile and the next)
    int flags[64];   // "all attended" flag of this tile (and the next 63)
  };
  __shared__ __attribute__((aligned(16))) Stage st0, st1, st2, st3;
  auto stage_ref = [&](auto bufc) __attribute__((always_inline)) -> Stage& {
    constexpr int buf = decltype(bufc)::value;
    return buf == 0 ? st0 : (buf == 1 ? st1 : (buf == 2 ? st2 : st3));
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;
  const int prow = perm23(l32);

  const int nqt = (a.Lq + BM - 1) / BM;
  const int total = nqt * a.B * a.Hq;
  const int bid = xcd_remap(blockIdx.x, total);
  const int qt = bid % nqt;
  const int bh = bid / nqt;
  const int b = bh / a.Hq, h = bh % a.Hq;
  const int hk = h / (a.Hq / a.Hkv);

  const int qrow = qt * BM + wave * 32 + l32;
  const bool qvalid = qrow < a.Lq;
  const int64_t srow = (int64_t)bh * a.Lqp + qrow;
  const float lse2 = qvalid ? a.lse2[srow] : kPosInf;
  const float ndelta = qvalid ? a.ndelta[srow] : 0.f;

  bf16x8 qf[KS], df[KS];
  {
    const bf16* qp = a.q + b * a.qsb + h * a.qsh + (int64_t)qrow * a.qsl + 8 * hh;
    const bf16* dp = a.dout + b * a.dosb + h * a.dosh + (int64_t)qrow * a.dosl + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
      if (qvalid) {
        x = *reinterpret_cast<const u32x4*>(qp + 16 * ks);
        y = *reinterpret_cast<const u32x4*>(dp + 16 * ks);
        if (a.cos_q) {
          const int64_t t = b * a.rqsb + (int64_t)qrow * (D / 2) + 8 * ks + 4 * hh;
          x = rotate8(x, *reinterpret_cast<const f32x4*>(a.cos_q + t), *reinterpret_cast<const f32x4*>(a.sin_q + t),
                      false);
        }
      }
      qf[ks] = bits_to_bf16x8(x);
      df[ks] = bits_to_bf16x8(y);
    }
  }

  const int64_t bhk = (int64_t)(b * a.Hkv + hk);
  const uint32_t slice = (uint32_t)a.Lkp * D * 2;
  const u32x4 rk = make_rsrc(a.kr + bhk * a.Lkp * D, slice);
  const u32x4 rv = make_rsrc(a.vr + bhk * a.Lkp * D, slice);
  const u32x4 rkt = make_rsrc(a.kt + bhk * D * a.Lkp, slice);
  // Biases and flags: both arrays are padded by 64 entries, so the 64 read
  // from a tile start stay inside them.
  const u32x4 rb = make_rsrc(a.kbias + (int64_t)b * a.Lkp, (uint32_t)(a.Lkp + 64) * 4);
  const u32x4 rf = make_rsrc(a.kfull + (int64_t)b * (a.Lkp / 32), (uint32_t)(a.Lkp / 32 + 64) * 4);

  using RowStager = TileStager<BN, D, NW>;  // 32 rows of D channels (row stride D)
  using ColStager = TileStager<D, BN, NW>;  // D rows of 32 keys (row stride Lkp)
  RowStager rst;
  ColStager ktst;
  rst.init(D, wave, lane);
  ktst.init(a.Lkp, wave, lane);
  // Vector-memory loads one stage issues per wave: K, V, K^T, bias, flags.
  constexpr int kStageLoads = 2 * RowStager::kPer + ColStager::kPer + 2;
  auto stage_op = [&](int t, auto bufc, int i) __attribute__((always_inline)) {
    Stage& sg = stage_ref(bufc);
    const uint32_t k0 = (uint32_t)t * BN;
    if (i < RowStager::kPer)
      rst.stage_one(sg.k, rk, k0 * D * 2, i);
    else if (i < 2 * RowStager::kPer)
      rst.stage_one(sg.v, rv, k0 * D * 2, i - RowStager::kPer);
    else if (i < 2 * RowStager::kPer + ColStager::kPer)
      ktst.stage_one(sg.kt, rkt, k0 * 2, i - 2 * RowStager::kPer);
    else if (i == kStageLoads - 2)
      dma4(rb, lds_addr(sg.bias), lane * 4, k0 * 4);
    else
      dma4(rf, lds_addr(sg.flags), lane * 4, (uint32_t)t * 4);
  };

  // Per-lane LDS byte offsets inside a tile.  Each iteration passes them
  // through opaque() once (Off), so every read of that iteration adds its
  // stage's base as an instruction immediate instead of the compiler keeping
  // one hoisted copy of every offset per stage in registers.
  struct Off {
    int k[KS];  // K/V row perm23(l32), chunk 16*ks + 8*hh
    int t[2];   // K^T row l32, key chunk 16*k2 + 8*hh (+32*dt rows)
  };
  Off off0;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) off0.k[ks] = 2 * TileLayout<D>::off(prow, 16 * ks + 8 * hh);
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) off0.t[k2] = 2 * TileLayout<BN>::off(l32, 16 * k2 + 8 * hh);
  auto fresh = [&]() __attribute__((always_inline)) {
    Off o;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) o.k[ks] = opaque(off0.k[ks]);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) o.t[k2] = opaque(off0.t[k2]);
    return o;
  };
  auto lds16 = [](const void* base, int byte_off) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(base) + byte_off);
  };

  f32x16 dq[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dq[i] = zero16();

  const float c = a.scale_log2;
  const int nkt = (a.Lk + BN - 1) / BN;

  // S^T and dP^T of one tile (2*KS MFMAs, the two chains alternating); dP^T
  // starts at ndelta (one value per query column, i.e. per lane), so the MFMAs
  // deliver dP^T + ndelta directly.  Operand reads run two k-steps (four
  // MFMAs) ahead; `slot(j)` runs extra work after MFMA j; sched_barrier(0)
  // pins the order.
  auto sdp = [&](const Stage& sg, const Off& o, f32x16& s, f32x16& dp, auto&& slot) __attribute__((always_inline)) {
    auto krow = [&](int ks) __attribute__((always_inline)) { return lds16(sg.k, o.k[ks]); };
    auto vrow = [&](int ks) __attribute__((always_inline)) { return lds16(sg.v, o.k[ks]); };
    bf16x8 ka[2], va[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      ka[j] = krow(j);
      va[j] = vrow(j);
    }
    s = zero16();
    dp = splat16(ndelta);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      s = mfma32(ka[ks & 1], qf[ks], s);
      if (ks + 2 < KS) ka[ks & 1] = krow(ks + 2);
      slot(2 * ks);
      __builtin_amdgcn_sched_barrier(0);
      dp = mfma32(va[ks & 1], df[ks], dp);
      if (ks + 2 < KS) va[ks & 1] = vrow(ks + 2);
      slot(2 * ks + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // dS^T of one tile (its S^T, dP^T and stage) as the bf16 B operands of dQ;
  // registers 8*k2 + e hold key 16*k2 + 8*hh + e.
  auto dsm = [&](const Stage& sg, f32x16& s, const f32x16& dp, bf16x8* dsb, auto&& slot) __attribute__((always_inline)) {
    if (!__builtin_amdgcn_readfirstlane(sg.flags[0])) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 bb = *reinterpret_cast<const f32x4*>(sg.bias + 16 * (g >> 1) + 8 * hh + 4 * (g & 1));
#pragma unroll
        for (int r = 0; r < 4; ++r) s[4 * g + r] += bb[r];
      }
    }
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      u32x4 u;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int r = 8 * k2 + 2 * e2;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(s[r], c, -lse2));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(s[r + 1], c, -lse2));
        u[e2] = pack_bf16x2(p0 * dp[r], p1 * dp[r + 1]);
        slot(4 * k2 + e2);
      }
      dsb[k2] = bits_to_bf16x8(u);
    }
  };
  // dQ^T += K^T dS^T (2*DT MFMAs).  The first four K^T operands are read
  // before dsm runs (their latency hides behind it), the rest four MFMAs
  // ahead.
  auto kt_op = [&](const Stage& sg, const Off& o, int j) __attribute__((always_inline)) {
    return lds16(sg.kt + (j % DT) * 32 * BN, o.t[j / DT]);
  };
  auto kt_read = [&](const Stage& sg, const Off& o, bf16x8* kta) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) kta[j] = kt_op(sg, o, j);
  };
  auto dqm = [&](const Stage& sg, const Off& o, bf16x8* kta, const bf16x8* dsb, auto&& slot) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2 * DT; ++j) {
      dq[j % DT] = mfma32(kta[j & 3], dsb[j / DT], dq[j % DT]);
      if (j + 4 < 2 * DT) kta[j & 3] = kt_op(sg, o, j + 4);
      slot(j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Where a tile's loads are issued: between the dQ MFMAs when they fit there
  // (measured ~1% faster than between the S/dP MFMAs), else between the S/dP
  // MFMAs (0); 2 would spread them over the dS VALU steps (measured slower).
  constexpr int kLoadsAt = kStageLoads <= 2 * DT ? 1 : 0;
  static_assert(kStageLoads <= 2 * KS && kStageLoads <= 8, "tile loads must fit the slots");
  auto no_slot = [](int) __attribute__((always_inline)) {};
  auto loads_in = [&](int t, auto nextc) __attribute__((always_inline)) {  // tile t's loads, one after each of the first MFMAs
    return [&, t, nextc](int j) __attribute__((always_inline)) {
      if (j < kStageLoads) stage_op(t, nextc, j);
    };
  };
  // Top of iteration t: tile t landed (only tile t+1's loads may still be in
  // flight) for every wave; the stage tile t-2 used is free for tile t+2.
  auto top = [&]() __attribute__((always_inline)) {
    wait_vmem_n<kStageLoads>();
    barrier_lds();
  };

  retire_prologue_loads();
  {
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
#pragma unroll
    for (int i = 0; i < kStageLoads; ++i) stage_op(0, B0(), i);
#pragma unroll
    for (int i = 0; i < kStageLoads; ++i) stage_op(min(1, nkt - 1), B1(), i);
  }

  f32x16 s, dp;
  bf16x8 kta[4], dsb[2];
  if (wave < NW / 2) {
    // Group A: S/dP(t), dS(t), dQ(t).
    auto body = [&](int t, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      using Next2 = std::integral_constant<int, (buf + 2) % 4>;
      top();
      const Stage& sg = stage_ref(bufc);
      const Off o = fresh();
      auto ld = loads_in(min(t + 2, nkt - 1), Next2());
      __builtin_amdgcn_s_setprio(2);
      if constexpr (kLoadsAt == 0) sdp(sg, o, s, dp, ld); else sdp(sg, o, s, dp, no_slot);
      kt_read(sg, o, kta);
      __builtin_amdgcn_s_setprio(0);
      if constexpr (kLoadsAt == 2) dsm(sg, s, dp, dsb, ld); else dsm(sg, s, dp, dsb, no_slot);
      __builtin_amdgcn_s_setprio(2);
      if constexpr (kLoadsAt == 1) dqm(sg, o, kta, dsb, ld); else dqm(sg, o, kta, dsb, no_slot);
    };
    for (int t = 0; t < nkt; t += 4) {
      body(t, std::integral_constant<int, 0>());
      if (t + 1 < nkt) body(t + 1, std::integral_constant<int, 1>());
      if (t + 2 < nkt) body(t + 2, std::integral_constant<int, 2>());
      if (t + 3 < nkt) body(t + 3, std::integral_constant<int, 3>());
    }
  } else {
    // Group B: dS(t-1), dQ(t-1), S/dP(t); S^T/dP^T of tile t are carried to
    // the next iteration.
    auto body = [&](int t, auto bufc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      using Prev = std::integral_constant<int, (buf + 3) % 4>;
      using Next2 = std::integral_constant<int, (buf + 2) % 4>;
      top();
      const Stage& sp = stage_ref(Prev());
      const Off o = fresh();
      auto ld = loads_in(min(t + 2, nkt - 1), Next2());
      kt_read(sp, o, kta);
      __builtin_amdgcn_s_setprio(0);
      if constexpr (kLoadsAt == 2) dsm(sp, s, dp, dsb, ld); else dsm(sp, s, dp, dsb, no_slot);
      __builtin_amdgcn_s_setprio(2);
      if constexpr (kLoadsAt == 1) dqm(sp, o, kta, dsb, ld); else dqm(sp, o, kta, dsb, no_slot);
      if constexpr (kLoadsAt == 0) sdp(stage_ref(bufc), o, s, dp, ld); else sdp(stage_ref(bufc), o, s, dp, no_slot);
    };
    {
      // Iteration 0: only S/dP(0).
      using B2 = std::integral_constant<int, 2>;
      top();
      const Off o = fresh();
      if constexpr (kLoadsAt == 0) {
        sdp(stage_ref(std::integral_constant<int, 0>()), o, s, dp, loads_in(min(2, nkt - 1), B2()));
      } else {
        sdp(stage_ref(std::integral_constant<int, 0>()), o, s, dp, no_slot);
#pragma unroll
        for (int i = 0; i < kStageLoads; ++i) stage_op(min(2, nkt - 1), B2(), i);
      }
    }
    for (int t = 1; t < nkt; t += 4) {
      body(t, std::integral_constant<int, 1>());
      if (t + 1 < nkt) body(t + 1, std::integral_constant<int, 2>());
      if (t + 2 < nkt) body(t + 2, std::integral_constant<int, 3>());
      if (t + 3 < nkt) body(t + 3, std::integral_constant<int, 0>());
    }
    // Tail: dS and dQ of the last tile (its stage is not refilled).
    const int bl = (nkt - 1) % 4;
    const Stage& sl = bl == 0 ? st0 : (bl == 1 ? st1 : (bl == 2 ? st2 : st3));
    const Off o = fresh();
    kt_read(sl, o, kta);
    __builtin_amdgcn_s_setprio(0);
    dsm(sl, s, dp, dsb, no_slot);
    dqm(sl, o, kta, dsb, no_slot);
  }
  __builtin_amdgcn_s_setprio(0);
  wait_vmem();  // the last (re-staged) tile loads

  if (qvalid && a.dq_acc) {
    // fp32 accumulation: dq_acc += this chunk's dq (each element owned by
    // exactly one lane, so a plain load-add-store).
    float* op = a.dq_acc + b * a.dqsb + h * a.dqsh + (int64_t)qrow * a.dqsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4* p = reinterpret_cast<f32x4*>(op + dt * 32 + 8 * g + 4 * hh);
        f32x4 w = *p;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] += dq[dt][4 * g + r] * a.scale;
        *p = w;
      }
  } else if (qvalid) {
    bf16* op = a.dq + b * a.dqsb + h * a.dqsh + (int64_t)qrow * a.dqsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w[0] = pack_bf16x2(dq[dt][4 * g] * a.scale, dq[dt][4 * g + 1] * a.scale);
        w[1] = pack_bf16x2(dq[dt][4 * g + 2] * a.scale, dq[dt][4 * g + 3] * a.scale);
        *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
      }
  }
}

// ---------------------------------------------------------------------------
// 3'. dQ from staged dS
// ---------------------------------------------------------------------------
// dQ^T[d, q] = scale * sum_key K^T[d, key] dS^T[key, q], a plain product
// (the S and dP recomputation of bwd_dq_kernel is replaced by reading the dS
// the dK/dV kernel stored).  One workgroup = 256 query rows of one (batch,
// head) of the pass: wave w owns query group 8*qb + w (32 rows, lane % 32 one
// row) and all D channels (DT accumulators).  64-key stages through three LDS
// buffers: K^T (D rows of 64 keys, TileLayout<64>, shared) and each wave's
// own 4 KB of dS, the stage's keys of its unit copied as stored
// ([k2][64 keys][16 rows]); the B operand (8 consecutive keys of one row per
// lane) comes from two transposed reads per 16-key step.  The kernel streams
// dS from HBM once; K^T comes from L2 (the query groups of one head run on
// one XCD).
// WIN: only the stages that meet the union of the workgroup's rows' key
// windows are staged, and a wave multiplies only those that meet its own
// 32 rows' windows (the dK/dV kernel wrote the dS of exactly those: a
// group's window union lies inside its 64-row tile's).
template <int D, int BK, int NSTG, bool WIN, bool CT>
__global__ __launch_bounds__(512, 1) void bwd_dq_ds_kernel(BwdArgs a) {
  static_assert(!CT || WIN, "the compact dS layout (BwdArgs::ds_tab) is for windows");
  constexpr int NW = 8, DT = D / 32;
  static_assert(BK == 32 || BK == 64, "stage of 32 or 64 keys");
  struct Stage {
    bf16 kt[D * BK];             // K^T: D rows of BK keys, TileLayout<BK>
    bf16 ds[NW][2 * BK * 16];    // per wave: [k2][BK keys][16 rows]
  };
  __shared__ __attribute__((aligned(16))) Stage st[NSTG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;

  const int group = a.Hq / a.Hkv;
  const int nqg = a.Lqp / 32;
  const int nqb = (nqg + NW - 1) / NW;
  const int total = nqb * a.nkv * group;
  const int bid = xcd_remap(blockIdx.x, total);
  const int qb = bid % nqb;
  const int bq_rel = bid / nqb;             // (b, hq) within the pass
  const int bq = a.kv0 * group + bq_rel;    // b*Hq + hq
  const int b = bq / a.Hq, h = bq % a.Hq;
  const int hk = h / group;
  const int qg = qb * NW + wave;
  const int qgl = min(qg, nqg - 1);  // groups past the end re-read the last one and write nothing
  const int qrow = qg * 32 + l32;
  const bool qvalid = qrow < a.Lq;
  const int nkt = (a.Lk + 127) / 128;
  int s0 = 0, s1 = a.Lkp / BK;  // stages of the workgroup
  int w0 = s0, w1 = s1;         // stages this wave multiplies
  if constexpr (WIN) {
    // Monotone windows: a row range's key union is [lo(first), hi(last)).
    const int* lo = a.wlo + b * a.wsb;
    const int* hi = a.whi + b * a.wsb;
    auto range = [&](int r0, int r1, int& st0, int& st1) {  // rows [r0, r1)
      r1 = min(r1, a.Lq);
      st0 = st1 = 0;
      if (r1 > r0) {
        const int l = min(max(lo[r0], 0), a.Lk);
        const int lol = min(max(lo[r1 - 1], 0), a.Lk);
        const int h = min(max(hi[r1 - 1], lol), a.Lk);
        if (h > l) {
          st0 = l / BK;
          st1 = (h + BK - 1) / BK;
        }
      }
    };
    range(qb * NW * 32, qb * NW * 32 + NW * 32, s0, s1);
    range(qg * 32, qg * 32 + 32, w0, w1);
    s0 = __builtin_amdgcn_readfirstlane(s0);
    s1 = __builtin_amdgcn_readfirstlane(s1);
    w0 = __builtin_amdgcn_readfirstlane(w0);
    w1 = __builtin_amdgcn_readfirstlane(w1);
  }

  const u32x4 rkt = make_rsrc(a.kt + (int64_t)(b * a.Hkv + hk) * D * a.Lkp, (uint32_t)a.Lkp * D * 2);
  // This wave's dS units: dense, every 128-key block of its group in order;
  // compact (WIN with a table), the blocks [kb_lo, kb_lo + nblk) of its
  // tile.  A stage is loaded by every wave (the counted waits need the same
  // loads everywhere); a stage outside this wave's blocks re-loads one of
  // them, or the head's first unit when the tile has none, and is not
  // multiplied (w0 .. w1 lies inside the tile's blocks).
  u32x4 rds;
  int ds_kb_lo = 0, ds_nblk = nkt;
  if (CT) {
    const int64_t e = ((int64_t)b * a.ds_tsb + (qgl >> 1)) * 4;
    const int kb_lo = __builtin_amdgcn_readfirstlane(load_const_i32(a.ds_tab, e));
    const int nblk = __builtin_amdgcn_readfirstlane(load_const_i32(a.ds_tab, e + 1));
    const int gbase = __builtin_amdgcn_readfirstlane(load_const_i32(a.ds_tab, e + 2));
    const bool ok = nblk > 0 && gbase >= 0 && (int64_t)gbase + 2 * nblk <= a.ds_units;
    const int64_t unit = (int64_t)bq_rel * a.ds_units + (ok ? gbase + (qgl & 1) * nblk : 0);
    ds_kb_lo = ok ? kb_lo : 0;
    ds_nblk = ok ? nblk : 1;
    rds = make_rsrc(reinterpret_cast<const char*>(a.ds) + unit * 8192, (uint32_t)ds_nblk * 8192);
  } else {
    rds = make_rsrc(reinterpret_cast<const char*>(a.ds) + ((int64_t)bq_rel * nqg + qgl) * nkt * 8192,
                    (uint32_t)nkt * 8192);
  }
  using KtStager = TileStager<D, BK, NW>;
  KtStager ktst;
  ktst.init(a.Lkp, wave, lane);
  constexpr int kPerK2 = BK / 32;            // 1 KB loads per k2 half and stage
  constexpr int kDsOps = 2 * kPerK2;         // this wave's 32 rows x BK keys
  constexpr int kStageLoads = KtStager::kPer + kDsOps;
  // Stage s = keys [BK s, BK s + BK): in unit BK*s/128, the BK*32 bytes at
  // (BK*s % 128)*32 of each k2 half (k2 at 4096 bytes).
  auto stage_load = [&](int s, Stage& sg) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < KtStager::kPer; ++i) ktst.stage_one(sg.kt, rkt, (uint32_t)s * BK * 2, i);
    // Unit of stage s among this wave's units (clamped into them), then the
    // stage's keys within it.
    const int ku = min(max(s * BK / 128 - ds_kb_lo, 0), ds_nblk - 1);
    const uint32_t soff = (uint32_t)ku * 8192 + DsUnit::stage_src<BK>(s % (128 / BK), 0, 0);
#pragma unroll
    for (int i = 0; i < kDsOps; ++i)
      dma16_nt(rds, lds_addr(&sg.ds[wave][512 * i]), DsUnit::stage_src<BK>(0, i, lane), soff);
  };
  // Transposed B-operand reads: in 16-lane group G (k2 = G % 2, hh = G / 2),
  // lane i reads rows 16*k2 + 4*(i%4) .. +3 of key 16*ks + 8*hh + i/4 (+4 for
  // the second read) and receives keys +0..3 (+4..7) of row 16*k2 + i.
  const int tr_off = DsUnit::tr_elem<BK>(lane, 0, 0);

  f32x16 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = zero16();

  auto compute = [&](const Stage& sg) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const bf16* src = sg.ds[wave] + tr_off + ks * 16 * 16;
      const bf16x4 lo = lds_read_tr16(src), hi = lds_read_tr16(src + 4 * 16);
      const bf16x8 bop = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        acc[dt] = mfma32(row_operand<BK>(sg.kt, 32 * dt + l32, 16 * ks + 8 * hh), bop, acc[dt]);
    }
  };

  retire_prologue_loads();
  if (s1 > s0) {  // same for every wave of the workgroup
#pragma unroll
    for (int p = 0; p < NSTG - 1; ++p) stage_load(min(s0 + p, s1 - 1), st[p]);
    // Iteration s: stage s is waited for (NSTG - 2 later stages may still be
    // in flight), then stage s + NSTG - 1 (clamped: the last stage is
    // re-loaded, same bytes) goes into the buffer stage s - 1 used.
    int cur = 0;
    for (int s = s0; s < s1; ++s) {
      wait_vmem_n<(NSTG - 2) * kStageLoads>();
      barrier_lds();
      const int nxt = cur == 0 ? NSTG - 1 : cur - 1;
      stage_load(min(s + NSTG - 1, s1 - 1), st[nxt]);
      if (!WIN || (s >= w0 && s < w1)) compute(st[cur]);
      cur = cur == NSTG - 1 ? 0 : cur + 1;
    }
  }
  wait_vmem();  // the last (re-staged) loads

  if (qvalid && a.dq_acc) {
    float* op = a.dq_acc + b * a.dqsb + h * a.dqsh + (int64_t)qrow * a.dqsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4* p = reinterpret_cast<f32x4*>(op + dt * 32 + 8 * g + 4 * hh);
        f32x4 w = *p;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] += acc[dt][4 * g + r] * a.scale;
        *p = w;
      }
  } else if (qvalid) {
    bf16* op = a.dq + b * a.dqsb + h * a.dqsh + (int64_t)qrow * a.dqsl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w[0] = pack_bf16x2(acc[dt][4 * g] * a.scale, acc[dt][4 * g + 1] * a.scale);
        w[1] = pack_bf16x2(acc[dt][4 * g + 2] * a.scale, acc[dt][4 * g + 3] * a.scale);
        *reinterpret_cast<u32x2*>(op + dt * 32 + 8 * g + 4 * hh) = w;
      }
  }
}

// Zero-fill rows of a strided (B, H, L, D) bf16 tensor (gradients of an empty
// attention).
__global__ void zero_rows_kernel(bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % (D / 8));
    const int64_t row = u / (D / 8);
    const int i = (int)(row % L);
    const int h = (int)((row / L) % H);
    const int b = (int)(row / ((int64_t)L * H));
    *reinterpret_cast<u32x4*>(x + b * sb + h * sh + (int64_t)i * sl + 8 * c) = u32x4{0u, 0u, 0u, 0u};
  }
}

// Compute units of the current device (0 if the query fails: no split).
static int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return n;
}

template <int D>
static void launch_dq_ds_d(const BwdArgs& a, hipStream_t stream) {
  const int group = a.Hq / a.Hkv;
  const int nqb = (a.Lqp / 32 + 7) / 8;  // 256 query rows per workgroup
  const dim3 grid(nqb * a.nkv * group);
  LaunchTimer timer(kKidBwdDqDs, stream);
  // 64-key stages, three buffers: measured faster than 32-key stages with
  // four or six buffers (4.75 vs 4.9-5.4 ms per c3 chunk).  The grid's
  // partial last round is not split as the dK/dV one is: this kernel is
  // bound by HBM, and the last round's workgroups share all of it (measured:
  // no gain at c3).
  if (a.wlo && a.ds_tab)
    hipLaunchKernelGGL((bwd_dq_ds_kernel<D, 64, 3, true, true>), grid, dim3(512), 0, stream, a);
  else if (a.wlo)
    hipLaunchKernelGGL((bwd_dq_ds_kernel<D, 64, 3, true, false>), grid, dim3(512), 0, stream, a);
  else
    hipLaunchKernelGGL((bwd_dq_ds_kernel<D, 64, 3, false, false>), grid, dim3(512), 0, stream, a);
}

template <int D>
static hipError_t launch_bwd_d(const BwdArgs& a, int kv_per_pass, hipStream_t stream) {
  const bool mask = a.mask != nullptr;
  {
    LaunchTimer timer(kKidTranspose, stream);
    hipError_t e = hipSuccess;
    if (!a.reuse_q) {
      // Row-major copies only: the dK/dV kernel reads its head_dim-major
      // operands from the same tiles by transposed LDS reads.
      e = launch_prep_copies(a.q, a.qsb, a.qsh, a.qsl, a.B, a.Hq, a.Lq, D, a.qr, nullptr, stream, nullptr, a.cos_q,
                             a.sin_q, a.rqsb);
      if (e == hipSuccess)
        e = launch_prep_copies(a.dout, a.dosb, a.dosh, a.dosl, a.B, a.Hq, a.Lq, D, a.dor, nullptr, stream);
    }
    // The dK/dV kernel reads its own key rows from k and v; the row-major
    // copies serve only the recomputing dQ kernel (no staged dS), the
    // head_dim-major k copy both dQ kernels.
    const bool rows = a.ds == nullptr;
    if (e == hipSuccess)
      e = launch_prep_copies(a.k, a.ksb, a.ksh, a.ksl, a.B, a.Hkv, a.Lk, D, rows ? a.kr : nullptr, a.kt, stream,
                             nullptr, a.cos_k, a.sin_k, a.rksb);
    if (e == hipSuccess && rows)
      e = launch_prep_copies(a.v, a.vsb, a.vsh, a.vsl, a.B, a.Hkv, a.Lk, D, a.vr, nullptr, stream);
    if (e == hipSuccess) e = launch_key_prep(a.mask, a.msb, a.B, a.Lk, a.kbias, a.kfull, stream);
    if (e != hipSuccess) return e;
  }
  if (!a.reuse_q) {
    constexpr int RPB = 256 / (D / 8);
    const int64_t rows = (int64_t)a.B * a.Hq * a.Lqp;
    LaunchTimer timer(kKidBwdPre, stream);
    hipLaunchKernelGGL(bwd_pre_kernel<D>, dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, stream, a);
  }
  // dK/dV (and, with staged dS, dQ) per pass over (b, kv head) pairs.
  const int nkv_all = a.B * a.Hkv;
  const int step = a.ds ? kv_per_pass : nkv_all;
  const int nkt = (a.Lk + 127) / 128;
  const int cus = cu_count();
  for (int kv0 = 0; kv0 < nkv_all; kv0 += step) {
    BwdArgs p = a;
    p.kv0 = kv0;
    p.nkv = min(step, nkv_all - kv0);
    // One 128-key block per workgroup, one workgroup per CU: a grid of
    // total blocks runs in ceil(total / cus) rounds, the last one with
    // total % cus blocks and the other CUs idle.  Those blocks are split
    // over several workgroups each (ranges of query tiles) so that the last
    // round is fuller and shorter.
    const int total = nkt * p.nkv;
    const TailSplit ts = p.split_part ? plan_tail_split(total, cus, kSplitSlots) : TailSplit{0, 0};
    p.nsplit = ts.nsplit;
    p.nparts = ts.nparts;
    {
      const dim3 grid(total - p.nsplit + p.nsplit * p.nparts);
      LaunchTimer timer(kKidBwdDkdv, stream);  // 1 workgroup (8 waves) per CU: LDS-bound occupancy
      if (p.wlo && p.ds_tab) {  // windows, compact dS layout
        if (mask)
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, true, true, true, true>), grid, dim3(512), 0, stream, p);
        else
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, false, true, true, true>), grid, dim3(512), 0, stream, p);
      } else if (p.wlo) {  // windows (staged dS only)
        if (mask)
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, true, true, true, false>), grid, dim3(512), 0, stream, p);
        else
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, false, true, true, false>), grid, dim3(512), 0, stream, p);
      } else if (mask) {
        if (p.ds)
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, true, true, false, false>), grid, dim3(512), 0, stream, p);
        else
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, true, false, false, false>), grid, dim3(512), 0, stream, p);
      } else {
        if (p.ds)
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, false, true, false, false>), grid, dim3(512), 0, stream, p);
        else
          hipLaunchKernelGGL((bwd_dkdv_kernel<D, false, false, false, false>), grid, dim3(512), 0, stream, p);
      }
    }
    if (p.nsplit > 0) {
      const int64_t threads = (int64_t)p.nsplit * 2 * 128 * (D / 4);
      LaunchTimer timer(kKidDkdvReduce, stream);
      hipLaunchKernelGGL(dkv_reduce_kernel<D>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
    }
    if (p.ds && !p.defer_dq) launch_dq_ds_d<D>(p, stream);
  }
  if (!a.ds) {
    constexpr int BM = 256;  // 8 waves x 32 query rows
    const int nqt = (a.Lq + BM - 1) / BM;
    const dim3 grid(nqt * a.B * a.Hq);
    LaunchTimer timer(kKidBwdDq, stream);
    hipLaunchKernelGGL(bwd_dq_kernel<D>, grid, dim3(512), 0, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdArgs& a, int head_dim, int kv_per_pass, hipStream_t stream) {
  return head_dim == 128 ? launch_bwd_d<128>(a, kv_per_pass, stream) : launch_bwd_d<64>(a, kv_per_pass, stream);
}

hipError_t launch_bwd_dq_staged(const BwdArgs& a, int head_dim, hipStream_t stream) {
  if (head_dim == 128)
    launch_dq_ds_d<128>(a, stream);
  else
    launch_dq_ds_d<64>(a, stream);
  return hipGetLastError();
}

hipError_t launch_zero_rows(bf16* x, int64_t sb, int64_t sh, int64_t sl, int B, int H, int L, int D,
                            hipStream_t stream) {
  const int64_t units = (int64_t)B * H * L * (D / 8);
  if (units == 0) return hipSuccess;
  const int64_t blocks = (units + 255) / 256;
  hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, stream, x,
                     sb, sh, sl, B, H, L, D);
  return hipGetLastError();
}

}  // namespace avattn
