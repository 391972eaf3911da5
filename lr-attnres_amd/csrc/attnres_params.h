// Kernel parameter blocks (passed by value as kernel arguments) and the
// launch helpers shared by the LR and base read kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/attnres_hip.h"
#include "attnres_device.h"

namespace attnres {

constexpr int kMaxSources = ATTNRES_MAX_SOURCES;
constexpr int kWaveSize = 64;  // CDNA wavefront
// Backward grids are capped so the per-workgroup partial sums stay small and
// the cross-token reduction order does not depend on the device.  The
// workspace holds kMaxBwdGroups rows; most backward kernels use at most
// kFullBwdGroups workgroups, the lean fast LR backward all of them.
constexpr int kMaxBwdGroups = 4096;
constexpr int kFullBwdGroups = 2048;
constexpr int kMaxFwdGroups = 65536;
constexpr int kPhase1SplitGroups = 65536;  // phase-1 split kernels: at most this many workgroups (one token each per step; one token per workgroup measured best)

// Smallest source count for which the host launches a fast LR kernel with nb
// value slots (it picks the smallest instantiated slot count that holds N:
// 8/12/14/16/20/24/32 for one column and two key chunks, else 8/16/32).  The
// kernels assume it, so their per-slot branches below it fold away.
__host__ __device__ constexpr int lr_fast_slot_floor(int cb, int rhc, int nb) {
  if (cb == 1 && rhc == 2)
    return nb <= 8 ? 1 : nb <= 12 ? 9 : nb <= 14 ? 13 : nb <= 16 ? 15 : nb <= 18 ? 17 : nb <= 20 ? 19 : nb <= 24 ? 21
                                                                                                             : 25;
  return nb <= 8 ? 1 : nb <= 16 ? 9 : 17;
}

// Optional code sets of the fast LR kernels (FEAT template parameter): per-token
// query and gate, output norm, per-source static key.
constexpr int kFeatDyn = 1, kFeatNorm = 2, kFeatStatic = 4, kFeatAll = 7;

// Value rows per token that the one-column 16-bit fast LR kernels load straight
// into LDS (global_load_lds_dwordx4) instead of VGPRs.  Rows loaded that way
// hold no registers while in flight and, measured at C3, stream faster than
// register loads (forward 87.6 -> 74.9 us, backward 183.5 -> 165.8 us with 6
// rows).  At most the slot floor (so every staged row is a real source), even
// (the mix and dW loops take source pairs), and 6 at most: each row costs
// 4 KB of LDS per workgroup, and at 8 the backward drops from 4 to 3
// workgroups per CU (188 us).  Only the static-query sets (no per-token query,
// no static keys): while a direct-to-LDS load is pending the compiler turns
// every wait on the vector-memory counter into a wait for all of them, and the
// per-token query chain then runs after the whole token has arrived (C4 with
// staging: forward 226 -> 243 us, backward 468 -> 507 us).
__host__ __device__ constexpr int lr_fast_staged_rows(int cb, int rhc, int nb, int elem_bytes, int feat) {
  if (cb != 1 || elem_bytes != 2 || (feat & (kFeatDyn | kFeatStatic)) != 0) return 0;
  const int f = lr_fast_slot_floor(cb, rhc, nb) & ~1;
  return f < 6 ? f : 6;
}


// Fast base backward (attnres_base_fast.h): LDS bytes beyond the source
// tables -- the fold rows of its four waves, n_part floats each padded to 16
// bytes (one lane's query slots are written as 16-byte vectors).
constexpr int kBaseFastWaves = 4;
__host__ __device__ constexpr size_t base_bwd_fast_lds(int n_part) {
  return (size_t)kBaseFastWaves * (((size_t)n_part + 3) / 4 * 4) * sizeof(float);
}

struct ReadParams {
  const void* val[kMaxSources];
  const void* key[kMaxSources];
  int32_t vstride[kMaxSources];  // row strides in elements
  int32_t kstride[kMaxSources];
  const void* q_static;  // LR [H*rh] / base [D]
  const void* q_dyn;     // [n_tok rows of R]
  const void* gate;      // [H] or [n_tok, H]
  const float* bias;     // [N]
  void* out;             // [n_tok, D]
  void* out_prenorm;     // [n_tok, D] read before the output norm (forward write / backward read)
  float* weights;        // [n_tok, H, N]
  float* out_inv_rms;    // [n_tok]
  int64_t n_tok;
  int64_t q_dyn_stride;
  int32_t n_src, D, H, R, rh, dh;
  int32_t ncols;         // vector columns per row: ceil(D / (64*E))
  int32_t wpt;           // waves per token
  int32_t key_norm, norm_out, mode;
  int32_t gate_per_token, gate_act;
  int32_t key_vec;       // keys / per-token queries allow 16-byte loads
  float scale, eps;
  // head-aligned work items (LR fast path): a wave owns `item_cols` columns
  // holding `nh` whole heads of one token; items per token = n_items; waves
  // with the same item index walk the tokens with stride `streams`
  int32_t n_items, nh, kch, streams;
  int32_t np;  // lanes per head in the (head, source) pair layout: next power of two >= n_src
  int32_t kdt;  // dtype code of the LR keys and their gradients (the value dtype unless the desc says otherwise)
  int32_t ldt;  // dtype code of the LR logit path: query, rounded keys, logits, their gradients
  const void* skey;  // LR static source keys [n_src, R] (key dtype) added to every key, or null
};

struct ReadBwdParams {
  ReadParams f;
  const void* gout;          // [n_tok, D]
  const float* saved_w;      // [n_tok, H, N]
  const float* saved_inv;    // [n_tok]
  void* dval[kMaxSources];   // [n_tok, D]
  void* dkey[kMaxSources];   // [n_tok, R]
  void* dq_dyn;              // [n_tok, R]
  void* dgate;               // per-token gate gradient [n_tok, H]
  float* partials;           // per-workgroup partial sums, layout part_layout (kPart*)
  int32_t n_part;            // slots per workgroup: q (R or D) | gate (H) | bias (N)
  int32_t part_q, part_gate, part_bias;  // slot offsets (-1 = unused)
  int32_t part_layout;       // kPart* layout of `partials` (fast base backward; the fast LR backward writes slot-major, the others row-major)
};

// Layouts of the per-workgroup partial sums (workgroup w, slot i):
//   row-major   [w][i]
//   slot-major  [i][w]                     (few slots: one reduction workgroup per slot)
//   tiled       [i / 16][w][i % 16]        (many slots: 64-byte runs both ways)
constexpr int kPartRowMajor = 0, kPartSlotMajor = 1, kPartTiled = 2;
constexpr int kPartTile = 16;
__host__ __device__ inline int64_t part_index(int layout, int64_t w, int i, int n_groups, int n_part) {
  if (layout == kPartSlotMajor) return (int64_t)i * n_groups + w;
  if (layout == kPartTiled) return ((int64_t)(i / kPartTile) * n_groups + w) * kPartTile + i % kPartTile;
  return w * n_part + i;
}
// slots per workgroup row in the workspace (tiled rows are padded to whole tiles)
__host__ __device__ inline int part_stride(int n_part) { return (n_part + kPartTile - 1) / kPartTile * kPartTile; }

// Token sums of the LR key gradients per source (the static keys' gradient):
// partial sums per (source, token chunk), then a fixed-order sum over chunks.
constexpr int kColsumMaxChunks = 128;  // <= 2 x 64: the finish pass gives each lane two chunks
static_assert(kColsumMaxChunks <= 2 * kWaveSize, "static-key finish pass: two chunks per lane");
constexpr int kColsumTokens = 128;  // tokens per chunk at least
struct ColsumParams {
  const void* dk[kMaxSources];  // [n_tok, R] dense, key dtype
  float* partials;              // [n_src][chunks][R]
  void* out;                    // [n_src, R] key dtype
  int64_t n_tok;
  int32_t n_src, R, chunks, kdt;
};

// Value-derived keys: rms-norm of every source row into one dense block
struct ValueNormParams {
  const void* val[kMaxSources];
  int32_t vstride[kMaxSources];  // row strides in elements
  void* dval[kMaxSources];       // backward: [n_tok, D] dense
  void* normed;                  // [n_src, n_tok, D] dense
  const void* gnormed;           // backward: its gradient, same layout
  float* inv;                    // [n_src, n_tok]
  int64_t n_tok;
  int32_t n_src, D;
  float eps;
};

struct ReduceParams {
  const float* partials;      // layout: kPart*
  int32_t n_groups, n_part;
  int32_t layout;
  int32_t part_q, n_q;        // static query slots
  int32_t part_gate, n_gate;  // per-site gate slots
  int32_t part_bias, n_bias;
  int32_t part_extra, n_extra;  // further fp32 slots (phase 2: value-scale gradient)
  void* dquery;               // dtype
  void* dgate;                // dtype
  float* dbias;
  float* dextra;
  int32_t q_rows, q_row;      // q_rows > 1: dquery is a [q_rows][n_q] bank, row q_row written, the others zeroed
};

// Phase 1 (cached-logit read of completed sources for Q read sites)
constexpr int kPhase1MaxQ = ATTNRES_PHASE1_MAX_QUERIES;
struct Phase1Params {
  const void* val[kMaxSources];
  void* dval[kMaxSources];     // backward: [n_tok, D] dense
  int32_t vstride[kMaxSources];
  const void* lsrc[kMaxSources];  // source s's logits: (q, t) at lsrc[s] + q*lq + t (elements)
  int64_t lq;
  void* dlsrc[kMaxSources];       // backward: source s's logit gradient, (q, t) at dlsrc[s] + q*dlq + t
  int64_t dlq;
  void* out;                   // [Q, n_tok, D]
  void* out_prenorm;           // [Q, n_tok, D] or null
  float* lse;                  // [Q, n_tok]
  float* out_inv_rms;          // [Q, n_tok] or null
  const void* gout[ATTNRES_PHASE1_MAX_QUERIES];   // backward: site q's output gradient [n_tok, D] dense
  const float* glse[ATTNRES_PHASE1_MAX_QUERIES];  // backward: site q's lse gradient [n_tok], null = zero
  // stacked: every table above is entry 0 plus a uniform stride (elements):
  // lsrc[s] = lsrc[0] + s*ls, dlsrc[s] = dlsrc[0] + s*dls, gout[q] = gout[0] +
  // q*gq, glse[q] = glse[0] + q*glq (or all null); the column-split kernels
  // then address rows from entry 0 instead of holding every table entry
  int32_t stacked;
  int64_t ls, dls, gq, glq;
  int64_t n_tok;
  int32_t n_src, n_q, D, ncols;
  int32_t ldt;                 // logits dtype code
  int32_t norm_out;
  int32_t np;                  // lanes per softmax row: next power of two >= n_src
  float eps;
};

// Entry idx (< K) of a pointer table in the kernel arguments: the K entries
// are read as scalars and the lane's one picked by a chain of selects, so that
// no lane waits on a per-lane load of its pointer before the load it addresses.
template <int K, class T, int M>
__device__ __forceinline__ T p1_pick(T const (&tab)[M], int idx) {
  static_assert(K <= M, "table smaller than the slots picked from");
  T r = tab[0];
#pragma unroll
  for (int i = 1; i < K; ++i) r = idx == i ? tab[i] : r;
  return r;
}

// Phase-1 accessors (the source and site indices may differ across lanes: the
// pointer tables are read from the kernel arguments per lane)
__device__ __forceinline__ float p1_logit(const Phase1Params& p, int q, int s, int64_t t) {
  return load_any(p.lsrc[s], (int64_t)q * p.lq + t, p.ldt);
}
__device__ __forceinline__ void p1_store_dlogit(const Phase1Params& p, int q, int s, int64_t t, float v) {
  store_any(p.dlsrc[s], (int64_t)q * p.dlq + t, p.ldt, v);
}
// site q's lse gradient (0 for a site without one; q < n_q; the table index is
// clamped so that a load the compiler hoists out of a lane condition stays
// inside the table)
__device__ __forceinline__ float p1_glse(const Phase1Params& p, int q, int64_t t) {
  const float* g = p.glse[q < kPhase1MaxQ ? q : kPhase1MaxQ - 1];
  return g ? g[t] : 0.f;
}
// dl = w (dW - <w, dW>) plus the lse term w * glse, rounded as the eager op
// rounds its logit gradient (a site without an lse gradient adds 0)
__device__ __forceinline__ float p1_dlogit(const Phase1Params& p, float dl, float gl) {
  return p.ldt == ATTNRES_DTYPE_F32 ? dl + gl : round_any(round_any(dl, p.ldt) + round_any(gl, p.ldt), p.ldt);
}

// Logits of one LR source against its read sites (attnres_site_logits.hip)
constexpr int kSiteLogitsMaxQ = ATTNRES_SITE_LOGITS_MAX_QUERIES;
struct SiteLogitsParams {
  const void* key;        // [n_tok] rows of R elements, row stride kstride (elements)
  int64_t kstride;
  const void* queries;    // [n_q, R] dense, dtype
  void* out;              // forward: [n_q, n_tok] dense, odt
  const void* dout[kSiteLogitsMaxQ];  // backward: site q's logit gradient [n_tok], odt
  void* dkey;             // backward: [n_tok, R] dense
  void* du;               // backward: [n_q, n_tok] dense, dtype
  void* khat;             // backward: [n_tok, R] dense, dtype
  int64_t n_tok;
  int32_t R, n_q, key_norm, odt, vec;
  float eps, scale, bias;
};

// Phase 2 (merge of a read site's phase-1 result with the partial block)
struct Phase2Params {
  const void* pv;              // partial value rows
  const void* pk;              // LR partial key rows
  const void* q;               // [D] or [R]
  const void* plogit;          // [n_tok] given logits
  const void* inter;           // interblock output rows
  const float* lse;            // [n_tok]
  const float* bias_dev;       // fp32 scalar or null
  const float* scale_dev;      // fp32 scalar or null
  void* out;                   // [n_tok, D]
  const void* gout;            // backward: [n_tok, D]
  void* dpv;                   // [n_tok, D]
  void* dpk;                   // [n_tok, R]
  void* dinter;                // [n_tok, D]
  float* dlse;                 // [n_tok]
  void* dplogit;               // [n_tok]
  float* partials;             // [gridDim.x, n_part]
  int64_t n_tok, pv_stride, pk_stride, inter_stride;
  int32_t n_part, part_q, part_bias, part_scale;  // slot offsets (-1 = unused)
  int32_t D, R, ncols;
  int32_t logit_given, merge, key_norm, norm_out, scale_key, pl_dt;
  float scale, eps, bias, vscale;
  // Block accumulation fused in front of the LR merge (the fast LR kernels'
  // ACC instantiations).  Forward: the partial block read here is the live
  // block grown by this sublayer -- value rnd(acc_pv_old + y[:D]), key
  // rnd(acc_pk_old + key(y[D:D+R])), the key rms-normed over heads of acc_hd
  // columns when acc_key_norm -- written to acc_pv_out / acc_pk_out with the
  // key's 1/rms in acc_inv [n_tok, acc_H]; pv / pk are not read.  Backward
  // (pv / pk = the grown block): the grown block's total gradient (the
  // merge's share plus acc_gv / acc_gk from its other consumers, if any) goes
  // to the projection gradient acc_gy [n_tok, acc_P] (value columns as they
  // are, key columns through the key norm, padding zero) and, for the key, to
  // acc_dpk_old (the old partial key's gradient); dpv / dpk are not written.
  const void* acc_y;           // [n_tok, acc_y_stride]
  int64_t acc_y_stride;
  int32_t acc_P, acc_H, acc_hd, acc_key_norm;
  float acc_eps;
  const void* acc_pv_old;      // [n_tok, D] or null (a block's first sublayer)
  const void* acc_pk_old;      // [n_tok, R] or null
  void* acc_pv_out;            // [n_tok, D]
  void* acc_pk_out;            // [n_tok, R]
  float* acc_inv;              // [n_tok, acc_H]
  const void* acc_gv;          // [n_tok, D] rows acc_gv_stride apart, or null
  int64_t acc_gv_stride;
  const void* acc_gk;          // [n_tok, R] or null
  void* acc_gy;                // [n_tok, acc_P]
  void* acc_dpk_old;           // [n_tok, R] or null
};

// Logits of a query bank against the sources' keys (phase 1 from a query bank)
constexpr int kKLMaxQ = 16;
struct KeyedLogitsParams {
  const void* val[kMaxSources];
  void* dval[kMaxSources];     // backward: [n_tok, D] dense
  int32_t vstride[kMaxSources];
  const void* queries;         // [n_q, D], value dtype
  void* logits;                // forward: [n_q, n_src, n_tok], value dtype
  const void* dlogits;         // backward: same layout
  float* inv;                  // [n_src, n_tok]: 1/rms of each key (forward writes, backward reads)
  float* partials;             // backward: [groups, n_q * D] query-gradient partial rows (null: no dqueries)
  int64_t n_tok;
  int32_t n_src, n_q, D, key_norm, n_part;
  float eps;
};

// Key-producer epilogue: split of the fused [out | key | pad] projection.
struct KeySplitParams {
  const void* y;     // [n_tok, y_stride]: the projection (GEMM output)
  void* out;         // forward: [n_tok, D]
  void* key;         // forward: [n_tok, R]
  float* inv;        // [n_tok, H]: 1/rms of each key head (key_norm)
  const void* gout;  // backward: [n_tok, D] or null
  const void* gkey;  // backward: [n_tok, R] or null
  void* gy;          // backward: [n_tok, P]
  int64_t n_tok, y_stride;
  int32_t D, R, P, H, hd, key_norm;
  float eps;
  // block-summary accumulation (attnres_block_accum_*): 0 = plain split
  int32_t accum;          // 1: add to the partial block; 2: form the completed block source
  const void* pv;         // partial value rows [n_tok, D] dense, or null
  const void* pk;         // partial key rows [n_tok, R] dense, or null
  int32_t value_norm, scale_key;
  float vscale;           // summary scale when scale_dev is null
  const float* scale_dev; // learned summary scale (fp32 scalar) or null
  float* vinv;            // [n_tok] 1/rms of the summary value (value_norm)
  int64_t gout_stride;    // backward: elements between rows of gout
  void* dpk;              // backward: partial-key gradient [n_tok, R] (complete with scale_key)
  float* partials;        // backward: learned-scale gradient partial sums [gridDim.x][2]
};

}  // namespace attnres
