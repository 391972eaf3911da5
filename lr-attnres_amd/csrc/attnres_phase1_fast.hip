// Phase 1 (cached-logit schedule) backward and forward, fast path: 16-bit rows that one
// wave covers exactly (D = 256 / 768 with 8-byte vectors in 1 / 3 columns,
// 512 / 1024 with 16-byte ones), at most 4 read sites and 8 sources, no output
// norm.  Semantics are those of phase1_bwd_kernel (attnres_phase1.hip, after
// the reference's eager op, attnres_ops.py:3956-3961):
//   dW[q, s] = rnd(<g[q], v[s]>),  dl = w (dW - sum_s w dW) (+ glse w),
//   dv[s]    = rnd(sum_q rnd(w[q, s]) g[q]).
// The general kernel spends its time on fp32 multiply-adds: Q x S row dot
// products and Q passes per value gradient, each element unpacked again.
// Here both are v_dot2 on packed words: a dot product costs half an
// instruction per element, and dv one v_dot2 per element and pair of sites
// (the upstream rows are interleaved by site pairs once per token).  The
// Q x S row sums are folded together by wave_sums.  Work layout as the other
// one-wave kernels: four token streams per workgroup, one resident round of
// waves, slots past n_src / n_q load a real row (the last one) and weigh 0.
// Workgroups take their tokens in XCD-major order (xcd_block): the logits
// [Q, S, n] and lse [Q, n] are token-minor, so the tokens sharing one of their
// cache lines run in one XCD and the line is fetched into one L2.
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

constexpr int kP1FastWaves = 4;  // token streams (waves) per workgroup
constexpr int kP1FastQ = 4;      // site slots

template <class DT, int VB, int CB, int SB>
__global__ void __launch_bounds__(256) phase1_bwd_fast_kernel(const Phase1Params p) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  constexpr int QB = kP1FastQ;
  constexpr int V = QB * SB;  // dot products per token
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform_i32(threadIdx.x / kWave);
  const int N = p.n_src, Q = p.n_q, D = p.D, np = p.np;
  // (site, source) lane of the softmax rows: lane = q * np + s
  const int sl = lane & (np - 1), ql = lane / np;
  const bool own = sl < N && ql < Q;
  // this lane's logits row pointers, picked once (loop-invariant)
  const void* lrow = p1_pick<SB>(p.lsrc, sl);
  const float* glrow = p1_pick<QB>(p.glse, ql);
  void* dlrow = p1_pick<SB>(p.dlsrc, sl);

  const int64_t t0 = (int64_t)xcd_block(blockIdx.x, gridDim.x) * kP1FastWaves + wave;  // XCD-major: logits / lse lines
  for (int64_t tok = t0; tok < p.n_tok; tok += (int64_t)gridDim.x * kP1FastWaves) {
    // ---- loads: upstream rows of the sites, value rows of the sources
    Raw<DT, E> gr[QB][CB], vr[SB][CB];
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const S* gp = (const S*)p.gout[min(q, Q - 1)] + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(gp + (c * kWave + lane) * E, gr[q][c]);
    }
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int j = min(s, N - 1);
      const S* vp = (const S*)p.val[j] + tok * (int64_t)p.vstride[j];
#pragma unroll
      for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(vp + (c * kWave + lane) * E, vr[s][c]);
    }
    // ---- softmax rows in the (site, source) lane layout
    const float l = own ? load_any(lrow, (int64_t)ql * p.lq + tok, p.ldt) : -INFINITY;
    const float lm = group_max(l, np);
    const float ex = own ? expf(l - lm) : 0.f;
    const float wt = ex / group_sum(ex, np);

    // ---- dW[q, s] = <g[q], v[s]>: one v_dot2 per word, all Q x S sums at once
    float part[V];
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
      for (int s = 0; s < SB; ++s) {
        float d = 0.f;
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int i = 0; i < W; ++i) d = dot2<DT>(gr[q][c].w[i], vr[s][c].w[i], d);
        part[q * SB + s] = d;
      }
    float z[V / 4];
    wave_sums<V>(part, z);
    float dw = 0.f;
#pragma unroll
    for (int q = 0; q < QB; ++q)
#pragma unroll
      for (int s = 0; s < SB; ++s)
        dw = wave_sums_pick<V>(z, q * SB + s, s < N && lane == q * np + s, dw);

    // ---- logits gradient (lane (q, s)): as phase1_bwd_kernel
    {
      const float dwb = DT::rnd(dw);  // gradient of the dtype-rounded weights
      const float inner = group_sum(own ? wt * dwb : 0.f, np);
      float dl = wt * (dwb - inner);
      dl = p1_dlogit(p, dl, own ? (glrow ? glrow[tok] : 0.f) * wt : 0.f);
      if (own) store_any(dlrow, (int64_t)ql * p.dlq + tok, p.ldt, dl);
    }

    // ---- dv[s] = rnd(sum_q rnd(w[q, s]) g[q]): upstream rows interleaved by
    // site pairs (element e of sites 2k, 2k+1 in one word), weights packed
    const uint32_t wb = own ? bits16<DT>(DT::rnd(wt)) : 0u;
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int i = 0; i < W; ++i)
#pragma unroll
        for (int k = 0; k < QB / 2; ++k) {
          const uint32_t a = gr[2 * k][c].w[i], b = gr[2 * k + 1][c].w[i];
          gr[2 * k][c].w[i] = lo_pair(a, b);
          gr[2 * k + 1][c].w[i] = hi_pair(a, b);
        }
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      if (s < N) {
        uint32_t wp[QB / 2];
#pragma unroll
        for (int k = 0; k < QB / 2; ++k)
          wp[k] = (uint32_t)__builtin_amdgcn_readlane((int)wb, (2 * k) * np + s) |
                  ((uint32_t)__builtin_amdgcn_readlane((int)wb, (2 * k + 1) * np + s) << 16);
        S* dp = (S*)p.dval[s] + tok * (int64_t)D;
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          float acc[E];
#pragma unroll
          for (int i = 0; i < W; ++i) {
            float lo = 0.f, hi = 0.f;
#pragma unroll
            for (int k = 0; k < QB / 2; ++k) {
              lo = dot2<DT>(gr[2 * k][c].w[i], wp[k], lo);
              hi = dot2<DT>(gr[2 * k + 1][c].w[i], wp[k], hi);
            }
            acc[2 * i] = lo;
            acc[2 * i + 1] = hi;
          }
          store_vec<DT, E, true>(dp + (c * kWave + lane) * E, acc);
        }
      }
    }
  }
}

// Forward on the same rows: w = softmax(logits) (fp32), lse = max + log(sum),
// out[q] = rnd(sum_s rnd(w[q, s]) v[s]).  The value rows are interleaved by
// source pairs once per token; each site then costs one v_dot2 per element
// and source pair.
template <class DT, int VB, int CB, int SB>
__global__ void __launch_bounds__(256) phase1_fwd_fast_kernel(const Phase1Params p) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  constexpr int QB = kP1FastQ;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform_i32(threadIdx.x / kWave);
  const int N = p.n_src, Q = p.n_q, D = p.D, np = p.np;
  const int sl = lane & (np - 1), ql = lane / np;
  const bool own = sl < N && ql < Q;
  // this lane's logits row pointers, picked once (loop-invariant)
  const void* lrow = p1_pick<SB>(p.lsrc, sl);

  const int64_t t0 = (int64_t)xcd_block(blockIdx.x, gridDim.x) * kP1FastWaves + wave;  // XCD-major: logits / lse lines
  for (int64_t tok = t0; tok < p.n_tok; tok += (int64_t)gridDim.x * kP1FastWaves) {
    Raw<DT, E> vr[SB][CB];
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int j = min(s, N - 1);
      const S* vp = (const S*)p.val[j] + tok * (int64_t)p.vstride[j];
#pragma unroll
      for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(vp + (c * kWave + lane) * E, vr[s][c]);
    }
    // softmax rows and lse in the (site, source) lane layout
    const float l = own ? load_any(lrow, (int64_t)ql * p.lq + tok, p.ldt) : -INFINITY;
    const float lm = group_max(l, np);
    const float ex = own ? expf(l - lm) : 0.f;
    const float z = group_sum(ex, np);
    if (own && sl == 0) p.lse[(int64_t)ql * p.n_tok + tok] = lm + logf(z);
    const uint32_t wb = own ? bits16<DT>(DT::rnd(ex / z)) : 0u;
    // value rows interleaved by source pairs
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int i = 0; i < W; ++i)
#pragma unroll
        for (int k = 0; k < SB / 2; ++k) {
          const uint32_t a = vr[2 * k][c].w[i], b = vr[2 * k + 1][c].w[i];
          vr[2 * k][c].w[i] = lo_pair(a, b);
          vr[2 * k + 1][c].w[i] = hi_pair(a, b);
        }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      if (q < Q) {
        uint32_t wp[SB / 2];
#pragma unroll
        for (int k = 0; k < SB / 2; ++k) {
          const uint32_t w0 = 2 * k < N ? (uint32_t)__builtin_amdgcn_readlane((int)wb, q * np + 2 * k) : 0u;
          const uint32_t w1 = 2 * k + 1 < N ? (uint32_t)__builtin_amdgcn_readlane((int)wb, q * np + 2 * k + 1) : 0u;
          wp[k] = w0 | (w1 << 16);
        }
        S* op = (S*)p.out + ((int64_t)q * p.n_tok + tok) * D;
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          float acc[E];
#pragma unroll
          for (int i = 0; i < W; ++i) {
            float lo = 0.f, hi = 0.f;
#pragma unroll
            for (int k = 0; k < SB / 2; ++k) {
              if (2 * k < N) {
                lo = dot2<DT>(vr[2 * k][c].w[i], wp[k], lo);
                hi = dot2<DT>(vr[2 * k + 1][c].w[i], wp[k], hi);
              }
            }
            acc[2 * i] = lo;
            acc[2 * i + 1] = hi;
          }
          store_vec<DT, E, true>(op + (c * kWave + lane) * E, acc);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- column split
// Phase 1 for the reference model's block widths (up to 16 read sites): a
// token's row is split over D / 256 waves of one workgroup, each wave owning
// 256 columns (8 bytes per lane), so a wave holds Q upstream and S value
// vectors of 2 words each instead of whole rows.  Softmax rows in the (site,
// source) lane layout, lane = q * np + s, so Q * np <= 64 (Q <= 16 with
// S <= 4, Q <= 8 with S <= 8, Q <= 4 with S <= 16).  Same arithmetic and
// rounding points as the one-wave kernels above; the forward needs nothing
// across waves, the backward sums the Q x S row dot products of its waves
// through LDS in a fixed order (one barrier per token) before rounding dW.
// Workgroups walk tokens in XCD-major order: the logits [Q, S, n] and lse
// [Q, n] are token-minor, so neighbouring tokens share their cache lines.
constexpr int kP1SplitCols = 256;  // columns per wave (64 lanes x 4 elements)

template <class DT, int QB, int SB, bool ST>
__global__ void __launch_bounds__(512) phase1_fwd_split_kernel(const Phase1Params p) {
  using S = typename DT::S;
  static_assert(QB * SB <= 64 && SB % 2 == 0, "one (site, source) pair per lane, sources in pairs");
  // per wave: the rounded weights [QB][SB] as 16-bit values, read back as
  // (source 2k, 2k + 1) words by every lane (broadcast reads)
  __shared__ uint16_t s_wh[8][64];
  const int lane = threadIdx.x & (kWave - 1);
  const int chunk = uniform_i32(threadIdx.x / kWave);  // this wave's 256 columns
  const int N = p.n_src, Q = p.n_q, D = p.D, np = p.np;
  const int sl = lane & (np - 1), ql = lane / np;
  const bool own = sl < N && ql < Q;
  // this lane's logits row pointer (loop-invariant), as in the backward
  const void* lrow = ST ? p.lsrc[0] : p1_pick<SB>(p.lsrc, sl);
  const int64_t loff = ST ? (int64_t)sl * p.ls : 0;
  const int col = chunk * kP1SplitCols + lane * 4;
  for (int64_t tok = xcd_block(blockIdx.x, gridDim.x); tok < p.n_tok; tok += gridDim.x) {
    Raw<DT, 4> vr[SB];
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int j = min(s, N - 1);
      load_raw<DT, 4, true>((const S*)p.val[j] + tok * (int64_t)p.vstride[j] + col, vr[s]);
    }
    const float l = own ? load_any(lrow, loff + (int64_t)ql * p.lq + tok, p.ldt) : -INFINITY;
    const float lm = group_max(l, np);
    const float ex = own ? expf(l - lm) : 0.f;
    const float z = group_sum(ex, np);
    if (chunk == 0 && own && sl == 0) p.lse[(int64_t)ql * p.n_tok + tok] = lm + logf(z);
    if (sl < SB && ql < QB) s_wh[chunk][ql * SB + sl] = (uint16_t)(own ? bits16<DT>(DT::rnd(ex / z)) : 0u);
    wave_sync();
    const uint32_t* s_wp = (const uint32_t*)s_wh[chunk];  // word q * SB / 2 + k: sources 2k, 2k + 1 of site q
    // value words interleaved by source pairs
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int k = 0; k < SB / 2; ++k) {
        const uint32_t a = vr[2 * k].w[i], b = vr[2 * k + 1].w[i];
        vr[2 * k].w[i] = lo_pair(a, b);
        vr[2 * k + 1].w[i] = hi_pair(a, b);
      }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      if (q < Q) {
        float acc[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float lo = 0.f, hi = 0.f;
#pragma unroll
          for (int k = 0; k < SB / 2; ++k) {
            if (2 * k < N) {
              const uint32_t wp = s_wp[q * (SB / 2) + k];  // zero weights past N
              lo = dot2<DT>(vr[2 * k].w[i], wp, lo);
              hi = dot2<DT>(vr[2 * k + 1].w[i], wp, hi);
            }
          }
          acc[2 * i] = lo;
          acc[2 * i + 1] = hi;
        }
        store_vec<DT, 4, true>((S*)p.out + ((int64_t)q * p.n_tok + tok) * D + col, acc);
      }
    }
    wave_sync();  // the table is read before the next token writes it
  }
}

template <class DT, int QB, int SB, bool ST>
__global__ void __launch_bounds__(512) phase1_bwd_split_kernel(const Phase1Params p) {
  using S = typename DT::S;
  static_assert(QB * SB <= 64 && QB % 2 == 0 && SB % 2 == 0, "one (site, source) pair per lane");
  constexpr int V = QB * SB;                 // row dot products per token (multiple of 4)
  // reduced 16 at a time (12 when V = 24; V itself up to 16)
  constexpr int VB16 = V <= 16 ? V : V % 16 == 0 ? 16 : 12;
  static_assert(V % VB16 == 0 && VB16 % 4 == 0, "the row dot products reduce in whole groups of four");
  __shared__ float s_dw[8][64];              // [wave][pair]: this wave's partial dW of pair (q, s) = q * SB + s
  __shared__ uint16_t s_wh[8][64];           // [wave][s * QB + q]: rounded weights, 16-bit
  const int lane = threadIdx.x & (kWave - 1);
  const int chunk = uniform_i32(threadIdx.x / kWave);
  const int nw = blockDim.x / kWave;
  const int N = p.n_src, Q = p.n_q, D = p.D, np = p.np;
  const int sl = lane & (np - 1), ql = lane / np;
  const bool own = sl < N && ql < Q;
  // this lane's logits row pointers (loop-invariant): from entry 0 and the
  // strides when the tables are stacked, else picked from the tables
  const void* lrow = ST ? p.lsrc[0] : p1_pick<SB>(p.lsrc, sl);
  const int64_t loff = ST ? (int64_t)sl * p.ls : 0;
  const float* glrow = ST ? p.glse[0] : p1_pick<QB>(p.glse, ql);
  const int64_t goff = ST ? (int64_t)ql * p.glq : 0;
  void* dlrow = ST ? p.dlsrc[0] : p1_pick<SB>(p.dlsrc, sl);
  const int64_t doff = ST ? (int64_t)sl * p.dls : 0;
  const int col = chunk * kP1SplitCols + lane * 4;
  for (int64_t tok = xcd_block(blockIdx.x, gridDim.x); tok < p.n_tok; tok += gridDim.x) {
    Raw<DT, 4> gr[QB], vr[SB];
#pragma unroll
    for (int q = 0; q < QB; ++q)
      load_raw<DT, 4, true>((ST ? (const S*)p.gout[0] + (int64_t)min(q, Q - 1) * p.gq : (const S*)p.gout[min(q, Q - 1)]) +
                                tok * (int64_t)D + col,
                            gr[q]);
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      const int j = min(s, N - 1);
      load_raw<DT, 4, true>((const S*)p.val[j] + tok * (int64_t)p.vstride[j] + col, vr[s]);
    }
    const float l = own ? load_any(lrow, loff + (int64_t)ql * p.lq + tok, p.ldt) : -INFINITY;
    const float glse = own ? (glrow ? glrow[goff + tok] : 0.f) : 0.f;
    const float lm = group_max(l, np);
    const float ex = own ? expf(l - lm) : 0.f;
    const float wt = ex / group_sum(ex, np);

    // partial dW[q, s] over this wave's columns, 16 pairs at a time; pair
    // (q, s) is value q * SB + s and lane q * np + s (SB == np: the host picks
    // the instantiation with SB = np)
#pragma unroll
    for (int b = 0; b < V; b += VB16) {
      if (b / SB < Q) {
        float part[VB16];
#pragma unroll
        for (int m = 0; m < VB16; ++m) {
          const int q = (b + m) / SB, s = (b + m) - ((b + m) / SB) * SB;
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 2; ++i) d = dot2<DT>(gr[q].w[i], vr[s].w[i], d);
          part[m] = d;
        }
        float z[VB16 / 4];
        wave_sums<VB16>(part, z);
        // register k holds value 4k + {0, 2, 1, 3}[row] in every lane of a
        // 16-lane row: the first lane of each row stores it
        if ((lane & 15) == 0) {
          const int r = lane >> 4, j = r == 1 ? 2 : r == 2 ? 1 : r;
#pragma unroll
          for (int k = 0; k < VB16 / 4; ++k) s_dw[chunk][b + 4 * k + j] = z[k];
        }
      }
    }
    __syncthreads();
    float dw = 0.f;
    for (int w = 0; w < nw; ++w) dw += s_dw[w][lane];  // fixed order
    __syncthreads();  // read before the next token writes

    // logits gradient (lane (q, s)), as the one-wave kernel
    {
      const float dwb = DT::rnd(dw);
      const float inner = group_sum(own ? wt * dwb : 0.f, np);
      float dl = wt * (dwb - inner);
      dl = p1_dlogit(p, dl, own ? glse * wt : 0.f);
      if (chunk == 0 && own) store_any(dlrow, doff + (int64_t)ql * p.dlq + tok, p.ldt, dl);
    }

    // dv[s] = rnd(sum_q rnd(w[q, s]) g[q]) over this wave's columns: upstream
    // words interleaved by site pairs, weights packed by site pairs
    if (sl < SB && ql < QB) s_wh[chunk][sl * QB + ql] = (uint16_t)(own ? bits16<DT>(DT::rnd(wt)) : 0u);
    wave_sync();
    const uint32_t* s_wp = (const uint32_t*)s_wh[chunk];  // word s * QB / 2 + k: sites 2k, 2k + 1 of source s
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int k = 0; k < QB / 2; ++k) {
        const uint32_t a = gr[2 * k].w[i], b = gr[2 * k + 1].w[i];
        gr[2 * k].w[i] = lo_pair(a, b);
        gr[2 * k + 1].w[i] = hi_pair(a, b);
      }
#pragma unroll
    for (int s = 0; s < SB; ++s) {
      if (s < N) {
        float acc[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float lo = 0.f, hi = 0.f;
#pragma unroll
          for (int k = 0; k < QB / 2; ++k) {
            if (2 * k < Q) {
              const uint32_t wp = s_wp[s * (QB / 2) + k];  // zero weights past Q
              lo = dot2<DT>(gr[2 * k].w[i], wp, lo);
              hi = dot2<DT>(gr[2 * k + 1].w[i], wp, hi);
            }
          }
          acc[2 * i] = lo;
          acc[2 * i + 1] = hi;
        }
        store_vec<DT, 4, true>((S*)p.dval[s] + tok * (int64_t)D + col, acc);
      }
    }
    wave_sync();  // the weight table is read before the next token writes it
  }
}

// L.wpt = waves per token (D / 256), L.nmax = source slots (np: 2/4/8/16)
template <class DT, bool BWD>
static hipError_t phase1_split_dt(const Phase1Params& p, const Launch& L, hipStream_t st) {
  const dim3 g(L.grid), b(L.wpt * kWave);
#define ATTNRES_P1S(QB, SB)                                                                               \
  if (p.stacked) {                                                                                        \
    if constexpr (BWD) hipLaunchKernelGGL((phase1_bwd_split_kernel<DT, QB, SB, true>), g, b, 0, st, p);    \
    else hipLaunchKernelGGL((phase1_fwd_split_kernel<DT, QB, SB, true>), g, b, 0, st, p);                  \
  } else {                                                                                                \
    if constexpr (BWD) hipLaunchKernelGGL((phase1_bwd_split_kernel<DT, QB, SB, false>), g, b, 0, st, p);   \
    else hipLaunchKernelGGL((phase1_fwd_split_kernel<DT, QB, SB, false>), g, b, 0, st, p);                 \
  }
  // L.nmax = source lanes np, L.teams = site slots (the site count rounded up
  // to 4, 6, 8, 12 or 16 within np * slots <= 64)
  switch (L.nmax * 100 + L.teams) {
    case 204: ATTNRES_P1S(4, 2) break;
    case 206: ATTNRES_P1S(6, 2) break;
    case 208: ATTNRES_P1S(8, 2) break;
    case 212: ATTNRES_P1S(12, 2) break;
    case 216: ATTNRES_P1S(16, 2) break;
    case 404: ATTNRES_P1S(4, 4) break;
    case 406: ATTNRES_P1S(6, 4) break;
    case 408: ATTNRES_P1S(8, 4) break;
    case 412: ATTNRES_P1S(12, 4) break;
    case 416: ATTNRES_P1S(16, 4) break;
    case 804: ATTNRES_P1S(4, 8) break;
    case 806: ATTNRES_P1S(6, 8) break;
    case 808: ATTNRES_P1S(8, 8) break;
    case 1604: ATTNRES_P1S(4, 16) break;
    default: return hipErrorInvalidValue;
  }
#undef ATTNRES_P1S
  return hipGetLastError();
}

hipError_t launch_phase1_split_forward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st) {
  if (dtype == ATTNRES_DTYPE_BF16) return phase1_split_dt<BF16, false>(p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return phase1_split_dt<F16, false>(p, L, st);
  return hipErrorInvalidValue;
}
hipError_t launch_phase1_split_backward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st) {
  if (dtype == ATTNRES_DTYPE_BF16) return phase1_split_dt<BF16, true>(p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return phase1_split_dt<F16, true>(p, L, st);
  return hipErrorInvalidValue;
}

// L.vb = vector bytes (8/16), L.wpt = columns per lane (1/2/3), L.nmax =
// source slots (2/4/6/8: the source count rounded up to a pair)
template <class DT, bool BWD>
static hipError_t phase1_fast_dt(const Phase1Params& p, const Launch& L, hipStream_t st) {
  const dim3 g(L.grid), b(kP1FastWaves * kWave);
#define ATTNRES_P1F(VB, CB, SB)                                                                    \
  case VB * 100 + CB * 10 + SB:                                                                    \
    if constexpr (BWD) hipLaunchKernelGGL((phase1_bwd_fast_kernel<DT, VB, CB, SB>), g, b, 0, st, p); \
    else hipLaunchKernelGGL((phase1_fwd_fast_kernel<DT, VB, CB, SB>), g, b, 0, st, p);             \
    break;
#define ATTNRES_P1F_SB(VB, CB) ATTNRES_P1F(VB, CB, 2) ATTNRES_P1F(VB, CB, 4) ATTNRES_P1F(VB, CB, 6) ATTNRES_P1F(VB, CB, 8)
  switch (L.vb * 100 + L.wpt * 10 + L.nmax) {
    ATTNRES_P1F_SB(8, 1)
    ATTNRES_P1F_SB(8, 3)
    ATTNRES_P1F_SB(16, 1)
    ATTNRES_P1F_SB(16, 2)
    default: return hipErrorInvalidValue;
  }
#undef ATTNRES_P1F_SB
#undef ATTNRES_P1F
  return hipGetLastError();
}

// 16-bit types only (the host plan never selects this path for fp32)
hipError_t launch_phase1_fast_forward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st) {
  if (dtype == ATTNRES_DTYPE_BF16) return phase1_fast_dt<BF16, false>(p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return phase1_fast_dt<F16, false>(p, L, st);
  return hipErrorInvalidValue;
}
hipError_t launch_phase1_fast_backward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st) {
  if (dtype == ATTNRES_DTYPE_BF16) return phase1_fast_dt<BF16, true>(p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return phase1_fast_dt<F16, true>(p, L, st);
  return hipErrorInvalidValue;
}

}  // namespace attnres
