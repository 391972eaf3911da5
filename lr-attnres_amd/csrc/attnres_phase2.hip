// Phase 2 of the cached-logit block-training schedule: merge of one read
// site's phase-1 result (interblock output + its log-sum-exp) with the live
// partial block.  Forward and backward, base and LR keys, or a given logit.
//
// Semantics follow the reference's eager merges at the same rounding points
// (attnres_ops.py:2630-2642, 4041-4068, 4085-4160):
//   p     = rnd(partial * value_scale)          block summary (model.py:990-1018)
//   key   = base: key_norm ? rnd(p / rms(p)) : p
//           LR:   key_norm ? rnd(k / rms(k)) : k   (k = partial key, fp32 norm)
//   logit = rnd(sum_i rnd(key_i * q_i))          torch.sum(key * query)
//           LR: rnd(logit * logit_scale)
//   prob  = rnd(sigmoid(logit + bias - lse))     fp32 sigmoid
//   out   = addcmul: rnd(inter + rnd(p - inter) * prob)
//           lerp:    rnd(torch.lerp(inter, p, prob))
//   optional out = rnd(out / rms(out))
// The backward recomputes these per token and follows the autograd graph of
// the same expressions (every dtype-tensor product rounded, fp32 sigmoid and
// norm backward).  Cross-token sums (query, learned bias and scale) go to
// per-workgroup partial rows, reduced in a fixed order afterwards.
//
// One workgroup of wpt waves owns one token at a time; a lane owns CB vectors
// of E elements of the D-wide rows, and thread t owns LR key elements
// t + j * blockDim (j < kP2KPT).
#include "attnres_block.h"
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

constexpr int kP2KPT = 4;  // LR key elements per thread

// Per-token forward state shared by both kernels.
template <int CB, int E>
struct P2State {
  float p[CB][E];    // scaled partial value (dtype-rounded)
  float pr[CB][E];   // partial value as loaded
  float it[CB][E];   // interblock output
  float key[CB][E];  // base key (dtype-rounded)
  float kl[kP2KPT];  // LR key (dtype-rounded)
  float kv[kP2KPT];  // LR key before the norm (scaled)
  float kr[kP2KPT];  // LR key as loaded
  float inv_key;     // 1/rms of the key (key_norm)
  float sg, prob;    // sigmoid and its dtype-rounded value
};

// One token's inputs as loaded (packed), so the next token's loads can be
// issued before the current token is processed.
template <class DT, int E, int CB>
struct P2Raw {
  Raw<DT, E> pv[CB], it[CB], g[CB];
  float kr[kP2KPT];
  float lse, logit;
};

template <class DT, int E, int CB, bool LR>
__device__ __forceinline__ void p2_load(const Phase2Params& p, int64_t tok, const Cols<CB, E>& cl, int tid,
                                        bool with_grad, P2Raw<DT, E, CB>& r) {
  using S = typename DT::S;
  const int bd = blockDim.x;
  const S* pvp = (const S*)p.pv + tok * p.pv_stride;
  const S* itp = (const S*)p.inter + tok * p.inter_stride;
  const S* gp = with_grad ? (const S*)p.gout + tok * (int64_t)p.D : nullptr;
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) {
      load_raw<DT, E, true>(pvp + cl.eoff[c], r.pv[c]);
      load_raw<DT, E, true>(itp + cl.eoff[c], r.it[c]);
      if (with_grad) load_raw<DT, E, true>(gp + cl.eoff[c], r.g[c]);
    }
  }
  uint32_t kb[kP2KPT];
  if (LR) row_bits_load<DT, kP2KPT>((const S*)p.pk + tok * p.pk_stride, p.R, tid, bd, kb);
  r.lse = p.lse[tok];
  r.logit = p.logit_given ? load_any(p.plogit, tok, p.pl_dt) : 0.f;
  if (LR) row_bits_floats<DT, kP2KPT>(kb, p.R, tid, bd, r.kr);
}

template <class DT, int E, int CB, bool LR>
__device__ __forceinline__ void p2_token(const Phase2Params& p, const P2Raw<DT, E, CB>& raw,
                                         const float (&qv)[CB][E], const float (&qk)[kP2KPT], float vs, float bias,
                                         const Cols<CB, E>& cl, float* s_red, int lane, int wave, int wpt,
                                         P2State<CB, E>& st) {
  const int D = p.D;
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) {
      unpack<DT, E>(raw.pv[c], st.pr[c]);
      unpack<DT, E>(raw.it[c], st.it[c]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) st.pr[c][e] = st.it[c][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) st.p[c][e] = DT::rnd(st.pr[c][e] * vs);
  }
#pragma unroll
  for (int j = 0; j < kP2KPT; ++j) st.kr[j] = raw.kr[j];
  const float lse = raw.lse;

  float logit;
  if (p.logit_given) {
    logit = raw.logit;
  } else if (LR) {
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) st.kv[j] = p.scale_key ? DT::rnd(st.kr[j] * vs) : st.kr[j];
    st.inv_key = 1.f;
    if (p.key_norm) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) ss += st.kv[j] * st.kv[j];
      ss = block_sum1(ss, s_red, lane, wave, wpt);
      st.inv_key = 1.0f / sqrtf(ss / (float)p.R + p.eps);
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) {
      st.kl[j] = p.key_norm ? DT::rnd(st.kv[j] * st.inv_key) : st.kv[j];
      dot += DT::rnd(st.kl[j] * qk[j]);
    }
    dot = block_sum1(dot, s_red, lane, wave, wpt);
    logit = DT::rnd(DT::rnd(dot) * p.scale);
  } else {
    st.inv_key = 1.f;
    if (p.key_norm) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) ss += st.p[c][e] * st.p[c][e];
      ss = block_sum1(ss, s_red, lane, wave, wpt);
      st.inv_key = 1.0f / sqrtf(ss / (float)D + p.eps);
    }
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        st.key[c][e] = p.key_norm ? DT::rnd(st.p[c][e] * st.inv_key) : st.p[c][e];
        dot += DT::rnd(st.key[c][e] * qv[c][e]);
      }
    logit = DT::rnd(block_sum1(dot, s_red, lane, wave, wpt));
  }
  const float x = (logit + bias) - lse;
  st.sg = 1.0f / (1.0f + expf(-x));
  st.prob = DT::rnd(st.sg);
}

// merged output (dtype-rounded, before the optional norm)
template <class DT, int E, int CB>
__device__ __forceinline__ void p2_merge(const Phase2Params& p, const P2State<CB, E>& st, float (&o)[CB][E]) {
  const float w = st.prob;
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float a = st.it[c][e], b = st.p[c][e];
      if (p.merge == ATTNRES_MERGE_LERP) o[c][e] = DT::rnd(fabsf(w) < 0.5f ? a + w * (b - a) : b - (b - a) * (1.0f - w));
      else o[c][e] = DT::rnd(a + DT::rnd(b - a) * w);
    }
}

// ============================================================== forward
template <class DT, int E, int CB, bool LR>
__global__ void __launch_bounds__(512) phase2_fwd_kernel(const Phase2Params p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  float* s_red = smem;  // [wpt]
  const int D = p.D, bd = blockDim.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave, wpt = bd / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;

  float qv[CB][E], qk[kP2KPT];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (!LR && !p.logit_given && cl.ok[c]) load_vec<DT, E>((const S*)p.q + cl.eoff[c], qv[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) qv[c][e] = 0.f;
  }
  if (LR && !p.logit_given) {
    uint32_t qb[kP2KPT];
    row_bits_load<DT, kP2KPT>((const S*)p.q, p.R, tid, bd, qb);
    row_bits_floats<DT, kP2KPT>(qb, p.R, tid, bd, qk);
  } else {
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) qk[j] = 0.f;
  }

  P2Raw<DT, E, CB> nxt;
  if ((int64_t)blockIdx.x < p.n_tok) p2_load<DT, E, CB, LR>(p, blockIdx.x, cl, tid, false, nxt);
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    const P2Raw<DT, E, CB> cur = nxt;
    if (tok + gridDim.x < p.n_tok) p2_load<DT, E, CB, LR>(p, tok + gridDim.x, cl, tid, false, nxt);
    P2State<CB, E> st;
    p2_token<DT, E, CB, LR>(p, cur, qv, qk, vs, bias, cl, s_red, lane, wave, wpt, st);
    float o[CB][E];
    p2_merge<DT, E, CB>(p, st, o);
    if (p.norm_out) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) ss += o[c][e] * o[c][e];
      ss = block_sum1(ss, s_red, lane, wave, wpt);
      const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) o[c][e] = DT::rnd(o[c][e] * inv);
    }
    S* op = (S*)p.out + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (cl.ok[c]) store_vec<DT, E, true>(op + cl.eoff[c], o[c]);
  }
}

// ============================================================== backward
template <class DT, int E, int CB, bool LR>
__global__ void __launch_bounds__(512) phase2_bwd_kernel(const Phase2Params p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  float* s_red = smem;  // [wpt]
  const int D = p.D, bd = blockDim.x;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave, wpt = bd / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;

  float qv[CB][E], qk[kP2KPT];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (!LR && !p.logit_given && cl.ok[c]) load_vec<DT, E>((const S*)p.q + cl.eoff[c], qv[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) qv[c][e] = 0.f;
  }
  if (LR && !p.logit_given) {
    uint32_t qb[kP2KPT];
    row_bits_load<DT, kP2KPT>((const S*)p.q, p.R, tid, bd, qb);
    row_bits_floats<DT, kP2KPT>(qb, p.R, tid, bd, qk);
  } else {
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) qk[j] = 0.f;
  }
  float dq_b[CB][E], dq_l[kP2KPT];
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) dq_b[c][e] = 0.f;
#pragma unroll
  for (int j = 0; j < kP2KPT; ++j) dq_l[j] = 0.f;
  float acc_bias = 0.f, acc_sv = 0.f, acc_sk = 0.f;  // bias, value-scale and key-scale gradient sums

  P2Raw<DT, E, CB> nxt;
  if ((int64_t)blockIdx.x < p.n_tok) p2_load<DT, E, CB, LR>(p, blockIdx.x, cl, tid, true, nxt);
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    const P2Raw<DT, E, CB> cur = nxt;
    if (tok + gridDim.x < p.n_tok) p2_load<DT, E, CB, LR>(p, tok + gridDim.x, cl, tid, true, nxt);
    P2State<CB, E> st;
    p2_token<DT, E, CB, LR>(p, cur, qv, qk, vs, bias, cl, s_red, lane, wave, wpt, st);
    float G[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if (cl.ok[c]) unpack<DT, E>(cur.g[c], G[c]);
      else
#pragma unroll
        for (int e = 0; e < E; ++e) G[c][e] = 0.f;
    }
    if (p.norm_out) {
      // G <- rms-norm backward from the recomputed pre-norm output o
      float o[CB][E];
      p2_merge<DT, E, CB>(p, st, o);
      float a[2] = {0.f, 0.f};
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          a[0] += o[c][e] * o[c][e];
          a[1] += G[c][e] * o[c][e];
        }
      block_allreduce<2>(a, 2, s_red, lane, wave, wpt);
      const float inv = 1.0f / sqrtf(a[0] / (float)D + p.eps);
      const float k3 = inv * inv * inv * (a[1] / (float)D);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) G[c][e] = cl.ok[c] ? DT::rnd(inv * G[c][e] - o[c][e] * k3) : 0.f;
    }

    // merge backward: gradients of the interblock output and of p through the
    // merge, and the per-element terms of d prob
    float dint[CB][E], dpm[CB][E];
    float dprob = 0.f;
    const float w = st.prob;
    const float omw = DT::rnd(1.0f - w);
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float diff = DT::rnd(st.p[c][e] - st.it[c][e]);
        if (p.merge == ATTNRES_MERGE_LERP) {
          dint[c][e] = DT::rnd(G[c][e] * omw);
          dpm[c][e] = DT::rnd(G[c][e] * w);
        } else {
          dpm[c][e] = DT::rnd(G[c][e] * w);
          dint[c][e] = DT::rnd(G[c][e] - dpm[c][e]);
        }
        dprob += DT::rnd(G[c][e] * diff);
      }
    dprob = DT::rnd(block_sum1(dprob, s_red, lane, wave, wpt));
    const float dx = dprob * (1.0f - st.sg) * st.sg;
    if (tid == 0) {
      p.dlse[tok] = -dx;
      acc_bias += dx;
      if (p.logit_given && p.dplogit) store_any(p.dplogit, tok, p.pl_dt, round_any(dx, p.pl_dt));
    }

    float dpk[CB][E];  // base: gradient of p through the key
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) dpk[c][e] = 0.f;
    if (!p.logit_given) {
      const float dlb = DT::rnd(dx);
      if (LR) {
        const float dsum = DT::rnd(dlb * p.scale);
        float dk[kP2KPT];
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < kP2KPT; ++j) {
          const bool in = tid + j * bd < p.R;
          dk[j] = in ? DT::rnd(dsum * qk[j]) : 0.f;
          if (in) dq_l[j] += DT::rnd(dsum * st.kl[j]);
          dot += dk[j] * st.kv[j];
        }
        if (p.key_norm) {
          dot = block_sum1(dot, s_red, lane, wave, wpt);
          const float iv = st.inv_key;
          const float k3 = iv * iv * iv * (dot / (float)p.R);
#pragma unroll
          for (int j = 0; j < kP2KPT; ++j) dk[j] = DT::rnd(iv * dk[j] - st.kv[j] * k3);
        }
        S* dkp = (S*)p.dpk + tok * (int64_t)p.R;
#pragma unroll
        for (int j = 0; j < kP2KPT; ++j) {
          const int r = tid + j * bd;
          if (r < p.R) {
            float g = dk[j];
            if (p.scale_key) {
              acc_sk += DT::rnd(g * st.kr[j]);
              g = DT::rnd(g * vs);
            }
            DT::store1(dkp + r, g);
          }
        }
      } else {
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float dk = DT::rnd(dlb * qv[c][e]);
            if (cl.ok[c]) dq_b[c][e] += DT::rnd(dlb * st.key[c][e]);
            dpk[c][e] = dk;
            dot += dk * st.p[c][e];
          }
        if (p.key_norm) {
          dot = block_sum1(dot, s_red, lane, wave, wpt);
          const float iv = st.inv_key;
          const float k3 = iv * iv * iv * (dot / (float)D);
#pragma unroll
          for (int c = 0; c < CB; ++c)
#pragma unroll
            for (int e = 0; e < E; ++e) dpk[c][e] = DT::rnd(iv * dpk[c][e] - st.p[c][e] * k3);
        }
      }
    }

    S* dpvp = (S*)p.dpv + tok * (int64_t)D;
    S* dip = (S*)p.dinter + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float dp[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float g = (!LR && !p.logit_given) ? DT::rnd(dpm[c][e] + dpk[c][e]) : dpm[c][e];
        if (cl.ok[c]) acc_sv += DT::rnd(g * st.pr[c][e]);
        dp[e] = DT::rnd(g * vs);
      }
      if (cl.ok[c]) {
        store_vec<DT, E, true>(dpvp + cl.eoff[c], dp);
        store_vec<DT, E, true>(dip + cl.eoff[c], dint[c]);
      }
    }
  }

  // this workgroup's partial sums
  float* part = p.partials ? p.partials + (int64_t)blockIdx.x * p.n_part : nullptr;
  if (part && p.part_q >= 0) {
    if (LR) {
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) {
        const int r = tid + j * bd;
        if (r < p.R) part[p.part_q + r] = dq_l[j];
      }
    } else {
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (cl.ok[c])
#pragma unroll
          for (int e = 0; e < E; ++e) part[p.part_q + cl.eoff[c] + e] = dq_b[c][e];
    }
  }
  if (part && p.part_bias >= 0 && tid == 0) part[p.part_bias] = acc_bias;
  if (part && p.part_scale >= 0) {
    // the value and key products are separate autograd edges of the scale:
    // kept apart so that each sum is rounded to the dtype on its own
    float a[2] = {acc_sv, acc_sk};
    block_allreduce<2>(a, 2, s_red, lane, wave, wpt);
    if (tid == 0) {
      part[p.part_scale] = a[0];
      if (p.scale_key) part[p.part_scale + 1] = a[1];
    }
  }
}

// ============================================================== one wave per token
// For rows that one wave covers (16-byte vectors, D <= 64 * E * CB): a wave
// owns a token, every reduction is a wave all-reduce (DPP and two lane
// shuffles) with no LDS round trip and no barrier, and a workgroup runs
// blockDim/64 tokens side by side.  Same per-token arithmetic as the kernels
// above; only the fp32 association order of the sums differs.

// Row sum of per-lane chunk partials, chunk by chunk: one wave sum per chunk,
// chunk totals added in order.  That is the association of the workgroup
// kernels above (chunk c on wave c, wave totals added in order), so 16-bit
// results do not depend on which of the two layouts ran.
template <int CB>
__device__ __forceinline__ float row_sum(const float (&x)[CB]) {
  float t = 0.f;
#pragma unroll
  for (int c = 0; c < CB; ++c) t += wave_sum(x[c]);
  return t;
}

template <class DT, int E, int CB, bool LR>
struct P2W {
  Raw<DT, E> pv[CB];  // partial value as loaded (packed)
  float p[CB][E];     // scaled partial value (dtype-rounded)
  float it[CB][E];    // interblock output
  float kl[kP2KPT];   // LR key (dtype-rounded)
  float kv[kP2KPT];   // LR key before the norm (scaled)
  float kr[kP2KPT];   // LR key as loaded
  float inv_key;      // 1/rms of the key (key_norm)
  float sg, prob;     // sigmoid and its dtype-rounded value
};

// Loads one token's partial value, interblock output and LR key, and
// recomputes the forward state (scaled value, key, logit, sigmoid).
template <class DT, int E, int CB, bool LR>
__device__ __forceinline__ void p2w_token(const Phase2Params& p, int64_t tok, const Cols<CB, E>& cl, int lane,
                                          const float (&qv)[CB][E], const float (&qk)[kP2KPT], float vs,
                                          float bias, P2W<DT, E, CB, LR>& st) {
  using S = typename DT::S;
  const S* pvp = (const S*)p.pv + tok * p.pv_stride;
  const S* itp = (const S*)p.inter + tok * p.inter_stride;
  Raw<DT, E> itr[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c)
    if (cl.ok[c]) {
      load_raw<DT, E, true>(pvp + cl.eoff[c], st.pv[c]);
      load_raw<DT, E, true>(itp + cl.eoff[c], itr[c]);
    }
  uint32_t kb[kP2KPT];
  if (LR) row_bits_load<DT, kP2KPT>((const S*)p.pk + tok * p.pk_stride, p.R, lane, kWave, kb);
  const float lse = p.lse[tok];
  const float given = p.logit_given ? load_any(p.plogit, tok, p.pl_dt) : 0.f;
  if (LR) row_bits_floats<DT, kP2KPT>(kb, p.R, lane, kWave, st.kr);
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    float pr[E];
    if (cl.ok[c]) {
      unpack<DT, E>(st.pv[c], pr);
      unpack<DT, E>(itr[c], st.it[c]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) pr[e] = st.it[c][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) st.p[c][e] = DT::rnd(pr[e] * vs);
  }

  float logit;
  st.inv_key = 1.f;
  if (p.logit_given) {
    logit = given;
  } else if (LR) {
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) st.kv[j] = p.scale_key ? DT::rnd(st.kr[j] * vs) : st.kr[j];
    if (p.key_norm) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) ss += st.kv[j] * st.kv[j];
      st.inv_key = 1.0f / sqrtf(wave_sum(ss) / (float)p.R + p.eps);
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) {
      st.kl[j] = p.key_norm ? DT::rnd(st.kv[j] * st.inv_key) : st.kv[j];
      dot += DT::rnd(st.kl[j] * qk[j]);
    }
    logit = DT::rnd(DT::rnd(wave_sum(dot)) * p.scale);
  } else {
    if (p.key_norm) {
      float ss[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        ss[c] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss[c] += st.p[c][e] * st.p[c][e];
      }
      st.inv_key = 1.0f / sqrtf(row_sum<CB>(ss) / (float)p.D + p.eps);
    }
    float dot[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      dot[c] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float key = p.key_norm ? DT::rnd(st.p[c][e] * st.inv_key) : st.p[c][e];
        dot[c] += DT::rnd(key * qv[c][e]);
      }
    }
    logit = DT::rnd(row_sum<CB>(dot));
  }
  const float x = (logit + bias) - lse;
  st.sg = 1.0f / (1.0f + expf(-x));
  st.prob = DT::rnd(st.sg);
}

template <class DT>
__device__ __forceinline__ float p2w_merge1(int merge, float a, float b, float w) {
  if (merge == ATTNRES_MERGE_LERP) return DT::rnd(fabsf(w) < 0.5f ? a + w * (b - a) : b - (b - a) * (1.0f - w));
  return DT::rnd(a + DT::rnd(b - a) * w);
}

template <class DT, int E, int CB, bool LR>
__device__ __forceinline__ void p2w_queries(const Phase2Params& p, const Cols<CB, E>& cl, int lane,
                                            float (&qv)[CB][E], float (&qk)[kP2KPT]) {
  using S = typename DT::S;
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (!LR && !p.logit_given && cl.ok[c]) load_vec<DT, E>((const S*)p.q + cl.eoff[c], qv[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) qv[c][e] = 0.f;
  }
  if (LR && !p.logit_given) {
    uint32_t qb[kP2KPT];
    row_bits_load<DT, kP2KPT>((const S*)p.q, p.R, lane, kWave, qb);
    row_bits_floats<DT, kP2KPT>(qb, p.R, lane, kWave, qk);
  } else {
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) qk[j] = 0.f;
  }
}

template <class DT, int E, int CB, bool LR>
__global__ void __launch_bounds__(256) phase2_wave_fwd_kernel(const Phase2Params p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const Cols<CB, E> cl(p.ncols, p.D, lane, 0, 1);
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;
  float qv[CB][E], qk[kP2KPT];
  p2w_queries<DT, E, CB, LR>(p, cl, lane, qv, qk);

  const int64_t stride = (int64_t)gridDim.x * wpb;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    P2W<DT, E, CB, LR> st;
    p2w_token<DT, E, CB, LR>(p, tok, cl, lane, qv, qk, vs, bias, st);
    float o[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) o[c][e] = p2w_merge1<DT>(p.merge, st.it[c][e], st.p[c][e], st.prob);
    if (p.norm_out) {
      float ss[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        ss[c] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss[c] += o[c][e] * o[c][e];
      }
      const float inv = 1.0f / sqrtf(row_sum<CB>(ss) / (float)p.D + p.eps);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) o[c][e] = DT::rnd(o[c][e] * inv);
    }
    S* op = (S*)p.out + tok * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (cl.ok[c]) store_vec<DT, E, true>(op + cl.eoff[c], o[c]);
  }
}

// An empty register barrier on packed words: the compiler must treat them as
// changed, so a later unpack is redone instead of keeping the unpacked floats
// of an earlier pass alive (no instruction is emitted).
template <class DT, int E, int CB>
__device__ __forceinline__ void reload(Raw<DT, E> (&r)[CB]) {
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int i = 0; i < Vec<DT, E>::kWords; ++i) asm volatile("" : "+v"(r[c].w[i]));
}

// Backward: one wave per token with the rows kept packed in the value dtype
// (partial value as loaded, scaled partial value, interblock output, upstream
// gradient): every per-element intermediate that is kept across a reduction
// is itself dtype-rounded, so it packs without loss, and a lane unpacks a
// vector where it uses it.  This halves the registers of a 16-bit row and
// keeps enough waves resident to cover the memory latency.
template <class DT, int E, int CB, bool LR>
__global__ void __launch_bounds__(256) phase2_wave_bwd_kernel(const Phase2Params p) {
  using S = typename DT::S;
  using R = Raw<DT, E>;
  extern __shared__ float smem[];  // [wpb][n_part]: each wave's partial sums
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int D = p.D;
  const Cols<CB, E> cl(p.ncols, D, lane, 0, 1);
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;
  const bool base_key = !LR && !p.logit_given;

  R qr[CB];  // base query (packed)
  float qk[kP2KPT];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (base_key && cl.ok[c]) load_raw<DT, E>((const S*)p.q + cl.eoff[c], qr[c]);
    else
#pragma unroll
      for (int i = 0; i < Vec<DT, E>::kWords; ++i) qr[c].w[i] = 0u;
  }
  if (LR && !p.logit_given) {
    uint32_t qb[kP2KPT];
    row_bits_load<DT, kP2KPT>((const S*)p.q, p.R, lane, kWave, qb);
    row_bits_floats<DT, kP2KPT>(qb, p.R, lane, kWave, qk);
  } else {
#pragma unroll
    for (int j = 0; j < kP2KPT; ++j) qk[j] = 0.f;
  }

  float dq_b[CB][E], dq_l[kP2KPT];
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) dq_b[c][e] = 0.f;
#pragma unroll
  for (int j = 0; j < kP2KPT; ++j) dq_l[j] = 0.f;
  float acc_bias = 0.f, acc_sv = 0.f, acc_sk = 0.f;
  const bool direct = LR || p.logit_given;  // d p has no key term: store it in the merge pass
  const bool want_sv = p.part_scale >= 0;

  const int64_t stride = (int64_t)gridDim.x * wpb;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    // ---- loads
    R gr[CB], pvr[CB], itr[CB], pp[CB];
    {
      const S* gp = (const S*)p.gout + tok * (int64_t)D;
      const S* pvp = (const S*)p.pv + tok * p.pv_stride;
      const S* itp = (const S*)p.inter + tok * p.inter_stride;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) {
          load_raw<DT, E, true>(gp + cl.eoff[c], gr[c]);
          load_raw<DT, E, true>(pvp + cl.eoff[c], pvr[c]);
          load_raw<DT, E, true>(itp + cl.eoff[c], itr[c]);
        } else {
#pragma unroll
          for (int i = 0; i < Vec<DT, E>::kWords; ++i) gr[c].w[i] = pvr[c].w[i] = itr[c].w[i] = 0u;
        }
      }
    }
    float kr[kP2KPT], kv[kP2KPT], kl[kP2KPT];
    uint32_t kb[kP2KPT];
    if (LR) row_bits_load<DT, kP2KPT>((const S*)p.pk + tok * p.pk_stride, p.R, lane, kWave, kb);
    const float lse = p.lse[tok];
    const float given = p.logit_given ? load_any(p.plogit, tok, p.pl_dt) : 0.f;
    if (LR) row_bits_floats<DT, kP2KPT>(kb, p.R, lane, kWave, kr);

    // ---- forward recompute: scaled partial (packed), key, logit, sigmoid
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float x[E];
      unpack<DT, E>(pvr[c], x);
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = x[e] * vs;
      pack_raw<DT, E>(x, pp[c]);  // packing rounds to the dtype
    }
    float logit, inv_key = 1.f;
    if (p.logit_given) {
      logit = given;
    } else if (LR) {
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) kv[j] = p.scale_key ? DT::rnd(kr[j] * vs) : kr[j];
      if (p.key_norm) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < kP2KPT; ++j) ss += kv[j] * kv[j];
        inv_key = 1.0f / sqrtf(wave_sum(ss) / (float)p.R + p.eps);
      }
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) {
        kl[j] = p.key_norm ? DT::rnd(kv[j] * inv_key) : kv[j];
        dot += DT::rnd(kl[j] * qk[j]);
      }
      logit = DT::rnd(DT::rnd(wave_sum(dot)) * p.scale);
    } else {
      if (p.key_norm) {
        float ss[CB];
        reload<DT, E, CB>(pp);
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          float x[E];
          unpack<DT, E>(pp[c], x);
          ss[c] = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) ss[c] += x[e] * x[e];
        }
        inv_key = 1.0f / sqrtf(row_sum<CB>(ss) / (float)D + p.eps);
      }
      float dot[CB];
      reload<DT, E, CB>(pp);
      reload<DT, E, CB>(qr);
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float x[E], q[E];
        unpack<DT, E>(pp[c], x);
        unpack<DT, E>(qr[c], q);
        dot[c] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float key = p.key_norm ? DT::rnd(x[e] * inv_key) : x[e];
          dot[c] += DT::rnd(key * q[e]);
        }
      }
      logit = DT::rnd(row_sum<CB>(dot));
    }
    const float xl = (logit + bias) - lse;
    const float sg = 1.0f / (1.0f + expf(-xl));
    const float w = DT::rnd(sg);

    // ---- output norm: sums of o*o and G*o over the recomputed merge o (kept packed)
    R orr[CB];
    float inv = 1.f, k3 = 0.f;
    if (p.norm_out) {
      float a0[CB], a1[CB];
      reload<DT, E, CB>(itr);
      reload<DT, E, CB>(pp);
      reload<DT, E, CB>(gr);
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float a[E], b[E], g[E], o[E];
        unpack<DT, E>(itr[c], a);
        unpack<DT, E>(pp[c], b);
        unpack<DT, E>(gr[c], g);
        a0[c] = a1[c] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          o[e] = p2w_merge1<DT>(p.merge, a[e], b[e], w);
          a0[c] += o[e] * o[e];
          a1[c] += g[e] * o[e];
        }
        pack_raw<DT, E>(o, orr[c]);  // o is dtype-rounded: packs exactly
      }
      inv = 1.0f / sqrtf(row_sum<CB>(a0) / (float)D + p.eps);
      k3 = inv * inv * inv * (row_sum<CB>(a1) / (float)D);
    }

    // ---- norm backward (G <- rnd(inv * G - o * k3)) and merge backward in one
    // pass; gr becomes d p through the merge (base keys)
    S* dpvp = (S*)p.dpv + tok * (int64_t)D;
    S* dip = (S*)p.dinter + tok * (int64_t)D;
    const float omw = DT::rnd(1.0f - w);
    float dpr[CB];
    reload<DT, E, CB>(itr);
    reload<DT, E, CB>(pp);
    reload<DT, E, CB>(gr);
    reload<DT, E, CB>(pvr);
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float a[E], b[E], g[E], dint[E], dpm[E];
      unpack<DT, E>(itr[c], a);
      unpack<DT, E>(pp[c], b);
      unpack<DT, E>(gr[c], g);
      if (p.norm_out) {
        float o[E];
        unpack<DT, E>(orr[c], o);
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = cl.ok[c] ? DT::rnd(inv * g[e] - o[e] * k3) : 0.f;
      }
      dpr[c] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float diff = DT::rnd(b[e] - a[e]);
        if (p.merge == ATTNRES_MERGE_LERP) {
          dint[e] = DT::rnd(g[e] * omw);
          dpm[e] = DT::rnd(g[e] * w);
        } else {
          dpm[e] = DT::rnd(g[e] * w);
          dint[e] = DT::rnd(g[e] - dpm[e]);
        }
        dpr[c] += DT::rnd(g[e] * diff);
      }
      if (cl.ok[c]) store_vec<DT, E, true>(dip + cl.eoff[c], dint);
      if (direct) {
        float pr[E], dp[E];
        unpack<DT, E>(pvr[c], pr);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if (want_sv && cl.ok[c]) acc_sv += DT::rnd(dpm[e] * pr[e]);
          dp[e] = DT::rnd(dpm[e] * vs);
        }
        if (cl.ok[c]) store_vec<DT, E, true>(dpvp + cl.eoff[c], dp);
      } else {
        pack_raw<DT, E>(dpm, gr[c]);
      }
    }
    const float dprob = DT::rnd(row_sum<CB>(dpr));
    const float dx = dprob * (1.0f - sg) * sg;
    if (lane == 0) {
      p.dlse[tok] = -dx;
      acc_bias += dx;
      if (p.logit_given && p.dplogit) store_any(p.dplogit, tok, p.pl_dt, round_any(dx, p.pl_dt));
    }
    if (p.logit_given) continue;

    const float dlb = DT::rnd(dx);
    if (LR) {
      const float dsum = DT::rnd(dlb * p.scale);
      float dk[kP2KPT];
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) {
        const bool in = lane + j * kWave < p.R;
        dk[j] = in ? DT::rnd(dsum * qk[j]) : 0.f;
        if (in) dq_l[j] += DT::rnd(dsum * kl[j]);
        dot += dk[j] * kv[j];
      }
      if (p.key_norm) {
        const float iv = inv_key;
        const float k3 = iv * iv * iv * (wave_sum(dot) / (float)p.R);
#pragma unroll
        for (int j = 0; j < kP2KPT; ++j) dk[j] = DT::rnd(iv * dk[j] - kv[j] * k3);
      }
      S* dkp = (S*)p.dpk + tok * (int64_t)p.R;
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) {
          float g = dk[j];
          if (p.scale_key) {
            acc_sk += DT::rnd(g * kr[j]);
            g = DT::rnd(g * vs);
          }
          DT::store1(dkp + r, g);
        }
      }
    } else {
      // base key: d p = d p (merge) + key-norm backward of dk, dk = rnd(dlb * q)
      float k3 = 0.f;
      const float iv = inv_key;
      {
        float dot[CB];
        reload<DT, E, CB>(pp);
        reload<DT, E, CB>(qr);
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          float x[E], q[E];
          unpack<DT, E>(pp[c], x);
          unpack<DT, E>(qr[c], q);
          dot[c] = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float key = p.key_norm ? DT::rnd(x[e] * iv) : x[e];
            const float dk = DT::rnd(dlb * q[e]);
            if (cl.ok[c]) dq_b[c][e] += DT::rnd(dlb * key);
            dot[c] += dk * x[e];
          }
        }
        if (p.key_norm) k3 = iv * iv * iv * (row_sum<CB>(dot) / (float)D);
      }
      reload<DT, E, CB>(pp);
      reload<DT, E, CB>(qr);
      reload<DT, E, CB>(gr);
      reload<DT, E, CB>(pvr);
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float x[E], q[E], dpm[E], pr[E], dp[E];
        unpack<DT, E>(pp[c], x);
        unpack<DT, E>(qr[c], q);
        unpack<DT, E>(gr[c], dpm);
        unpack<DT, E>(pvr[c], pr);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float dk = DT::rnd(dlb * q[e]);
          const float dpk = p.key_norm ? DT::rnd(iv * dk - x[e] * k3) : dk;
          const float g = DT::rnd(dpm[e] + dpk);
          if (want_sv && cl.ok[c]) acc_sv += DT::rnd(g * pr[e]);
          dp[e] = DT::rnd(g * vs);
        }
        if (cl.ok[c]) store_vec<DT, E, true>(dpvp + cl.eoff[c], dp);
      }
    }
  }

  // partial sums: each wave's row in LDS, then the workgroup's row (fixed order)
  if (!p.partials) return;
  float* mine = smem + wave * p.n_part;
  if (p.part_q >= 0) {
    if (LR) {
#pragma unroll
      for (int j = 0; j < kP2KPT; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) mine[p.part_q + r] = dq_l[j];
      }
    } else {
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (cl.ok[c])
#pragma unroll
          for (int e = 0; e < E; ++e) mine[p.part_q + cl.eoff[c] + e] = dq_b[c][e];
    }
  }
  if (p.part_bias >= 0 && lane == 0) mine[p.part_bias] = acc_bias;
  if (p.part_scale >= 0) {
    // the value and key products are separate autograd edges of the scale:
    // kept apart so that each sum is rounded to the dtype on its own
    const float sv = wave_sum(acc_sv), sk = wave_sum(acc_sk);
    if (lane == 0) {
      mine[p.part_scale] = sv;
      if (p.scale_key) mine[p.part_scale + 1] = sk;
    }
  }
  __syncthreads();
  // tiled partials: 16 consecutive slots of this workgroup are one 64-byte run
  for (int i = threadIdx.x; i < p.n_part; i += blockDim.x) {
    float t = 0.f;
    for (int w2 = 0; w2 < wpb; ++w2) t += smem[w2 * p.n_part + i];
    p.partials[part_index(kPartTiled, blockIdx.x, i, gridDim.x, p.n_part)] = t;
  }
}

// ============================================================== launchers
// L.teams > 0 selects the one-wave-per-token kernels: teams = waves per
// workgroup, vb = vector bytes (16, or 8 for 16-bit rows where 16-byte
// vectors would leave lanes idle), wpt = vectors per lane.
template <class DT, bool LR, int E, int CB>
static void phase2_wave_launch(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  const dim3 g(L.grid), b(L.teams * kWave);
  if (bwd) hipLaunchKernelGGL((phase2_wave_bwd_kernel<DT, E, CB, LR>), g, b, L.lds, st, p);
  else hipLaunchKernelGGL((phase2_wave_fwd_kernel<DT, E, CB, LR>), g, b, 0, st, p);
}
template <class DT, bool LR>
static void phase2_wave(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  if constexpr (sizeof(typename DT::S) == 4) {
    switch (L.wpt) {
      case 1: phase2_wave_launch<DT, LR, 4, 1>(bwd, p, L, st); break;
      case 2: phase2_wave_launch<DT, LR, 4, 2>(bwd, p, L, st); break;
      case 3: phase2_wave_launch<DT, LR, 4, 3>(bwd, p, L, st); break;
      default: phase2_wave_launch<DT, LR, 4, 4>(bwd, p, L, st); break;
    }
  } else if (L.vb == 8) {
    if (L.wpt == 1) phase2_wave_launch<DT, LR, 4, 1>(bwd, p, L, st);
    else phase2_wave_launch<DT, LR, 4, 3>(bwd, p, L, st);
  } else {
    if (L.wpt == 1) phase2_wave_launch<DT, LR, 8, 1>(bwd, p, L, st);
    else phase2_wave_launch<DT, LR, 8, 2>(bwd, p, L, st);
  }
}

template <class DT, bool LR>
static hipError_t phase2_fwd_t(const Phase2Params& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  constexpr int CBV = sizeof(typename DT::S) == 4 ? 2 : 1;
  const dim3 g(L.grid), b(L.wpt * kWave);
  if (L.teams > 0) phase2_wave<DT, LR>(false, p, L, st);
  else if (L.vec) hipLaunchKernelGGL((phase2_fwd_kernel<DT, EV, CBV, LR>), g, b, L.lds, st, p);
  else hipLaunchKernelGGL((phase2_fwd_kernel<DT, 1, 8, LR>), g, b, L.lds, st, p);
  return hipGetLastError();
}
template <class DT, bool LR>
static hipError_t phase2_bwd_t(const Phase2Params& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  constexpr int CBV = sizeof(typename DT::S) == 4 ? 2 : 1;
  const dim3 g(L.grid), b(L.wpt * kWave);
  if (L.teams > 0) phase2_wave<DT, LR>(true, p, L, st);
  else if (L.vec) hipLaunchKernelGGL((phase2_bwd_kernel<DT, EV, CBV, LR>), g, b, L.lds, st, p);
  else hipLaunchKernelGGL((phase2_bwd_kernel<DT, 1, 8, LR>), g, b, L.lds, st, p);
  return hipGetLastError();
}
template <class DT>
static hipError_t phase2_fwd_dt(const Phase2Params& p, const Launch& L, hipStream_t st) {
  return L.nmax ? phase2_fwd_t<DT, true>(p, L, st) : phase2_fwd_t<DT, false>(p, L, st);
}
template <class DT>
static hipError_t phase2_bwd_dt(const Phase2Params& p, const Launch& L, hipStream_t st) {
  return L.nmax ? phase2_bwd_t<DT, true>(p, L, st) : phase2_bwd_t<DT, false>(p, L, st);
}

#define ATTNRES_P2_DISPATCH(dtype, fn, ...)                \
  switch (dtype) {                                         \
    case ATTNRES_DTYPE_F32: return fn<F32>(__VA_ARGS__);   \
    case ATTNRES_DTYPE_BF16: return fn<BF16>(__VA_ARGS__); \
    default: return fn<F16>(__VA_ARGS__);                  \
  }

hipError_t launch_phase2_forward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st) {
  ATTNRES_P2_DISPATCH(dtype, phase2_fwd_dt, p, L, st);
}
hipError_t launch_phase2_backward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st) {
  ATTNRES_P2_DISPATCH(dtype, phase2_bwd_dt, p, L, st);
}

}  // namespace attnres
