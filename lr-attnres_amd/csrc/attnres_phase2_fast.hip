// Phase 2, fast path for 16-bit rows that one wave covers exactly: D = 64
// lanes x CB columns x one VB-byte vector (256 / 768 with 8-byte vectors,
// 512 / 1024 with 16-byte ones).  Base keys (rms-norm of the scaled partial
// block, scored against the query) with the addcmul merge and no output norm
// (reference: attention_residual_phase2, attnres_ops.py:3964-4035); LR keys
// (r <= 256) with either merge and the optional output norm (reference:
// lrid_attention_residual_phase2[_torch], attnres_ops.py:4075-4160).  Other
// forms run the general kernels in attnres_phase2.hip.
//
// The arithmetic and every rounding point are those of the general one-wave
// kernels (the eager op's step-by-step roundings); only the instruction forms
// change, because those kernels spend about twice the token's HBM time in VALU
// work (phase 2 moves only 3 rows forward and 5 backward per token):
//   * rows stay packed in the dtype; a rounding that feeds a packed consumer is
//     one v_cvt_pk for two elements,
//   * sums of dtype-rounded products (the logit <rnd(key), q> as the eager op
//     forms it, <g, rnd(p - it)>) add the packed products with one v_dot2
//     against (1, 1); <p, p> is one v_dot2,
//   * the query gradient adds rnd(dlb * key) from packed products with one
//     v_dot2 against (1, 0) / (0, 1) per element.
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

namespace {

constexpr int kP2FastWaves = 4;  // tokens (waves) per workgroup

// (1, 1), (1, 0), (0, 1) as packed 16-bit words of the dtype
template <class DT>
__device__ __forceinline__ uint32_t one_pair() {
  return DT::kCode == 1 ? 0x3f803f80u : 0x3c003c00u;
}
template <class DT>
__device__ __forceinline__ uint32_t one_lo() {
  return DT::kCode == 1 ? 0x00003f80u : 0x00003c00u;
}
template <class DT>
__device__ __forceinline__ uint32_t one_hi() {
  return DT::kCode == 1 ? 0x3f800000u : 0x3c000000u;
}

template <class DT>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  Raw<DT, 2> r;
  r.w[0] = w;
  float t[2];
  unpack<DT, 2>(r, t);
  lo = t[0];
  hi = t[1];
}

// The recomputed forward state of one token: scaled partial block p (packed,
// dtype-rounded), rnd(p * inv) (packed, key norm), inv, sigmoid and its
// dtype-rounded value.
template <class DT, int VB, int CB, bool KN>
struct P2Fast {
  static constexpr int W = VB / 4;
  uint32_t pw[CB][W];
  uint32_t kw[CB][W];
  float inv, sg, prob;
};

template <class DT, int VB, int CB, bool KN>
__device__ __forceinline__ void p2fast_forward_state(const Phase2Params& p, const Raw<DT, VB / 2> (&pvr)[CB],
                                                     const float (&q)[CB][VB / 2], float vs, float bias, float lse,
                                                     P2Fast<DT, VB, CB, KN>& st) {
  constexpr int W = VB / 4;
  // p = rnd(pv * vs), packed; <p, p>
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int i = 0; i < W; ++i) {
      float a, b;
      unpack2<DT>(pvr[c].w[i], a, b);
      st.pw[c][i] = pack2<DT>(a * vs, b * vs);
      if constexpr (KN) ss = dot2<DT>(st.pw[c][i], st.pw[c][i], ss);
    }
  st.inv = 1.f;
  if constexpr (KN) st.inv = 1.0f / sqrtf(wave_sum(ss) / (float)p.D + p.eps);
  // logit = rnd(sum_e rnd(key_e * q_e)), key = rnd(p * inv) (or p)
  float t = 0.f;
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int i = 0; i < W; ++i) {
      float k0, k1;
      if constexpr (KN) {
        float a, b;
        unpack2<DT>(st.pw[c][i], a, b);
        st.kw[c][i] = pack2<DT>(a * st.inv, b * st.inv);
        unpack2<DT>(st.kw[c][i], k0, k1);
      } else {
        st.kw[c][i] = st.pw[c][i];
        unpack2<DT>(st.pw[c][i], k0, k1);
      }
      t = dot2<DT>(pack2<DT>(k0 * q[c][2 * i], k1 * q[c][2 * i + 1]), one_pair<DT>(), t);
    }
  const float logit = DT::rnd(wave_sum(t));
  const float x = (logit + bias) - lse;
  st.sg = 1.0f / (1.0f + expf(-x));
  st.prob = DT::rnd(st.sg);
}

// The query row as raw words (loaded once per wave) and as floats (unpacked
// per token after the token's loads are issued, so that a wave's first token
// does not wait for the query's load first).
template <class DT, int VB, int CB>
__device__ __forceinline__ void p2fast_query_load(const Phase2Params& p, int lane, Raw<DT, VB / 2> (&qr)[CB]) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
#pragma unroll
  for (int c = 0; c < CB; ++c) load_raw<DT, E>((const S*)p.q + (c * kWave + lane) * E, qr[c]);
}
template <class DT, int VB, int CB>
__device__ __forceinline__ void p2fast_query(const Raw<DT, VB / 2> (&qr)[CB], float (&q)[CB][VB / 2]) {
#pragma unroll
  for (int c = 0; c < CB; ++c) unpack<DT, VB / 2>(qr[c], q[c]);
}

}  // namespace

template <class DT, int VB, int CB, bool KN>
__global__ void __launch_bounds__(256) phase2_fwd_fast_kernel(const Phase2Params p) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform_i32(threadIdx.x / kWave);
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;
  Raw<DT, E> qr[CB];
  p2fast_query_load<DT, VB, CB>(p, lane, qr);

  const int64_t stride = (int64_t)gridDim.x * kP2FastWaves;
  for (int64_t tok = (int64_t)blockIdx.x * kP2FastWaves + wave; tok < p.n_tok; tok += stride) {
    Raw<DT, E> pvr[CB], itr[CB];
    const S* pvp = (const S*)p.pv + tok * p.pv_stride;
    const S* itp = (const S*)p.inter + tok * p.inter_stride;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      load_raw<DT, E, true>(pvp + (c * kWave + lane) * E, pvr[c]);
      load_raw<DT, E, true>(itp + (c * kWave + lane) * E, itr[c]);
    }
    float q[CB][E];
    p2fast_query<DT, VB, CB>(qr, q);
    P2Fast<DT, VB, CB, KN> st;
    p2fast_forward_state<DT, VB, CB, KN>(p, pvr, q, vs, bias, p.lse[tok], st);
    const float w = st.prob;
    S* op = (S*)p.out + tok * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float o[E];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        // addcmul merge: rnd(a + rnd(b - a) * w), a = interblock output, b = p
        float a0, a1, b0, b1, d0, d1;
        unpack2<DT>(itr[c].w[i], a0, a1);
        unpack2<DT>(st.pw[c][i], b0, b1);
        unpack2<DT>(pack2<DT>(b0 - a0, b1 - a1), d0, d1);
        o[2 * i] = a0 + d0 * w;
        o[2 * i + 1] = a1 + d1 * w;
      }
      store_vec<DT, E, true>(op + (c * kWave + lane) * E, o);
    }
  }
}

template <class DT, int VB, int CB, bool KN>
__global__ void __launch_bounds__(256) phase2_bwd_fast_kernel(const Phase2Params p) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  extern __shared__ float smem[];  // [waves][n_part]: each wave's partial sums
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform_i32(threadIdx.x / kWave);
  const int D = p.D;
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;
  const bool want_sv = p.part_scale >= 0;
  float q[CB][E];  // unpacked once: a backward wave walks several tokens
  {
    Raw<DT, E> qr[CB];
    p2fast_query_load<DT, VB, CB>(p, lane, qr);
    p2fast_query<DT, VB, CB>(qr, q);
  }
  float dq[CB][E];
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) dq[c][e] = 0.f;
  float acc_bias = 0.f, acc_sv = 0.f;
  // (1, 0) and (0, 1) in scalar registers the compiler cannot see through: as
  // a constant, (1, 0) is emitted as the inline operand "1.0", which the packed
  // v_dot2c reads as (0, 1) (found on gfx950: every query-gradient element
  // then took its neighbour's value)
  uint32_t e_lo = one_lo<DT>(), e_hi = one_hi<DT>();
  asm volatile("" : "+s"(e_lo), "+s"(e_hi));

  const int64_t stride = (int64_t)gridDim.x * kP2FastWaves;
  for (int64_t tok = (int64_t)blockIdx.x * kP2FastWaves + wave; tok < p.n_tok; tok += stride) {
    Raw<DT, E> pvr[CB], itr[CB], gr[CB];
    {
      const S* pvp = (const S*)p.pv + tok * p.pv_stride;
      const S* itp = (const S*)p.inter + tok * p.inter_stride;
      const S* gp = (const S*)p.gout + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        load_raw<DT, E, true>(gp + (c * kWave + lane) * E, gr[c]);
        load_raw<DT, E, true>(pvp + (c * kWave + lane) * E, pvr[c]);
        load_raw<DT, E, true>(itp + (c * kWave + lane) * E, itr[c]);
      }
    }
    P2Fast<DT, VB, CB, KN> st;
    p2fast_forward_state<DT, VB, CB, KN>(p, pvr, q, vs, bias, p.lse[tok], st);
    const float w = st.prob;

    // ---- merge backward: d inter stored; d p (merge part) kept packed in gr;
    // dprob = rnd(sum_e rnd(g * rnd(p - it)))
    S* dip = (S*)p.dinter + tok * (int64_t)D;
    float t = 0.f;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float di[E];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float a0, a1, b0, b1, g0, g1;
        unpack2<DT>(itr[c].w[i], a0, a1);
        unpack2<DT>(st.pw[c][i], b0, b1);
        unpack2<DT>(gr[c].w[i], g0, g1);
        const uint32_t diff = pack2<DT>(b0 - a0, b1 - a1);
        float f0, f1;
        unpack2<DT>(diff, f0, f1);
        t = dot2<DT>(pack2<DT>(g0 * f0, g1 * f1), one_pair<DT>(), t);
        // d p (merge part) = rnd(g w), d inter = rnd(g - rnd(g w))
        const uint32_t dpm = pack2<DT>(g0 * w, g1 * w);
        float m0, m1;
        unpack2<DT>(dpm, m0, m1);
        di[2 * i] = g0 - m0;
        di[2 * i + 1] = g1 - m1;
        gr[c].w[i] = dpm;
      }
      store_vec<DT, E, true>(dip + (c * kWave + lane) * E, di);
    }
    const float dprob = DT::rnd(wave_sum(t));
    const float dx = dprob * (1.0f - st.sg) * st.sg;
    if (lane == 0) {
      p.dlse[tok] = -dx;
      acc_bias += dx;
    }
    const float dlb = DT::rnd(dx);

    // ---- key backward: dq += rnd(dlb * key); <rnd(dlb q), p> for the rms-norm chain
    float k3 = 0.f;
    {
      float m = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int i = 0; i < W; ++i) {
          float k0, k1;
          unpack2<DT>(st.kw[c][i], k0, k1);
          const uint32_t pr = pack2<DT>(dlb * k0, dlb * k1);
          dq[c][2 * i] = dot2<DT>(pr, e_lo, dq[c][2 * i]);
          dq[c][2 * i + 1] = dot2<DT>(pr, e_hi, dq[c][2 * i + 1]);
          if constexpr (KN) m = dot2<DT>(pack2<DT>(dlb * q[c][2 * i], dlb * q[c][2 * i + 1]), st.pw[c][i], m);
        }
      if constexpr (KN) k3 = st.inv * st.inv * st.inv * (wave_sum(m) / (float)D);
    }
    // ---- d p = rnd(rnd(dpm + dpk) * vs), dpk = rnd(inv * rnd(dlb q) - p * k3) (or rnd(dlb q))
    S* dpvp = (S*)p.dpv + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float dp[E];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float d0, d1;
        unpack2<DT>(pack2<DT>(dlb * q[c][2 * i], dlb * q[c][2 * i + 1]), d0, d1);
        if constexpr (KN) {
          float x0, x1;
          unpack2<DT>(st.pw[c][i], x0, x1);
          unpack2<DT>(pack2<DT>(st.inv * d0 - x0 * k3, st.inv * d1 - x1 * k3), d0, d1);
        }
        float m0, m1;
        unpack2<DT>(gr[c].w[i], m0, m1);
        const float s0 = DT::rnd(m0 + d0);
        const float s1 = DT::rnd(m1 + d1);
        if (want_sv) {
          float r0, r1;
          unpack2<DT>(pvr[c].w[i], r0, r1);
          acc_sv += DT::rnd(s0 * r0);
          acc_sv += DT::rnd(s1 * r1);
        }
        dp[2 * i] = s0 * vs;
        dp[2 * i + 1] = s1 * vs;
      }
      store_vec<DT, E, true>(dpvp + (c * kWave + lane) * E, dp);
    }
  }

  // partial sums: each wave's row in LDS, then the workgroup's row in 16-slot tiles
  if (!p.partials) return;
  float* mine = smem + wave * p.n_part;
  if (p.part_q >= 0) {
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) mine[p.part_q + (c * kWave + lane) * E + e] = dq[c][e];
  }
  if (p.part_bias >= 0 && lane == 0) mine[p.part_bias] = acc_bias;
  if (p.part_scale >= 0) {
    const float sv = wave_sum(acc_sv);
    if (lane == 0) mine[p.part_scale] = sv;
  }
  __syncthreads();
  const int wpb = blockDim.x / kWave;
  for (int i = threadIdx.x; i < p.n_part; i += blockDim.x) {
    float a = 0.f;
    for (int w2 = 0; w2 < wpb; ++w2) a += smem[w2 * p.n_part + i];
    p.partials[part_index(kPartTiled, blockIdx.x, i, gridDim.x, p.n_part)] = a;
  }
}

// ---------------------------------------------------------------- LR keys
// The LR merge (attnres_ops.py:4075-4160, single head): the partial block's
// logit comes from its r-dim LR key, rnd(rnd(<rnd(khat), q>) * scale) with
// khat = rms-norm of the (optionally scaled) key, and the merge is either
// addcmul or torch.lerp (MERGE template flag, true = lerp); the output norm of
// the next sublayer may be fused (runtime flag, one wave holds the row).  The
// value rows stay packed as in the base kernels; the key row is KJ elements
// per lane (r <= 64 KJ), loaded as raw bits after the rows' loads are issued.

// The merge of one element pair: addcmul rnd(a + rnd(b - a) w), lerp
// rnd(|w| < 1/2 ? a + w (b - a) : b - (b - a)(1 - w)) with b - a in fp32 (the
// eager lerp's opmath); w is wave-uniform, so is the lerp branch.
template <class DT, bool LERP>
__device__ __forceinline__ uint32_t p2lr_merge2(uint32_t aw, uint32_t bw, float w) {
  float a0, a1, b0, b1;
  unpack2<DT>(aw, a0, a1);
  unpack2<DT>(bw, b0, b1);
  if constexpr (LERP) {
    if (fabsf(w) < 0.5f) return pack2<DT>(a0 + w * (b0 - a0), a1 + w * (b1 - a1));
    const float omw = 1.0f - w;
    return pack2<DT>(b0 - (b0 - a0) * omw, b1 - (b1 - a1) * omw);
  } else {
    float d0, d1;
    unpack2<DT>(pack2<DT>(b0 - a0, b1 - a1), d0, d1);
    return pack2<DT>(a0 + d0 * w, a1 + d1 * w);
  }
}

// Sums over the row in the general kernels' order (per column, fp32 adds in
// element order, then one wave sum per column added in column order), so the
// per-token results are bit-identical to theirs.
template <int CB>
__device__ __forceinline__ float p2lr_row_sum(const float (&x)[CB]) {
  float t = 0.f;
#pragma unroll
  for (int c = 0; c < CB; ++c) t += wave_sum(x[c]);
  return t;
}

// Recomputed forward state of one LR token: p = rnd(pv vs) packed, the key
// as scored (kv: scaled key, kl: normed and rounded key), 1/rms of the key,
// sigmoid and its rounded value.
template <class DT, int VB, int CB, int KJ>
struct P2LR {
  static constexpr int W = VB / 4;
  uint32_t pw[CB][W];
  float kv[KJ], kl[KJ];
  float inv_key, sg, prob;
};

template <class DT, int VB, int CB, int KJ>
__device__ __forceinline__ void p2lr_forward_state(const Phase2Params& p, int lane, const Raw<DT, VB / 2> (&pvr)[CB],
                                                   const float (&kr)[KJ], const float (&qk)[KJ], float vs, float bias,
                                                   float lse, P2LR<DT, VB, CB, KJ>& st) {
  constexpr int W = VB / 4;
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int i = 0; i < W; ++i) {
      float a, b;
      unpack2<DT>(pvr[c].w[i], a, b);
      st.pw[c][i] = pack2<DT>(a * vs, b * vs);
    }
  // key: kv = rnd(k vs) when the block scale applies to it; khat = rnd(kv / rms(kv))
#pragma unroll
  for (int j = 0; j < KJ; ++j) st.kv[j] = p.scale_key ? DT::rnd(kr[j] * vs) : kr[j];
  st.inv_key = 1.f;
  if (p.key_norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < KJ; ++j) ss += st.kv[j] * st.kv[j];
    st.inv_key = 1.0f / sqrtf(wave_sum(ss) / (float)p.R + p.eps);
  }
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    st.kl[j] = p.key_norm ? DT::rnd(st.kv[j] * st.inv_key) : st.kv[j];
    dot += DT::rnd(st.kl[j] * qk[j]);  // 0 past R (q and the key read as 0 there)
  }
  const float logit = DT::rnd(DT::rnd(wave_sum(dot)) * p.scale);
  const float x = (logit + bias) - lse;
  st.sg = 1.0f / (1.0f + expf(-x));
  st.prob = DT::rnd(st.sg);
}

// The block accumulation fused in front of the merge (ACC): this sublayer's
// projection y = [out | key | pad] grows the live partial block, value
// rnd(pv_old + y[:D]) and key rnd(pk_old + k) with k = rnd(x inv) over each
// key head (x = y[D:D+R]; the key split's arithmetic and sum order), and the
// grown block is what the merge reads.  One token's loads (raw bits) and the
// grown rows: pvr (packed, as the merge's partial rows) and kr (floats).
template <class DT, int VB, int CB, int KJ>
__device__ __forceinline__ void p2lr_accumulate(const Phase2Params& p, int64_t tok, int lane,
                                                const Raw<DT, VB / 2> (&yv)[CB], const Raw<DT, VB / 2> (&po)[CB],
                                                const uint32_t (&xb)[KJ], const uint32_t (&ob)[KJ],
                                                Raw<DT, VB / 2> (&pvr)[CB], float (&kr)[KJ]) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  const bool old = p.acc_pv_old != nullptr;
  S* pvo = (S*)p.acc_pv_out + tok * (int64_t)p.D;
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    float f[E];
#pragma unroll
    for (int i = 0; i < W; ++i) {
      float y0, y1;
      unpack2<DT>(yv[c].w[i], y0, y1);
      if (old) {
        float a0, a1;
        unpack2<DT>(po[c].w[i], a0, a1);
        pvr[c].w[i] = pack2<DT>(a0 + y0, a1 + y1);
      } else {
        pvr[c].w[i] = yv[c].w[i];
      }
      unpack2<DT>(pvr[c].w[i], f[2 * i], f[2 * i + 1]);
    }
    store_vec<DT, E, true>(pvo + (c * kWave + lane) * E, f);
  }
  float x[KJ];
  row_bits_floats<DT, KJ>(xb, p.R, lane, kWave, x);
#pragma unroll
  for (int j = 0; j < KJ; ++j) kr[j] = x[j];
  if (p.acc_key_norm) {
    float sq[KJ], ss[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) sq[j] = x[j] * x[j];
    key_head_sums<KJ>(p.acc_hd, sq, ss);
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int r = lane + j * kWave;
      const float inv = 1.0f / sqrtf(ss[j] / (float)p.acc_hd + p.acc_eps);
      kr[j] = DT::rnd(x[j] * inv);
      if (r < p.R && r % p.acc_hd == 0) p.acc_inv[tok * p.acc_H + r / p.acc_hd] = inv;
    }
  }
  if (p.acc_pk_old) {
    float o[KJ];
    row_bits_floats<DT, KJ>(ob, p.R, lane, kWave, o);
#pragma unroll
    for (int j = 0; j < KJ; ++j) kr[j] = DT::rnd(o[j] + kr[j]);
  }
  S* pko = (S*)p.acc_pk_out + tok * (int64_t)p.R;
#pragma unroll
  for (int j = 0; j < KJ; ++j) {
    const int r = lane + j * kWave;
    if (r < p.R) DT::store1(pko + r, kr[j]);
  }
}

template <class DT, int VB, int CB, int KJ, bool LERP, bool ACC>
__global__ void __launch_bounds__(256) phase2_lr_fwd_fast_kernel(const Phase2Params p) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform_i32(threadIdx.x / kWave);
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;
  // the query as raw bits, converted per token after the token's loads are
  // issued (a wave often has one token: converting here would put the query's
  // load latency in front of the rows')
  uint32_t qb[KJ];
  row_bits_load<DT, KJ>((const S*)p.q, p.R, lane, kWave, qb);

  const int64_t stride = (int64_t)gridDim.x * kP2FastWaves;
  for (int64_t tok = (int64_t)blockIdx.x * kP2FastWaves + wave; tok < p.n_tok; tok += stride) {
    Raw<DT, E> pvr[CB], itr[CB];
    const S* itp = (const S*)p.inter + tok * p.inter_stride;
    float kr[KJ], qk[KJ];
    float lse;
    if constexpr (ACC) {
      const S* yr = (const S*)p.acc_y + tok * p.acc_y_stride;
      const S* pop = p.acc_pv_old ? (const S*)p.acc_pv_old + tok * (int64_t)p.D : nullptr;
      Raw<DT, E> yv[CB], po[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        load_raw<DT, E, true>(yr + (c * kWave + lane) * E, yv[c]);
        if (pop) load_raw<DT, E, true>(pop + (c * kWave + lane) * E, po[c]);
        load_raw<DT, E, true>(itp + (c * kWave + lane) * E, itr[c]);
      }
      uint32_t xb[KJ], ob[KJ];
      row_bits_load<DT, KJ>(yr + p.D, p.R, lane, kWave, xb);
      if (p.acc_pk_old) row_bits_load<DT, KJ>((const S*)p.acc_pk_old + tok * (int64_t)p.R, p.R, lane, kWave, ob);
      lse = p.lse[tok];
      row_bits_floats<DT, KJ>(qb, p.R, lane, kWave, qk);
      p2lr_accumulate<DT, VB, CB, KJ>(p, tok, lane, yv, po, xb, ob, pvr, kr);
    } else {
      const S* pvp = (const S*)p.pv + tok * p.pv_stride;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        load_raw<DT, E, true>(pvp + (c * kWave + lane) * E, pvr[c]);
        load_raw<DT, E, true>(itp + (c * kWave + lane) * E, itr[c]);
      }
      uint32_t kb[KJ];
      row_bits_load<DT, KJ>((const S*)p.pk + tok * p.pk_stride, p.R, lane, kWave, kb);
      lse = p.lse[tok];
      row_bits_floats<DT, KJ>(qb, p.R, lane, kWave, qk);
      row_bits_floats<DT, KJ>(kb, p.R, lane, kWave, kr);
    }
    P2LR<DT, VB, CB, KJ> st;
    p2lr_forward_state<DT, VB, CB, KJ>(p, lane, pvr, kr, qk, vs, bias, lse, st);
    const float w = st.prob;
    uint32_t ow[CB][W];
    float ss[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      ss[c] = 0.f;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        ow[c][i] = p2lr_merge2<DT, LERP>(itr[c].w[i], st.pw[c][i], w);
        float o0, o1;
        unpack2<DT>(ow[c][i], o0, o1);
        ss[c] += o0 * o0;
        ss[c] += o1 * o1;
      }
    }
    const float inv = p.norm_out ? 1.0f / sqrtf(p2lr_row_sum<CB>(ss) / (float)p.D + p.eps) : 1.f;
    S* op = (S*)p.out + tok * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float o[E];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        unpack2<DT>(ow[c][i], o[2 * i], o[2 * i + 1]);
        o[2 * i] *= inv;  // the store rounds (exact when inv = 1)
        o[2 * i + 1] *= inv;
      }
      store_vec<DT, E, true>(op + (c * kWave + lane) * E, o);
    }
  }
}

template <class DT, int VB, int CB, int KJ, bool LERP, bool ACC>
__global__ void __launch_bounds__(256) phase2_lr_bwd_fast_kernel(const Phase2Params p) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
  constexpr int W = VB / 4;
  extern __shared__ float smem[];  // [waves][n_part]: each wave's partial sums
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = uniform_i32(threadIdx.x / kWave);
  const int D = p.D;
  const float vs = summary_scale<DT>(p.scale_dev, p.vscale);
  const float bias = p.bias_dev ? *p.bias_dev : p.bias;
  const bool want_sv = p.part_scale >= 0;
  uint32_t qb[KJ];  // raw bits, converted per token (see the forward)
  row_bits_load<DT, KJ>((const S*)p.q, p.R, lane, kWave, qb);
  float dq[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) dq[j] = 0.f;
  float acc_bias = 0.f, acc_sv = 0.f, acc_sk = 0.f;

  const int64_t stride = (int64_t)gridDim.x * kP2FastWaves;
  for (int64_t tok = (int64_t)blockIdx.x * kP2FastWaves + wave; tok < p.n_tok; tok += stride) {
    Raw<DT, E> pvr[CB], itr[CB], gr[CB];
    {
      const S* pvp = (const S*)p.pv + tok * p.pv_stride;
      const S* itp = (const S*)p.inter + tok * p.inter_stride;
      const S* gp = (const S*)p.gout + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        load_raw<DT, E, true>(gp + (c * kWave + lane) * E, gr[c]);
        load_raw<DT, E, true>(pvp + (c * kWave + lane) * E, pvr[c]);
        load_raw<DT, E, true>(itp + (c * kWave + lane) * E, itr[c]);
      }
    }
    uint32_t kb[KJ];
    row_bits_load<DT, KJ>((const S*)p.pk + tok * p.pk_stride, p.R, lane, kWave, kb);
    // ACC: the grown block's gradients from its other consumers, the
    // projection's key columns and their 1/rms (the accumulation's backward)
    Raw<DT, E> gvr[CB];
    uint32_t gkb[KJ], xab[KJ];
    float ia[KJ];
    if constexpr (ACC) {
      if (p.acc_gv) {
        const S* gvp = (const S*)p.acc_gv + tok * p.acc_gv_stride;
#pragma unroll
        for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(gvp + (c * kWave + lane) * E, gvr[c]);
      }
      if (p.acc_gk) row_bits_load<DT, KJ>((const S*)p.acc_gk + tok * (int64_t)p.R, p.R, lane, kWave, gkb);
      if (p.acc_key_norm) {
        row_bits_load<DT, KJ>((const S*)p.acc_y + tok * p.acc_y_stride + D, p.R, lane, kWave, xab);
#pragma unroll
        for (int j = 0; j < KJ; ++j) ia[j] = p.acc_inv[tok * p.acc_H + min(lane + j * kWave, p.R - 1) / p.acc_hd];
      }
    }
    const float lse = p.lse[tok];
    float kr[KJ], qk[KJ];
    row_bits_floats<DT, KJ>(qb, p.R, lane, kWave, qk);
    row_bits_floats<DT, KJ>(kb, p.R, lane, kWave, kr);
    P2LR<DT, VB, CB, KJ> st;
    p2lr_forward_state<DT, VB, CB, KJ>(p, lane, pvr, kr, qk, vs, bias, lse, st);
    const float w = st.prob;

    // ---- output norm backward: G <- rnd(inv G - o k3), o the recomputed merge
    if (p.norm_out) {
      uint32_t ow[CB][W];
      float a0[CB], a1[CB];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        a0[c] = a1[c] = 0.f;
#pragma unroll
        for (int i = 0; i < W; ++i) {
          ow[c][i] = p2lr_merge2<DT, LERP>(itr[c].w[i], st.pw[c][i], w);
          float o0, o1, g0, g1;
          unpack2<DT>(ow[c][i], o0, o1);
          unpack2<DT>(gr[c].w[i], g0, g1);
          a0[c] += o0 * o0;
          a1[c] += g0 * o0;
          a0[c] += o1 * o1;
          a1[c] += g1 * o1;
        }
      }
      const float inv = 1.0f / sqrtf(p2lr_row_sum<CB>(a0) / (float)D + p.eps);
      const float k3 = inv * inv * inv * (p2lr_row_sum<CB>(a1) / (float)D);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int i = 0; i < W; ++i) {
          float g0, g1, o0, o1;
          unpack2<DT>(gr[c].w[i], g0, g1);
          unpack2<DT>(ow[c][i], o0, o1);
          gr[c].w[i] = pack2<DT>(inv * g0 - o0 * k3, inv * g1 - o1 * k3);
        }
    }

    // ---- merge backward: d inter stored, d p (merge part) kept packed in gr,
    // dprob = rnd(sum_e rnd(g rnd(p - it)))
    S* dip = (S*)p.dinter + tok * (int64_t)D;
    const float omw = DT::rnd(1.0f - w);
    float t[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      t[c] = 0.f;
      float di[E];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float a0, a1, b0, b1, g0, g1, f0, f1;
        unpack2<DT>(itr[c].w[i], a0, a1);
        unpack2<DT>(st.pw[c][i], b0, b1);
        unpack2<DT>(gr[c].w[i], g0, g1);
        unpack2<DT>(pack2<DT>(b0 - a0, b1 - a1), f0, f1);
        t[c] += DT::rnd(g0 * f0);
        t[c] += DT::rnd(g1 * f1);
        const uint32_t dpm = pack2<DT>(g0 * w, g1 * w);
        if constexpr (LERP) {
          di[2 * i] = g0 * omw;  // the store rounds
          di[2 * i + 1] = g1 * omw;
        } else {
          float m0, m1;
          unpack2<DT>(dpm, m0, m1);
          di[2 * i] = g0 - m0;
          di[2 * i + 1] = g1 - m1;
        }
        gr[c].w[i] = dpm;
      }
      store_vec<DT, E, true>(dip + (c * kWave + lane) * E, di);
    }
    const float dprob = DT::rnd(p2lr_row_sum<CB>(t));
    const float dx = dprob * (1.0f - st.sg) * st.sg;
    if (lane == 0) {
      p.dlse[tok] = -dx;
      acc_bias += dx;
    }
    const float dlb = DT::rnd(dx);

    // ---- LR key backward: dk = rnd(rnd(dlb scale) q), rms-norm chain, the
    // key's share of the block scale; dq += rnd(rnd(dlb scale) khat)
    {
      const float dsum = DT::rnd(dlb * p.scale);
      float dk[KJ];
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const bool in = lane + j * kWave < p.R;
        dk[j] = in ? DT::rnd(dsum * qk[j]) : 0.f;
        if (in) dq[j] += DT::rnd(dsum * st.kl[j]);
        m += dk[j] * st.kv[j];
      }
      if (p.key_norm) {
        const float iv = st.inv_key;
        const float k3 = iv * iv * iv * (wave_sum(m) / (float)p.R);
#pragma unroll
        for (int j = 0; j < KJ; ++j) dk[j] = DT::rnd(iv * dk[j] - st.kv[j] * k3);
      }
      if constexpr (ACC) {
        // the grown key's total gradient rnd(merge share + other consumers'),
        // the old partial key's too; through the key norm into the projection
        float tot[KJ], gd[KJ];
        if (p.acc_gk) row_bits_floats<DT, KJ>(gkb, p.R, lane, kWave, gd);
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
          const int r = lane + j * kWave;
          float gk = dk[j];
          if (p.scale_key) {
            acc_sk += DT::rnd(gk * kr[j]);
            gk = gk * vs;
          }
          gk = DT::rnd(gk);
          tot[j] = r < p.R ? (p.acc_gk ? DT::rnd(gk + gd[j]) : gk) : 0.f;
          if (r < p.R && p.acc_dpk_old) DT::store1((S*)p.acc_dpk_old + tok * (int64_t)p.R + r, tot[j]);
        }
        S* gyr = (S*)p.acc_gy + tok * (int64_t)p.acc_P;
        if (p.acc_key_norm) {
          float xa[KJ], gx[KJ], kd[KJ];
          row_bits_floats<DT, KJ>(xab, p.R, lane, kWave, xa);
#pragma unroll
          for (int j = 0; j < KJ; ++j) gx[j] = tot[j] * xa[j];
          key_head_sums<KJ>(p.acc_hd, gx, kd);
#pragma unroll
          for (int j = 0; j < KJ; ++j) {
            const int r = lane + j * kWave;
            if (r < p.R) {
              const float k3k = ia[j] * ia[j] * ia[j] * (kd[j] / (float)p.acc_hd);
              DT::store1(gyr + D + r, ia[j] * tot[j] - xa[j] * k3k);
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < KJ; ++j) {
            const int r = lane + j * kWave;
            if (r < p.R) DT::store1(gyr + D + r, tot[j]);
          }
        }
        for (int cc = D + p.R + lane; cc < p.acc_P; cc += kWave) DT::store1(gyr + cc, 0.f);
      } else {
        S* dkp = (S*)p.dpk + tok * (int64_t)p.R;
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
          const int r = lane + j * kWave;
          if (r < p.R) {
            float gk = dk[j];
            if (p.scale_key) {
              acc_sk += DT::rnd(gk * kr[j]);
              gk = gk * vs;  // the store rounds
            }
            DT::store1(dkp + r, gk);
          }
        }
      }
    }

    // ---- d p = rnd(dpm vs); the value's share of the block scale: rnd(dpm pv).
    // ACC: plus the other consumers' gradient, into the projection's value
    // columns (the old partial value's gradient too)
    S* dpvp = ACC ? (S*)p.acc_gy + tok * (int64_t)p.acc_P : (S*)p.dpv + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float dp[E];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float m0, m1;
        unpack2<DT>(gr[c].w[i], m0, m1);
        if (want_sv) {
          float r0, r1;
          unpack2<DT>(pvr[c].w[i], r0, r1);
          acc_sv += DT::rnd(m0 * r0);
          acc_sv += DT::rnd(m1 * r1);
        }
        dp[2 * i] = m0 * vs;  // the store rounds
        dp[2 * i + 1] = m1 * vs;
        if (ACC && p.acc_gv) {
          float g0, g1;
          unpack2<DT>(gvr[c].w[i], g0, g1);
          dp[2 * i] = DT::rnd(dp[2 * i]) + g0;
          dp[2 * i + 1] = DT::rnd(dp[2 * i + 1]) + g1;
        }
      }
      store_vec<DT, E, true>(dpvp + (c * kWave + lane) * E, dp);
    }
  }

  // partial sums: each wave's row in LDS, then the workgroup's row in 16-slot tiles
  if (!p.partials) return;
  float* mine = smem + wave * p.n_part;
  if (p.part_q >= 0) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int r = lane + j * kWave;
      if (r < p.R) mine[p.part_q + r] = dq[j];
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
  const int wpb = blockDim.x / kWave;
  for (int i = threadIdx.x; i < p.n_part; i += blockDim.x) {
    float a = 0.f;
    for (int w2 = 0; w2 < wpb; ++w2) a += smem[w2 * p.n_part + i];
    p.partials[part_index(kPartTiled, blockIdx.x, i, gridDim.x, p.n_part)] = a;
  }
}

// ---------------------------------------------------------------- launchers
// L.vb = vector bytes (8/16), L.wpt = columns per lane (1/2/3), L.feat bit 0 =
// key norm (base keys; the LR kernels read p.key_norm), L.nmax = 1 for LR keys.
namespace {

template <class DT, int VB, int CB, bool KN>
hipError_t p2fast_launch(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  const dim3 g(L.grid), b(kP2FastWaves * kWave);
  if (bwd) hipLaunchKernelGGL((phase2_bwd_fast_kernel<DT, VB, CB, KN>), g, b, L.lds, st, p);
  else hipLaunchKernelGGL((phase2_fwd_fast_kernel<DT, VB, CB, KN>), g, b, 0, st, p);
  return hipGetLastError();
}

template <class DT, bool KN>
hipError_t p2fast_shape(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  switch (L.vb * 10 + L.wpt) {
    case 81: return p2fast_launch<DT, 8, 1, KN>(bwd, p, L, st);
    case 83: return p2fast_launch<DT, 8, 3, KN>(bwd, p, L, st);
    case 161: return p2fast_launch<DT, 16, 1, KN>(bwd, p, L, st);
    case 162: return p2fast_launch<DT, 16, 2, KN>(bwd, p, L, st);
    default: return hipErrorInvalidValue;
  }
}

template <class DT>
hipError_t p2fast_dt(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  return (L.feat & 1) ? p2fast_shape<DT, true>(bwd, p, L, st) : p2fast_shape<DT, false>(bwd, p, L, st);
}

// LR keys (L.nmax == 1): KJ key elements per lane from p.R, L.feat bit 1 =
// lerp merge, bit 2 = the block accumulation fused in front
template <class DT, int VB, int CB, int KJ, bool LERP>
hipError_t p2lr_launch(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  const dim3 g(L.grid), b(kP2FastWaves * kWave);
  if (L.feat & 4) {
    if (bwd) hipLaunchKernelGGL((phase2_lr_bwd_fast_kernel<DT, VB, CB, KJ, LERP, true>), g, b, L.lds, st, p);
    else hipLaunchKernelGGL((phase2_lr_fwd_fast_kernel<DT, VB, CB, KJ, LERP, true>), g, b, 0, st, p);
    return hipGetLastError();
  }
  if (bwd) hipLaunchKernelGGL((phase2_lr_bwd_fast_kernel<DT, VB, CB, KJ, LERP, false>), g, b, L.lds, st, p);
  else hipLaunchKernelGGL((phase2_lr_fwd_fast_kernel<DT, VB, CB, KJ, LERP, false>), g, b, 0, st, p);
  return hipGetLastError();
}

template <class DT, int KJ, bool LERP>
hipError_t p2lr_shape(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  switch (L.vb * 10 + L.wpt) {
    case 81: return p2lr_launch<DT, 8, 1, KJ, LERP>(bwd, p, L, st);
    case 83: return p2lr_launch<DT, 8, 3, KJ, LERP>(bwd, p, L, st);
    case 161: return p2lr_launch<DT, 16, 1, KJ, LERP>(bwd, p, L, st);
    case 162: return p2lr_launch<DT, 16, 2, KJ, LERP>(bwd, p, L, st);
    default: return hipErrorInvalidValue;
  }
}

template <class DT, bool LERP>
hipError_t p2lr_kj(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  if (p.R <= kWave) return p2lr_shape<DT, 1, LERP>(bwd, p, L, st);
  if (p.R <= 2 * kWave) return p2lr_shape<DT, 2, LERP>(bwd, p, L, st);
  if (p.R <= 4 * kWave) return p2lr_shape<DT, 4, LERP>(bwd, p, L, st);
  return hipErrorInvalidValue;
}

template <class DT>
hipError_t p2lr_dt(bool bwd, const Phase2Params& p, const Launch& L, hipStream_t st) {
  return (L.feat & 2) ? p2lr_kj<DT, true>(bwd, p, L, st) : p2lr_kj<DT, false>(bwd, p, L, st);
}

hipError_t p2fast(bool bwd, int dtype, const Phase2Params& p, const Launch& L, hipStream_t st) {
  const bool lr = L.nmax == 1;
  if (dtype == ATTNRES_DTYPE_BF16) return lr ? p2lr_dt<BF16>(bwd, p, L, st) : p2fast_dt<BF16>(bwd, p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return lr ? p2lr_dt<F16>(bwd, p, L, st) : p2fast_dt<F16>(bwd, p, L, st);
  return hipErrorInvalidValue;  // 16-bit types only (the host plan never selects this path for fp32)
}

}  // namespace

hipError_t launch_phase2_fast_forward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st) {
  return p2fast(false, dtype, p, L, st);
}
hipError_t launch_phase2_fast_backward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st) {
  return p2fast(true, dtype, p, L, st);
}

}  // namespace attnres
