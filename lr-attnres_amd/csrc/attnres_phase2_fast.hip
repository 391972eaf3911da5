// Phase 2 with base keys (rms-norm of the scaled partial block, scored against
// the query), fast path for 16-bit rows that one wave covers exactly:
// D = 64 lanes x CB columns x one VB-byte vector (256 / 768 with 8-byte
// vectors, 512 / 1024 with 16-byte ones), addcmul merge, no output norm.  Reference:
// attention_residual_phase2[_torch], attnres_ops.py:3964-4035 (merge by
// addcmul); other forms run the general kernels in attnres_phase2.hip.
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

template <class DT, int VB, int CB>
__device__ __forceinline__ void p2fast_query(const Phase2Params& p, int lane, float (&q)[CB][VB / 2]) {
  using S = typename DT::S;
  constexpr int E = VB / 2;
#pragma unroll
  for (int c = 0; c < CB; ++c) load_vec<DT, E>((const S*)p.q + (c * kWave + lane) * E, q[c]);
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
  float q[CB][E];
  p2fast_query<DT, VB, CB>(p, lane, q);

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
  float q[CB][E];
  p2fast_query<DT, VB, CB>(p, lane, q);
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

// ---------------------------------------------------------------- launchers
// L.vb = vector bytes (8/16), L.wpt = columns per lane (1/2/3), L.feat bit 0 =
// key norm.
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

hipError_t p2fast(bool bwd, int dtype, const Phase2Params& p, const Launch& L, hipStream_t st) {
  if (dtype == ATTNRES_DTYPE_BF16) return p2fast_dt<BF16>(bwd, p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return p2fast_dt<F16>(bwd, p, L, st);
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
