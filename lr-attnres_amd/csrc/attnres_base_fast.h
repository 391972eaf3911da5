// Base AttnRes read (keys = rms_norm of the full values), fast path for 16-bit
// rows that one wave covers exactly: D = 64 lanes x CB columns x one VB-byte
// vector (256 / 768 with 8-byte vectors, 512 / 1024 with 16-byte ones).
//
// Numerics are those of the step-by-step kernels (the reference's eager op,
// which the oracle restates): the forward scores the dtype-rounded key
// rnd(v * inv) (inv = 1/sqrt(<v, v>/D + eps), IEEE), rounds the logit and mixes
// with dtype-rounded weights; the backward rounds dW, the logit gradient ge,
// rnd(ge q), the rms-norm gradient and rnd(w g) where the eager op does.  The
// speed comes from doing the same arithmetic in fewer instructions: row dot
// products and the mix as v_dot2 on packed 16-bit words, the query-gradient
// products of two sources as one v_dot2 with (ge_0, ge_1), rnd(a) + rnd(b) as
// one v_cvt_pk + one v_dot2 with (1, 1), the per-source scalars (inverse rms,
// softmax) computed once per lane instead of once per source in every lane,
// and many row sums folded together by wave_sums.  The step-by-step kernels
// at d=768 spent about twice the token's HBM time in VALU work.
//
// Work layout as in the fast LR kernels: four independent one-wave token
// streams per workgroup, per-source row tables in LDS read as scalars, every
// load of a token issued before any arithmetic, stores last, non-temporal
// policy on the row streams.  Source slots past n_src repeat the last source
// (their rows are cache hits and their values are never used), so the loads
// over NB slots carry no branches.
#pragma once

#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_lr_fast.h"
#include "attnres_params.h"

namespace attnres {

// this lane's words of the static query (dtype-exact, packed two per word)
template <class DT, int VB, int CB>
__device__ __forceinline__ void base_fast_query(const ReadParams& p, int lane, uint32_t (&qw)[CB][VB / 4]) {
  using S = typename DT::S;
  constexpr int E = VB / (int)sizeof(S);
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    Raw<DT, E> r;
    load_raw<DT, E>((const S*)p.q_static + (c * kWave + lane) * E, r);
#pragma unroll
    for (int i = 0; i < VB / 4; ++i) qw[c][i] = r.w[i];
  }
}

template <class DT, int VB, int CB, int NB, bool KN>
__global__ void __launch_bounds__(256) base_fwd_fast_kernel(const ReadParams p) {
  using S = typename DT::S;
  constexpr int E = VB / (int)sizeof(S);
  constexpr int W = VB / 4;
  constexpr int NP = NB <= 4 ? 4 : NB <= 8 ? 8 : 16;  // lanes of the softmax group
  constexpr int NB1 = (NB + 3) / 4 * 4;               // wave_sums takes groups of four values
  extern __shared__ float smem[];
  SrcTab* tab = (SrcTab*)smem;
  const int lane = threadIdx.x & (kWave - 1);
  const int wslot = uniform_i32(threadIdx.x / kWave);
  const int N = p.n_src;
  for (int i = threadIdx.x; i < kMaxSources; i += blockDim.x) {
    const int j = min(i, N - 1);
    tab->vptr[i] = (uint64_t)p.val[j];
    tab->vstrb[i] = (uint32_t)p.vstride[j] * (uint32_t)sizeof(S);
  }
  __syncthreads();
  uint32_t qw[CB][W];
  base_fast_query<DT, VB, CB>(p, lane, qw);

  const int64_t t0 = (int64_t)blockIdx.x * kFastWaves + wslot;
  for (int64_t tok = t0 < p.streams ? t0 : p.n_tok; tok < p.n_tok; tok += p.streams) {
    Raw<DT, E> vr[NB][CB];
    {
      uint64_t base[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) base[s] = row_base(tab, s, tok);
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        const S* vp = global_ptr<const S>(uniform_u64(base[s]));
#pragma unroll
        for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(vp + (c * kWave + lane) * E, vr[s][c]);
      }
    }
    // ---- <v, v> of every slot -> lane s holds source s's inverse rms
    float inv[NB];
    if constexpr (KN) {
      float ssp[NB1];
#pragma unroll
      for (int s = NB; s < NB1; ++s) ssp[s] = 0.f;
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int i = 0; i < W; ++i) ss = dot2<DT>(vr[s][c].w[i], vr[s][c].w[i], ss);
        ssp[s] = ss;
      }
      float z[NB1 / 4];
      wave_sums<NB1>(ssp, z);
      float mine = 0.f;
#pragma unroll
      for (int s = 0; s < NB; ++s)
        mine = wave_sums_pick<NB1>(z, s, lane == s, mine);
      const float inv_l = 1.0f / sqrtf(mine / (float)p.D + p.eps);
#pragma unroll
      for (int s = 0; s < NB; ++s) inv[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_l), s));
    }
    // ---- logits <rnd(v * inv), q> (or <v, q>) -> lane s holds source s's logit
    float tp[NB1];
#pragma unroll
    for (int s = NB; s < NB1; ++s) tp[s] = 0.f;
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      float t = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if constexpr (KN) {
          float v[E];
          unpack<DT, E>(vr[s][c], v);
#pragma unroll
          for (int i = 0; i < W; ++i) t = dot2<DT>(pack2<DT>(v[2 * i] * inv[s], v[2 * i + 1] * inv[s]), qw[c][i], t);
        } else {
#pragma unroll
          for (int i = 0; i < W; ++i) t = dot2<DT>(vr[s][c].w[i], qw[c][i], t);
        }
      }
      tp[s] = t;
    }
    float z[NB1 / 4];
    wave_sums<NB1>(tp, z);
    float lg = -INFINITY;
#pragma unroll
    for (int s = 0; s < NB; ++s)
      lg = wave_sums_pick<NB1>(z, s, lane == s && s < N, lg);
    {
      const float bl = p.bias ? p.bias[min(lane, N - 1)] : 0.f;
      lg = lane < N ? DT::rnd(lg) + bl : -INFINITY;
    }
    // ---- softmax across lanes 0..NB-1
    const float mx = group_max(lg, NP);
    const float ex = lane < N ? expf(lg - mx) : 0.f;
    const float pw = ex / group_sum(ex, NP);
    if (p.weights && lane < N) p.weights[tok * N + lane] = pw;
    // dtype-rounded weights, two sources per word (spare slots and lanes weigh 0)
    const uint32_t wb = lane < N ? bits16<DT>(DT::rnd(pw)) : 0u;
    constexpr int NJ = (NB + 1) / 2;
    uint32_t wp[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      wp[j] = (uint32_t)__builtin_amdgcn_readlane((int)wb, 2 * j) |
              ((uint32_t)__builtin_amdgcn_readlane((int)wb, 2 * j + 1) << 16);
    // ---- mix: one v_dot2 per element and source pair (an odd last slot is
    // paired with +0, so no product of a zero weight with a row is formed)
    float acc[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (2 * j < N) {
        const bool has1 = 2 * j + 1 < NB;
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const uint32_t a = vr[2 * j][c].w[i], b = has1 ? vr[has1 ? 2 * j + 1 : 2 * j][c].w[i] : 0u;
            acc[c][2 * i] = dot2<DT>(lo_pair(a, b), wp[j], acc[c][2 * i]);
            acc[c][2 * i + 1] = dot2<DT>(hi_pair(a, b), wp[j], acc[c][2 * i + 1]);
          }
      }
    }
    S* op = global_ptr<S>((uint64_t)p.out) + tok * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < CB; ++c) store_vec<DT, E, true>(op + (c * kWave + lane) * E, acc[c]);
  }
}

static_assert(kFastWaves == kBaseFastWaves, "base fast kernels: four token streams per workgroup");

template <class DT, int VB, int CB, int NB, bool KN>
__global__ void __launch_bounds__(256) base_bwd_fast_kernel(const ReadBwdParams bp) {
  using S = typename DT::S;
  constexpr int E = VB / (int)sizeof(S);
  constexpr int W = VB / 4;
  constexpr int NB2 = (2 * NB + 3) / 4 * 4;  // wave_sums takes groups of four values
  constexpr int NB1 = (NB + 3) / 4 * 4;
  const ReadParams& p = bp.f;
  extern __shared__ float smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wslot = uniform_i32(threadIdx.x / kWave);
  // LDS: source tables | fold rows [waves][fstride]
  SrcTab* tab = (SrcTab*)smem;
  const int fstride = (bp.n_part + 3) & ~3;
  float* s_fold = smem + kSrcTabFloats;
  const int N = p.n_src, D = p.D;
  const uint32_t rowb = (uint32_t)D * (uint32_t)sizeof(S);
  for (int i = threadIdx.x; i < kMaxSources; i += blockDim.x) {
    const int j = min(i, N - 1);
    tab->vptr[i] = (uint64_t)p.val[j];
    tab->vstrb[i] = (uint32_t)p.vstride[j] * (uint32_t)sizeof(S);
    tab->dvptr[i] = (uint64_t)bp.dval[j];
  }
  __syncthreads();
  uint32_t qw[CB][W];
  base_fast_query<DT, VB, CB>(p, lane, qw);
  float qacc[CB][E];
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) qacc[c][e] = 0.f;
  float bacc = 0.f;  // bias slot `lane` (lane < N)

  const int64_t t0 = (int64_t)blockIdx.x * kFastWaves + wslot;
  for (int64_t tok = t0 < p.streams ? t0 : p.n_tok; tok < p.n_tok; tok += p.streams) {
    Raw<DT, E> gr[CB];
    Raw<DT, E> vr[NB][CB];
    {
      const S* gp = global_ptr<const S>(row_addr((uint64_t)bp.gout, tok, rowb));
#pragma unroll
      for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(gp + (c * kWave + lane) * E, gr[c]);
      uint64_t base[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) base[s] = row_base(tab, s, tok);
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        const S* vp = global_ptr<const S>(uniform_u64(base[s]));
#pragma unroll
        for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(vp + (c * kWave + lane) * E, vr[s][c]);
      }
    }
    const float* wrow = bp.saved_w + tok * N;
    float pw[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) pw[s] = wrow[min(s, N - 1)];
    // ---- stage 1: <g, v> and <v, v> of every slot, summed over the wave
    float part[NB2];
#pragma unroll
    for (int i = 2 * NB; i < NB2; ++i) part[i] = 0.f;
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      float dw = 0.f, ss = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        const Raw<DT, E> v = vr[s][c];
#pragma unroll
        for (int i = 0; i < W; ++i) {
          dw = dot2<DT>(gr[c].w[i], v.w[i], dw);
          ss = dot2<DT>(v.w[i], v.w[i], ss);
        }
      }
      part[2 * s] = dw;
      part[2 * s + 1] = ss;
    }
    // per-source scalars live in scalar registers (wave-uniform)
    float b[NB], ge[NB], mr[NB], b_l = 1.f;
    {
      float z[NB2 / 4];
      wave_sums<NB2>(part, z);
      // lane s: source s's inverse rms (IEEE, as the forward)
      if constexpr (KN) {
        float mine = 0.f;
#pragma unroll
        for (int s = 0; s < NB; ++s)
          mine = wave_sums_pick<NB2>(z, 2 * s + 1, lane == s, mine);
        b_l = 1.0f / sqrtf(mine / (float)D + p.eps);
      }
      // ---- softmax backward: dW and the logit gradient rounded like the
      // reference's 16-bit contraction gradients
      float wdot = 0.f;
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        part[s] = DT::rnd(wave_sums_get<NB2>(z, 2 * s));
        if (s < N) wdot += pw[s] * part[s];
      }
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        b[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b_l), s));
        float dl = 0.f;
        if (s < N) {
          dl = pw[s] * (part[s] - wdot);
          if (lane == s) bacc += dl;
        }
        ge[s] = uniform_f32(DT::rnd(dl));                   // 0 past N
        pw[s] = uniform_f32(s < N ? DT::rnd(pw[s]) : 0.f);  // weight as the mix used it
      }
    }
    // ---- stage 2 (key norm): m_s = <rnd(ge_s q), v_s>, mr_s = m_s inv_s / D
    if constexpr (KN) {
      float mp[NB1];
#pragma unroll
      for (int s = 0; s < NB1; ++s) mp[s] = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float q[E];
        {
          Raw<DT, E> qr;
#pragma unroll
          for (int i = 0; i < W; ++i) qr.w[i] = qw[c][i];
          unpack<DT, E>(qr, q);
        }
#pragma unroll
        for (int s = 0; s < NB; ++s)
#pragma unroll
          for (int i = 0; i < W; ++i)
            mp[s] = dot2<DT>(pack2<DT>(ge[s] * q[2 * i], ge[s] * q[2 * i + 1]), vr[s][c].w[i], mp[s]);
      }
      float z2[NB1 / 4];
      wave_sums<NB1>(mp, z2);
      float mine = 0.f;
#pragma unroll
      for (int s = 0; s < NB; ++s)
        mine = wave_sums_pick<NB1>(z2, s, lane == s, mine);
      const float mr_l = mine * b_l / (float)D;
#pragma unroll
      for (int s = 0; s < NB; ++s) mr[s] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mr_l), s));
    }
    // Stage 3 recomputes ge q rather than keeping stage 2's products (one
    // register per element and source): the empty asm hides that they are the
    // same values, and the barrier keeps stage 3's mr-independent half from
    // being hoisted above the stage-2 reduction (same register cost).
#pragma unroll
    for (int s = 0; s < NB; ++s) asm volatile("" : "+s"(ge[s]));
    __builtin_amdgcn_sched_barrier(0);
    // ---- stage 3, per column, two sources at a time (one for an odd last slot):
    //   dv  = rnd(rnd(w g) + dvk),  dvk = rnd(inv (rnd(ge q) - v inv mr))  (key norm; else rnd(ge q))
    //   dq += ge rnd(v inv)
    // rnd(a) + rnd(b) is one v_dot2 of the packed pair with (1, 1), and the
    // query-gradient products of a source pair one v_dot2 with (ge_0, ge_1).
    const uint32_t one2 = DT::kCode == 1 ? 0x3f803f80u : 0x3c003c00u;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      float q[E], g[E];
      {
        Raw<DT, E> qr;
#pragma unroll
        for (int i = 0; i < W; ++i) qr.w[i] = qw[c][i];
        unpack<DT, E>(qr, q);
        unpack<DT, E>(gr[c], g);
      }
#pragma unroll
      for (int j = 0; j < (NB + 1) / 2; ++j) {
        const int s0 = 2 * j;
        const bool has1 = 2 * j + 1 < NB;
        const int s1 = has1 ? 2 * j + 1 : s0;
        if (s0 < N) {
          const float ge1 = has1 ? ge[s1] : 0.f;
          const uint32_t gep = uniform_u32(bits16<DT>(ge[s0]) | (bits16<DT>(ge1) << 16));
          float v0[E], v1[E], d0[E], d1[E];
          unpack<DT, E>(vr[s0][c], v0);
          if (has1) unpack<DT, E>(vr[s1][c], v1);
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float vb0 = KN ? v0[e] * b[s0] : v0[e];
            if (has1) {
              const float vb1 = KN ? v1[e] * b[s1] : v1[e];
              qacc[c][e] = dot2<DT>(pack2<DT>(vb0, vb1), gep, qacc[c][e]);
              float dk0, dk1;
              {
                Raw<DT, 2> dk;
                dk.w[0] = pack2<DT>(ge[s0] * q[e], ge1 * q[e]);
                float t[2];
                unpack<DT, 2>(dk, t);
                dk0 = t[0];
                dk1 = t[1];
              }
              if constexpr (KN) {
                dk0 = b[s0] * (dk0 - vb0 * mr[s0]);
                dk1 = b[s1] * (dk1 - vb1 * mr[s1]);
              }
              d0[e] = dot2<DT>(pack2<DT>(pw[s0] * g[e], dk0), one2, 0.f);
              d1[e] = dot2<DT>(pack2<DT>(pw[s1] * g[e], dk1), one2, 0.f);
            } else {
              qacc[c][e] = dot2<DT>(pack2<DT>(vb0, 0.f), gep, qacc[c][e]);
              float dk0 = DT::rnd(ge[s0] * q[e]);
              if constexpr (KN) dk0 = b[s0] * (dk0 - vb0 * mr[s0]);
              d0[e] = dot2<DT>(pack2<DT>(pw[s0] * g[e], dk0), one2, 0.f);
            }
          }
          S* dvp0 = global_ptr<S>(uniform_u64(row_addr(tab->dvptr[s0], tok, rowb)));
          store_vec<DT, E, true>(dvp0 + (c * kWave + lane) * E, d0);
          if (has1 && s1 < N) {
            S* dvp1 = global_ptr<S>(uniform_u64(row_addr(tab->dvptr[s1], tok, rowb)));
            store_vec<DT, E, true>(dvp1 + (c * kWave + lane) * E, d1);
          }
        }
      }
    }
  }

  // ---- fold the waves' accumulators into this workgroup's partial row
  // (16-byte LDS writes: one lane's E query slots are consecutive)
  if (!bp.partials) return;
  float* fold = s_fold + wslot * fstride;
  if (bp.part_q >= 0) {
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; e += 4)
        *(float4*)&fold[bp.part_q + (c * kWave + lane) * E + e] =
            make_float4(qacc[c][e], qacc[c][e + 1], qacc[c][e + 2], qacc[c][e + 3]);
  }
  if (bp.part_bias >= 0 && lane < N) fold[bp.part_bias + lane] = bacc;
  __syncthreads();
  for (int i = threadIdx.x; i < bp.n_part; i += blockDim.x) {
    float a = 0.f;
    for (int w = 0; w < kFastWaves; ++w) a += s_fold[w * fstride + i];
    bp.partials[part_index(bp.part_layout, blockIdx.x, i, gridDim.x, bp.n_part)] = a;
  }
}

// Launch switch: L.vb = vector bytes (8/16), L.wpt = columns (1/2/3), L.nmax =
// source slots: the exact count up to 8 sources (no wasted slot at the common
// block counts), then 10/12/14/16; KNV = rms-norm keys (compile time: the
// key-norm code and the plain-key code are separate instantiations).
#define ATTNRES_BASE_FAST_NB(fn, P, VB, CB, KNV)         \
  switch (L.nmax) {                                    \
    case 2: return fn<DT, VB, CB, 2, KNV>(P, L, st);   \
    case 3: return fn<DT, VB, CB, 3, KNV>(P, L, st);   \
    case 4: return fn<DT, VB, CB, 4, KNV>(P, L, st);   \
    case 5: return fn<DT, VB, CB, 5, KNV>(P, L, st);   \
    case 6: return fn<DT, VB, CB, 6, KNV>(P, L, st);   \
    case 7: return fn<DT, VB, CB, 7, KNV>(P, L, st);   \
    case 8: return fn<DT, VB, CB, 8, KNV>(P, L, st);   \
    case 10: return fn<DT, VB, CB, 10, KNV>(P, L, st); \
    case 12: return fn<DT, VB, CB, 12, KNV>(P, L, st); \
    case 14: return fn<DT, VB, CB, 14, KNV>(P, L, st); \
    case 16: return fn<DT, VB, CB, 16, KNV>(P, L, st); \
    default: return hipErrorInvalidValue;              \
  }
#define ATTNRES_BASE_FAST_SWITCH(fn, P, KNV)                         \
  switch (L.vb * 10 + L.wpt) {                                     \
    case 81: ATTNRES_BASE_FAST_NB(fn, P, 8, 1, KNV)                \
    case 83: ATTNRES_BASE_FAST_NB(fn, P, 8, 3, KNV)                \
    case 161: ATTNRES_BASE_FAST_NB(fn, P, 16, 1, KNV)              \
    case 162: ATTNRES_BASE_FAST_NB(fn, P, 16, 2, KNV)              \
    default: return hipErrorInvalidValue;                          \
  }

}  // namespace attnres
