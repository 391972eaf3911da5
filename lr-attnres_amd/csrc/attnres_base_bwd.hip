// Base AttnRes read (keys = rms_norm of the values), backward kernels and
// launch (the forward, the average read and the partial-sum reduction are in
// attnres_base.hip).
#include "attnres_block.h"
#include "attnres_device.h"
#include "attnres_params.h"
#include "attnres_launch.h"

namespace attnres {

// ============================================================== base backward
// A workgroup holds `teams` independent one-wave token streams when a token
// fits one wave (every reduction is then a wave butterfly, no LDS, no
// barrier); otherwise one team of wpt waves.  The teams' query/bias
// accumulators are folded in team order at the end.
template <class DT, int E, int CB, int NMAX, int MAXT>
__global__ void __launch_bounds__(MAXT) base_bwd_kernel(const ReadBwdParams bp) {
  using S = typename DT::S;
  // 16-bit vector path: the row dot products run on packed words (v_dot2)
  constexpr bool kPk = sizeof(S) == 2 && E >= 2;
  constexpr int W = Vec<DT, E>::kWords;
  const ReadParams& p = bp.f;
  extern __shared__ float smem[];
  float* s_red = smem;  // [wpt * NMAX] (only used when wpt > 1, then teams == 1)
  const int N = p.n_src, D = p.D;
  const int wpt = p.wpt;
  const int team_threads = wpt * kWave;
  const int teams = blockDim.x / team_threads;
  const int team = threadIdx.x / team_threads;
  const int tid = threadIdx.x - team * team_threads;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);

  float q[CB][E], qacc[CB][E];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) load_vec<DT, E>((const S*)p.q_static + cl.eoff[c], q[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) q[c][e] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) qacc[c][e] = 0.f;
  }
  float bacc = 0.f;  // bias slot `tid` (tid < N)

  const int64_t tstride = (int64_t)gridDim.x * teams;
  for (int64_t tok = (int64_t)blockIdx.x * teams + team; tok < p.n_tok; tok += tstride) {
    Raw<DT, E> gr[CB];
    const S* gp = (const S*)bp.gout + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if (cl.ok[c]) load_raw<DT, E, true>(gp + cl.eoff[c], gr[c]);
      else
#pragma unroll
        for (int i = 0; i < W; ++i) gr[c].w[i] = 0u;
    }
    Raw<DT, E> r[NMAX][CB];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
        const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if (cl.ok[c]) load_raw<DT, E, true>(vp + cl.eoff[c], r[s][c]);
          else
#pragma unroll
            for (int i = 0; i < W; ++i) r[s][c].w[i] = 0u;
        }
      }
    }
    float pw[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) pw[s] = s < N ? bp.saved_w[tok * N + s] : 0.f;
    float g[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c) unpack<DT, E>(gr[c], g[c]);
    if (p.norm_out) {
      norm_output_backward<DT, CB, E>(g, (const S*)p.out_prenorm + tok * (int64_t)D, bp.saved_inv[tok], cl, D, s_red, lane,
                                      wave, wpt);
      if constexpr (kPk) {
#pragma unroll
        for (int c = 0; c < CB; ++c) pack_raw<DT, E>(g[c], gr[c]);  // g is dtype-exact
      }
    }

    // stage 1: dW = <g, v> and (key_norm) sum of squares
    float a[NMAX], b[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      a[s] = 0.f;
      b[s] = 0.f;
      if (s < N) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if constexpr (kPk) {
#pragma unroll
            for (int i = 0; i < W; ++i) {
              a[s] = dot2<DT>(gr[c].w[i], r[s][c].w[i], a[s]);
              b[s] = dot2<DT>(r[s][c].w[i], r[s][c].w[i], b[s]);
            }
          } else {
            float v[E];
            unpack<DT, E>(r[s][c], v);
#pragma unroll
            for (int e = 0; e < E; ++e) {
              a[s] += g[c][e] * v[e];
              b[s] += v[e] * v[e];
            }
          }
        }
      }
    }
    block_allreduce<NMAX>(a, N, s_red, lane, wave, wpt);
    if (p.key_norm) block_allreduce<NMAX>(b, N, s_red, lane, wave, wpt);

    float dot = 0.f;
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      a[s] = DT::rnd(a[s]);  // dW, rounded like the reference's contraction grad
      b[s] = p.key_norm ? 1.0f / sqrtf(b[s] / (float)D + p.eps) : 1.f;  // inv rms
      if (s < N) dot += pw[s] * a[s];
    }
    float ge[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      const float dl = pw[s] * (a[s] - dot);
      if (tid == s) bacc += dl;
      ge[s] = DT::rnd(dl);
    }
    // stage 2 (key_norm): m_s = <d key_hat, v> * inv for the rms-norm backward
    float mm[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      mm[s] = 0.f;
      if (p.key_norm && s < N) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if constexpr (kPk) {
#pragma unroll
            for (int i = 0; i < W; ++i) {
              const uint32_t dk2 = bits16<DT>(DT::rnd(ge[s] * q[c][2 * i])) |
                                   (bits16<DT>(DT::rnd(ge[s] * q[c][2 * i + 1])) << 16);
              mm[s] = dot2<DT>(dk2, r[s][c].w[i], mm[s]);
            }
          } else {
            float v[E];
            unpack<DT, E>(r[s][c], v);
#pragma unroll
            for (int e = 0; e < E; ++e) mm[s] += DT::rnd(ge[s] * q[c][e]) * v[e];
          }
        }
      }
    }
    if (p.key_norm) block_allreduce<NMAX>(mm, N, s_red, lane, wave, wpt);
    // stage 3: dv = w g + key path; query gradient accumulation
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
        const float ws = DT::rnd(pw[s]);
        const float mr = mm[s] * b[s] / (float)D;
        S* dvp = (S*)bp.dval[s] + tok * (int64_t)D;
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if (cl.ok[c]) {
            float v[E], dv[E];
            unpack<DT, E>(r[s][c], v);
#pragma unroll
            for (int e = 0; e < E; ++e) {
              const float kh = p.key_norm ? DT::rnd(v[e] * b[s]) : v[e];
              qacc[c][e] += ge[s] * kh;
              const float dkh = DT::rnd(ge[s] * q[c][e]);
              const float dvk = p.key_norm ? DT::rnd(b[s] * (dkh - v[e] * b[s] * mr)) : dkh;
              dv[e] = DT::rnd(DT::rnd(ws * g[c][e]) + dvk);
            }
            store_vec<DT, E, true>(dvp + cl.eoff[c], dv);
          }
        }
      }
    }
  }

  if (!bp.partials) return;
  if (teams == 1) {
    float* part = bp.partials + (int64_t)blockIdx.x * bp.n_part;
    if (bp.part_q >= 0) {
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (cl.ok[c])
#pragma unroll
          for (int e = 0; e < E; ++e) part[bp.part_q + cl.eoff[c] + e] = qacc[c][e];
    }
    if (bp.part_bias >= 0 && tid < N) part[bp.part_bias + tid] = bacc;
    return;
  }
  // several teams: stage each team's accumulators in LDS, fold in team order
  __syncthreads();
  float* fold = smem + team * bp.n_part;
  if (bp.part_q >= 0) {
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (cl.ok[c])
#pragma unroll
        for (int e = 0; e < E; ++e) fold[bp.part_q + cl.eoff[c] + e] = qacc[c][e];
  }
  if (bp.part_bias >= 0 && tid < N) fold[bp.part_bias + tid] = bacc;
  __syncthreads();
  for (int i = threadIdx.x; i < bp.n_part; i += blockDim.x) {
    float a = 0.f;
    for (int t = 0; t < teams; ++t) a += smem[t * bp.n_part + i];
    bp.partials[(int64_t)blockIdx.x * bp.n_part + i] = a;
  }
}


template <class DT, int E, int CB>
__global__ void __launch_bounds__(1024) base_bwd_stream_kernel(const ReadBwdParams bp) {
  using S = typename DT::S;
  const ReadParams& p = bp.f;
  extern __shared__ float smem[];
  const int N = p.n_src, D = p.D;
  float* s_dw = smem;          // [N]
  float* s_inv = smem + N;     // [N]
  float* s_red = smem + 2 * N; // [32]
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);
  float q[CB][E], qacc[CB][E];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) load_vec<DT, E>((const S*)p.q_static + cl.eoff[c], q[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) q[c][e] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) qacc[c][e] = 0.f;
  }
  float bacc = 0.f;
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    float g[CB][E];
    const S* gp = (const S*)bp.gout + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if (cl.ok[c]) load_vec<DT, E>(gp + cl.eoff[c], g[c]);
      else
#pragma unroll
        for (int e = 0; e < E; ++e) g[c][e] = 0.f;
    }
    if (p.norm_out)
      norm_output_backward<DT, CB, E>(g, (const S*)p.out_prenorm + tok * (int64_t)D, bp.saved_inv[tok], cl, D, s_red, lane,
                                      wave, wpt);
    for (int s = 0; s < N; ++s) {
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) {
          float v[E];
          load_vec<DT, E>(vp + cl.eoff[c], v);
#pragma unroll
          for (int e = 0; e < E; ++e) {
            a += g[c][e] * v[e];
            b += v[e] * v[e];
          }
        }
      }
      a = block_sum1(a, s_red, lane, wave, wpt);
      if (p.key_norm) b = block_sum1(b, s_red, lane, wave, wpt);
      if (tid == 0) {
        s_dw[s] = DT::rnd(a);
        s_inv[s] = p.key_norm ? 1.0f / sqrtf(b / (float)D + p.eps) : 1.f;
      }
    }
    __syncthreads();
    float dot = 0.f;
    for (int s = 0; s < N; ++s) dot += bp.saved_w[tok * N + s] * s_dw[s];
    for (int s = 0; s < N; ++s) {
      const float pw = bp.saved_w[tok * N + s];
      const float dl = pw * (s_dw[s] - dot);
      if (tid == s) bacc += dl;
      const float ge = DT::rnd(dl);
      const float inv = s_inv[s];
      const float ws = DT::rnd(pw);
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
      float v[CB][E];
      float mm = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) load_vec<DT, E>(vp + cl.eoff[c], v[c]);
        else
#pragma unroll
          for (int e = 0; e < E; ++e) v[c][e] = 0.f;
        if (p.key_norm)
#pragma unroll
          for (int e = 0; e < E; ++e) mm += DT::rnd(ge * q[c][e]) * (v[c][e] * inv);
      }
      if (p.key_norm) mm = block_sum1(mm, s_red, lane, wave, wpt);
      const float mr = mm / (float)D;
      S* dvp = (S*)bp.dval[s] + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) {
          float dv[E];
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float kh = p.key_norm ? DT::rnd(v[c][e] * inv) : v[c][e];
            qacc[c][e] += ge * kh;
            const float dkh = DT::rnd(ge * q[c][e]);
            const float dvk = p.key_norm ? DT::rnd(inv * (dkh - v[c][e] * inv * mr)) : dkh;
            dv[e] = DT::rnd(DT::rnd(ws * g[c][e]) + dvk);
          }
          store_vec<DT, E, true>(dvp + cl.eoff[c], dv);
        }
      }
    }
    __syncthreads();
  }
  if (bp.partials) {
    float* part = bp.partials + (int64_t)blockIdx.x * bp.n_part;
    if (bp.part_q >= 0) {
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (cl.ok[c])
#pragma unroll
          for (int e = 0; e < E; ++e) part[bp.part_q + cl.eoff[c] + e] = qacc[c][e];
    }
    if (bp.part_bias >= 0 && tid < N) part[bp.part_bias + tid] = bacc;
  }
}

// ============================================================== launchers
template <class DT, int E, int CB, int NMAX, bool ONLY256 = false>
static hipError_t base_bwd_t(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  const int threads = L.wpt * kWave * L.teams;
  if (ONLY256 || threads <= 256)
    hipLaunchKernelGGL((base_bwd_kernel<DT, E, CB, NMAX, 256>), dim3(L.grid), dim3(threads), L.lds, st, p);
  else if constexpr (!ONLY256)
    hipLaunchKernelGGL((base_bwd_kernel<DT, E, CB, NMAX, 1024>), dim3(L.grid), dim3(threads), L.lds, st, p);
  return hipGetLastError();
}

// Resident path (N <= 16), 8-byte rows and streaming beyond 16 sources, as
// in the forward.
template <class DT>
static hipError_t base_bwd_dt(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  if constexpr (sizeof(typename DT::S) == 2) {
    if (L.vec && L.vb == 8) {
      if (L.wpt == 1 && p.f.ncols == 1)
        return L.nmax == 8 ? base_bwd_t<DT, EV / 2, 1, 8, true>(p, L, st) : base_bwd_t<DT, EV / 2, 1, 16, true>(p, L, st);
      return L.nmax == 8 ? base_bwd_t<DT, EV / 2, 3, 8, true>(p, L, st) : base_bwd_t<DT, EV / 2, 3, 16, true>(p, L, st);
    }
  }
  if (L.vec) {
    switch (L.nmax) {
      case 8: return base_bwd_t<DT, EV, 2, 8>(p, L, st);
      case 16: return base_bwd_t<DT, EV, 2, 16>(p, L, st);
      default:
        hipLaunchKernelGGL((base_bwd_stream_kernel<DT, EV, 2>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
        return hipGetLastError();
    }
  }
  switch (L.nmax) {
    case 8: return base_bwd_t<DT, 1, 4, 8>(p, L, st);
    case 16: return base_bwd_t<DT, 1, 4, 16>(p, L, st);
    default:
      hipLaunchKernelGGL((base_bwd_stream_kernel<DT, 1, 4>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
      return hipGetLastError();
  }
}

hipError_t launch_base_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, base_bwd_dt, p, L, st);
}
}  // namespace attnres
