// Base AttnRes read (keys are the values, rms-normed over the full width when
// key_norm), the uniform average read, and the deterministic reduction of the
// backward's per-workgroup partial sums.
//
// Semantics follow the reference's eager op (attnres_ops.py:2176-2190): keys
// rms_norm(values) rounded to the tensor dtype, logits a dtype-rounded
// contraction with the query (+ fp32 bias), fp32 softmax, dtype-rounded
// weights, fp32-accumulated mix.
//
// The base read needs every value row twice (norm + logit, then the mix), so
// a token's N rows stay resident in VGPRs as packed raw words: the kernel is
// templated on NMAX (the register slots) and reads HBM exactly once per row.
// Per-source reductions over the row width are wave butterflies, combined
// across waves through LDS when a token spans several waves.
#include "attnres_block.h"
#include "attnres_device.h"
#include "attnres_params.h"
#include "attnres_launch.h"

namespace attnres {

// store the pre-norm output (when a backward will need it)
template <class DT, int CB, int E>
__device__ __forceinline__ void store_prenorm(const ReadParams& p, int64_t tok, const float (&acc)[CB][E],
                                              const Cols<CB, E>& cl) {
  if (!p.out_prenorm) return;
  typename DT::S* xp = (typename DT::S*)p.out_prenorm + tok * (int64_t)p.D;
#pragma unroll
  for (int c = 0; c < CB; ++c)
    if (cl.ok[c]) store_vec<DT, E, true>(xp + cl.eoff[c], acc[c]);
}

// ============================================================== base forward
template <class DT, int E, int CB, int NMAX, int MAXT>
__global__ void __launch_bounds__(MAXT) base_fwd_kernel(const ReadParams p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  float* s_red = smem;  // [wpt * NMAX]
  const int N = p.n_src, D = p.D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);

  float q[CB][E];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) load_vec<DT, E>((const S*)p.q_static + cl.eoff[c], q[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) q[c][e] = 0.f;
  }

  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    Raw<DT, E> r[NMAX][CB];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
        const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
#pragma unroll
        for (int c = 0; c < CB; ++c)
          if (cl.ok[c]) load_raw<DT, E, true>(vp + cl.eoff[c], r[s][c]);
      }
    }
    // stage 1: sum of squares (key_norm) or the raw logit
    float a[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      a[s] = 0.f;
      if (s < N) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if (cl.ok[c]) {
            float v[E];
            unpack<DT, E>(r[s][c], v);
#pragma unroll
            for (int e = 0; e < E; ++e) a[s] += p.key_norm ? v[e] * v[e] : v[e] * q[c][e];
          }
        }
      }
    }
    block_allreduce<NMAX>(a, N, s_red, lane, wave, wpt);
    if (p.key_norm) {
      // stage 2: logit against the dtype-rounded normalised key
#pragma unroll
      for (int s = 0; s < NMAX; ++s) {
        const float inv = 1.0f / sqrtf(a[s] / (float)D + p.eps);
        float t = 0.f;
        if (s < N) {
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            if (cl.ok[c]) {
              float v[E];
              unpack<DT, E>(r[s][c], v);
#pragma unroll
              for (int e = 0; e < E; ++e) t += DT::rnd(v[e] * inv) * q[c][e];
            }
          }
        }
        a[s] = t;
      }
      block_allreduce<NMAX>(a, N, s_red, lane, wave, wpt);
    }
    // softmax over sources, redundantly in every lane
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
        a[s] = DT::rnd(a[s]) + (p.bias ? p.bias[s] : 0.f);
        m = fmaxf(m, a[s]);
      }
    }
    float den = 0.f;
#pragma unroll
    for (int s = 0; s < NMAX; ++s)
      if (s < N) den += expf(a[s] - m);
    float w[NMAX];
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
        const float pw = expf(a[s] - m) / den;
        if (p.weights && tid == s) p.weights[tok * N + s] = pw;
        w[s] = DT::rnd(pw);
      }
    }
    // mix
    float acc[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = 0.f;
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if (cl.ok[c]) {
            float v[E];
            unpack<DT, E>(r[s][c], v);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[c][e] += w[s] * v[e];
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = DT::rnd(acc[c][e]);
    if (p.norm_out) {
      store_prenorm<DT, CB, E>(p, tok, acc, cl);
      const float inv = norm_output<DT, CB, E>(acc, cl, D, p.eps, s_red, lane, wave, wpt);
      if (tid == 0 && p.out_inv_rms) p.out_inv_rms[tok] = inv;
    }
    S* op = (S*)p.out + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (cl.ok[c]) store_vec<DT, E, true>(op + cl.eoff[c], acc[c]);
  }
}

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


// ============================================================== base, streaming (N > 16)
// Same math as the resident kernels, one source at a time: the logit pass and
// the mix pass each read the value rows (twice the value traffic), per-source
// scalars live in LDS.
template <class DT, int E, int CB>
__global__ void __launch_bounds__(1024) base_fwd_stream_kernel(const ReadParams p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  const int N = p.n_src, D = p.D;
  float* s_l = smem;         // [N] logits, then weights
  float* s_red = smem + N;   // [32]
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);
  float q[CB][E];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) load_vec<DT, E>((const S*)p.q_static + cl.eoff[c], q[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) q[c][e] = 0.f;
  }
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    for (int s = 0; s < N; ++s) {
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
      float v[CB][E];
      float a = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) load_vec<DT, E>(vp + cl.eoff[c], v[c]);
        else
#pragma unroll
          for (int e = 0; e < E; ++e) v[c][e] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) a += p.key_norm ? v[c][e] * v[c][e] : v[c][e] * q[c][e];
      }
      a = block_sum1(a, s_red, lane, wave, wpt);
      if (p.key_norm) {
        const float inv = 1.0f / sqrtf(a / (float)D + p.eps);
        a = 0.f;
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) a += DT::rnd(v[c][e] * inv) * q[c][e];
        a = block_sum1(a, s_red, lane, wave, wpt);
      }
      if (tid == 0) s_l[s] = DT::rnd(a) + (p.bias ? p.bias[s] : 0.f);
    }
    __syncthreads();
    float m = -INFINITY;
    for (int s = 0; s < N; ++s) m = fmaxf(m, s_l[s]);
    float den = 0.f;
    for (int s = 0; s < N; ++s) den += expf(s_l[s] - m);
    float acc[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = 0.f;
    for (int s = 0; s < N; ++s) {
      const float pw = expf(s_l[s] - m) / den;
      if (p.weights && tid == 0) p.weights[tok * N + s] = pw;
      const float w = DT::rnd(pw);
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) {
          float v[E];
          load_vec<DT, E>(vp + cl.eoff[c], v);
#pragma unroll
          for (int e = 0; e < E; ++e) acc[c][e] += w * v[e];
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = DT::rnd(acc[c][e]);
    if (p.norm_out) {
      store_prenorm<DT, CB, E>(p, tok, acc, cl);
      const float inv = norm_output<DT, CB, E>(acc, cl, D, p.eps, s_red, lane, wave, wpt);
      if (tid == 0 && p.out_inv_rms) p.out_inv_rms[tok] = inv;
    }
    S* op = (S*)p.out + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (cl.ok[c]) store_vec<DT, E, true>(op + cl.eoff[c], acc[c]);
    __syncthreads();
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

// ============================================================== average read
template <class DT, int E, int CB>
__global__ void __launch_bounds__(1024) avg_fwd_kernel(const ReadParams p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  float* s_red = smem;
  const int N = p.n_src, D = p.D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    float acc[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = 0.f;
    for (int s = 0; s < N; ++s) {
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) {
          float v[E];
          load_vec<DT, E, true>(vp + cl.eoff[c], v);
#pragma unroll
          for (int e = 0; e < E; ++e) acc[c][e] += v[e];
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = DT::rnd(acc[c][e] / (float)N);
    if (p.norm_out) {
      store_prenorm<DT, CB, E>(p, tok, acc, cl);
      const float inv = norm_output<DT, CB, E>(acc, cl, D, p.eps, s_red, lane, wave, wpt);
      if (tid == 0 && p.out_inv_rms) p.out_inv_rms[tok] = inv;
    }
    S* op = (S*)p.out + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (cl.ok[c]) store_vec<DT, E, true>(op + cl.eoff[c], acc[c]);
  }
}

template <class DT, int E, int CB>
__global__ void __launch_bounds__(1024) avg_bwd_kernel(const ReadBwdParams bp) {
  using S = typename DT::S;
  const ReadParams& p = bp.f;
  extern __shared__ float smem[];
  float* s_red = smem;
  const int N = p.n_src, D = p.D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    float g[CB][E];
    const S* gp = (const S*)bp.gout + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if (cl.ok[c]) load_vec<DT, E, true>(gp + cl.eoff[c], g[c]);
      else
#pragma unroll
        for (int e = 0; e < E; ++e) g[c][e] = 0.f;
    }
    if (p.norm_out)
      norm_output_backward<DT, CB, E>(g, (const S*)p.out_prenorm + tok * (int64_t)D, bp.saved_inv[tok], cl, D, s_red, lane,
                                      wave, wpt);
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) g[c][e] = DT::rnd(g[c][e] / (float)N);
    for (int s = 0; s < N; ++s) {
      S* dvp = (S*)bp.dval[s] + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (cl.ok[c]) store_vec<DT, E, true>(dvp + cl.eoff[c], g[c]);
    }
  }
}

// ============================================================== partial-sum reduction
// A workgroup of 1024 threads owns SPB consecutive slots; thread (rl, sl) sums
// rows rl, rl + RL, ... of slot sl (RL = 1024 / SPB row lanes, reading SPB-wide
// coalesced row segments), and the RL row sums of each slot are added by a
// fixed tree.  The order is fixed, so the result is bit-reproducible run to
// run.  Few slots (the LR static query: R floats) use narrow, deep workgroups
// so that enough of them share the rows.
template <class DT, int SPB>
__global__ void __launch_bounds__(1024) reduce_partials_kernel(const ReduceParams rp) {
  constexpr int RL = 1024 / SPB;
  const int tid = threadIdx.x;
  const int n_slot_blocks = (rp.n_part + SPB - 1) / SPB;
  if ((int)blockIdx.x < n_slot_blocks) {
    __shared__ float sh[RL][SPB + 1];
    const int sl = tid % SPB, rl = tid / SPB;
    const int slot = (int)blockIdx.x * SPB + sl;
    const bool regular = slot < rp.n_part && !(slot >= rp.part_extra && slot < rp.part_extra + rp.n_extra);
    float a = 0.f;
    if (regular) {
#pragma unroll 8
      for (int w = rl; w < rp.n_groups; w += RL) a += rp.partials[(int64_t)w * rp.n_part + slot];
    }
    sh[rl][sl] = a;
    __syncthreads();
    for (int o = RL / 2; o > 0; o >>= 1) {
      if (rl < o) sh[rl][sl] += sh[rl + o][sl];
      __syncthreads();
    }
    if (rl == 0 && regular) {
      const float t = sh[0][sl];
      if (slot >= rp.part_q && slot < rp.part_q + rp.n_q) {
        if (rp.dquery) DT::store1((typename DT::S*)rp.dquery + (slot - rp.part_q), t);
      } else if (slot >= rp.part_gate && slot < rp.part_gate + rp.n_gate) {
        if (rp.dgate) DT::store1((typename DT::S*)rp.dgate + (slot - rp.part_gate), t);
      } else if (slot >= rp.part_bias && slot < rp.part_bias + rp.n_bias) {
        if (rp.dbias) rp.dbias[slot - rp.part_bias] = t;
      }
    }
    return;
  }
  // the last workgroup: extra slots are the summands of one fp32 gradient,
  // each summed over the rows and rounded to the dtype on its own (separate
  // autograd edges reduced in the dtype), then added in slot order
  __shared__ float tree[1024];
  float tot = 0.f;
  for (int k = 0; k < rp.n_extra; ++k) {
    float b = 0.f;
    for (int w = tid; w < rp.n_groups; w += 1024) b += rp.partials[(int64_t)w * rp.n_part + rp.part_extra + k];
    tree[tid] = b;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
      if (tid < o) tree[tid] += tree[tid + o];
      __syncthreads();
    }
    tot += DT::rnd(tree[0]);
    __syncthreads();
  }
  if (tid == 0 && rp.dextra) rp.dextra[0] = tot;
}

// ============================================================== launchers
template <class DT, int E, int CB, int NMAX>
static hipError_t base_fwd_t(const ReadParams& p, const Launch& L, hipStream_t st) {
  // workgroups of at most 256 threads may use up to 256 VGPRs per lane (the
  // rows of 16 sources stay resident without spilling)
  if (L.wpt * kWave <= 256)
    hipLaunchKernelGGL((base_fwd_kernel<DT, E, CB, NMAX, 256>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  else
    hipLaunchKernelGGL((base_fwd_kernel<DT, E, CB, NMAX, 1024>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  return hipGetLastError();
}
template <class DT, int E, int CB, int NMAX>
static hipError_t base_bwd_t(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  // workgroups of at most 256 threads may use up to 256 VGPRs per lane
  const int threads = L.wpt * kWave * L.teams;
  if (threads <= 256)
    hipLaunchKernelGGL((base_bwd_kernel<DT, E, CB, NMAX, 256>), dim3(L.grid), dim3(threads), L.lds, st, p);
  else
    hipLaunchKernelGGL((base_bwd_kernel<DT, E, CB, NMAX, 1024>), dim3(L.grid), dim3(threads), L.lds, st, p);
  return hipGetLastError();
}

// Resident path (N <= 16): vector path keeps two columns per lane.  More
// sources take the streaming kernels, which read each value row twice.
// 16-bit rows of 256 or 768 elements use 8-byte vectors in one or three
// columns, so that every lane of the wave holds part of the row (16-byte
// vectors would leave half of the last column's lanes idle).
template <class DT>
static hipError_t base_fwd_dt(const ReadParams& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  if constexpr (sizeof(typename DT::S) == 2) {
    if (L.vec && L.vb == 8) {
      if (L.wpt == 1 && p.ncols == 1)
        return L.nmax == 8 ? base_fwd_t<DT, EV / 2, 1, 8>(p, L, st) : base_fwd_t<DT, EV / 2, 1, 16>(p, L, st);
      return L.nmax == 8 ? base_fwd_t<DT, EV / 2, 3, 8>(p, L, st) : base_fwd_t<DT, EV / 2, 3, 16>(p, L, st);
    }
  }
  if (L.vec) {
    switch (L.nmax) {
      case 8: return base_fwd_t<DT, EV, 2, 8>(p, L, st);
      case 16: return base_fwd_t<DT, EV, 2, 16>(p, L, st);
      default:
        hipLaunchKernelGGL((base_fwd_stream_kernel<DT, EV, 2>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
        return hipGetLastError();
    }
  }
  switch (L.nmax) {
    case 8: return base_fwd_t<DT, 1, 4, 8>(p, L, st);
    case 16: return base_fwd_t<DT, 1, 4, 16>(p, L, st);
    default:
      hipLaunchKernelGGL((base_fwd_stream_kernel<DT, 1, 4>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
      return hipGetLastError();
  }
}
template <class DT>
static hipError_t base_bwd_dt(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  if constexpr (sizeof(typename DT::S) == 2) {
    if (L.vec && L.vb == 8) {
      if (L.wpt == 1 && p.f.ncols == 1)
        return L.nmax == 8 ? base_bwd_t<DT, EV / 2, 1, 8>(p, L, st) : base_bwd_t<DT, EV / 2, 1, 16>(p, L, st);
      return L.nmax == 8 ? base_bwd_t<DT, EV / 2, 3, 8>(p, L, st) : base_bwd_t<DT, EV / 2, 3, 16>(p, L, st);
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

template <class DT>
static hipError_t avg_fwd_dt(const ReadParams& p, const Launch& L, hipStream_t st) {
  if (L.vec)
    hipLaunchKernelGGL((avg_fwd_kernel<DT, 16 / sizeof(typename DT::S), 2>), dim3(L.grid), dim3(L.wpt * kWave), L.lds,
                       st, p);
  else
    hipLaunchKernelGGL((avg_fwd_kernel<DT, 1, 4>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  return hipGetLastError();
}
template <class DT>
static hipError_t avg_bwd_dt(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  if (L.vec)
    hipLaunchKernelGGL((avg_bwd_kernel<DT, 16 / sizeof(typename DT::S), 2>), dim3(L.grid), dim3(L.wpt * kWave), L.lds,
                       st, p);
  else
    hipLaunchKernelGGL((avg_bwd_kernel<DT, 1, 4>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  return hipGetLastError();
}

#define ATTNRES_DISPATCH(dtype, fn, ...)                          \
  switch (dtype) {                                                \
    case ATTNRES_DTYPE_F32: return fn<F32>(__VA_ARGS__);          \
    case ATTNRES_DTYPE_BF16: return fn<BF16>(__VA_ARGS__);        \
    default: return fn<F16>(__VA_ARGS__);                         \
  }

hipError_t launch_base_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, base_fwd_dt, p, L, st);
}
hipError_t launch_base_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, base_bwd_dt, p, L, st);
}
hipError_t launch_average_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, avg_fwd_dt, p, L, st);
}
hipError_t launch_average_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, avg_bwd_dt, p, L, st);
}

template <class DT>
static hipError_t reduce_dt(const ReduceParams& rp, hipStream_t st) {
  const int extra = rp.n_extra > 0 ? 1 : 0;
  if (rp.n_part <= 512)
    hipLaunchKernelGGL((reduce_partials_kernel<DT, 8>), dim3((rp.n_part + 7) / 8 + extra), dim3(1024), 0, st, rp);
  else if (rp.n_part <= 2048)
    hipLaunchKernelGGL((reduce_partials_kernel<DT, 16>), dim3((rp.n_part + 15) / 16 + extra), dim3(1024), 0, st, rp);
  else
    hipLaunchKernelGGL((reduce_partials_kernel<DT, 64>), dim3((rp.n_part + 63) / 64 + extra), dim3(1024), 0, st, rp);
  return hipGetLastError();
}
hipError_t launch_reduce_partials(int dtype, const ReduceParams& rp, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, reduce_dt, rp, st);
}

}  // namespace attnres
