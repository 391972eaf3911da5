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
// A workgroup of 1024 threads (16 waves) owns SPB consecutive slots; thread
// (rl, sl) sums rows rl, rl + RL, ... of slot sl (RL = 1024 / SPB row lanes,
// reading SPB-wide coalesced row segments; the loads are issued ahead of the
// adds).  The row sums of a slot are then added inside each wave (lane
// shuffles across the wave's row lanes) and the 16 wave sums in wave order by
// one thread: one workgroup barrier.  The order is fixed, so the result is
// bit-reproducible run to run.  Few slots (the LR static query: R floats) use
// narrow, deep workgroups so that enough of them share the rows.
template <class DT, int SPB>
__global__ void __launch_bounds__(1024) reduce_partials_kernel(const ReduceParams rp) {
  static_assert(SPB >= 1 && SPB <= kWave && kWave % SPB == 0, "slots per workgroup divide the wave");
  constexpr int RL = 1024 / SPB;
  constexpr int kWaves = 1024 / kWave;
  constexpr int kExtraChunk = 4;
  __shared__ float sh[kWaves][kWave];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  const int n_slot_blocks = (rp.n_part + SPB - 1) / SPB;
  if ((int)blockIdx.x < n_slot_blocks) {
    const int sl = tid % SPB, rl = tid / SPB;
    const int slot = (int)blockIdx.x * SPB + sl;
    const bool regular = slot < rp.n_part && !(slot >= rp.part_extra && slot < rp.part_extra + rp.n_extra);
    float a = 0.f;
    if (regular) {
      // kRowLoads rows per pass, all loads issued before the first add (rows
      // past the end re-read the last row and add +0, which leaves the sum
      // as it is: the adds run in row order either way)
      constexpr int kRowLoads = 8;
      for (int w0 = rl; w0 < rp.n_groups; w0 += kRowLoads * RL) {
        float x[kRowLoads];
#pragma unroll
        for (int u = 0; u < kRowLoads; ++u) {
          const int w = min(w0 + u * RL, rp.n_groups - 1);
          x[u] = rp.partials[part_index(rp.layout, w, slot, rp.n_groups, rp.n_part)];
        }
#pragma unroll
        for (int u = 0; u < kRowLoads; ++u) a += w0 + u * RL < rp.n_groups ? x[u] : 0.f;
      }
    }
    // the wave's row lanes of slot sl are the lanes congruent to sl mod SPB
    if constexpr (SPB == 1) {
      a = wave_sum(a);
    } else {
#pragma unroll
      for (int o = SPB; o < kWave; o <<= 1) a += __shfl_xor(a, o, kWave);
    }
    if (lane < SPB) sh[wv][lane] = a;
    __syncthreads();
    if (tid < SPB && regular) {
      float t = 0.f;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) t += sh[v][tid];
      if (slot >= rp.part_q && slot < rp.part_q + rp.n_q) {
        if (rp.dquery) {
          typename DT::S* dq = (typename DT::S*)rp.dquery + (slot - rp.part_q);
          if (rp.q_rows > 1) {
            for (int r = 0; r < rp.q_rows; ++r) DT::store1(dq + (int64_t)r * rp.n_q, r == rp.q_row ? t : 0.f);
          } else {
            DT::store1(dq, t);
          }
        }
      } else if (slot >= rp.part_gate && slot < rp.part_gate + rp.n_gate) {
        if (rp.dgate) DT::store1((typename DT::S*)rp.dgate + (slot - rp.part_gate), t);
      } else if (slot >= rp.part_bias && slot < rp.part_bias + rp.n_bias) {
        if (rp.dbias) rp.dbias[slot - rp.part_bias] = t;
      }
    }
    return;
  }
  // the last workgroup: extra slots are the summands of one gradient, each
  // summed over the rows and rounded to the dtype on its own (separate autograd
  // edges reduced in the dtype), then accumulated in slot order with a rounding
  // after each add (autograd's accumulation of gradients in the dtype); up to
  // four slots are read in one pass over the rows
  float tot = 0.f;
  for (int k0 = 0; k0 < rp.n_extra; k0 += kExtraChunk) {
    float b[kExtraChunk];
#pragma unroll
    for (int k = 0; k < kExtraChunk; ++k) b[k] = 0.f;
    for (int w = tid; w < rp.n_groups; w += 1024) {
#pragma unroll
      for (int k = 0; k < kExtraChunk; ++k)
        if (k0 + k < rp.n_extra) b[k] += rp.partials[part_index(rp.layout, w, rp.part_extra + k0 + k, rp.n_groups, rp.n_part)];
    }
#pragma unroll
    for (int k = 0; k < kExtraChunk; ++k) {
      b[k] = wave_sum(b[k]);
      if (lane == 0) sh[wv][k] = b[k];
    }
    __syncthreads();
    if (tid == 0) {
      for (int k = 0; k < kExtraChunk && k0 + k < rp.n_extra; ++k) {
        float t = 0.f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) t += sh[v][k];
        tot = DT::rnd(tot + DT::rnd(t));
      }
    }
    __syncthreads();
  }
  if (tid == 0 && rp.dextra) rp.dextra[0] = tot;
}

// ============================================================== launchers
// Workgroups of at most 256 threads may use up to 256 VGPRs per lane (the rows
// of 16 sources stay resident without spilling); ONLY256 instantiates just
// that bound, for layouts that always run one wave per token.
template <class DT, int E, int CB, int NMAX, bool ONLY256 = false>
static hipError_t base_fwd_t(const ReadParams& p, const Launch& L, hipStream_t st) {
  if (ONLY256 || L.wpt * kWave <= 256)
    hipLaunchKernelGGL((base_fwd_kernel<DT, E, CB, NMAX, 256>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  else if constexpr (!ONLY256)
    hipLaunchKernelGGL((base_fwd_kernel<DT, E, CB, NMAX, 1024>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
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
        return L.nmax == 8 ? base_fwd_t<DT, EV / 2, 1, 8, true>(p, L, st) : base_fwd_t<DT, EV / 2, 1, 16, true>(p, L, st);
      return L.nmax == 8 ? base_fwd_t<DT, EV / 2, 3, 8, true>(p, L, st) : base_fwd_t<DT, EV / 2, 3, 16, true>(p, L, st);
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

hipError_t launch_base_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, base_fwd_dt, p, L, st);
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
  // slot-major partials: one workgroup per slot reads that slot's rows as one
  // contiguous run
  if (rp.layout == kPartSlotMajor && rp.n_part <= 1024)
    hipLaunchKernelGGL((reduce_partials_kernel<DT, 1>), dim3(rp.n_part + extra), dim3(1024), 0, st, rp);
  else if (rp.layout == kPartTiled)
    hipLaunchKernelGGL((reduce_partials_kernel<DT, kPartTile>), dim3((rp.n_part + kPartTile - 1) / kPartTile + extra),
                       dim3(1024), 0, st, rp);
  else if (rp.n_part <= 512)
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
