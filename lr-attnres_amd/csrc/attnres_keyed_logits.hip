// Logits of a query bank against the sources' keys, the first half of phase 1
// from a query bank (attention_residual_phase1, attnres_ops.py:3862-3907; eager
// form _attnres_phase1_read_torch :2620-2627; fused form
// _attnres_phase1_forward_kernel / _backward_kernel :785-930):
//   key[s, t]      = rnd(rms_norm(v[s, t]))    (or v with key_norm off)
//   logits[q, s, t] = rnd(<queries[q], key[s, t]>)
// The second half -- softmax over the sources, lse and the mix -- is exactly
// phase 1 from these logits (attnres_phase1_forward), so the op composes the
// two.  Backward, as the eager op's autograd:
//   dkey = rnd(sum_q dl[q] queries[q]),  dv = rnd(inv (dkey - v inv mr)),
//   mr = <dkey, v> inv / D  (key_norm; else dv = dkey),
//   dqueries[q] = rnd(sum_{s,t} dl[q, s, t] key[s, t]).
// Not on the model's training path: one workgroup of wpt waves per token, one
// element per lane and column (any width, any alignment), queries re-read from
// L2.  The query gradient is a cross-token reduction: workgroup (g, q) sums
// query q over the tokens g, g + G, ... into a partial row, reduced in a
// fixed order by reduce_partials_kernel.
#include "attnres_block.h"
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

constexpr int kKLCols = 8;  // columns per lane (one element each)

template <class DT>
__global__ void __launch_bounds__(512) keyed_logits_fwd_kernel(const KeyedLogitsParams p) {
  using S = typename DT::S;
  extern __shared__ float smem[];  // [wpt][kKLMaxQ]
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave, wpt = blockDim.x / kWave;
  const int N = p.n_src, Q = p.n_q, D = p.D;
  const Cols<kKLCols, 1> cl((D + kWave - 1) / kWave, D, lane, wave, wpt);
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    for (int s = 0; s < N; ++s) {
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
      float key[kKLCols];
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < kKLCols; ++c) {
        key[c] = cl.ok[c] ? DT::load1(vp + cl.eoff[c]) : 0.f;
        ss += key[c] * key[c];
      }
      float inv = 1.f;
      if (p.key_norm) {
        inv = 1.0f / sqrtf(block_sum1(ss, smem, lane, wave, wpt) / (float)D + p.eps);
#pragma unroll
        for (int c = 0; c < kKLCols; ++c) key[c] = DT::rnd(key[c] * inv);
      }
      float t[kKLMaxQ];
#pragma unroll
      for (int q = 0; q < kKLMaxQ; ++q) {
        t[q] = 0.f;
        if (q < Q) {
          const S* qp = (const S*)p.queries + (int64_t)q * D;
#pragma unroll
          for (int c = 0; c < kKLCols; ++c)
            if (cl.ok[c]) t[q] += key[c] * DT::load1(qp + cl.eoff[c]);
        }
      }
      block_allreduce<kKLMaxQ>(t, Q, smem, lane, wave, wpt);
      S* lp = (S*)p.logits;
#pragma unroll
      for (int q = 0; q < kKLMaxQ; ++q)
        if (q < Q && tid == q) DT::store1(lp + ((int64_t)q * N + s) * p.n_tok + tok, DT::rnd(t[q]));
      if (p.inv && tid == 0) p.inv[(int64_t)s * p.n_tok + tok] = inv;
    }
  }
}

// value gradients through the key (and its rms norm)
template <class DT>
__global__ void __launch_bounds__(512) keyed_logits_dv_kernel(const KeyedLogitsParams p) {
  using S = typename DT::S;
  extern __shared__ float smem[];  // [wpt] partial sums
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave, wpt = blockDim.x / kWave;
  const int N = p.n_src, Q = p.n_q, D = p.D;
  const Cols<kKLCols, 1> cl((D + kWave - 1) / kWave, D, lane, wave, wpt);
  const S* dlp = (const S*)p.dlogits;
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    for (int s = 0; s < N; ++s) {
      float dk[kKLCols];
#pragma unroll
      for (int c = 0; c < kKLCols; ++c) dk[c] = 0.f;
      for (int q = 0; q < Q; ++q) {
        const float dl = DT::load1(dlp + ((int64_t)q * N + s) * p.n_tok + tok);
        const S* qp = (const S*)p.queries + (int64_t)q * D;
#pragma unroll
        for (int c = 0; c < kKLCols; ++c)
          if (cl.ok[c]) dk[c] += dl * DT::load1(qp + cl.eoff[c]);
      }
#pragma unroll
      for (int c = 0; c < kKLCols; ++c) dk[c] = DT::rnd(dk[c]);
      S* dvp = (S*)p.dval[s] + tok * (int64_t)D;
      if (p.key_norm) {
        const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
        const float inv = p.inv[(int64_t)s * p.n_tok + tok];
        float v[kKLCols];
        float mm = 0.f;
#pragma unroll
        for (int c = 0; c < kKLCols; ++c) {
          v[c] = cl.ok[c] ? DT::load1(vp + cl.eoff[c]) : 0.f;
          mm += dk[c] * v[c];
        }
        const float mr = block_sum1(mm, smem, lane, wave, wpt) * inv / (float)D;
#pragma unroll
        for (int c = 0; c < kKLCols; ++c)
          if (cl.ok[c]) DT::store1(dvp + cl.eoff[c], DT::rnd(inv * (dk[c] - v[c] * inv * mr)));
      } else {
#pragma unroll
        for (int c = 0; c < kKLCols; ++c)
          if (cl.ok[c]) DT::store1(dvp + cl.eoff[c], dk[c]);
      }
    }
  }
}

// query gradient partials: workgroup (g, q) sums dl[q, s, t] * key[s, t] over
// the sources and the tokens t = g, g + G, ... into row g, slots q*D .. q*D+D-1
template <class DT>
__global__ void __launch_bounds__(512) keyed_logits_dq_kernel(const KeyedLogitsParams p) {
  using S = typename DT::S;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave, wpt = blockDim.x / kWave;
  const int N = p.n_src, D = p.D, q = blockIdx.y;
  const Cols<kKLCols, 1> cl((D + kWave - 1) / kWave, D, lane, wave, wpt);
  const S* dlp = (const S*)p.dlogits;
  float acc[kKLCols];
#pragma unroll
  for (int c = 0; c < kKLCols; ++c) acc[c] = 0.f;
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    for (int s = 0; s < N; ++s) {
      const float dl = DT::load1(dlp + ((int64_t)q * N + s) * p.n_tok + tok);
      const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
      const float inv = p.key_norm ? p.inv[(int64_t)s * p.n_tok + tok] : 1.f;
#pragma unroll
      for (int c = 0; c < kKLCols; ++c) {
        if (cl.ok[c]) {
          const float v = DT::load1(vp + cl.eoff[c]);
          acc[c] += dl * (p.key_norm ? DT::rnd(v * inv) : v);
        }
      }
    }
  }
  float* row = p.partials + (int64_t)blockIdx.x * p.n_part + (int64_t)q * D;
#pragma unroll
  for (int c = 0; c < kKLCols; ++c)
    if (cl.ok[c]) row[cl.eoff[c]] = acc[c];
  (void)tid;
}

template <class DT>
static hipError_t kl_fwd_dt(const KeyedLogitsParams& p, const Launch& L, hipStream_t st) {
  hipLaunchKernelGGL((keyed_logits_fwd_kernel<DT>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  return hipGetLastError();
}
template <class DT>
static hipError_t kl_bwd_dt(const KeyedLogitsParams& p, const Launch& L, hipStream_t st) {
  hipLaunchKernelGGL((keyed_logits_dv_kernel<DT>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !p.partials) return e;
  hipLaunchKernelGGL((keyed_logits_dq_kernel<DT>), dim3(L.teams, p.n_q), dim3(L.wpt * kWave), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_keyed_logits_forward(int dtype, const KeyedLogitsParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, kl_fwd_dt, p, L, st);
}
hipError_t launch_keyed_logits_backward(int dtype, const KeyedLogitsParams& p, const Launch& L, hipStream_t st) {
  ATTNRES_DISPATCH(dtype, kl_bwd_dt, p, L, st);
}

}  // namespace attnres
