// Logits of one completed LR source against the read sites that will read it
// (the block decoder's per-source logit cache, model.py:1838-1865
// make_source_logits):
//   khat[t]      = rnd(rms_norm(key[t]))        (fp32 norm, rounded to the dtype; or the key itself)
//   logit[q, t]  = rnd(rnd(<khat[t], query[q]>) * scale)   (+ bias in fp32 when the count prior is on)
// Eight lanes per token, each with the token's key row (R <= 128) in
// registers and every eighth site; the site queries sit in LDS (read as
// broadcasts).  The backward follows the eager op's
// autograd: the bias add hands the 16-bit branch rnd(g), the scale gives
// du = rnd(g * scale), the linear gives dkhat = rnd(sum_q du[q] query[q]) and
// the rms-norm backward dkey = rnd(inv (dkhat - khat_f32 <dkhat, khat_f32> / R));
// it also writes du and khat, from which the caller forms the queries'
// gradient du^T khat with one library GEMM (the reference's linear backward).
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

constexpr int kSLWaves = 4;  // waves per workgroup
constexpr int kSLBatch = 4;  // backward: site gradients a lane loads per batch
constexpr int kSLLanes = 8;  // lanes per token

// this lane's key row (R elements, RM >= R slots; slots past R are 0)
template <class DT, int RM>
__device__ __forceinline__ void sl_load_key(const SiteLogitsParams& p, int64_t tok, float (&k)[RM]) {
  using S = typename DT::S;
  const S* kp = (const S*)p.key + tok * p.kstride;
  constexpr int E = 16 / (int)sizeof(S);
  if (p.vec) {
#pragma unroll
    for (int c = 0; c < RM / E; ++c) {
      if (c * E < p.R) {
        float v[E];
        load_vec<DT, E>(kp + c * E, v);
#pragma unroll
        for (int e = 0; e < E; ++e) k[c * E + e] = v[e];
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) k[c * E + e] = 0.f;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < RM; ++j) k[j] = j < p.R ? DT::load1(kp + j) : 0.f;
  }
}

// inverse rms of the key row (IEEE divide and square root, as the read kernels)
template <int RM>
__device__ __forceinline__ float sl_inv_rms(const SiteLogitsParams& p, const float (&k)[RM]) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < RM; ++j) ss += k[j] * k[j];
  return 1.0f / sqrtf(ss / (float)p.R + p.eps);
}

// the site queries as fp32 into LDS ([n_q][RM], rows padded to RM)
template <class DT, int RM>
__device__ __forceinline__ void sl_queries_to_lds(const SiteLogitsParams& p, float* s_q) {
  using S = typename DT::S;
  for (int i = threadIdx.x; i < p.n_q * RM; i += blockDim.x) {
    const int q = i / RM, j = i - (i / RM) * RM;
    s_q[i] = j < p.R ? DT::load1((const S*)p.queries + (int64_t)q * p.R + j) : 0.f;
  }
  __syncthreads();
}

// Eight lanes per token (kSLLanes): lane c of a token's group takes the sites
// c, c + 8, ..., so that short inputs (a 2048-token batch has 2048 tokens to
// spread over 256 CUs) still have 8 waves per 64 tokens; the group's lanes are
// adjacent, and the token loop runs wave-uniformly (the last tokens clamped,
// their stores dropped) so that the group sums stay inside full groups.
template <class DT, int RM>
__global__ void __launch_bounds__(kSLWaves * kWave) site_logits_fwd_kernel(const SiteLogitsParams p) {
  using S = typename DT::S;
  extern __shared__ float s_q[];
  sl_queries_to_lds<DT, RM>(p, s_q);
  const int c = threadIdx.x & (kSLLanes - 1);
  const int64_t per_wave = kWave / kSLLanes;
  const int64_t step = (int64_t)gridDim.x * kSLWaves * per_wave;
  for (int64_t w0 = ((int64_t)blockIdx.x * kSLWaves + threadIdx.x / kWave) * per_wave; w0 < p.n_tok; w0 += step) {
    const int64_t tok = w0 + (threadIdx.x & (kWave - 1)) / kSLLanes;
    const bool live = tok < p.n_tok;
    float k[RM];
    sl_load_key<DT, RM>(p, live ? tok : p.n_tok - 1, k);
    if (p.key_norm) {
      const float inv = sl_inv_rms<RM>(p, k);
#pragma unroll
      for (int j = 0; j < RM; ++j) k[j] = DT::rnd(k[j] * inv);
    }
    for (int q = c; q < p.n_q; q += kSLLanes) {
      const float4* qr = (const float4*)(s_q + q * RM);
      float dot = 0.f;
#pragma unroll
      for (int j4 = 0; j4 < RM / 4; ++j4) {
        const float4 w = qr[j4];
        dot = fmaf(k[4 * j4], w.x, dot);
        dot = fmaf(k[4 * j4 + 1], w.y, dot);
        dot = fmaf(k[4 * j4 + 2], w.z, dot);
        dot = fmaf(k[4 * j4 + 3], w.w, dot);
      }
      const float t = DT::rnd(DT::rnd(dot) * p.scale);
      const int64_t o = (int64_t)q * p.n_tok + tok;
      if (live) {
        if (p.odt == ATTNRES_DTYPE_F32) ((float*)p.out)[o] = t + p.bias;
        else DT::store1((S*)p.out + o, t);
      }
    }
  }
}

template <class DT, int RM>
__global__ void __launch_bounds__(kSLWaves * kWave) site_logits_bwd_kernel(const SiteLogitsParams p) {
  using S = typename DT::S;
  extern __shared__ float s_q[];
  sl_queries_to_lds<DT, RM>(p, s_q);
  // the bias add hands a 16-bit branch its gradient rounded to the dtype
  const bool round_in = p.odt == ATTNRES_DTYPE_F32 && DT::kCode != 0;
  const int c = threadIdx.x & (kSLLanes - 1);
  const int64_t per_wave = kWave / kSLLanes;
  const int64_t step = (int64_t)gridDim.x * kSLWaves * per_wave;
  for (int64_t w0 = ((int64_t)blockIdx.x * kSLWaves + threadIdx.x / kWave) * per_wave; w0 < p.n_tok; w0 += step) {
    const int64_t tok = w0 + (threadIdx.x & (kWave - 1)) / kSLLanes;
    const bool live = tok < p.n_tok;
    const int64_t t = live ? tok : p.n_tok - 1;
    float inv = 1.f;
    if (p.key_norm) {
      float k[RM];
      sl_load_key<DT, RM>(p, t, k);
      inv = sl_inv_rms<RM>(p, k);
    }
    // this lane's sites: loads issued in batches, then du and its share of dkhat
    float dk[RM];
#pragma unroll
    for (int j = 0; j < RM; ++j) dk[j] = 0.f;
    for (int q0 = c; q0 < p.n_q; q0 += kSLBatch * kSLLanes) {
      float g[kSLBatch];
#pragma unroll
      for (int i = 0; i < kSLBatch; ++i)
        g[i] = load_any(p.dout[min(q0 + i * kSLLanes, p.n_q - 1)], t, p.odt);
#pragma unroll
      for (int i = 0; i < kSLBatch; ++i) {
        const int q = q0 + i * kSLLanes;
        if (q < p.n_q) {
          const float du = DT::rnd((round_in ? DT::rnd(g[i]) : g[i]) * p.scale);
          if (live) DT::store1((S*)p.du + (int64_t)q * p.n_tok + tok, du);
          const float4* qr = (const float4*)(s_q + q * RM);
#pragma unroll
          for (int j4 = 0; j4 < RM / 4; ++j4) {
            const float4 w = qr[j4];
            dk[4 * j4] = fmaf(du, w.x, dk[4 * j4]);
            dk[4 * j4 + 1] = fmaf(du, w.y, dk[4 * j4 + 1]);
            dk[4 * j4 + 2] = fmaf(du, w.z, dk[4 * j4 + 2]);
            dk[4 * j4 + 3] = fmaf(du, w.w, dk[4 * j4 + 3]);
          }
        }
      }
    }
    // dkhat summed over the token's eight lanes (every lane ends with the sum)
#pragma unroll
    for (int j = 0; j < RM; ++j) dk[j] = DT::rnd(group_sum(dk[j], kSLLanes));
    float k[RM];  // loaded again: not held through the site loop
    sl_load_key<DT, RM>(p, t, k);
    float mr = 0.f;
    if (p.key_norm) {
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < RM; ++j) m += dk[j] * (k[j] * inv);
      mr = m / (float)p.R;
    }
    // lane c writes elements c, c + 8, ... of khat and dkey
    S* khp = (S*)p.khat + tok * (int64_t)p.R;
    S* dkp = (S*)p.dkey + tok * (int64_t)p.R;
#pragma unroll
    for (int j = 0; j < RM; ++j) {
      if ((j & (kSLLanes - 1)) == c && j < p.R && live) {
        if (p.key_norm) {
          DT::store1(khp + j, DT::rnd(k[j] * inv));
          DT::store1(dkp + j, DT::rnd(inv * (dk[j] - k[j] * inv * mr)));
        } else {
          DT::store1(khp + j, k[j]);
          DT::store1(dkp + j, dk[j]);
        }
      }
    }
  }
}

template <class DT, bool BWD>
static hipError_t sl_launch_dt(const SiteLogitsParams& p, const Launch& L, hipStream_t st) {
#define ATTNRES_SL_CASE(RMV)                                                                                       \
  case RMV:                                                                                                        \
    if (BWD)                                                                                                       \
      hipLaunchKernelGGL((site_logits_bwd_kernel<DT, RMV>), dim3(L.grid), dim3(kSLWaves * kWave), L.lds, st, p); \
    else                                                                                                           \
      hipLaunchKernelGGL((site_logits_fwd_kernel<DT, RMV>), dim3(L.grid), dim3(kSLWaves * kWave), L.lds, st, p); \
    return hipGetLastError();
  switch (L.nmax) {
    ATTNRES_SL_CASE(32)
    ATTNRES_SL_CASE(64)
    ATTNRES_SL_CASE(128)
    default: return hipErrorInvalidValue;
  }
#undef ATTNRES_SL_CASE
}

hipError_t launch_site_logits_forward(int dtype, const SiteLogitsParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return sl_launch_dt<F32, false>(p, L, st);
    case ATTNRES_DTYPE_BF16: return sl_launch_dt<BF16, false>(p, L, st);
    default: return sl_launch_dt<F16, false>(p, L, st);
  }
}
hipError_t launch_site_logits_backward(int dtype, const SiteLogitsParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return sl_launch_dt<F32, true>(p, L, st);
    case ATTNRES_DTYPE_BF16: return sl_launch_dt<BF16, true>(p, L, st);
    default: return sl_launch_dt<F16, true>(p, L, st);
  }
}

}  // namespace attnres
