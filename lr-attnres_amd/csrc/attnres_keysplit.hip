// Key-producer epilogue: split of a sublayer's fused output projection
// y = [out | key | pad] (model.py:316-388, LRIDFusedProjection).
//
// Forward, per token:  out = y[:D];  key = y[D:D+R], rms-normed over each of
// H heads of hd = R/H columns when key_norm: key = rnd(x / sqrt(mean_h(x^2) +
// eps)) in fp32 (F.rms_norm with eps=None, model.py:28-37), saving 1/rms.
// Backward, per token: gy[:D] = g_out;  gy[D:D+R] = rnd(inv * g - x * inv^3 *
// sum_h(g * x) / hd) (rms-norm backward, or g itself without the norm);
// gy[D+R:P] = 0.  That is the sum of the two slice gradients autograd builds
// (each zero outside its slice, so the sum is exact).
//
// One wave per token.  Output columns move as 16-byte vectors when rows are
// aligned; the key lives one element per lane (element lane + 64 j), so a
// head of hd < 64 columns is an aligned group of hd lanes and a head of
// hd >= 64 columns is a run of whole 64-element chunks.
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

constexpr int kKsJ = 4;  // key chunks of 64 (R <= 256)

// per-element head sums of a[j] over each key head (all lanes get their head's sum)
__device__ __forceinline__ void head_sums(const KeySplitParams& p, const float (&a)[kKsJ], float (&s)[kKsJ]) {
  if (p.hd < kWave) {
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) s[j] = group_sum(a[j], p.hd);
  } else {
    float t[kKsJ];
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) t[j] = wave_sum(a[j]);
    const int cph = p.hd / kWave;  // chunks per head
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) {
      const int h0 = (j / cph) * cph;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kKsJ; ++k)
        if (k >= h0 && k < h0 + cph) acc += t[k];
      s[j] = acc;
    }
  }
}

template <class DT, int E>
__global__ void __launch_bounds__(256) keyed_split_fwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    const S* yr = (const S*)p.y + tok * p.y_stride;
    float x[kKsJ];
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) {
      const int r = lane + j * kWave;
      x[j] = r < p.R ? DT::load1(yr + p.D + r) : 0.f;
    }
    S* orow = (S*)p.out + tok * (int64_t)p.D;
    for (int v = lane; v < nv; v += kWave) {
      Raw<DT, E> t;
      load_raw<DT, E, true>(yr + v * E, t);
      float f[E];
      unpack<DT, E>(t, f);
      store_vec<DT, E, true>(orow + v * E, f);
    }
    S* krow = (S*)p.key + tok * (int64_t)p.R;
    if (p.key_norm) {
      float sq[kKsJ], ss[kKsJ];
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) sq[j] = x[j] * x[j];
      head_sums(p, sq, ss);
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        const float inv = 1.0f / sqrtf(ss[j] / (float)p.hd + p.eps);
        if (r < p.R) {
          DT::store1(krow + r, x[j] * inv);
          if (r % p.hd == 0) p.inv[tok * p.H + r / p.hd] = inv;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) DT::store1(krow + r, x[j]);
      }
    }
  }
}

template <class DT, int E>
__global__ void __launch_bounds__(256) keyed_split_bwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    S* gyr = (S*)p.gy + tok * (int64_t)p.P;
    // output columns: the output gradient (or zero)
    const S* gor = p.gout ? (const S*)p.gout + tok * (int64_t)p.D : nullptr;
    for (int v = lane; v < nv; v += kWave) {
      float f[E];
      if (gor) {
        Raw<DT, E> t;
        load_raw<DT, E, true>(gor + v * E, t);
        unpack<DT, E>(t, f);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) f[e] = 0.f;
      }
      store_vec<DT, E, true>(gyr + v * E, f);
    }
    // key columns
    float g[kKsJ];
    const S* gkr = p.gkey ? (const S*)p.gkey + tok * (int64_t)p.R : nullptr;
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) {
      const int r = lane + j * kWave;
      g[j] = (gkr && r < p.R) ? DT::load1(gkr + r) : 0.f;
    }
    if (p.key_norm && gkr) {
      const S* yr = (const S*)p.y + tok * p.y_stride + p.D;
      float x[kKsJ], gx[kKsJ], dot[kKsJ];
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        x[j] = r < p.R ? DT::load1(yr + r) : 0.f;
        gx[j] = g[j] * x[j];
      }
      head_sums(p, gx, dot);
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) {
          const float inv = p.inv[tok * p.H + r / p.hd];
          const float k3 = inv * inv * inv * (dot[j] / (float)p.hd);
          DT::store1(gyr + p.D + r, inv * g[j] - x[j] * k3);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) DT::store1(gyr + p.D + r, g[j]);
      }
    }
    // padding columns of the projection: zero
    for (int c = p.D + p.R + lane; c < p.P; c += kWave) DT::store1(gyr + c, 0.f);
  }
}

template <class DT>
static hipError_t keyed_split_t(bool bwd, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  const dim3 g(L.grid), b(L.teams * kWave);
  if (bwd) {
    if (L.vec) hipLaunchKernelGGL((keyed_split_bwd_kernel<DT, EV>), g, b, 0, st, p);
    else hipLaunchKernelGGL((keyed_split_bwd_kernel<DT, 1>), g, b, 0, st, p);
  } else {
    if (L.vec) hipLaunchKernelGGL((keyed_split_fwd_kernel<DT, EV>), g, b, 0, st, p);
    else hipLaunchKernelGGL((keyed_split_fwd_kernel<DT, 1>), g, b, 0, st, p);
  }
  return hipGetLastError();
}

static hipError_t keyed_split(int dtype, bool bwd, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return keyed_split_t<F32>(bwd, p, L, st);
    case ATTNRES_DTYPE_BF16: return keyed_split_t<BF16>(bwd, p, L, st);
    default: return keyed_split_t<F16>(bwd, p, L, st);
  }
}

hipError_t launch_keyed_split_forward(int dtype, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  return keyed_split(dtype, false, p, L, st);
}
hipError_t launch_keyed_split_backward(int dtype, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  return keyed_split(dtype, true, p, L, st);
}

}  // namespace attnres
