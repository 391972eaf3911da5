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
    const S* gor = p.gout ? (const S*)p.gout + tok * p.gout_stride : nullptr;
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

// ============================================================ block accumulation
// The split above, fused with the live partial block's update and, at a block
// end, the block source (include/attnres_hip.h, attnres_block_accum_*).  Per
// token (one wave): the key as in the split, added to the partial key; the
// output columns added to the partial value; with accum == 2 the block source
// -- value * s (or rms_norm(value)), key (* s) -- instead of the sums.  Each
// add and product is rounded to the dtype, as the reference's eager ops do.

// row v (E elements) of the grown partial value for token tok: pv + y[:D]
template <class DT, int E>
__device__ __forceinline__ void grown_value(const KeySplitParams& p, const typename DT::S* yr, const typename DT::S* pvr,
                                            int v, float (&f)[E]) {
  Raw<DT, E> t;
  load_raw<DT, E, true>(yr + v * E, t);
  unpack<DT, E>(t, f);
  if (pvr) {
    float a[E];
    Raw<DT, E> u;
    load_raw<DT, E, true>(pvr + v * E, u);
    unpack<DT, E>(u, a);
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = DT::rnd(a[e] + f[e]);
  }
}

template <class DT, int E>
__global__ void __launch_bounds__(256) block_accum_fwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  const bool complete = p.accum == 2;
  const bool vnorm = complete && p.value_norm;
  const float s = complete ? summary_scale<DT>(p.scale_dev, p.vscale) : 1.f;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    const S* yr = (const S*)p.y + tok * p.y_stride;
    const S* pvr = p.pv ? (const S*)p.pv + tok * (int64_t)p.D : nullptr;
    // ---- key: split (and per-head norm), + partial key, (* s)
    float x[kKsJ], k[kKsJ];
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) {
      const int r = lane + j * kWave;
      x[j] = r < p.R ? DT::load1(yr + p.D + r) : 0.f;
      k[j] = x[j];
    }
    if (p.key_norm) {
      float sq[kKsJ], ss[kKsJ];
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) sq[j] = x[j] * x[j];
      head_sums(p, sq, ss);
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        const float inv = 1.0f / sqrtf(ss[j] / (float)p.hd + p.eps);
        k[j] = DT::rnd(x[j] * inv);
        if (r < p.R && r % p.hd == 0 && p.inv) p.inv[tok * p.H + r / p.hd] = inv;
      }
    }
    S* krow = (S*)p.key + tok * (int64_t)p.R;
    const S* pkr = p.pk ? (const S*)p.pk + tok * (int64_t)p.R : nullptr;
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) {
      const int r = lane + j * kWave;
      if (r < p.R) {
        float kv = pkr ? DT::rnd(DT::load1(pkr + r) + k[j]) : k[j];
        if (complete && !vnorm && p.scale_key) kv = DT::rnd(kv * s);
        DT::store1(krow + r, kv);
      }
    }
    // ---- value: y[:D] + partial value, (* s or rms-normed)
    S* orow = (S*)p.out + tok * (int64_t)p.D;
    float inv_v = 1.f;
    if (vnorm) {  // first pass: the grown row's sum of squares
      float ss = 0.f;
      for (int v = lane; v < nv; v += kWave) {
        float f[E];
        grown_value<DT, E>(p, yr, pvr, v, f);
#pragma unroll
        for (int e = 0; e < E; ++e) ss += f[e] * f[e];
      }
      inv_v = 1.0f / sqrtf(wave_sum(ss) / (float)p.D + p.eps);
      if (lane == 0 && p.vinv) p.vinv[tok] = inv_v;
    }
    for (int v = lane; v < nv; v += kWave) {
      float f[E];
      grown_value<DT, E>(p, yr, pvr, v, f);
      if (vnorm) {
#pragma unroll
        for (int e = 0; e < E; ++e) f[e] = DT::rnd(f[e] * inv_v);
      } else if (complete) {
#pragma unroll
        for (int e = 0; e < E; ++e) f[e] = DT::rnd(f[e] * s);
      }
      store_vec<DT, E, true>(orow + v * E, f);
    }
  }
}

template <class DT, int E>
__global__ void __launch_bounds__(256) block_accum_bwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  __shared__ float s_fold[2 * 16];  // two sums per wave (at most 16 waves)
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  const bool complete = p.accum == 2;
  const bool vnorm = complete && p.value_norm;
  const float s = complete ? summary_scale<DT>(p.scale_dev, p.vscale) : 1.f;
  const bool want_ds = complete && !vnorm && p.partials;
  float acc_v = 0.f, acc_k = 0.f;  // learned-scale gradient: sum of rnd(g * grown value / key)
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    const S* yr = (const S*)p.y + tok * p.y_stride;
    const S* pvr = p.pv ? (const S*)p.pv + tok * (int64_t)p.D : nullptr;
    S* gyr = (S*)p.gy + tok * (int64_t)p.P;
    const S* gor = p.gout ? (const S*)p.gout + tok * p.gout_stride : nullptr;
    // ---- value columns: the grown partial value's gradient
    float dot = 0.f;
    if (vnorm && gor) {  // rms-norm backward needs <g, x> over the row first
      for (int v = lane; v < nv; v += kWave) {
        float f[E], g[E];
        grown_value<DT, E>(p, yr, pvr, v, f);
        load_vec<DT, E, true>(gor + v * E, g);
#pragma unroll
        for (int e = 0; e < E; ++e) dot += g[e] * f[e];
      }
      dot = wave_sum(dot);
    }
    const float inv_v = (vnorm && gor) ? p.vinv[tok] : 1.f;  // the host requires vinv with a value gradient
    const float k3 = inv_v * inv_v * inv_v * (dot / (float)p.D);
    for (int v = lane; v < nv; v += kWave) {
      float g[E];
      if (gor) {
        load_vec<DT, E, true>(gor + v * E, g);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = 0.f;
      }
      if (vnorm && gor) {
        float f[E];
        grown_value<DT, E>(p, yr, pvr, v, f);
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = DT::rnd(inv_v * g[e] - f[e] * k3);
      } else if (complete) {
        if (want_ds) {
          float f[E];
          grown_value<DT, E>(p, yr, pvr, v, f);
#pragma unroll
          for (int e = 0; e < E; ++e) acc_v += DT::rnd(g[e] * f[e]);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = DT::rnd(g[e] * s);
      }
      store_vec<DT, E, true>(gyr + v * E, g);
    }
    // ---- key columns
    const S* gkr = p.gkey ? (const S*)p.gkey + tok * (int64_t)p.R : nullptr;
    const S* pkr = p.pk ? (const S*)p.pk + tok * (int64_t)p.R : nullptr;
    float x[kKsJ], g[kKsJ], inv[kKsJ];
#pragma unroll
    for (int j = 0; j < kKsJ; ++j) {
      const int r = lane + j * kWave;
      x[j] = r < p.R ? DT::load1(yr + p.D + r) : 0.f;
      g[j] = (gkr && r < p.R) ? DT::load1(gkr + r) : 0.f;
      inv[j] = (p.key_norm && r < p.R) ? p.inv[tok * p.H + r / p.hd] : 1.f;
    }
    if (complete && !vnorm && p.scale_key) {
      // key = rnd(grown key * s): the grown key's gradient is rnd(g * s)
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        if (want_ds && gkr && r < p.R) {
          const float kt = p.key_norm ? DT::rnd(x[j] * inv[j]) : x[j];
          const float kg = pkr ? DT::rnd(DT::load1(pkr + r) + kt) : kt;
          acc_k += DT::rnd(g[j] * kg);
        }
        g[j] = DT::rnd(g[j] * s);
        if (r < p.R && p.dpk) DT::store1((S*)p.dpk + tok * (int64_t)p.R + r, g[j]);
      }
    }
    if (p.key_norm) {
      float gx[kKsJ], kd[kKsJ];
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) gx[j] = g[j] * x[j];
      head_sums(p, gx, kd);
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) {
          const float k3k = inv[j] * inv[j] * inv[j] * (kd[j] / (float)p.hd);
          DT::store1(gyr + p.D + r, inv[j] * g[j] - x[j] * k3k);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kKsJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) DT::store1(gyr + p.D + r, g[j]);
      }
    }
    for (int c = p.D + p.R + lane; c < p.P; c += kWave) DT::store1(gyr + c, 0.f);
  }
  // ---- learned-scale gradient: this workgroup's two partial sums (value, key)
  if (!want_ds) return;
  acc_v = wave_sum(acc_v);
  acc_k = wave_sum(acc_k);
  if (lane == 0) {
    s_fold[2 * wave] = acc_v;
    s_fold[2 * wave + 1] = acc_k;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float a = 0.f;
    for (int w = 0; w < wpb; ++w) a += s_fold[2 * w + threadIdx.x];
    p.partials[(int64_t)blockIdx.x * 2 + threadIdx.x] = a;
  }
}

template <class DT>
static hipError_t keyed_split_t(bool bwd, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  const dim3 g(L.grid), b(L.teams * kWave);
  if (p.accum) {
    if (bwd) {
      if (L.vec) hipLaunchKernelGGL((block_accum_bwd_kernel<DT, EV>), g, b, 0, st, p);
      else hipLaunchKernelGGL((block_accum_bwd_kernel<DT, 1>), g, b, 0, st, p);
    } else {
      if (L.vec) hipLaunchKernelGGL((block_accum_fwd_kernel<DT, EV>), g, b, 0, st, p);
      else hipLaunchKernelGGL((block_accum_fwd_kernel<DT, 1>), g, b, 0, st, p);
    }
  } else if (bwd) {
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
