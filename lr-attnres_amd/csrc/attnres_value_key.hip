// Value-derived LR keys (config 4's key producer): the rms-norm around the
// projection GEMM of LRIDSourceKeyProjection (model.py:391-428 with
// lrid_key_from_value and lrid_key_value_norm):
//     key_s = rms_norm(v_s) @ W^T      (norm in fp32, one rounding to the dtype)
// The GEMM stays a library GEMM (hipBLASLt); these kernels write the normed
// rows of every source into one dense [n_src, n_tok, dim] block (so one GEMM
// covers all sources) with the fp32 inverse rms, and in the backward turn the
// GEMM's input gradient into the values' gradient through the rms-norm
// backward, dv = inv * g - x * inv^3 * <g, x> / dim, rounded once.
//
// One wave per row: every load of the row is issued before the first store
// (rows of up to 4096 16-bit elements, 8 vectors per lane, stay in registers).
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

namespace {

constexpr int kVkWaves = 4;  // rows (waves) per workgroup
constexpr int kVkMaxV = 8;   // 16-byte vectors per lane held at once (dim <= 64 * 8 * E)

template <class DT, int E>
__global__ void __launch_bounds__(256) value_norm_fwd_kernel(const ValueNormParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int nv = p.D / E;
  const int64_t rows = (int64_t)p.n_src * p.n_tok;
  const int64_t stride = (int64_t)gridDim.x * kVkWaves;
  for (int64_t row = (int64_t)blockIdx.x * kVkWaves + wave; row < rows; row += stride) {
    const int s = (int)(row / p.n_tok);
    const int64_t tok = row - (int64_t)s * p.n_tok;
    const S* vr = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
    Raw<DT, E> r[kVkMaxV];
#pragma unroll
    for (int c = 0; c < kVkMaxV; ++c) {
      const int v = lane + c * kWave;
      if (v < nv) load_raw<DT, E, true>(vr + v * E, r[c]);
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kVkMaxV; ++c) {
      if (lane + c * kWave < nv) {
        float x[E];
        unpack<DT, E>(r[c], x);
#pragma unroll
        for (int e = 0; e < E; ++e) ss += x[e] * x[e];
      }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)p.D + p.eps);
    if (lane == 0) p.inv[row] = inv;
    S* out = (S*)p.normed + row * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < kVkMaxV; ++c) {
      const int v = lane + c * kWave;
      if (v < nv) {
        float x[E];
        unpack<DT, E>(r[c], x);
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = x[e] * inv;
        store_vec<DT, E, true>(out + v * E, x);
      }
    }
  }
}

template <class DT, int E>
__global__ void __launch_bounds__(256) value_norm_bwd_kernel(const ValueNormParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int nv = p.D / E;
  const int64_t rows = (int64_t)p.n_src * p.n_tok;
  const int64_t stride = (int64_t)gridDim.x * kVkWaves;
  for (int64_t row = (int64_t)blockIdx.x * kVkWaves + wave; row < rows; row += stride) {
    const int s = (int)(row / p.n_tok);
    const int64_t tok = row - (int64_t)s * p.n_tok;
    const S* vr = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
    const S* gr = (const S*)p.gnormed + row * (int64_t)p.D;
    Raw<DT, E> xr[kVkMaxV], g[kVkMaxV];
#pragma unroll
    for (int c = 0; c < kVkMaxV; ++c) {
      const int v = lane + c * kWave;
      if (v < nv) {
        load_raw<DT, E, true>(vr + v * E, xr[c]);
        load_raw<DT, E, true>(gr + v * E, g[c]);
      }
    }
    const float inv = p.inv[row];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < kVkMaxV; ++c) {
      if (lane + c * kWave < nv) {
        float x[E], gg[E];
        unpack<DT, E>(xr[c], x);
        unpack<DT, E>(g[c], gg);
#pragma unroll
        for (int e = 0; e < E; ++e) dot += gg[e] * x[e];
      }
    }
    const float k3 = inv * inv * inv * (wave_sum(dot) / (float)p.D);
    S* dv = (S*)p.dval[s] + tok * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < kVkMaxV; ++c) {
      const int v = lane + c * kWave;
      if (v < nv) {
        float x[E], gg[E];
        unpack<DT, E>(xr[c], x);
        unpack<DT, E>(g[c], gg);
#pragma unroll
        for (int e = 0; e < E; ++e) gg[e] = inv * gg[e] - x[e] * k3;
        store_vec<DT, E, true>(dv + v * E, gg);
      }
    }
  }
}

template <class DT>
hipError_t value_norm_t(bool bwd, const ValueNormParams& p, int grid, bool vec, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  const dim3 g(grid), b(kVkWaves * kWave);
  if (bwd) {
    if (vec) hipLaunchKernelGGL((value_norm_bwd_kernel<DT, EV>), g, b, 0, st, p);
    else hipLaunchKernelGGL((value_norm_bwd_kernel<DT, 1>), g, b, 0, st, p);
  } else {
    if (vec) hipLaunchKernelGGL((value_norm_fwd_kernel<DT, EV>), g, b, 0, st, p);
    else hipLaunchKernelGGL((value_norm_fwd_kernel<DT, 1>), g, b, 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_value_norm(int dtype, bool bwd, const ValueNormParams& p, int grid, bool vec, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return value_norm_t<F32>(bwd, p, grid, vec, st);
    case ATTNRES_DTYPE_BF16: return value_norm_t<BF16>(bwd, p, grid, vec, st);
    default: return value_norm_t<F16>(bwd, p, grid, vec, st);
  }
}

}  // namespace attnres
