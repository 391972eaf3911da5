// Workgroup-level helpers shared by the kernels that give one token to a
// workgroup of `wpt` waves (base read, phase-1 and phase-2 merges): column
// ownership, block all-reduces through LDS, and the output rms-norm with its
// backward.
#pragma once

#include "attnres_device.h"

namespace attnres {

// all-reduce NMAX per-lane values over the workgroup's waves (first N used)
template <int NMAX>
__device__ __forceinline__ void block_allreduce(float (&a)[NMAX], int N, float* s_red, int lane, int wave,
                                                int wpt) {
#pragma unroll
  for (int s = 0; s < NMAX; ++s)
    if (s < N) a[s] = wave_sum(a[s]);
  if (wpt > 1) {
    if (lane == 0) {
#pragma unroll
      for (int s = 0; s < NMAX; ++s)
        if (s < N) s_red[wave * NMAX + s] = a[s];
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < NMAX; ++s) {
      if (s < N) {
        float t = 0.f;
        for (int w = 0; w < wpt; ++w) t += s_red[w * NMAX + s];
        a[s] = t;
      }
    }
    __syncthreads();
  }
}

__device__ __forceinline__ float block_sum1(float x, float* s_red, int lane, int wave, int wpt) {
  x = wave_sum(x);
  if (wpt > 1) {
    if (lane == 0) s_red[wave] = x;
    __syncthreads();
    x = 0.f;
    for (int w = 0; w < wpt; ++w) x += s_red[w];
    __syncthreads();
  }
  return x;
}

template <int CB, int E>
struct Cols {
  int eoff[CB];
  bool ok[CB];
  __device__ __forceinline__ Cols(int ncols, int D, int lane, int wave, int wpt) {
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int col = wave + c * wpt;
      const int e = (col * kWave + lane) * E;
      ok[c] = col < ncols && e < D;
      eoff[c] = e;
    }
  }
};

// rms-norm the token's output (already rounded to the dtype) in place
template <class DT, int CB, int E>
__device__ __forceinline__ float norm_output(float (&acc)[CB][E], const Cols<CB, E>& cl, int D, float eps,
                                             float* s_red, int lane, int wave, int wpt) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (cl.ok[c]) ss += acc[c][e] * acc[c][e];
  ss = block_sum1(ss, s_red, lane, wave, wpt);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[c][e] = DT::rnd(acc[c][e] * inv);
  return inv;
}

// g <- d rms_norm backward from the saved pre-norm output x (dtype-rounded, as
// the reference's autograd keeps it) and 1/rms:
//   dx = inv*g - x*inv^3*mean(g*x), one rounding to the dtype
template <class DT, int CB, int E>
__device__ __forceinline__ void norm_output_backward(float (&g)[CB][E], const typename DT::S* xp, float inv,
                                                     const Cols<CB, E>& cl, int D, float* s_red, int lane,
                                                     int wave, int wpt) {
  float x[CB][E];
  float dot = 0.f;
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    if (cl.ok[c]) load_vec<DT, E>(xp + cl.eoff[c], x[c]);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) x[c][e] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) dot += g[c][e] * x[c][e];
  }
  dot = block_sum1(dot, s_red, lane, wave, wpt);
  const float k3 = inv * inv * inv * (dot / (float)D);
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int e = 0; e < E; ++e) g[c][e] = cl.ok[c] ? DT::rnd(inv * g[c][e] - x[c][e] * k3) : 0.f;
}

}  // namespace attnres
