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

// A token's key row is held as KJ chunks of 64 lanes (KJ = 1, 2 or 4: R <= 64,
// 128 or 256), a template parameter so that short keys keep few registers.

// Key rows are short (R <= 256): the lane holds elements r = lane + 64 j for
// j < nj = ceil(R / 64), loaded as raw bits (row_bits_load) and converted after
// every load of the token is issued.
template <class DT, int KJ>
__device__ __forceinline__ void key_load(const typename DT::S* row, int R, int nj, int lane, uint32_t (&b)[KJ]) {
  row_bits_load<DT, KJ>(row, R, lane, kWave, b);
}

template <class DT, int KJ>
__device__ __forceinline__ void key_floats(const uint32_t (&b)[KJ], int R, int nj, int lane, float (&f)[KJ]) {
  row_bits_floats<DT, KJ>(b, R, lane, kWave, f);
}

// the key heads' 1/rms values of the lane's elements (forward's saved values)
template <int KJ>
__device__ __forceinline__ void key_inv_load(const KeySplitParams& p, int64_t tok, int nj, int lane, float (&inv)[KJ]) {
#pragma unroll
  for (int j = 0; j < KJ; ++j)
    inv[j] = (p.key_norm && j < nj) ? p.inv[tok * p.H + min(lane + j * kWave, p.R - 1) / p.hd] : 1.f;
}

// per-element head sums of a[j] over each key head (all lanes get their head's sum)
template <int KJ>
__device__ __forceinline__ void head_sums(const KeySplitParams& p, const float (&a)[KJ], float (&s)[KJ]) {
  key_head_sums<KJ>(p.hd, a, s);
}

template <class DT, int E, int KJ>
__global__ void __launch_bounds__(256) keyed_split_fwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  const int nj = (p.R + kWave - 1) / kWave;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    const S* yr = (const S*)p.y + tok * p.y_stride;
    uint32_t xb[KJ];
    key_load<DT, KJ>(yr + p.D, p.R, nj, lane, xb);
    S* orow = (S*)p.out + tok * (int64_t)p.D;
    for (int v = lane; v < nv; v += kWave) {
      Raw<DT, E> t;
      load_raw<DT, E, true>(yr + v * E, t);
      float f[E];
      unpack<DT, E>(t, f);
      store_vec<DT, E, true>(orow + v * E, f);
    }
    float x[KJ];
    key_floats<DT, KJ>(xb, p.R, nj, lane, x);
    S* krow = (S*)p.key + tok * (int64_t)p.R;
    if (p.key_norm) {
      float sq[KJ], ss[KJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j) sq[j] = x[j] * x[j];
      head_sums<KJ>(p, sq, ss);
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int r = lane + j * kWave;
        const float inv = 1.0f / sqrtf(ss[j] / (float)p.hd + p.eps);
        if (r < p.R) {
          DT::store1(krow + r, x[j] * inv);
          if (r % p.hd == 0) p.inv[tok * p.H + r / p.hd] = inv;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) DT::store1(krow + r, x[j]);
      }
    }
  }
}

template <class DT, int E, int KJ>
__global__ void __launch_bounds__(256) keyed_split_bwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  const int nj = (p.R + kWave - 1) / kWave;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    S* gyr = (S*)p.gy + tok * (int64_t)p.P;
    // key loads first (raw bits), then the output columns
    const S* gkr = p.gkey ? (const S*)p.gkey + tok * (int64_t)p.R : nullptr;
    const bool norm_bwd = p.key_norm && gkr;
    uint32_t gb[KJ], xb[KJ];
    float inv[KJ];
    if (gkr) key_load<DT, KJ>(gkr, p.R, nj, lane, gb);
    if (norm_bwd) {
      key_load<DT, KJ>((const S*)p.y + tok * p.y_stride + p.D, p.R, nj, lane, xb);
      key_inv_load<KJ>(p, tok, nj, lane, inv);
    }
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
    float g[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) g[j] = 0.f;
    if (gkr) key_floats<DT, KJ>(gb, p.R, nj, lane, g);
    if (norm_bwd) {
      float x[KJ], gx[KJ], dot[KJ];
      key_floats<DT, KJ>(xb, p.R, nj, lane, x);
#pragma unroll
      for (int j = 0; j < KJ; ++j) gx[j] = g[j] * x[j];
      head_sums<KJ>(p, gx, dot);
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) {
          const float k3 = inv[j] * inv[j] * inv[j] * (dot[j] / (float)p.hd);
          DT::store1(gyr + p.D + r, inv[j] * g[j] - x[j] * k3);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
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

// Rows of up to AV vectors per lane (AV = 2 or 4: D <= 1024 or 2048 for 16-bit
// types; AV = 0: a loop over the row) are held in registers: every load of a
// token -- key, partial key, y[:D], partial value -- is issued before the first
// store.  The stores may alias the loads as far as
// the compiler knows, so it would otherwise keep each load behind the previous
// store and serialise a token into several memory round trips.  Longer rows
// take a loop over the row (twice for the value norm).
template <class DT, int E, int AV>
struct AccRow {  // raw bits of the lane's vectors of y[:D] and of the partial value
  Raw<DT, E> y[AV > 0 ? AV : 1], pv[AV > 0 ? AV : 1];
};

// issue the loads of the lane's vectors (c < nc); lanes past the row's end
// re-read its last vector (a cache hit) and drop the result
template <class DT, int E, int AV>
__device__ __forceinline__ void acc_row_load(const typename DT::S* yr, const typename DT::S* pvr, int nv, int nc,
                                             int lane, AccRow<DT, E, AV>& a) {
#pragma unroll
  for (int c = 0; c < AV; ++c) {
    if (c < nc) {
      const int v = min(lane + c * kWave, nv - 1);
      load_raw<DT, E, true>(yr + v * E, a.y[c]);
      if (pvr) load_raw<DT, E, true>(pvr + v * E, a.pv[c]);
    }
  }
}

// vector c of the grown partial value pv + y[:D] from the loaded bits
template <class DT, int E, int AV>
__device__ __forceinline__ void acc_row_grown(const AccRow<DT, E, AV>& a, bool has_pv, int c, float (&f)[E]) {
  unpack<DT, E>(a.y[c], f);
  if (has_pv) {
    float b[E];
    unpack<DT, E>(a.pv[c], b);
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = DT::rnd(b[e] + f[e]);
  }
}

// row v (E elements) of the grown partial value for token tok: pv + y[:D] (long rows)
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

template <class DT, int E, int AV, int KJ>
__global__ void __launch_bounds__(256) block_accum_fwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int nc = (nv + kWave - 1) / kWave;  // the host launches AV > 0 only for nc <= AV
  constexpr bool resident = AV > 0;
  const int nj = (p.R + kWave - 1) / kWave;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  const bool complete = p.accum == 2;
  const bool vnorm = complete && p.value_norm;
  const float s = complete ? summary_scale<DT>(p.scale_dev, p.vscale) : 1.f;
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    const S* yr = (const S*)p.y + tok * p.y_stride;
    const S* pvr = p.pv ? (const S*)p.pv + tok * (int64_t)p.D : nullptr;
    const S* pkr = p.pk ? (const S*)p.pk + tok * (int64_t)p.R : nullptr;
    // ---- every load of the token
    uint32_t xb[KJ], pb[KJ];
    key_load<DT, KJ>(yr + p.D, p.R, nj, lane, xb);
    if (pkr) key_load<DT, KJ>(pkr, p.R, nj, lane, pb);
    AccRow<DT, E, AV> a;
    if constexpr (resident) acc_row_load<DT, E, AV>(yr, pvr, nv, nc, lane, a);
    // ---- key: split (and per-head norm), + partial key, (* s)
    float x[KJ], pkv[KJ], k[KJ];
    key_floats<DT, KJ>(xb, p.R, nj, lane, x);
    if (pkr) key_floats<DT, KJ>(pb, p.R, nj, lane, pkv);
#pragma unroll
    for (int j = 0; j < KJ; ++j) k[j] = x[j];
    if (p.key_norm) {
      float sq[KJ], ss[KJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j) sq[j] = x[j] * x[j];
      head_sums<KJ>(p, sq, ss);
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int r = lane + j * kWave;
        const float inv = 1.0f / sqrtf(ss[j] / (float)p.hd + p.eps);
        k[j] = DT::rnd(x[j] * inv);
        if (r < p.R && r % p.hd == 0 && p.inv) p.inv[tok * p.H + r / p.hd] = inv;
      }
    }
    S* krow = (S*)p.key + tok * (int64_t)p.R;
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int r = lane + j * kWave;
      if (r < p.R) {
        float kv = pkr ? DT::rnd(pkv[j] + k[j]) : k[j];
        if (complete && !vnorm && p.scale_key) kv = DT::rnd(kv * s);
        DT::store1(krow + r, kv);
      }
    }
    // ---- value: y[:D] + partial value, (* s or rms-normed)
    S* orow = (S*)p.out + tok * (int64_t)p.D;
    if constexpr (resident) {
      float f[AV][E];
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < AV; ++c) {
        if (c < nc) {
          acc_row_grown<DT, E, AV>(a, pvr != nullptr, c, f[c]);
          if (vnorm && lane + c * kWave < nv) {
#pragma unroll
            for (int e = 0; e < E; ++e) ss += f[c][e] * f[c][e];
          }
        }
      }
      float inv_v = 1.f;
      if (vnorm) {
        inv_v = 1.0f / sqrtf(wave_sum(ss) / (float)p.D + p.eps);
        if (lane == 0 && p.vinv) p.vinv[tok] = inv_v;
      }
#pragma unroll
      for (int c = 0; c < AV; ++c) {
        const int v = lane + c * kWave;
        if (c < nc && v < nv) {
          if (vnorm) {
#pragma unroll
            for (int e = 0; e < E; ++e) f[c][e] = DT::rnd(f[c][e] * inv_v);
          } else if (complete) {
#pragma unroll
            for (int e = 0; e < E; ++e) f[c][e] = DT::rnd(f[c][e] * s);
          }
          store_vec<DT, E, true>(orow + v * E, f[c]);
        }
      }
      continue;
    }
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

// the gradient of the grown value's vector from its upstream gradient g (in place):
// rms-norm backward, or the scale (adding rnd(g * value) to the scale's gradient)
template <class DT, int E>
__device__ __forceinline__ void grown_grad(bool vnorm, bool complete, bool want_ds, float s, float inv_v, float k3,
                                           const float (&f)[E], float (&g)[E], float& acc_v) {
  if (vnorm) {
#pragma unroll
    for (int e = 0; e < E; ++e) g[e] = DT::rnd(inv_v * g[e] - f[e] * k3);
  } else if (complete) {
    if (want_ds) {
#pragma unroll
      for (int e = 0; e < E; ++e) acc_v += DT::rnd(g[e] * f[e]);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) g[e] = DT::rnd(g[e] * s);
  }
}

// G: the grown value may be read back (value norm or a learned scale's gradient);
// without it the kernel keeps fewer registers
template <class DT, int E, int AV, int KJ, bool G>
__global__ void __launch_bounds__(256) block_accum_bwd_kernel(const KeySplitParams p) {
  using S = typename DT::S;
  __shared__ float s_fold[2 * 16];  // two sums per wave (at most 16 waves)
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave, wpb = blockDim.x / kWave;
  const int nv = p.D / E;
  const int nc = (nv + kWave - 1) / kWave;  // the host launches AV > 0 only for nc <= AV
  constexpr bool resident = AV > 0;
  const int nj = (p.R + kWave - 1) / kWave;
  const int64_t stride = (int64_t)gridDim.x * wpb;
  const bool complete = p.accum == 2;
  const bool vnorm = G && complete && p.value_norm;
  const float s = complete ? summary_scale<DT>(p.scale_dev, p.vscale) : 1.f;
  const bool want_ds = G && complete && !vnorm && p.partials;
  const bool key_ds = want_ds && p.scale_key && p.gkey;
  // the grown value is read back only for the norm's backward or the scale's gradient
  const bool need_grown = p.gout && (vnorm || want_ds);
  float acc_v = 0.f, acc_k = 0.f;  // learned-scale gradient: sum of rnd(g * grown value / key)
  for (int64_t tok = (int64_t)blockIdx.x * wpb + wave; tok < p.n_tok; tok += stride) {
    const S* yr = (const S*)p.y + tok * p.y_stride;
    const S* pvr = p.pv ? (const S*)p.pv + tok * (int64_t)p.D : nullptr;
    const S* pkr = p.pk ? (const S*)p.pk + tok * (int64_t)p.R : nullptr;
    const S* gor = p.gout ? (const S*)p.gout + tok * p.gout_stride : nullptr;
    const S* gkr = p.gkey ? (const S*)p.gkey + tok * (int64_t)p.R : nullptr;
    S* gyr = (S*)p.gy + tok * (int64_t)p.P;
    // ---- every load of the token
    uint32_t xb[KJ], gb[KJ], pb[KJ];
    float inv[KJ];
    key_load<DT, KJ>(yr + p.D, p.R, nj, lane, xb);
    if (gkr) key_load<DT, KJ>(gkr, p.R, nj, lane, gb);
    if (key_ds && pkr) key_load<DT, KJ>(pkr, p.R, nj, lane, pb);
    key_inv_load<KJ>(p, tok, nj, lane, inv);
    Raw<DT, E> graw[AV > 0 ? AV : 1];
    AccRow<DT, E, AV> a;
    if constexpr (resident) {
      if (gor) {
#pragma unroll
        for (int c = 0; c < AV; ++c)
          if (c < nc) load_raw<DT, E, true>(gor + min(lane + c * kWave, nv - 1) * E, graw[c]);
      }
      if (need_grown) acc_row_load<DT, E, AV>(yr, pvr, nv, nc, lane, a);
    }
    const float inv_v = (vnorm && gor) ? p.vinv[tok] : 1.f;  // the host requires vinv with a value gradient
    float x[KJ], g[KJ], pkv[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) g[j] = pkv[j] = 0.f;
    key_floats<DT, KJ>(xb, p.R, nj, lane, x);
    if (gkr) key_floats<DT, KJ>(gb, p.R, nj, lane, g);
    if (key_ds && pkr) key_floats<DT, KJ>(pb, p.R, nj, lane, pkv);
    // ---- value columns: the grown partial value's gradient
    if constexpr (resident) {
      float gv[AV][E], f[AV][E];
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < AV; ++c) {
        if (c < nc) {
          if (gor) {
            unpack<DT, E>(graw[c], gv[c]);
          } else {
#pragma unroll
            for (int e = 0; e < E; ++e) gv[c][e] = 0.f;
          }
          if (need_grown) {
            acc_row_grown<DT, E, AV>(a, pvr != nullptr, c, f[c]);
          } else {
#pragma unroll
            for (int e = 0; e < E; ++e) f[c][e] = 0.f;
          }
          if (lane + c * kWave >= nv) {  // a re-read vector: contributes nothing
#pragma unroll
            for (int e = 0; e < E; ++e) gv[c][e] = 0.f;
          }
          if (vnorm) {
#pragma unroll
            for (int e = 0; e < E; ++e) dot += gv[c][e] * f[c][e];
          }
        }
      }
      const float k3 = vnorm && gor ? inv_v * inv_v * inv_v * (wave_sum(dot) / (float)p.D) : 0.f;
#pragma unroll
      for (int c = 0; c < AV; ++c) {
        const int v = lane + c * kWave;
        if (c < nc && v < nv) {
          grown_grad<DT, E>(vnorm && gor, complete, want_ds, s, inv_v, k3, f[c], gv[c], acc_v);
          store_vec<DT, E, true>(gyr + v * E, gv[c]);
        }
      }
    } else {
      float dot = 0.f;
      if (vnorm && gor) {  // rms-norm backward needs <g, x> over the row first
        for (int v = lane; v < nv; v += kWave) {
          float f[E], gg[E];
          grown_value<DT, E>(p, yr, pvr, v, f);
          load_vec<DT, E, true>(gor + v * E, gg);
#pragma unroll
          for (int e = 0; e < E; ++e) dot += gg[e] * f[e];
        }
        dot = wave_sum(dot);
      }
      const float k3 = inv_v * inv_v * inv_v * (dot / (float)p.D);
      for (int v = lane; v < nv; v += kWave) {
        float gg[E], f[E];
        if (gor) {
          load_vec<DT, E, true>(gor + v * E, gg);
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) gg[e] = 0.f;
        }
        if (need_grown) {
          grown_value<DT, E>(p, yr, pvr, v, f);
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) f[e] = 0.f;
        }
        grown_grad<DT, E>(vnorm && gor, complete, want_ds, s, inv_v, k3, f, gg, acc_v);
        store_vec<DT, E, true>(gyr + v * E, gg);
      }
    }
    // ---- key columns
    if (complete && !vnorm && p.scale_key) {
      // key = rnd(grown key * s): the grown key's gradient is rnd(g * s)
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int r = lane + j * kWave;
        if (key_ds && r < p.R) {
          const float kt = p.key_norm ? DT::rnd(x[j] * inv[j]) : x[j];
          const float kg = pkr ? DT::rnd(pkv[j] + kt) : kt;
          acc_k += DT::rnd(g[j] * kg);
        }
        g[j] = DT::rnd(g[j] * s);
        if (r < p.R && p.dpk) DT::store1((S*)p.dpk + tok * (int64_t)p.R + r, g[j]);
      }
    }
    if (p.key_norm) {
      float gx[KJ], kd[KJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j) gx[j] = g[j] * x[j];
      head_sums<KJ>(p, gx, kd);
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        const int r = lane + j * kWave;
        if (r < p.R) {
          const float k3k = inv[j] * inv[j] * inv[j] * (kd[j] / (float)p.hd);
          DT::store1(gyr + p.D + r, inv[j] * g[j] - x[j] * k3k);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
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

template <class DT, int KJ>
static hipError_t keyed_split_t(bool bwd, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  const dim3 g(L.grid), b(L.teams * kWave);
  if (p.accum) {
    // vectors per lane of a value row: up to 2 or 4 (held in registers) or more (a loop)
    const int nc = (p.D / (L.vec ? EV : 1) + kWave - 1) / kWave;
    if (bwd && p.accum == 2 && (p.value_norm || p.partials)) {
      if (L.vec && nc <= 2) hipLaunchKernelGGL((block_accum_bwd_kernel<DT, EV, 2, KJ, true>), g, b, 0, st, p);
      else if (L.vec) hipLaunchKernelGGL((block_accum_bwd_kernel<DT, EV, 0, KJ, true>), g, b, 0, st, p);
      else hipLaunchKernelGGL((block_accum_bwd_kernel<DT, 1, 0, KJ, true>), g, b, 0, st, p);
    } else if (bwd) {
      if (L.vec && nc <= 2) hipLaunchKernelGGL((block_accum_bwd_kernel<DT, EV, 2, KJ, false>), g, b, 0, st, p);
      else if (L.vec && nc <= 4) hipLaunchKernelGGL((block_accum_bwd_kernel<DT, EV, 4, KJ, false>), g, b, 0, st, p);
      else if (L.vec) hipLaunchKernelGGL((block_accum_bwd_kernel<DT, EV, 0, KJ, false>), g, b, 0, st, p);
      else hipLaunchKernelGGL((block_accum_bwd_kernel<DT, 1, 0, KJ, false>), g, b, 0, st, p);
    } else {
      if (L.vec && nc <= 2) hipLaunchKernelGGL((block_accum_fwd_kernel<DT, EV, 2, KJ>), g, b, 0, st, p);
      else if (L.vec && nc <= 4) hipLaunchKernelGGL((block_accum_fwd_kernel<DT, EV, 4, KJ>), g, b, 0, st, p);
      else if (L.vec) hipLaunchKernelGGL((block_accum_fwd_kernel<DT, EV, 0, KJ>), g, b, 0, st, p);
      else hipLaunchKernelGGL((block_accum_fwd_kernel<DT, 1, 0, KJ>), g, b, 0, st, p);
    }
  } else if (bwd) {
    if (L.vec) hipLaunchKernelGGL((keyed_split_bwd_kernel<DT, EV, KJ>), g, b, 0, st, p);
    else hipLaunchKernelGGL((keyed_split_bwd_kernel<DT, 1, KJ>), g, b, 0, st, p);
  } else {
    if (L.vec) hipLaunchKernelGGL((keyed_split_fwd_kernel<DT, EV, KJ>), g, b, 0, st, p);
    else hipLaunchKernelGGL((keyed_split_fwd_kernel<DT, 1, KJ>), g, b, 0, st, p);
  }
  return hipGetLastError();
}

template <int KJ>
static hipError_t keyed_split_kj(int dtype, bool bwd, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return keyed_split_t<F32, KJ>(bwd, p, L, st);
    case ATTNRES_DTYPE_BF16: return keyed_split_t<BF16, KJ>(bwd, p, L, st);
    default: return keyed_split_t<F16, KJ>(bwd, p, L, st);
  }
}

static hipError_t keyed_split(int dtype, bool bwd, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  const int nj = (p.R + kWave - 1) / kWave;  // the host keeps R <= 256
  if (nj <= 1) return keyed_split_kj<1>(dtype, bwd, p, L, st);
  if (nj <= 2) return keyed_split_kj<2>(dtype, bwd, p, L, st);
  return keyed_split_kj<4>(dtype, bwd, p, L, st);
}

hipError_t launch_keyed_split_forward(int dtype, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  return keyed_split(dtype, false, p, L, st);
}
hipError_t launch_keyed_split_backward(int dtype, const KeySplitParams& p, const Launch& L, hipStream_t st) {
  return keyed_split(dtype, true, p, L, st);
}

}  // namespace attnres
