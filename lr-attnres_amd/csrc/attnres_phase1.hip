// Phase 1 of the cached-logit block-training schedule: one read of the S
// completed block summaries serves Q upcoming read sites whose logits were
// computed ahead.  Forward and backward.
//
// Semantics follow the reference's eager op (attnres_ops.py:3956-3961):
//   w[q, s]  = softmax_s(float(logits[q, s, t]))          (fp32)
//   out[q]   = rnd(sum_s rnd(w[q, s]) * v[s])             (fp32 accumulate)
//   lse[q]   = max_s l + log(sum_s exp(l - max))          (fp32)
//   optional out[q] = rnd(out[q] / rms(out[q]))
// and the backward of that graph: dW = rnd(<g[q], v[s]>) (a dtype
// contraction), dl = w * (dW - sum_s w * dW) + glse * w (fp32; summed in the
// logits dtype when that is not fp32, as autograd adds the two branches),
// dv[s] = rnd(sum_q rnd(w[q, s]) * g[q]).
//
// One workgroup of wpt waves owns one token at a time; each lane owns CB
// vectors of E elements of the D-wide rows.  Forward: every wave computes the
// token's softmax rows itself in a (site, source) lane layout and reads its
// weights back from its own LDS region (no workgroup barrier unless the output
// is normed), and the next token's value rows are loaded before this token's
// stores.  Backward: wave 0 computes the softmax rows while the other waves'
// loads are in flight; the per-wave partial dots meet in LDS (double-buffered
// by token parity, so one barrier per token suffices).
#include "attnres_block.h"
#include "attnres_device.h"
#include "attnres_launch.h"
#include "attnres_params.h"

namespace attnres {

constexpr int kP1QC = 8;  // read sites accumulated per pass of the forward
constexpr int kP1SC = 8;  // source rows loaded per batch

// Softmax rows of one token by one wave: lane = site * np + source, np lanes
// per site (np = next power of two >= S), 64 / np sites per round.  Writes the
// fp32 weights to w[q * S + s] and, when asked, lse[q * n_tok + tok].
__device__ __forceinline__ void phase1_softmax(const Phase1Params& p, int64_t tok, int lane, float* w,
                                               bool write_lse) {
  const int N = p.n_src, Q = p.n_q, np = p.np, qpr = kWave / np;
  const int sl = lane & (np - 1), ql = lane / np;
  for (int q0 = 0; q0 < Q; q0 += qpr) {
    const int q = q0 + ql;
    const bool ok = sl < N && q < Q;
    const float l = ok ? p1_logit(p, q, sl, tok) : -INFINITY;
    const float m = group_max(l, np);
    const float e = ok ? expf(l - m) : 0.f;
    const float z = group_sum(e, np);
    if (ok) w[q * N + sl] = e / z;
    if (write_lse && ok && sl == 0) p.lse[(int64_t)q * p.n_tok + tok] = m + logf(z);
  }
}

template <class DT, int E, int CB>
__device__ __forceinline__ void phase1_load_rows(const Phase1Params& p, int64_t tok, int s0,
                                                 Raw<DT, E> (&r)[kP1SC][CB], const Cols<CB, E>& cl) {
  using S = typename DT::S;
#pragma unroll
  for (int j = 0; j < kP1SC; ++j) {
    if (s0 + j < p.n_src) {
      const S* vp = (const S*)p.val[s0 + j] + tok * (int64_t)p.vstride[s0 + j];
#pragma unroll
      for (int c = 0; c < CB; ++c)
        if (cl.ok[c]) load_raw<DT, E, true>(vp + cl.eoff[c], r[j][c]);
    }
  }
}

// ============================================================== forward
// QC read sites accumulate per pass over the source rows (kP1QC; 4 when a
// lane holds three columns, to stay within the register budget)
template <class DT, int E, int CB, int QC = kP1QC>
__global__ void __launch_bounds__(512) phase1_fwd_kernel(const Phase1Params p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  const int N = p.n_src, Q = p.n_q, D = p.D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  float* w = smem + wave * Q * N;    // this wave's weights [Q * N]
  float* s_red = smem + wpt * Q * N;  // [wpt * QC]
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);

  Raw<DT, E> r[kP1SC][CB];
  if ((int64_t)blockIdx.x < p.n_tok) phase1_load_rows<DT, E, CB>(p, blockIdx.x, 0, r, cl);
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    // every wave computes the token's softmax rows itself: no workgroup
    // barrier (the first batch of value rows is already in flight)
    phase1_softmax(p, tok, lane, w, wave == 0);
    wave_sync();

    for (int q0 = 0; q0 < Q; q0 += QC) {
      float acc[QC][CB][E];
#pragma unroll
      for (int qq = 0; qq < QC; ++qq)
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) acc[qq][c][e] = 0.f;
      for (int s0 = 0; s0 < N; s0 += kP1SC) {
        if (s0 > 0 || q0 > 0) phase1_load_rows<DT, E, CB>(p, tok, s0, r, cl);
#pragma unroll
        for (int j = 0; j < kP1SC; ++j) {
          if (s0 + j < N) {
            float v[CB][E];
#pragma unroll
            for (int c = 0; c < CB; ++c) unpack<DT, E>(r[j][c], v[c]);
#pragma unroll
            for (int qq = 0; qq < QC; ++qq) {
              if (q0 + qq < Q) {
                const float wq = DT::rnd(w[(q0 + qq) * N + s0 + j]);
#pragma unroll
                for (int c = 0; c < CB; ++c)
#pragma unroll
                  for (int e = 0; e < E; ++e) acc[qq][c][e] += wq * v[c][e];
              }
            }
          }
        }
      }
      // the next token's first batch of value rows goes out before this
      // token's stores
      if (q0 + QC >= Q && tok + gridDim.x < p.n_tok) phase1_load_rows<DT, E, CB>(p, tok + gridDim.x, 0, r, cl);
      float ss[QC];
#pragma unroll
      for (int qq = 0; qq < QC; ++qq) {
        ss[qq] = 0.f;
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) {
            acc[qq][c][e] = DT::rnd(acc[qq][c][e]);
            if (cl.ok[c]) ss[qq] += acc[qq][c][e] * acc[qq][c][e];
          }
      }
      const int nq = Q - q0 < QC ? Q - q0 : QC;
      if (p.norm_out) {
#pragma unroll
        for (int qq = 0; qq < QC; ++qq) {
          if (qq < nq && p.out_prenorm) {
            S* xp = (S*)p.out_prenorm + ((int64_t)(q0 + qq) * p.n_tok + tok) * D;
#pragma unroll
            for (int c = 0; c < CB; ++c)
              if (cl.ok[c]) store_vec<DT, E, true>(xp + cl.eoff[c], acc[qq][c]);
          }
        }
        block_allreduce<QC>(ss, nq, s_red, lane, wave, wpt);
#pragma unroll
        for (int qq = 0; qq < QC; ++qq) {
          if (qq < nq) {
            const float inv = 1.0f / sqrtf(ss[qq] / (float)D + p.eps);
#pragma unroll
            for (int c = 0; c < CB; ++c)
#pragma unroll
              for (int e = 0; e < E; ++e) acc[qq][c][e] = DT::rnd(acc[qq][c][e] * inv);
            if (tid == 0 && p.out_inv_rms) p.out_inv_rms[(int64_t)(q0 + qq) * p.n_tok + tok] = inv;
          }
        }
      }
#pragma unroll
      for (int qq = 0; qq < QC; ++qq) {
        if (qq < nq) {
          S* op = (S*)p.out + ((int64_t)(q0 + qq) * p.n_tok + tok) * D;
#pragma unroll
          for (int c = 0; c < CB; ++c)
            if (cl.ok[c]) store_vec<DT, E, true>(op + cl.eoff[c], acc[qq][c]);
        }
      }
    }
    wave_sync();  // this token's weights are read before the next token writes them
  }
}

// ============================================================== backward
// QMAX register slots for the Q upstream gradient rows (kept packed).
template <class DT, int E, int CB, int QMAX>
__global__ void __launch_bounds__(512) phase1_bwd_kernel(const Phase1Params p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  const int N = p.n_src, Q = p.n_q, D = p.D, QN = p.n_q * p.n_src;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;
  float* s_w = smem;                   // [2][Q * N] weights
  float* s_dw = smem + 2 * QN;         // [2][wpt][Q * N] per-wave partial dots
  float* s_red = s_dw + 2 * wpt * QN;  // [wpt * QMAX]
  const Cols<CB, E> cl(p.ncols, D, lane, wave, wpt);

  Raw<DT, E> r[kP1SC][CB];
  if ((int64_t)blockIdx.x < p.n_tok) phase1_load_rows<DT, E, CB>(p, blockIdx.x, 0, r, cl);
  int par = 0;
  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x, par ^= 1) {
    float* w = s_w + par * QN;
    float* dwp = s_dw + par * wpt * QN;
    Raw<DT, E> gr[QMAX][CB];
#pragma unroll
    for (int q = 0; q < QMAX; ++q) {
      if (q < Q) {
        const S* gp = (const S*)p.gout[q] + tok * (int64_t)D;
#pragma unroll
        for (int c = 0; c < CB; ++c)
          if (cl.ok[c]) load_raw<DT, E, true>(gp + cl.eoff[c], gr[q][c]);
      }
    }
    if (wave == 0) phase1_softmax(p, tok, lane, w, false);

    if (p.norm_out) {
      // g <- rms-norm backward of each site's output from its pre-norm row x:
      // rnd(inv * g - x * inv^3 * mean(g * x))
      Raw<DT, E> xr[QMAX][CB];
      float dot[QMAX];
#pragma unroll
      for (int q = 0; q < QMAX; ++q) {
        dot[q] = 0.f;
        if (q < Q) {
          const S* xp = (const S*)p.out_prenorm + ((int64_t)q * p.n_tok + tok) * D;
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            if (cl.ok[c]) {
              load_raw<DT, E, true>(xp + cl.eoff[c], xr[q][c]);
              float g[E], x[E];
              unpack<DT, E>(gr[q][c], g);
              unpack<DT, E>(xr[q][c], x);
#pragma unroll
              for (int e = 0; e < E; ++e) dot[q] += g[e] * x[e];
            }
          }
        }
      }
      block_allreduce<QMAX>(dot, Q, s_red, lane, wave, wpt);
#pragma unroll
      for (int q = 0; q < QMAX; ++q) {
        if (q < Q) {
          const float inv = p.out_inv_rms[(int64_t)q * p.n_tok + tok];
          const float k3 = inv * inv * inv * (dot[q] / (float)D);
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            if (cl.ok[c]) {
              float g[E], x[E];
              unpack<DT, E>(gr[q][c], g);
              unpack<DT, E>(xr[q][c], x);
#pragma unroll
              for (int e = 0; e < E; ++e) g[e] = DT::rnd(inv * g[e] - x[e] * k3);
              pack_raw<DT, E>(g, gr[q][c]);
            }
          }
        }
      }
    }

    // per-wave partial dots <g[q], v[s]>
    for (int s0 = 0; s0 < N; s0 += kP1SC) {
      if (s0 > 0) phase1_load_rows<DT, E, CB>(p, tok, s0, r, cl);
#pragma unroll
      for (int j = 0; j < kP1SC; ++j) {
        if (s0 + j < N) {
          float v[CB][E];
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            if (cl.ok[c]) unpack<DT, E>(r[j][c], v[c]);
            else
#pragma unroll
              for (int e = 0; e < E; ++e) v[c][e] = 0.f;
          }
#pragma unroll
          for (int q = 0; q < QMAX; ++q) {
            if (q < Q) {
              float d = 0.f;
#pragma unroll
              for (int c = 0; c < CB; ++c) {
                if (cl.ok[c]) {
                  float g[E];
                  unpack<DT, E>(gr[q][c], g);
#pragma unroll
                  for (int e = 0; e < E; ++e) d += g[e] * v[c][e];
                }
              }
              d = wave_sum(d);
              if (lane == 0) dwp[wave * QN + q * N + s0 + j] = d;
            }
          }
        }
      }
    }
    // the next token's first batch of value rows is in flight during the
    // logits and value gradients of this one
    if (tok + gridDim.x < p.n_tok) phase1_load_rows<DT, E, CB>(p, tok + gridDim.x, 0, r, cl);
    __syncthreads();

    if (wave == 0) {
      // logits gradient in the (site, source) lane layout
      const int np = p.np, qpr = kWave / np;
      const int sl = lane & (np - 1), ql = lane / np;
      for (int q0 = 0; q0 < Q; q0 += qpr) {
        const int q = q0 + ql;
        const bool ok = sl < N && q < Q;
        float dw = 0.f, wt = 0.f;
        if (ok) {
          for (int k = 0; k < wpt; ++k) dw += dwp[k * QN + q * N + sl];
          wt = w[q * N + sl];
        }
        const float dwb = DT::rnd(dw);  // gradient of the dtype-rounded weights
        const float inner = group_sum(wt * dwb, np);
        float dl = wt * (dwb - inner);
        dl = p1_dlogit(p, dl, ok ? p1_glse(p, q, tok) * wt : 0.f);
        if (ok) p1_store_dlogit(p, q, sl, tok, dl);
      }
    }

    // value gradients
    for (int s = 0; s < N; ++s) {
      float acc[CB][E];
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[c][e] = 0.f;
#pragma unroll
      for (int q = 0; q < QMAX; ++q) {
        if (q < Q) {
          const float wq = DT::rnd(w[q * N + s]);
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            float g[E];
            unpack<DT, E>(gr[q][c], g);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[c][e] += wq * g[e];
          }
        }
      }
      S* dp = (S*)p.dval[s] + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (cl.ok[c]) {
#pragma unroll
          for (int e = 0; e < E; ++e) acc[c][e] = DT::rnd(acc[c][e]);
          store_vec<DT, E, true>(dp + cl.eoff[c], acc[c]);
        }
      }
    }
  }
}

// ============================================================== launchers
// Vector path: one 16-byte vector per column (fp32: two columns per lane);
// unaligned rows: eight single-element columns per lane.
// 16-bit rows of 256 / 768 elements: one wave of 8-byte vectors, one or three
// columns per lane.
template <class DT>
static hipError_t phase1_fwd_dt(const Phase1Params& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  constexpr int CBV = sizeof(typename DT::S) == 4 ? 2 : 1;
  if constexpr (sizeof(typename DT::S) == 2) {
    if (L.vec && L.vb == 8) {
      if (p.ncols == 1)
        hipLaunchKernelGGL((phase1_fwd_kernel<DT, EV / 2, 1>), dim3(L.grid), dim3(kWave), L.lds, st, p);
      else
        hipLaunchKernelGGL((phase1_fwd_kernel<DT, EV / 2, 3, 4>), dim3(L.grid), dim3(kWave), L.lds, st, p);
      return hipGetLastError();
    }
  }
  if (L.vec)
    hipLaunchKernelGGL((phase1_fwd_kernel<DT, EV, CBV>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  else
    hipLaunchKernelGGL((phase1_fwd_kernel<DT, 1, 8>), dim3(L.grid), dim3(L.wpt * kWave), L.lds, st, p);
  return hipGetLastError();
}

template <class DT>
static hipError_t phase1_bwd_dt(const Phase1Params& p, const Launch& L, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  constexpr int CBV = sizeof(typename DT::S) == 4 ? 2 : 1;
  const dim3 g(L.grid), b(L.wpt * kWave);
  if constexpr (sizeof(typename DT::S) == 2) {
    if (L.vec && L.vb == 8) {
      if (p.ncols == 1) {
        if (L.nmax <= 4) hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV / 2, 1, 4>), g, b, L.lds, st, p);
        else if (L.nmax <= 8) hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV / 2, 1, 8>), g, b, L.lds, st, p);
        else hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV / 2, 1, kPhase1MaxQ>), g, b, L.lds, st, p);
      } else {
        // three columns: the host picks this layout for at most 4 sites
        if (L.nmax > 4) return hipErrorInvalidValue;
        hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV / 2, 3, 4>), g, b, L.lds, st, p);
      }
      return hipGetLastError();
    }
  }
  if (L.vec) {
    if (L.nmax <= 4) hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV, CBV, 4>), g, b, L.lds, st, p);
    else if (L.nmax <= 8) hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV, CBV, 8>), g, b, L.lds, st, p);
    else hipLaunchKernelGGL((phase1_bwd_kernel<DT, EV, CBV, kPhase1MaxQ>), g, b, L.lds, st, p);
  } else {
    if (L.nmax <= 4) hipLaunchKernelGGL((phase1_bwd_kernel<DT, 1, 8, 4>), g, b, L.lds, st, p);
    else if (L.nmax <= 8) hipLaunchKernelGGL((phase1_bwd_kernel<DT, 1, 8, 8>), g, b, L.lds, st, p);
    else hipLaunchKernelGGL((phase1_bwd_kernel<DT, 1, 8, kPhase1MaxQ>), g, b, L.lds, st, p);
  }
  return hipGetLastError();
}

#define ATTNRES_P1_DISPATCH(dtype, fn, ...)                \
  switch (dtype) {                                         \
    case ATTNRES_DTYPE_F32: return fn<F32>(__VA_ARGS__);   \
    case ATTNRES_DTYPE_BF16: return fn<BF16>(__VA_ARGS__); \
    default: return fn<F16>(__VA_ARGS__);                  \
  }

hipError_t launch_phase1_forward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st) {
  ATTNRES_P1_DISPATCH(dtype, phase1_fwd_dt, p, L, st);
}
hipError_t launch_phase1_backward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st) {
  ATTNRES_P1_DISPATCH(dtype, phase1_bwd_dt, p, L, st);
}

}  // namespace attnres
