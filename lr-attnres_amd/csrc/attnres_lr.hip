// LR AttnRes read: low-rank keys, multi-head depth softmax, forward and backward.
//
// Semantics follow the reference's eager op (attnres_ops.py:4163-4192) with its
// rounding points mirrored: keys are rms-normed per head in fp32 and rounded to
// the tensor dtype, logits are a dtype-rounded contraction times the scale
// (rounded again) plus an fp32 bias, the softmax is fp32 and the mix uses the
// dtype-rounded weights with fp32 accumulation.
//
// Work decomposition (one workgroup = one token at a time, persistent over
// tokens):
//   phase A  one thread per (head, source) pair scores its key slice
//   phase B  the same pairs turn logits into softmax weights (saved as fp32)
//   phase C  each wave streams its columns of the N value rows (16-byte loads,
//            up to 8 sources x CB columns in flight per lane) and mixes them
// The backward streams the value rows once more: dW partials and dv = w*g are
// produced in the same pass, dW is reduced per (head, source) through LDS, and
// the key/query chain runs on the (head, source) pairs.  Cross-token sums
// (static query, per-site gate, bias) go to per-workgroup partials that
// attnres_reduce_partials_kernel folds in a fixed order: no atomics.
#include "attnres_device.h"
#include "attnres_params.h"
#include "attnres_launch.h"

namespace attnres {

constexpr int kSrcGroup = 8;

// Keys are read through the key dtype (p.kdt) and the logit path -- query,
// rounded keys, logits and their gradients -- is rounded in the logit dtype
// (p.ldt).  Both equal the value dtype unless keys of another dtype are read
// (the reference norms such keys in fp32 and rounds them to the value dtype:
// attnres_ops.py:4179-4186); the fast kernels handle only equal dtypes.
__host__ __device__ __forceinline__ int dtype_bytes(int code) { return code == 0 ? 4 : 2; }

// query element j of head h for token tok (fp32 of a logit-dtype value;
// composed queries are rounded to that dtype, as the reference casts the
// composed query)
template <class DT>
struct QueryView {
  const void* qs;
  const void* qd;
  int ldt;
  float gf;
  __device__ __forceinline__ float at(int j) const {
    float q = qs ? load_any(qs, j, ldt) : 0.f;
    if (qd) q = round_any(q + gf * load_any(qd, j, ldt), ldt);
    return q;
  }
};

template <class DT>
__device__ __forceinline__ QueryView<DT> query_view(const ReadParams& p, int64_t tok, int h) {
  using S = typename DT::S;
  const int qb = dtype_bytes(p.ldt);
  QueryView<DT> v;
  v.qs = p.q_static ? (const char*)p.q_static + (int64_t)h * p.rh * qb : nullptr;
  v.qd = p.q_dyn ? (const char*)p.q_dyn + (tok * p.q_dyn_stride + (int64_t)h * p.rh) * qb : nullptr;
  v.ldt = p.ldt;
  v.gf = 1.f;
  if (v.qd && p.gate) {
    const S* gp = (const S*)p.gate + (p.gate_per_token ? tok * p.H : 0) + h;
    v.gf = gate_value(DT::load1(gp), p.gate_act);
  }
  return v;
}

// byte address of the key slice of (source s, head h) for token tok
__device__ __forceinline__ const char* key_slice(const ReadParams& p, int s, int64_t tok, int h) {
  return (const char*)p.key[s] + (tok * (int64_t)p.kstride[s] + (int64_t)h * p.rh) * dtype_bytes(p.kdt);
}

// Key element j of (source s, head h) as the read scores it: the key plus the
// source's static key, rounded to the key dtype as the eager add is, when there
// is one.
__device__ __forceinline__ float key_at(const ReadParams& p, const char* kp, int s, int h, int j) {
  const float k = load_any(kp, j, p.kdt);
  if (!p.skey) return k;
  return round_any(k + load_any(p.skey, (int64_t)s * p.R + h * p.rh + j, p.kdt), p.kdt);
}

// Sum of squares of one key slice (rh elements): 16-byte loads when the keys
// have the value dtype and are aligned for them (and no static key is added),
// else one element at a time.
template <class DT>
__device__ __forceinline__ float key_sumsq(const ReadParams& p, const char* kp, int s, int h) {
  constexpr int KV = 16 / (int)sizeof(typename DT::S);
  const int rh = p.rh;
  float ss = 0.f;
  if (p.key_vec && !p.skey) {
    for (int j = 0; j < rh; j += KV) {
      float k[KV];
      load_vec<DT, KV>((const typename DT::S*)kp + j, k);
#pragma unroll
      for (int i = 0; i < KV; ++i) ss += k[i] * k[i];
    }
  } else {
    for (int j = 0; j < rh; ++j) {
      const float k = key_at(p, kp, s, h, j);
      ss += k * k;
    }
  }
  return ss;
}

// logit of (head h, source s) for token tok
template <class DT>
__device__ float lr_logit(const ReadParams& p, int64_t tok, int h, int s) {
  using S = typename DT::S;
  constexpr int KV = 16 / (int)sizeof(S);
  const int rh = p.rh, ldt = p.ldt;
  const char* kp = key_slice(p, s, tok, h);
  const QueryView<DT> q = query_view<DT>(p, tok, h);
  float inv = 1.f;
  if (p.key_norm) inv = 1.0f / sqrtf(key_sumsq<DT>(p, kp, s, h) / (float)rh + p.eps);
  float dot = 0.f;
  if (p.key_vec && !p.skey) {
    for (int j = 0; j < rh; j += KV) {
      float k[KV];
      load_vec<DT, KV>((const S*)kp + j, k);
#pragma unroll
      for (int i = 0; i < KV; ++i) {
        const float kh = p.key_norm ? round_any(k[i] * inv, ldt) : k[i];
        dot += kh * q.at(j + i);
      }
    }
  } else {
    for (int j = 0; j < rh; ++j) {
      const float k = key_at(p, kp, s, h, j);
      const float kh = p.key_norm ? round_any(k * inv, ldt) : k;
      dot += kh * q.at(j);
    }
  }
  float logit = round_any(round_any(dot, ldt) * p.scale, ldt);
  if (p.bias) logit += p.bias[s];
  return logit;
}

// softmax over the N sources of head h (logits in LDS); returns weight of pair pi
__device__ __forceinline__ float softmax_pair(const float* s_logit, int N, int h, int pi) {
  const float* lg = s_logit + h * N;
  float m = lg[0];
  for (int s = 1; s < N; ++s) m = fmaxf(m, lg[s]);
  float den = 0.f;
  for (int s = 0; s < N; ++s) den += expf(lg[s] - m);
  return expf(s_logit[pi] - m) / den;
}

// ============================================================== forward
template <class DT, int E, int CB>
__global__ void __launch_bounds__(1024) lr_fwd_kernel(const ReadParams p) {
  using S = typename DT::S;
  extern __shared__ float smem[];
  const int N = p.n_src, H = p.H, HN = H * N;
  float* s_logit = smem;
  float* s_w = smem + HN;
  float* s_red = smem + 2 * HN;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int wpt = blockDim.x / kWave;

  int eoff[CB], hd[CB];
  bool ok[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    const int col = wave + c * wpt;
    const int e = (col * kWave + lane) * E;
    ok[c] = col < p.ncols && e < p.D;
    eoff[c] = e;
    hd[c] = ok[c] ? e / p.dh : 0;
  }

  for (int64_t tok = blockIdx.x; tok < p.n_tok; tok += gridDim.x) {
    for (int pi = tid; pi < HN; pi += blockDim.x) {
      const int h = pi / N;
      s_logit[pi] = lr_logit<DT>(p, tok, h, pi - h * N);
    }
    __syncthreads();
    for (int pi = tid; pi < HN; pi += blockDim.x) {
      const float pr = softmax_pair(s_logit, N, pi / N, pi);
      if (p.weights) p.weights[tok * HN + pi] = pr;
      s_w[pi] = DT::rnd(pr);
    }
    __syncthreads();

    float acc[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int i = 0; i < E; ++i) acc[c][i] = 0.f;

    for (int s0 = 0; s0 < N; s0 += kSrcGroup) {
      Raw<DT, E> r[kSrcGroup][CB];
#pragma unroll
      for (int i = 0; i < kSrcGroup; ++i) {
        const int s = s0 + i;
        if (s < N) {
          const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
#pragma unroll
          for (int c = 0; c < CB; ++c)
            if (ok[c]) load_raw<DT, E, true>(vp + eoff[c], r[i][c]);
        }
      }
#pragma unroll
      for (int i = 0; i < kSrcGroup; ++i) {
        const int s = s0 + i;
        if (s < N) {
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            if (ok[c]) {
              float v[E];
              unpack<DT, E>(r[i][c], v);
              const float w = s_w[hd[c] * N + s];
#pragma unroll
              for (int e = 0; e < E; ++e) acc[c][e] += w * v[e];
            }
          }
        }
      }
    }

    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        acc[c][e] = DT::rnd(acc[c][e]);
        if (ok[c]) ss += acc[c][e] * acc[c][e];
      }
    if (p.norm_out) {
      if (p.out_prenorm) {
        S* xp = (S*)p.out_prenorm + tok * (int64_t)p.D;
#pragma unroll
        for (int c = 0; c < CB; ++c)
          if (ok[c]) store_vec<DT, E, true>(xp + eoff[c], acc[c]);
      }
      ss = wave_sum(ss);
      if (wpt > 1) {
        if (lane == 0) s_red[wave] = ss;
        __syncthreads();
        ss = 0.f;
        for (int w = 0; w < wpt; ++w) ss += s_red[w];
      }
      const float inv = 1.0f / sqrtf(ss / (float)p.D + p.eps);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[c][e] = DT::rnd(acc[c][e] * inv);
      if (tid == 0 && p.out_inv_rms) p.out_inv_rms[tok] = inv;
    }
    S* op = (S*)p.out + tok * (int64_t)p.D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (ok[c]) store_vec<DT, E, true>(op + eoff[c], acc[c]);
    __syncthreads();
  }
}

// ============================================================== backward
// A workgroup holds `teams` token teams of `wpt` waves each.  With one wave
// per token (wpt == 1) the teams run independent token streams and synchronise
// at wavefront scope only, so a workgroup keeps several tokens in flight
// without workgroup barriers; with wpt > 1 there is one team and the team
// barrier is the workgroup barrier.  Each team owns an LDS region; the teams'
// cross-token accumulators are summed in team order at the end.
__device__ __forceinline__ void team_sync(int wpt) {
  if (wpt == 1) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();
  }
}

template <class DT, int E, int CB>
__global__ void __launch_bounds__(1024) lr_bwd_kernel(const ReadBwdParams bp) {
  using S = typename DT::S;
  const ReadParams& p = bp.f;
  extern __shared__ float smem[];
  const int N = p.n_src, H = p.H, HN = H * N, R = p.R, rh = p.rh, D = p.D;
  const int wpt = p.wpt;
  const int team_threads = wpt * kWave;
  const int teams = blockDim.x / team_threads;
  const int team = threadIdx.x / team_threads;
  const int tid = threadIdx.x - team * team_threads;  // thread index inside the team
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  // lanes per dW pre-reduction group: largest power of two dividing the
  // vectors per head, at most a wave
  const int cph_full = p.dh / E;
  int gl = cph_full & (-cph_full);
  if (gl > kWave) gl = kWave;
  const int gpc = kWave / gl;       // groups per column
  const int cph = cph_full / gl;    // groups per head

  const int team_floats = 5 * HN + N * p.ncols * gpc + N * R + R + bp.n_part + 32;
  float* s_p = smem + team * team_floats;
  float* s_w = s_p + HN;
  float* s_dw = s_w + HN;
  float* s_ge = s_dw + HN;
  float* s_dl = s_ge + HN;
  float* s_part = s_dl + HN;                   // [N * ncols * gpc]
  float* s_kh = s_part + N * p.ncols * gpc;    // [N * R]
  float* s_dq = s_kh + N * R;                  // [R]
  float* s_acc = s_dq + R;                     // [n_part]
  float* s_red = s_acc + bp.n_part;            // [32]

  for (int i = tid; i < bp.n_part; i += team_threads) s_acc[i] = 0.f;

  int eoff[CB], hd[CB];
  bool ok[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    const int col = wave + c * wpt;
    const int e = (col * kWave + lane) * E;
    ok[c] = col < p.ncols && e < D;
    eoff[c] = e;
    hd[c] = ok[c] ? e / p.dh : 0;
  }
  team_sync(wpt);

  const int64_t stride = (int64_t)gridDim.x * teams;
  for (int64_t tok = (int64_t)blockIdx.x * teams + team; tok < p.n_tok; tok += stride) {
    // ---- A: saved weights, upstream gradient (through the output norm)
    for (int pi = tid; pi < HN; pi += team_threads) {
      const float pr = bp.saved_w[tok * HN + pi];
      s_p[pi] = pr;
      s_w[pi] = DT::rnd(pr);
    }
    float g[CB][E];
    const S* gp = (const S*)bp.gout + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if (ok[c]) load_vec<DT, E, true>(gp + eoff[c], g[c]);
      else
#pragma unroll
        for (int e = 0; e < E; ++e) g[c][e] = 0.f;
    }
    if (p.norm_out) {
      // rms-norm backward from the pre-norm output x: inv*g - x*inv^3*mean(g*x)
      float x[CB][E];
      const S* xp = (const S*)p.out_prenorm + tok * (int64_t)D;
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        if (ok[c]) load_vec<DT, E, true>(xp + eoff[c], x[c]);
        else
#pragma unroll
          for (int e = 0; e < E; ++e) x[c][e] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) dot += g[c][e] * x[c][e];
      }
      dot = wave_sum(dot);
      if (wpt > 1) {
        if (lane == 0) s_red[wave] = dot;
        team_sync(wpt);
        dot = 0.f;
        for (int w = 0; w < wpt; ++w) dot += s_red[w];
      }
      const float inv = bp.saved_inv[tok];
      const float k3 = inv * inv * inv * (dot / (float)D);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) g[c][e] = ok[c] ? DT::rnd(inv * g[c][e] - x[c][e] * k3) : 0.f;
    }
    team_sync(wpt);

    // ---- B: stream the value rows: dW partials and dv = w * g
    for (int s0 = 0; s0 < N; s0 += kSrcGroup) {
      Raw<DT, E> r[kSrcGroup][CB];
#pragma unroll
      for (int i = 0; i < kSrcGroup; ++i) {
        const int s = s0 + i;
        if (s < N) {
          const S* vp = (const S*)p.val[s] + tok * (int64_t)p.vstride[s];
#pragma unroll
          for (int c = 0; c < CB; ++c)
            if (ok[c]) load_raw<DT, E, true>(vp + eoff[c], r[i][c]);
        }
      }
#pragma unroll
      for (int i = 0; i < kSrcGroup; ++i) {
        const int s = s0 + i;
        if (s < N) {
          S* dvp = (S*)bp.dval[s] + tok * (int64_t)D;
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            float part = 0.f;
            if (ok[c]) {
              float v[E], dv[E];
              unpack<DT, E>(r[i][c], v);
              const float w = s_w[hd[c] * N + s];
#pragma unroll
              for (int e = 0; e < E; ++e) {
                part += g[c][e] * v[e];
                dv[e] = DT::rnd(w * g[c][e]);
              }
              store_vec<DT, E, true>(dvp + eoff[c], dv);
            }
            part = group_sum(part, gl);
            const int col = wave + c * wpt;
            if (ok[c] && (lane & (gl - 1)) == 0) s_part[(s * p.ncols + col) * gpc + lane / gl] = part;
          }
        }
      }
    }
    team_sync(wpt);

    // ---- C: dW per (head, source)
    for (int pi = tid; pi < HN; pi += team_threads) {
      const int h = pi / N, s = pi - h * N;
      const float* sp = s_part + s * p.ncols * gpc + h * cph;
      float dw = 0.f;
      for (int j = 0; j < cph; ++j) dw += sp[j];
      s_dw[pi] = DT::rnd(dw);
    }
    team_sync(wpt);

    // ---- D: softmax backward, key gradient, normalised keys for dq
    for (int pi = tid; pi < HN; pi += team_threads) {
      const int h = pi / N, s = pi - h * N;
      float dot = 0.f;
      for (int t = 0; t < N; ++t) dot += s_p[h * N + t] * s_dw[h * N + t];
      const float dl = s_p[pi] * (s_dw[pi] - dot);
      s_dl[pi] = dl;
      const int ldt = p.ldt;
      const float ge = round_any(round_any(dl, ldt) * p.scale, ldt);
      s_ge[pi] = ge;

      const char* kp = key_slice(p, s, tok, h);
      const QueryView<DT> q = query_view<DT>(p, tok, h);
      float inv = 1.f;
      if (p.key_norm) inv = 1.0f / sqrtf(key_sumsq<DT>(p, kp, s, h) / (float)rh + p.eps);
      float m = 0.f;
      for (int j = 0; j < rh; ++j) {
        const float k = key_at(p, kp, s, h, j);
        const float kh = p.key_norm ? round_any(k * inv, ldt) : k;
        s_kh[s * R + h * rh + j] = kh;
        if (p.key_norm) m += round_any(ge * q.at(j), ldt) * (k * inv);
      }
      // dk in the key dtype: the rms-norm backward of the rounded-key gradient
      // (fp32), or that gradient itself without key_norm
      void* dkp = (char*)bp.dkey[s] + (tok * (int64_t)R + h * rh) * dtype_bytes(p.kdt);
      const float mr = m / (float)rh;
      for (int j = 0; j < rh; ++j) {
        const float dkh = round_any(ge * q.at(j), ldt);
        float dk = dkh;
        if (p.key_norm) {
          const float yk = key_at(p, kp, s, h, j) * inv;
          dk = inv * (dkh - yk * mr);
        }
        store_any(dkp, j, p.kdt, dk);
      }
    }
    team_sync(wpt);

    // ---- E: query gradient (per token or accumulated), bias accumulation
    for (int j = tid; j < R; j += team_threads) {
      const int h = j / rh;
      float a = 0.f;
      for (int s = 0; s < N; ++s) a += s_ge[h * N + s] * s_kh[s * R + j];
      const float t = p.q_dyn ? round_any(a, p.ldt) : a;
      if (bp.part_q >= 0) s_acc[bp.part_q + j] += t;
      if (p.q_dyn) {
        const QueryView<DT> q = query_view<DT>(p, tok, h);
        if (bp.dq_dyn) store_any(bp.dq_dyn, tok * (int64_t)R + j, p.ldt, round_any(q.gf * t, p.ldt));
        if (p.gate) s_dq[j] = t * load_any(q.qd, j - h * rh, p.ldt);
      }
    }
    if (bp.part_bias >= 0) {
      for (int s = tid; s < N; s += team_threads) {
        float b = 0.f;
        for (int h = 0; h < H; ++h) b += s_dl[h * N + s];
        s_acc[bp.part_bias + s] += b;
      }
    }
    if (p.q_dyn && p.gate) {
      team_sync(wpt);
      for (int h = tid; h < H; h += team_threads) {
        float c = 0.f;
        for (int j = 0; j < rh; ++j) c += s_dq[h * rh + j];
        const S* gptr = (const S*)p.gate + (p.gate_per_token ? tok * H : 0) + h;
        if (p.gate_act == ATTNRES_GATE_SIGMOID) {
          const float sg = gate_value(DT::load1(gptr), p.gate_act);
          c *= sg * (1.f - sg);
        }
        if (p.gate_per_token) {
          if (bp.dgate) DT::store1((S*)bp.dgate + tok * H + h, DT::rnd(c));
        } else if (bp.part_gate >= 0) {
          s_acc[bp.part_gate + h] += c;
        }
      }
    }
    team_sync(wpt);
  }

  // fold the teams' accumulators in team order into this workgroup's partials
  __syncthreads();
  if (bp.partials) {
    for (int i = threadIdx.x; i < bp.n_part; i += blockDim.x) {
      float a = 0.f;
      for (int t = 0; t < teams; ++t) a += smem[t * team_floats + 5 * HN + N * p.ncols * gpc + N * R + R + i];
      bp.partials[(int64_t)blockIdx.x * bp.n_part + i] = a;
    }
  }
}

// ============================================================== launchers
template <class DT, int E, int CB>
static hipError_t launch_lr_fwd_t(const ReadParams& p, int wpt, int grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((lr_fwd_kernel<DT, E, CB>), dim3(grid), dim3(wpt * kWave), lds, st, p);
  return hipGetLastError();
}

template <class DT, int E, int CB>
static hipError_t launch_lr_bwd_t(const ReadBwdParams& p, int threads, int grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((lr_bwd_kernel<DT, E, CB>), dim3(grid), dim3(threads), lds, st, p);
  return hipGetLastError();
}

template <class DT>
static hipError_t lr_fwd_dt(const ReadParams& p, const Launch& L, hipStream_t st) {
  if (L.vec) return launch_lr_fwd_t<DT, 16 / sizeof(typename DT::S), 2>(p, L.wpt, L.grid, L.lds, st);
  return launch_lr_fwd_t<DT, 1, 4>(p, L.wpt, L.grid, L.lds, st);
}

template <class DT>
static hipError_t lr_bwd_dt(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  const int threads = L.wpt * kWave * L.teams;
  if (L.vec) return launch_lr_bwd_t<DT, 16 / sizeof(typename DT::S), 2>(p, threads, L.grid, L.lds, st);
  return launch_lr_bwd_t<DT, 1, 4>(p, threads, L.grid, L.lds, st);
}

// ---------------------------------------------------------------- static-key gradient
// d static_s = rnd(sum over tokens of dk_s): the reference's `key + static`
// expands the static key over (B, T), whose backward sums the key-dtype
// gradient rows with fp32 accumulation and rounds once.  Pass 1: workgroup
// (chunk, source) sums its chunk of tokens: a thread owns V consecutive
// columns (one 16-byte load per row when the rows allow it) and one of P
// token phases; the phases are folded in a fixed order through LDS.  Pass 2:
// thread (source, column) adds the chunks in order and rounds.
template <class DT, int V>
__global__ void __launch_bounds__(256) key_colsum_kernel(const ColsumParams p) {
  using S = typename DT::S;
  __shared__ float s_part[256 * V];
  const int c = blockIdx.x, s = blockIdx.y, R = p.R;
  const int64_t tpc = (p.n_tok + p.chunks - 1) / p.chunks;
  const int64_t t0 = (int64_t)c * tpc;
  const int64_t t1 = t0 + tpc < p.n_tok ? t0 + tpc : p.n_tok;
  const int cg = R / V;               // column groups (the host keeps cg <= 256)
  const int P = 256 / cg;             // token phases
  const int tid = threadIdx.x;
  const int ph = tid / cg, col = tid - (tid / cg) * cg;
  const S* dk = (const S*)p.dk[s] + col * V;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.f;
  if (ph < P) {
#pragma unroll 8
    for (int64_t t = t0 + ph; t < t1; t += P) {
      float x[V];
      load_vec<DT, V, true>(dk + t * R, x);
#pragma unroll
      for (int v = 0; v < V; ++v) acc[v] += x[v];
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) s_part[tid * V + v] = acc[v];
  __syncthreads();
  float* out = p.partials + ((int64_t)s * p.chunks + c) * R;
  for (int r = tid; r < R; r += 256) {
    const int g = r / V, v = r - (r / V) * V;
    float sum = 0.f;
    for (int k = 0; k < P; ++k) sum += s_part[(k * cg + g) * V + v];
    out[r] = sum;
  }
}

// Pass 2: one wave per (source, column): lane l adds chunks l and l + 64 (the
// host keeps chunks <= 128), then a fixed-order wave sum (deterministic), one
// rounding to the key dtype.  One memory round trip per output instead of a
// thread walking every chunk.
__global__ void __launch_bounds__(256) key_colsum_finish_kernel(const ColsumParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t i = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (i >= (int64_t)p.n_src * p.R) return;  // wave-uniform
  const int s = (int)(i / p.R), r = (int)(i - (int64_t)s * p.R);
  const float* row = p.partials + (int64_t)s * p.chunks * p.R + r;
  float a = lane < p.chunks ? row[(int64_t)lane * p.R] : 0.f;
  if (lane + kWave < p.chunks) a += row[(int64_t)(lane + kWave) * p.R];
  a = wave_sum(a);
  if (lane == 0) store_any(p.out, i, p.kdt, a);
}

template <class DT>
static void key_colsum_t(const ColsumParams& p, bool vec, hipStream_t st) {
  constexpr int EV = 16 / sizeof(typename DT::S);
  const dim3 g(p.chunks, p.n_src), b(256);
  if (vec) hipLaunchKernelGGL((key_colsum_kernel<DT, EV>), g, b, 0, st, p);
  else hipLaunchKernelGGL((key_colsum_kernel<DT, 1>), g, b, 0, st, p);
}

hipError_t launch_key_colsum(const ColsumParams& p, hipStream_t st) {
  // 16-byte rows when every source's dk rows are aligned for them; column
  // groups must fit the 256 threads (rank <= 256 scalar, <= 2048 / 1024 vector)
  const int es = dtype_bytes(p.kdt);
  bool vec = (p.R * es) % 16 == 0;
  for (int s = 0; vec && s < p.n_src; ++s) vec = ((uintptr_t)p.dk[s] & 15u) == 0;
  const int cg = vec ? p.R * es / 16 : p.R;
  if (cg > 256) return hipErrorInvalidValue;
  switch (p.kdt) {
    case ATTNRES_DTYPE_F32: key_colsum_t<F32>(p, vec, st); break;
    case ATTNRES_DTYPE_BF16: key_colsum_t<BF16>(p, vec, st); break;
    default: key_colsum_t<F16>(p, vec, st); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t n = (int64_t)p.n_src * p.R;  // one wave per output, four per workgroup
  if (p.chunks > 2 * kWaveSize) return hipErrorInvalidValue;
  hipLaunchKernelGGL(key_colsum_finish_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_lr_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return lr_fwd_dt<F32>(p, L, st);
    case ATTNRES_DTYPE_BF16: return lr_fwd_dt<BF16>(p, L, st);
    default: return lr_fwd_dt<F16>(p, L, st);
  }
}

hipError_t launch_lr_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return lr_bwd_dt<F32>(p, L, st);
    case ATTNRES_DTYPE_BF16: return lr_bwd_dt<BF16>(p, L, st);
    default: return lr_bwd_dt<F16>(p, L, st);
  }
}

}  // namespace attnres
