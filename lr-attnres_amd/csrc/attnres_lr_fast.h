// LR AttnRes read, fast path: one wave per (token, head-aligned column group).
//
// A "column" is 64 lanes x one 16-byte vector (512 bf16/fp16 or 256 fp32
// elements).  When the head width divides the column width (or spans exactly
// two columns), every wave can own whole heads of a token, so a wave computes
// everything for its heads -- logits, softmax, mix, and in the backward dW,
// the softmax and key-norm chains, dk and the query gradient -- with no
// cross-wave synchronisation and no duplicated work.  Work items are
// (token, item) with item in [0, n_items); a wave keeps one item index and
// walks tokens with a fixed stride, so its heads (and static query) never
// change and its query-gradient accumulators live in registers.
//
// Memory order: every load a token needs (keys, per-token query, upstream
// gradient, all N value vectors) is issued first; stores go last.  On CDNA the
// vector-memory counter also counts stores, so a load issued after a store
// cannot be waited on without draining that store -- keeping stores at the end
// removes those round trips from the token's critical path.
//
// Staged rows: with one 16-bit column per wave, the first SL value rows of a
// token (lr_fast_staged_rows) go straight into a per-wave LDS area
// (global_load_lds_dwordx4), issued after the register rows; the mix (and the
// backward's dW) takes the register rows first, then waits for everything and
// reads the staged rows back.  They hold no VGPRs in flight (85 / 95 instead
// of 109 / 111 at C3) and stream faster than register loads.
//
// Addressing: the per-source pointer / stride tables are copied to LDS once
// and read back as wave-uniform scalars inside the token loop, so row
// addresses are scalar (SGPR base + one VGPR lane offset) and the tables do
// not pin dozens of SGPRs for the whole kernel.
//
// Requirements (checked on the host, else the general kernels run):
// 16-byte vector path, N <= NB (8/16/32, or 12/14/20/24 for one column
// and two key chunks), N * heads_per_item <= 64 pairs,
// key slice of a head = kch 16-byte chunks with kch <= RHC, heads_per_item *
// (R/H) <= 64 (a power of two when the backward has a gate), output norm only
// when one item covers the whole row.
#pragma once

#include "attnres_device.h"
#include "attnres_params.h"
#include "attnres_launch.h"

namespace attnres {

constexpr int kFastWaves = 4;  // waves per workgroup (independent token streams)

// FEAT selects at compile time which optional code an instantiation carries:
// kFeatDyn = per-token query and gate, kFeatNorm = output norm, kFeatStatic =
// a static key per source added to every key.  The host picks the smallest
// instantiated set a read needs (0, kFeatDyn, kFeatDyn | kFeatStatic, or all):
// without them the static-query backward fits 4 waves per SIMD instead of 3,
// and the gated one 3 instead of 2.
// (the kFeat* constants are in attnres_params.h, shared with the host)

// per-source tables in LDS
struct SrcTab {
  uint64_t vptr[kMaxSources];
  uint64_t kptr[kMaxSources];
  uint64_t dvptr[kMaxSources];
  uint64_t dkptr[kMaxSources];
  uint32_t vstrb[kMaxSources];  // row strides in bytes (< 2^32, checked on the host)
  uint32_t kstrb[kMaxSources];
};
constexpr int kSrcTabFloats = (int)(sizeof(SrcTab) / sizeof(float));

template <class DT, int RHC>
struct KeySlice {
  static constexpr int KV = 16 / (int)sizeof(typename DT::S);
  Raw<DT, KV> r[RHC];
};

// Static source keys (kFeatStatic): the [n_src, R] table is copied to LDS once
// per workgroup (16-byte chunks; the host checks R * elem is a multiple of 16),
// and every token's key slice gets its source's slice added from there,
// rounded to the dtype as the eager `key + static` is -- token-invariant data
// kept out of the loop-carried registers.  Rows sit one 16-byte chunk more
// than R apart: the pair lanes of one head read the same offset in every
// source's row, which with a row stride of a multiple of 256 bytes would all
// fall in the same LDS banks.
template <class DT>
__device__ __forceinline__ int static_key_row(int R) {
  return R + 16 / (int)sizeof(typename DT::S);  // elements
}
template <class DT>
__device__ __forceinline__ void static_keys_to_lds(const ReadParams& p, typename DT::S* dst) {
  using S = typename DT::S;
  const int row16 = p.R * (int)sizeof(S) / 16;  // chunks per row
  const int n16 = p.n_src * row16;
  const u32x4* src = (const u32x4*)p.skey;
  for (int i = threadIdx.x; i < n16; i += blockDim.x) {
    const int s = i / row16;
    ((u32x4*)dst)[i + s] = src[i];  // row s starts s chunks further on
  }
}

template <class DT, int RHC>
__device__ __forceinline__ void add_static_key(const typename DT::S* sk, int kch, KeySlice<DT, RHC>& kr) {
#pragma unroll
  for (int j = 0; j < RHC; ++j) {
    if (j < kch) {
      const u32x4 w = *(const u32x4*)(sk + j * KeySlice<DT, RHC>::KV);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
      // word by word (two 16-bit elements, or one fp32), so few values are live at once
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(typename DT::S) == 2) {
          Raw<DT, 2> a, b;
          a.w[0] = kr.r[j].w[i];
          b.w[0] = ww[i];
          float x[2], y[2];
          unpack<DT, 2>(a, x);
          unpack<DT, 2>(b, y);
          kr.r[j].w[i] = pack2<DT>(x[0] + y[0], x[1] + y[1]);  // packing rounds to the dtype
        } else {
          kr.r[j].w[i] = __float_as_uint(__uint_as_float(kr.r[j].w[i]) + __uint_as_float(ww[i]));
        }
      }
    }
  }
}

// the staged rows of this lane back from LDS into the register rows' array
// (after every load of the token has completed)
template <int SL, class DT, int E, int NB, int CB>
__device__ __forceinline__ void read_staged_rows(const char* stage, int lane, Raw<DT, E> (&vr)[NB][CB]) {
  wait_staged();
#pragma unroll
  for (int r = 0; r < SL; ++r) {
    const u32x4 w = *(const u32x4*)(stage + r * 1024 + lane * 16);
    vr[r][0].w[0] = w.x;
    vr[r][0].w[1] = w.y;
    vr[r][0].w[2] = w.z;
    vr[r][0].w[3] = w.w;
  }
}

// byte address of a row: base + tok * stride, one 32 x 32 -> 64-bit
// multiply-add (tok and the byte stride fit 32 bits on this path)
__device__ __forceinline__ uint64_t row_addr(uint64_t base, int64_t tok, uint32_t strideb) {
  return base + (uint64_t)(uint32_t)tok * strideb;
}

// byte address of source s's row for a wave-uniform token tok (the table
// has kMaxSources slots, so reading a slot past n_src is harmless; its value
// is never used).  The table entries move to scalar registers first, so the
// address arithmetic runs on the scalar unit.
__device__ __forceinline__ uint64_t row_base(const SrcTab* tab, int s, int64_t tok) {
  return row_addr(uniform_u64(tab->vptr[s]), tok, uniform_u32(tab->vstrb[s]));
}


template <class DT, int RHC>
__device__ __forceinline__ float key_inv_rms(const KeySlice<DT, RHC>& kr, int kch, int rh, float eps) {
  constexpr int KV = KeySlice<DT, RHC>::KV;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < RHC; ++j) {
    if (j < kch) {
      float k[KV];
      unpack<DT, KV>(kr.r[j], k);
#pragma unroll
      for (int i = 0; i < KV; ++i) ss += k[i] * k[i];
    }
  }
  return 1.0f / sqrtf(ss / (float)rh + eps);
}

// The pair lane's query slice for one token, in registers: static part
// (dtype-exact, token-invariant) plus, with a per-token query, the gated
// dynamic part composed and rounded like the reference: rnd(q_s + g * q_d).
// 16-bit types keep the (exact) values packed two per word.
template <class DT, int RHC>
struct QSlice {
  static constexpr int KV = KeySlice<DT, RHC>::KV;
  static constexpr bool kPacked = sizeof(typename DT::S) == 2;
  static constexpr int kWords = kPacked ? RHC * KV / 2 : RHC * KV;
  uint32_t w[kWords];
  __device__ __forceinline__ float get(int j) const {
    if constexpr (kPacked) {
      const uint32_t x = w[j >> 1];
      if constexpr (DT::kCode == 1) return __uint_as_float((j & 1) ? (x & 0xffff0000u) : (x << 16));
      else return f16_bits_to_f32((j & 1) ? (x >> 16) : x);
    } else {
      return __uint_as_float(w[j]);
    }
  }
  __device__ __forceinline__ void set2(int j, float a, float b) {  // elements j, j + 1 (j even), dtype-exact
    if constexpr (kPacked) {
      w[j >> 1] = bits16<DT>(a) | (bits16<DT>(b) << 16);
    } else {
      w[j] = __float_as_uint(a);
      w[j + 1] = __float_as_uint(b);
    }
  }
};

template <class DT, int RHC>
__device__ __forceinline__ void static_query(const float* s_qh, bool has_static, int kch, QSlice<DT, RHC>& qs) {
  constexpr int KV = QSlice<DT, RHC>::KV;
#pragma unroll
  for (int j = 0; j < RHC * KV; j += 2) {
    const bool in = has_static && j < kch * KV;
    qs.set2(j, in ? s_qh[j] : 0.f, in ? s_qh[j + 1] : 0.f);
  }
}

template <class DT, int RHC>
__device__ __forceinline__ void token_query(const QSlice<DT, RHC>& qs, const KeySlice<DT, RHC>& qr, bool dyn, float gf,
                                            QSlice<DT, RHC>& q) {
  constexpr int KV = QSlice<DT, RHC>::KV;
  if (dyn) {
#pragma unroll
    for (int j = 0; j < RHC; ++j) {
      float t[KV];
      unpack<DT, KV>(qr.r[j], t);
#pragma unroll
      for (int i = 0; i < KV; i += 2)
        q.set2(j * KV + i, DT::rnd(qs.get(j * KV + i) + gf * t[i]), DT::rnd(qs.get(j * KV + i + 1) + gf * t[i + 1]));
    }
  } else {
#pragma unroll
    for (int j = 0; j < QSlice<DT, RHC>::kWords; ++j) q.w[j] = qs.w[j];
  }
}

// <khat, q> of a pair lane, khat = rnd(k * inv) (key_norm) or k.  16-bit
// types: one v_dot2 per element pair on the (exact) 16-bit values.
template <class DT, int RHC>
__device__ __forceinline__ float key_query_dot(const KeySlice<DT, RHC>& kr, const QSlice<DT, RHC>& q, bool key_norm,
                                               float inv, int kch) {
  constexpr int KV = QSlice<DT, RHC>::KV;
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < RHC; ++j) {
    if (j < kch) {
      float k[KV];
      unpack<DT, KV>(kr.r[j], k);
#pragma unroll
      for (int i = 0; i < KV; ++i) k[i] = key_norm ? DT::rnd(k[i] * inv) : k[i];
      if constexpr (QSlice<DT, RHC>::kPacked) {
#pragma unroll
        for (int i = 0; i < KV / 2; ++i) {
          const uint32_t kk = bits16<DT>(k[2 * i]) | (bits16<DT>(k[2 * i + 1]) << 16);
          dot = dot2<DT>(kk, q.w[(j * KV) / 2 + i], dot);
        }
      } else {
#pragma unroll
        for (int i = 0; i < KV; ++i) dot += k[i] * q.get(j * KV + i);
      }
    }
  }
  return dot;
}

// ============================================================== forward
// (the static-key instantiations with 20+ slots would cross 168 VGPRs by one
// register: they ask for 3 waves per SIMD, which the compiler meets without spills)
template <class DT, int VB, int CB, int NB, int RHC, int FEAT>
__global__ void __launch_bounds__(256, (FEAT & kFeatStatic) && NB >= 20 ? 3 : 1) lr_fwd_fast_kernel(const ReadParams p) {
  using S = typename DT::S;
  constexpr int E = VB / (int)sizeof(S);        // value elements per lane vector
  constexpr int KV = 16 / (int)sizeof(S);       // key elements per 16-byte chunk
  constexpr int colw = kWave * E;
  extern __shared__ float lds_base[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wslot = uniform_i32(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int N = p.n_src, H = p.H, rh = p.rh, dh = p.dh, D = p.D, R = p.R;
  __builtin_assume(N >= lr_fast_slot_floor(CB, RHC, NB));
  constexpr int SL = lr_fast_staged_rows(CB, RHC, NB, (int)sizeof(S), FEAT);
  // LDS: per wave SL staged rows of 1 KB | source tables | static query [R] |
  // per wave: the softmax weights, 64 words (16-bit types: the rounded
  // weights of lanes 2i and 2i + 1 packed in word i; fp32: one word per lane)
  char* stage = (char*)lds_base + wslot * SL * 1024;
  float* smem = lds_base + nwaves * SL * 256;
  SrcTab* tab = (SrcTab*)smem;
  float* s_q = smem + kSrcTabFloats;
  uint32_t* s_w = (uint32_t*)(s_q + R) + wslot * 64;
  // slots past n_src repeat the last source, so the unrolled loads over NB
  // slots read the table at constant offsets (their values are never used)
  for (int i = threadIdx.x; i < kMaxSources; i += blockDim.x) {
    const int j = min(i, N - 1);
    tab->vptr[i] = (uint64_t)p.val[j];
    tab->vstrb[i] = (uint32_t)p.vstride[j] * (uint32_t)sizeof(S);
    tab->kptr[i] = (uint64_t)p.key[j];
    tab->kstrb[i] = (uint32_t)p.kstride[j] * (uint32_t)sizeof(S);
  }
  if (p.q_static)
    for (int i = threadIdx.x; i < R; i += blockDim.x) s_q[i] = DT::load1((const S*)p.q_static + i);
  // static keys after the per-wave weight words
  S* s_sk = (S*)(s_q + R + nwaves * 64);
  const bool skey = (FEAT & kFeatStatic) && p.skey != nullptr;
  if (skey) static_keys_to_lds<DT>(p, s_sk);
  __syncthreads();

  // staged-row kernels: XCD-major workgroup order (C3 fwd 77.9 -> 73.7 us, bwd
  // 169.2 -> 165.0 us; neutral to slightly slower for the other kernels)
  const int wv = (SL > 0 ? xcd_block(blockIdx.x, gridDim.x) : (int)blockIdx.x) * nwaves + wslot;
  const int item = wv % p.n_items;
  // waves past n_items * streams (the last workgroup's spare slots) stay idle
  const int64_t t0 = wv < p.n_items * p.streams ? wv / p.n_items : p.n_tok;
  const int h0 = (item * CB * colw) / dh;
  const int nh = min(p.nh, H - h0);
  // (head, source) pairs: lane = head_in_item * np + source, np = pow2 >= N,
  // so per-head softmax reductions are butterflies inside np-lane groups
  const int np = p.np;
  const int lh = lane / np, lsrc = lane - (lane / np) * np;
  const bool has_pair = lh < nh && lsrc < N;
  const int ph = h0 + (lh < nh ? lh : 0);
  const int ps = has_pair ? lsrc : 0;
  const int kch = p.kch;
  const bool dyn = (FEAT & kFeatDyn) && p.q_dyn != nullptr;
  const bool has_static = p.q_static != nullptr;
  const uint64_t kbase = tab->kptr[ps] + (uint64_t)(ph * rh) * sizeof(S);
  const uint32_t kstrb = tab->kstrb[ps];
  const float bias = (p.bias && has_pair) ? p.bias[ps] : 0.f;  // token-invariant

  // lanes past the row end load from the row start (valid memory) and store nothing
  int eoff[CB], hd[CB];
  bool ok[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    const int e = (item * CB + c) * colw + lane * E;
    ok[c] = e < D;
    eoff[c] = ok[c] ? e : 0;
    hd[c] = ok[c] ? e / dh - h0 : 0;
  }

  // ---- every load a token needs: keys (and per-token query), values.  No
  // branches: every lane loads valid addresses -- lanes without a pair read
  // pair 0's slice, slots past kch / N re-read the last chunk / row -- so the
  // loads issue back to back.
  QSlice<DT, RHC> qstat;
  static_query<DT, RHC>(s_q + ph * rh, has_static, kch, qstat);
  KeySlice<DT, RHC> kr, qr;
  S graw = 0;
  Raw<DT, E> vr[NB][CB];
  auto issue_loads = [&](int64_t t) {
    {
      const S* kp = global_ptr<const S>(row_addr(kbase, t, kstrb));
#pragma unroll
      for (int j = 0; j < RHC; ++j) load_raw<DT, KV>(kp + min(j, kch - 1) * KV, kr.r[j]);
    }
    if (dyn) {
      const S* qp = global_ptr<const S>((uint64_t)p.q_dyn) + t * p.q_dyn_stride + ph * rh;
#pragma unroll
      for (int j = 0; j < RHC; ++j) load_raw<DT, KV>(qp + min(j, kch - 1) * KV, qr.r[j]);
      if (p.gate) graw = *(global_ptr<const S>((uint64_t)p.gate) + (p.gate_per_token ? t * H : 0) + ph);
    }
    uint64_t base[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) base[s] = row_base(tab, s, t);
#pragma unroll
    for (int s = SL; s < NB; ++s) {
      const S* vp = global_ptr<const S>(base[s]);
#pragma unroll
      for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(vp + eoff[c], vr[s][c]);
    }
    // the first SL rows straight into LDS, issued last (CB == 1 here)
#pragma unroll
    for (int s = 0; s < SL; ++s) stage16(global_ptr<const S>(base[s]) + eoff[0], stage + s * 1024);
  };

  for (int64_t tok = t0; tok < p.n_tok; tok += p.streams) {
    issue_loads(tok);
    // ---- logits of this wave's (head, source) pairs
    float logit = -INFINITY;
    if (has_pair) {
      if (skey) add_static_key<DT, RHC>(s_sk + ps * static_key_row<DT>(R) + ph * rh, kch, kr);
      const float gf = (dyn && p.gate) ? gate_value(DT::load1(&graw), p.gate_act) : 1.f;
      const float inv = p.key_norm ? key_inv_rms<DT, RHC>(kr, kch, rh, p.eps) : 1.f;
      QSlice<DT, RHC> q;
      token_query<DT, RHC>(qstat, qr, dyn, gf, q);
      const float dot = key_query_dot<DT, RHC>(kr, q, p.key_norm, inv, kch);
      logit = DT::rnd(DT::rnd(dot) * p.scale) + bias;
    }
    // softmax over each head's np-lane group (lanes without a pair carry -inf / 0)
    const float lmax = group_max(logit, np);
    const float ex = has_pair ? expf(logit - lmax) : 0.f;
    const float pw = ex / group_sum(ex, np);
    if constexpr (sizeof(S) == 2) {
      // 16-bit weights, zero for lanes without a pair (so an odd source count
      // pairs its last source with a zero weight); even lanes store the word
      // of their pair with lane + 1
      const float wr = has_pair ? DT::rnd(pw) : 0.f;
      const uint32_t hi = bits16<DT>(lane_xor1(wr));
      if ((lane & 1) == 0) s_w[lane >> 1] = bits16<DT>(wr) | (hi << 16);
    } else {
      s_w[lane] = __float_as_uint(has_pair ? pw : 0.f);
    }
    wave_sync();

    // ---- mix
    float acc[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[c][e] = 0.f;
    if constexpr (sizeof(S) == 2) {
      // register rows first (as they arrive), then the staged rows
#pragma unroll
      for (int s0 = SL; s0 < NB + SL; s0 += 2) {
        const int s = s0 < NB ? s0 : s0 - NB;
        if (s0 == NB) read_staged_rows<SL>(stage, lane, vr);
        if (s < N) {
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            const uint32_t wp = s_w[(hd[c] * np + s) >> 1];
#pragma unroll
            for (int i = 0; i < E / 2; ++i) {
              acc[c][2 * i] = dot2<DT>(lo_pair(vr[s][c].w[i], vr[s + 1][c].w[i]), wp, acc[c][2 * i]);
              acc[c][2 * i + 1] = dot2<DT>(hi_pair(vr[s][c].w[i], vr[s + 1][c].w[i]), wp, acc[c][2 * i + 1]);
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        if (s < N) {
#pragma unroll
          for (int c = 0; c < CB; ++c) {
            float v[E];
            unpack<DT, E>(vr[s][c], v);
            const float w = __uint_as_float(s_w[hd[c] * np + s]);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[c][e] += w * v[e];
          }
        }
      }
    }
    // ---- stores (each store's packing rounds the mix to the dtype)
    if ((FEAT & kFeatNorm) && p.norm_out) {  // one item covers the whole row here
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          acc[c][e] = DT::rnd(acc[c][e]);
          if (ok[c]) ss += acc[c][e] * acc[c][e];
        }
      if (p.out_prenorm) {
        S* xp = global_ptr<S>((uint64_t)p.out_prenorm) + tok * (int64_t)D;
#pragma unroll
        for (int c = 0; c < CB; ++c)
          if (ok[c]) store_vec<DT, E, true>(xp + eoff[c], acc[c]);
      }
      const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + p.eps);
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[c][e] = acc[c][e] * inv;
      if (lane == 0 && p.out_inv_rms) p.out_inv_rms[tok] = inv;
    }
    S* op = global_ptr<S>((uint64_t)p.out) + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c)
      if (ok[c]) store_vec<DT, E, true>(op + eoff[c], acc[c]);
    if (has_pair && p.weights) p.weights[(tok * H + ph) * N + ps] = pw;
    wave_sync();  // this token's weights are read before the next token writes them
  }
}

// ============================================================== backward
template <class DT, int VB, int CB, int NB, int RHC, int FEAT>
__global__ void __launch_bounds__(256) lr_bwd_fast_kernel(const ReadBwdParams bp) {
  using S = typename DT::S;
  constexpr int E = VB / (int)sizeof(S);
  constexpr int KV = 16 / (int)sizeof(S);
  constexpr int colw = kWave * E;
  const ReadParams& p = bp.f;
  extern __shared__ float lds_base[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wslot = uniform_i32(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int N = p.n_src, H = p.H, rh = p.rh, dh = p.dh, D = p.D, R = p.R;
  __builtin_assume(N >= lr_fast_slot_floor(CB, RHC, NB));
  constexpr int SL = lr_fast_staged_rows(CB, RHC, NB, (int)sizeof(S), FEAT);
  // LDS: per wave SL staged rows of 1 KB | source tables | static query [R] |
  // per wave: p [64], dW [64], dl [64], contributions [nh*np][rh] | fold
  // [nwaves][n_part]
  char* stage = (char*)lds_base + wslot * SL * 1024;
  float* smem = lds_base + nwaves * SL * 256;
  SrcTab* tab = (SrcTab*)smem;
  float* s_q = smem + kSrcTabFloats;
  const int wave_floats = 3 * 64 + p.np * p.nh * (rh + 1);
  float* s_p = s_q + R + wslot * wave_floats;
  float* s_dw = s_p + 64;
  float* s_dl = s_dw + 64;
  // s_c rows are rh + 1 floats apart: with an odd stride the pair lanes' writes
  // and the owner lanes' reads fall in distinct LDS banks
  float* s_c = s_dl + 64;  // [npairs][rh + 1] = ge * khat
  float* s_fold = s_q + R + nwaves * wave_floats;
  for (int i = threadIdx.x; i < kMaxSources; i += blockDim.x) {
    const int j = min(i, N - 1);
    tab->vptr[i] = (uint64_t)p.val[j];
    tab->vstrb[i] = (uint32_t)p.vstride[j] * (uint32_t)sizeof(S);
    tab->kptr[i] = (uint64_t)p.key[j];
    tab->kstrb[i] = (uint32_t)p.kstride[j] * (uint32_t)sizeof(S);
    tab->dvptr[i] = (uint64_t)bp.dval[j];
    tab->dkptr[i] = (uint64_t)bp.dkey[j];
  }
  if (p.q_static)
    for (int i = threadIdx.x; i < R; i += blockDim.x) s_q[i] = DT::load1((const S*)p.q_static + i);
  // static keys after the fold rows, on a 16-byte boundary
  S* s_sk = (S*)(s_fold + (nwaves * bp.n_part + 3) / 4 * 4);
  const bool skey = (FEAT & kFeatStatic) && p.skey != nullptr;
  if (skey) static_keys_to_lds<DT>(p, s_sk);
  __syncthreads();

  // staged-row kernels: XCD-major workgroup order (C3 fwd 77.9 -> 73.7 us, bwd
  // 169.2 -> 165.0 us; neutral to slightly slower for the other kernels)
  const int wv = (SL > 0 ? xcd_block(blockIdx.x, gridDim.x) : (int)blockIdx.x) * nwaves + wslot;
  const int item = wv % p.n_items;
  const int64_t t0 = wv < p.n_items * p.streams ? wv / p.n_items : p.n_tok;
  const int h0 = (item * CB * colw) / dh;
  const int nh = min(p.nh, H - h0);
  const int np = p.np;
  const int lh = lane / np, lsrc = lane - (lane / np) * np;
  const bool has_pair = lh < nh && lsrc < N;
  const int ph = h0 + (lh < nh ? lh : 0);
  const int ps = has_pair ? lsrc : 0;
  const int kch = p.kch;
  const bool dyn = (FEAT & kFeatDyn) && p.q_dyn != nullptr;
  const bool has_static = p.q_static != nullptr;
  // query-gradient owner lanes: (head h0 + lane / rh, element lane % rh)
  const int nq = nh * rh;
  const bool q_owner = lane < nq;
  const int qh = lane / rh, qj = lane - (lane / rh) * rh;
  // dW lane groups: lanes of one head inside a column
  const int gl = CB == 2 ? kWave : (dh / E < kWave ? dh / E : kWave);
  const uint64_t kbase = tab->kptr[ps] + (uint64_t)(ph * rh) * sizeof(S);
  S* dkbase = global_ptr<S>(tab->dkptr[ps]) + ph * rh;
  const uint32_t kstrb = tab->kstrb[ps];
  const uint32_t rowb = (uint32_t)D * (uint32_t)sizeof(S);  // dense gradient rows

  int eoff[CB], hd[CB];
  bool ok[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    const int e = (item * CB + c) * colw + lane * E;
    ok[c] = e < D;
    eoff[c] = ok[c] ? e : 0;
    hd[c] = ok[c] ? e / dh - h0 : 0;
  }

  float qacc = 0.f;  // static-query gradient of (h0 + qh, qj), over this wave's tokens
  float bacc = 0.f;  // bias gradient of source `lane`
  float gacc = 0.f;  // per-site gate gradient of head h0 + qh (lanes with qj == 0)
  const bool gated = dyn && p.gate != nullptr;
  const int64_t gate_tok = p.gate_per_token ? H : 0;  // gate row stride over tokens

  for (int64_t tok = t0; tok < p.n_tok; tok += p.streams) {
    // ---- issue every load of the token
    // (branch-free: see the forward)
    KeySlice<DT, RHC> kr, qr;
    float pr = bp.saved_w[(tok * H + ph) * N + ps];
    {
      const S* kp = global_ptr<const S>(row_addr(kbase, tok, kstrb));
#pragma unroll
      for (int j = 0; j < RHC; ++j) load_raw<DT, KV>(kp + min(j, kch - 1) * KV, kr.r[j]);
    }
    // gate of the pair lane's head, and for the query-gradient owner lanes the
    // gate and per-token query element of (h0 + qh, qj)
    S graw_p = 0, graw_o = 0, qd_o = 0;
    if (dyn) {
      const S* qp = global_ptr<const S>((uint64_t)p.q_dyn) + tok * p.q_dyn_stride + ph * rh;
#pragma unroll
      for (int j = 0; j < RHC; ++j) load_raw<DT, KV>(qp + min(j, kch - 1) * KV, qr.r[j]);
      if (gated) {
        const S* gt = global_ptr<const S>((uint64_t)p.gate) + tok * gate_tok;
        graw_p = gt[ph];
        graw_o = gt[h0 + (q_owner ? qh : 0)];
        qd_o = *(global_ptr<const S>((uint64_t)p.q_dyn) + tok * p.q_dyn_stride + h0 * rh + (q_owner ? lane : 0));
      }
    }
    Raw<DT, E> gr[CB];
    const S* gp = global_ptr<const S>((uint64_t)bp.gout) + tok * (int64_t)D;
#pragma unroll
    for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(gp + eoff[c], gr[c]);
    Raw<DT, E> xr[CB];
    if ((FEAT & kFeatNorm) && p.norm_out) {
      const S* xp = global_ptr<const S>((uint64_t)p.out_prenorm) + tok * (int64_t)D;
#pragma unroll
      for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(xp + eoff[c], xr[c]);
    }
    Raw<DT, E> vr[NB][CB];
    {
      uint64_t base[NB];
#pragma unroll
      for (int s = 0; s < NB; ++s) base[s] = row_base(tab, s, tok);
#pragma unroll
      for (int s = SL; s < NB; ++s) {
        const S* vp = global_ptr<const S>(base[s]);
#pragma unroll
        for (int c = 0; c < CB; ++c) load_raw<DT, E, true>(vp + eoff[c], vr[s][c]);
      }
      // the first SL rows straight into LDS, issued last (CB == 1 here)
#pragma unroll
      for (int s = 0; s < SL; ++s) stage16(global_ptr<const S>(base[s]) + eoff[0], stage + s * 1024);
    }
    float g[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      unpack<DT, E>(gr[c], g[c]);
#pragma unroll
      for (int e = 0; e < E; ++e) g[c][e] = ok[c] ? g[c][e] : 0.f;
    }

    // ---- upstream gradient through the output norm (item = whole row)
    if ((FEAT & kFeatNorm) && p.norm_out) {
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float x[E];
        unpack<DT, E>(xr[c], x);
#pragma unroll
        for (int e = 0; e < E; ++e) dot += g[c][e] * x[e];
      }
      const float inv = bp.saved_inv[tok];
      const float k3 = inv * inv * inv * (wave_sum(dot) / (float)D);
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float x[E];
        unpack<DT, E>(xr[c], x);
#pragma unroll
        for (int e = 0; e < E; ++e) g[c][e] = ok[c] ? DT::rnd(inv * g[c][e] - x[e] * k3) : 0.f;
      }
    }

    if (has_pair) s_p[lane] = pr;

    // ---- dW = <g, v> per (head, source), reduced over the head's lanes
    // (16-bit types: packed g against the packed value words, one v_dot2 per
    // element pair; g is dtype-exact, so packing it loses nothing)
    uint32_t gpk[CB][E / 2 > 0 ? E / 2 : 1];
    if constexpr (sizeof(S) == 2) {
#pragma unroll
      for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int i = 0; i < E / 2; ++i) gpk[c][i] = bits16<DT>(g[c][2 * i]) | (bits16<DT>(g[c][2 * i + 1]) << 16);
    }
    // this lane's share of <g, v_s> over the wave's columns (one head's lanes
    // of a column, or a head spanning both columns)
    auto dw_part = [&](int s) {
      float part = 0.f;
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        float pc = 0.f;
        if constexpr (sizeof(S) == 2) {
#pragma unroll
          for (int i = 0; i < E / 2; ++i) pc = dot2<DT>(gpk[c][i], vr[s][c].w[i], pc);
        } else {
          float v[E];
          unpack<DT, E>(vr[s][c], v);
#pragma unroll
          for (int e = 0; e < E; ++e) pc += g[c][e] * v[e];
        }
        part = c == 0 ? pc : part + pc;
      }
      return part;
    };
    // Sources two at a time.  Two heads per wave (32-lane groups): one
    // v_permlane16_swap fold and one DPP all-reduce give both sums, and lane
    // 16 r writes (head r / 2, source 2 j + r % 2); otherwise a butterfly per
    // source over the head's lane group.
    const int r16 = lane >> 4;
    // register rows first (as they arrive), then the staged rows
    constexpr int NJ = (NB + 1) / 2;
#pragma unroll
    for (int j0 = SL / 2; j0 < NJ + SL / 2; ++j0) {
      const int j = j0 < NJ ? j0 : j0 - NJ;
      if (SL > 0 && j0 == NJ) read_staged_rows<SL>(stage, lane, vr);
      if (2 * j < N) {
        float x[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int s = 2 * j + i;
          x[i] = 0.f;
          if (s < NB && s < N) x[i] = dw_part(s);
        }
        if (CB == 1 && gl == 32) {
          float z[1];
          half_sums<2>(x, z);
          const int src = 2 * j + (r16 & 1), head = r16 >> 1;
          if ((lane & 15) == 0 && src < N && head < nh) s_dw[head * np + src] = z[0];
        } else {
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int s = 2 * j + i;
            if (s < NB && s < N) {
              if (CB == 2) {
                const float t = wave_sum(x[i]);  // one head spans both columns
                if (lane == 0) s_dw[s] = t;
              } else {
                const float t = group_sum(x[i], gl);
                if (ok[0] && (lane & (gl - 1)) == 0) s_dw[hd[0] * np + s] = t;
              }
            }
          }
        }
      }
    }
    wave_sync();

    // ---- per pair: softmax backward, key-norm backward state, contributions to dq
    float ge = 0.f, kinv = 1.f, mr = 0.f;
    // softmax backward: dl = p (dW - sum_s p dW), the sum a butterfly over the head's group
    const float dwr = has_pair ? DT::rnd(s_dw[lane]) : 0.f;
    const float pdot = group_sum(has_pair ? pr * dwr : 0.f, np);
    QSlice<DT, RHC> q;
    {
      QSlice<DT, RHC> qs;  // read per token: keeps the slice out of the loop-carried registers
      static_query<DT, RHC>(s_q + ph * rh, has_static, kch, qs);
      token_query<DT, RHC>(qs, qr, dyn, gated ? gate_value(DT::load1(&graw_p), p.gate_act) : 1.f, q);
    }
    if (has_pair) {
      const float dl = pr * (dwr - pdot);
      s_dl[lane] = dl;
      ge = DT::rnd(DT::rnd(dl) * p.scale);
      if (skey) add_static_key<DT, RHC>(s_sk + ps * static_key_row<DT>(R) + ph * rh, kch, kr);  // the scored key; dk is its gradient
      if (p.key_norm) kinv = key_inv_rms<DT, RHC>(kr, kch, rh, p.eps);
      float m = 0.f;
#pragma unroll
      for (int j = 0; j < RHC; ++j) {
        if (j < kch) {
          float k[KV];
          unpack<DT, KV>(kr.r[j], k);
#pragma unroll
          for (int i = 0; i < KV; ++i) {
            const int jj = j * KV + i;
            const float kh = p.key_norm ? DT::rnd(k[i] * kinv) : k[i];
            s_c[lane * (rh + 1) + jj] = ge * kh;
            if (p.key_norm) {
              const float dkh = DT::rnd(ge * q.get(jj));
              m += dkh * (k[i] * kinv);
            }
          }
        }
      }
      mr = m / (float)rh;
    }
    wave_sync();

    // ---- query gradient and bias accumulation (owner lanes)
    float dqt = 0.f;
    if (q_owner) {
      for (int s = 0; s < N; ++s) dqt += s_c[(qh * np + s) * (rh + 1) + qj];
      if (dyn) dqt = DT::rnd(dqt);
      qacc += dqt;
    }
    float dqd = dqt;  // per-token query gradient: rnd(act(gate) * dq) when gated
    if (gated) {
      // gate gradient of head h0 + qh: sum_j dq_j * q_dyn_j over the head's
      // rh owner lanes (an aligned power-of-two group), times the sigmoid slope
      const float gv = gate_value(DT::load1(&graw_o), p.gate_act);
      dqd = DT::rnd(gv * dqt);
      float c = group_sum(q_owner ? dqt * DT::load1(&qd_o) : 0.f, rh);
      if (p.gate_act == ATTNRES_GATE_SIGMOID) c *= gv * (1.f - gv);
      if (q_owner && qj == 0) {
        if (p.gate_per_token) {
          if (bp.dgate) DT::store1(global_ptr<S>((uint64_t)bp.dgate) + tok * H + h0 + qh, DT::rnd(c));
        } else {
          gacc += c;
        }
      }
    }
    if (p.bias && lane < N) {
      float b = 0.f;
      for (int h = 0; h < nh; ++h) b += s_dl[h * np + lane];
      bacc += b;
    }

    // ---- stores: dv = w * g, dk, per-token dq
    // 16-bit types: g again from its packed (dtype-exact) words, unpacked once
    // here, so the unpacked row is not held through the dW loop
    float gv[CB][E];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if constexpr (sizeof(S) == 2) {
        Raw<DT, E> r;
#pragma unroll
        for (int i = 0; i < E / 2; ++i) r.w[i] = gpk[c][i];
        unpack<DT, E>(r, gv[c]);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) gv[c][e] = g[c][e];
      }
    }
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      if (s < N) {
        S* dvp = global_ptr<S>(row_addr(uniform_u64(tab->dvptr[s]), tok, rowb));
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          if (ok[c]) {
            const float w = DT::rnd(s_p[hd[c] * np + s]);
            // the store's packing is the one rounding of w * g to the dtype
            float dv[E];
#pragma unroll
            for (int e = 0; e < E; ++e) dv[e] = w * gv[c][e];
            store_vec<DT, E, true>(dvp + eoff[c], dv);
          }
        }
      }
    }
    if (has_pair) {
      // dk = inv * (dkhat - khat_f32 * <dkhat, khat_f32>/rh) (rms-norm backward), dkhat = rnd(ge * q)
      S* dkp = dkbase + tok * (int64_t)R;
#pragma unroll
      for (int j = 0; j < RHC; ++j) {
        if (j < kch) {
          float k[KV], t[KV];
          unpack<DT, KV>(kr.r[j], k);
#pragma unroll
          for (int i = 0; i < KV; ++i) {
            const float dkh = DT::rnd(ge * q.get(j * KV + i));
            t[i] = p.key_norm ? kinv * (dkh - k[i] * kinv * mr) : dkh;  // rounded by the store
          }
          store_vec<DT, KV>(dkp + j * KV, t);
        }
      }
    }
    if (dyn && q_owner && bp.dq_dyn)
      DT::store1(global_ptr<S>((uint64_t)bp.dq_dyn) + tok * (int64_t)R + h0 * rh + lane, dqd);
    wave_sync();  // this token's LDS is read before the next token writes it
  }

  // ---- fold the waves' accumulators into this workgroup's partial row
  if (!bp.partials) return;
  for (int i = threadIdx.x; i < nwaves * bp.n_part; i += blockDim.x) s_fold[i] = 0.f;
  __syncthreads();
  float* fold = s_fold + wslot * bp.n_part;
  if (bp.part_q >= 0 && q_owner) fold[bp.part_q + h0 * rh + lane] = qacc;
  if (bp.part_bias >= 0 && lane < N) fold[bp.part_bias + lane] = bacc;
  if (bp.part_gate >= 0 && q_owner && qj == 0) fold[bp.part_gate + h0 + qh] = gacc;
  __syncthreads();
  for (int i = threadIdx.x; i < bp.n_part; i += blockDim.x) {
    float a = 0.f;
    for (int w = 0; w < nwaves; ++w) a += s_fold[w * bp.n_part + i];
    bp.partials[(int64_t)i * gridDim.x + blockIdx.x] = a;  // slot-major: each slot's rows contiguous
  }
}

// Launch switch shared by the forward and backward translation units:
// L.vec = value vector bytes (16), L.wpt = columns per item (1/2), L.nmax =
// source slots (8/16/32; also 12/14/18/20/24 for one column and two key chunks),
// L.teams = key chunks per head slot (2/8); FEATV is the FEAT set.
#define ATTNRES_FAST_SWITCH(fn, P, FEATV)                            \
  switch (L.vec * 10000 + L.wpt * 1000 + L.nmax * 10 + L.teams) {     \
    case 161082: return fn<DT, 16, 1, 8, 2, FEATV>(P, L, st);        \
    case 161122: return fn<DT, 16, 1, 12, 2, FEATV>(P, L, st);       \
    case 161142: return fn<DT, 16, 1, 14, 2, FEATV>(P, L, st);       \
    case 161162: return fn<DT, 16, 1, 16, 2, FEATV>(P, L, st);       \
    case 161182: return fn<DT, 16, 1, 18, 2, FEATV>(P, L, st);       \
    case 161202: return fn<DT, 16, 1, 20, 2, FEATV>(P, L, st);       \
    case 161242: return fn<DT, 16, 1, 24, 2, FEATV>(P, L, st);       \
    case 161322: return fn<DT, 16, 1, 32, 2, FEATV>(P, L, st);       \
    case 161088: return fn<DT, 16, 1, 8, 8, FEATV>(P, L, st);        \
    case 161168: return fn<DT, 16, 1, 16, 8, FEATV>(P, L, st);       \
    case 162082: return fn<DT, 16, 2, 8, 2, FEATV>(P, L, st);        \
    case 162162: return fn<DT, 16, 2, 16, 2, FEATV>(P, L, st);       \
    case 162088: return fn<DT, 16, 2, 8, 8, FEATV>(P, L, st);        \
    default: return hipErrorInvalidValue;                            \
  }

}  // namespace attnres
