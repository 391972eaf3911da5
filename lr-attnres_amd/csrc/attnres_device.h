// Device-side helpers shared by the AttnRes read kernels (gfx950 / CDNA4).
//
// Storage types are raw bits (fp32 as float, bf16 and fp16 as 16-bit words);
// every computation is fp32.  The rounding helpers reproduce PyTorch's
// round-to-nearest-even casts, which is how the kernels mirror the points
// where the reference's eager op rounds to the tensor dtype.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace attnres {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bits_to_f32(uint32_t u) { return __uint_as_float(u); }

// bf16 <-> fp32, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
// gfx950 converts to bf16 in hardware (v_cvt_pk_bf16_f32, round to nearest even)
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float round_bf16(float f) { return (float)(__bf16)f; }
// two fp32 values -> one word of two bf16 (low element in the low half)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xffffu));
}
__device__ __forceinline__ float round_f16(float f) { return (float)(_Float16)f; }

// ---------------------------------------------------------------- dtype tags
struct F32 {
  using S = float;
  static constexpr int kCode = 0;
  __device__ __forceinline__ static float rnd(float x) { return x; }
  __device__ __forceinline__ static float from_bits(uint32_t u) { return __uint_as_float(u); }
  __device__ __forceinline__ static float load1(const S* p) { return *p; }
  __device__ __forceinline__ static void store1(S* p, float x) { *p = x; }
};
struct BF16 {
  using S = uint16_t;
  static constexpr int kCode = 1;
  __device__ __forceinline__ static float rnd(float x) { return round_bf16(x); }
  __device__ __forceinline__ static float load1(const S* p) { return __uint_as_float(((uint32_t)*p) << 16); }
  __device__ __forceinline__ static void store1(S* p, float x) { *p = (S)f32_to_bf16_bits(x); }
};
struct F16 {
  using S = uint16_t;
  static constexpr int kCode = 2;
  __device__ __forceinline__ static float rnd(float x) { return round_f16(x); }
  __device__ __forceinline__ static float load1(const S* p) { return f16_bits_to_f32(*p); }
  __device__ __forceinline__ static void store1(S* p, float x) { *p = (S)f32_to_f16_bits(x); }
};

// one element's raw bits (zero-extended for 16-bit types), converted by bits_to_float
template <class DT>
__device__ __forceinline__ uint32_t load_bits1(const typename DT::S* p) {
  if constexpr (sizeof(typename DT::S) == 4) return __float_as_uint(*p);
  else return (uint32_t)*p;
}
template <class DT>
__device__ __forceinline__ float bits_to_float(uint32_t u) {
  if constexpr (DT::kCode == 0) return __uint_as_float(u);
  else if constexpr (DT::kCode == 1) return __uint_as_float(u << 16);
  else return f16_bits_to_f32(u);
}

// Elements r = lane + stride * j (j < K) of a short row of R elements: loaded
// as raw bits and converted only after every load of the row's token is issued
// -- a 16-bit element converted right after its load would make the wave wait
// for that load (and every earlier one) before it issues the next.  Every
// lane issues all K loads, unconditionally: indices past R re-read element
// R - 1 (in bounds, a cache hit) and convert to 0; a load under a branch
// would be merged with a zero-extension that again waits for it.
template <class DT, int K>
__device__ __forceinline__ void row_bits_load(const typename DT::S* row, int R, int lane, int stride,
                                              uint32_t (&b)[K]) {
#pragma unroll
  for (int j = 0; j < K; ++j) b[j] = load_bits1<DT>(row + min(lane + j * stride, R - 1));
}
template <class DT, int K>
__device__ __forceinline__ void row_bits_floats(const uint32_t (&b)[K], int R, int lane, int stride, float (&f)[K]) {
#pragma unroll
  for (int j = 0; j < K; ++j) f[j] = lane + j * stride < R ? bits_to_float<DT>(b[j]) : 0.f;
}

// A block summary's scale: a python number scales in fp32; a scale tensor takes
// the value dtype first (model.py:985 casts the learned scale; a 0-dim fp32
// device tensor multiplying a 16-bit tensor is cast to that dtype the same way)
template <class DT>
__device__ __forceinline__ float summary_scale(const float* dev, float host) { return dev ? DT::rnd(*dev) : host; }

// ---------------------------------------------------------------- vectors
// A "vector" is E consecutive elements loaded or stored with one access:
// 16 bytes on the fast path (8 bf16/fp16 or 4 fp32), one element otherwise.
template <class DT, int E> struct Vec {
  static constexpr int kBytes = E * (int)sizeof(typename DT::S);
  static constexpr int kWords = kBytes >= 4 ? kBytes / 4 : 1;
};

template <class DT, int E>
struct Raw {  // raw bits of one vector, kept packed in VGPRs until used
  uint32_t w[Vec<DT, E>::kWords];
};

// Streaming accesses.  Rows that a kernel touches exactly once (source values,
// upstream gradients, outputs and value gradients: hundreds of MB per launch,
// far beyond L2 and the MALL) go through the non-temporal cache policy
// (NT = true): they then neither displace lines other waves still use nor sit
// dirty in the caches until a later kernel's traffic forces their write-back.
// Small rows that are re-read (keys, queries, tables) keep the default policy.
template <class T, bool NT>
__device__ __forceinline__ T ld(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <class T, bool NT>
__device__ __forceinline__ void st(T* p, T v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <class DT, int E, bool NT = false>
__device__ __forceinline__ void load_raw(const typename DT::S* __restrict__ p, Raw<DT, E>& r) {
  constexpr int B = Vec<DT, E>::kBytes;
  if constexpr (B == 16) {
    u32x4 v = ld<u32x4, NT>(reinterpret_cast<const u32x4*>(p));
    r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  } else if constexpr (B == 8) {
    u32x2 v = ld<u32x2, NT>(reinterpret_cast<const u32x2*>(p));
    r.w[0] = v.x; r.w[1] = v.y;
  } else if constexpr (B == 4) {
    r.w[0] = ld<uint32_t, NT>(reinterpret_cast<const uint32_t*>(p));
  } else {
    r.w[0] = (uint32_t)ld<uint16_t, NT>(reinterpret_cast<const uint16_t*>(p));
  }
}

template <class DT, int E>
__device__ __forceinline__ void unpack(const Raw<DT, E>& r, float (&o)[E]) {
  if constexpr (sizeof(typename DT::S) == 4) {
#pragma unroll
    for (int i = 0; i < E; ++i) o[i] = __uint_as_float(r.w[i]);
  } else if constexpr (E == 1) {
    if constexpr (DT::kCode == 1) o[0] = __uint_as_float(r.w[0] << 16);
    else o[0] = f16_bits_to_f32(r.w[0]);
  } else {
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
      if constexpr (DT::kCode == 1) {
        o[2 * i] = __uint_as_float(r.w[i] << 16);
        o[2 * i + 1] = __uint_as_float(r.w[i] & 0xffff0000u);
      } else {
        o[2 * i] = f16_bits_to_f32(r.w[i]);
        o[2 * i + 1] = f16_bits_to_f32(r.w[i] >> 16);
      }
    }
  }
}

template <class DT, int E, bool NT = false>
__device__ __forceinline__ void load_vec(const typename DT::S* __restrict__ p, float (&o)[E]) {
  Raw<DT, E> r;
  load_raw<DT, E, NT>(p, r);
  unpack<DT, E>(r, o);
}

// store E fp32 values (already rounded where the caller wants) as DT
template <class DT, int E, bool NT = false>
__device__ __forceinline__ void store_vec(typename DT::S* __restrict__ p, const float (&x)[E]) {
  if constexpr (sizeof(typename DT::S) == 4) {
    if constexpr (E == 4) {
      u32x4 v = {__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
      st<u32x4, NT>(reinterpret_cast<u32x4*>(p), v);
    } else if constexpr (E == 2) {
      u32x2 v = {__float_as_uint(x[0]), __float_as_uint(x[1])};
      st<u32x2, NT>(reinterpret_cast<u32x2*>(p), v);
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) st<float, NT>(p + i, x[i]);
    }
  } else {
    auto pack2 = [](float lo, float hi) -> uint32_t {
      if constexpr (DT::kCode == 1) return pack_bf16x2(lo, hi);
      else return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
    };
    if constexpr (E == 8) {
      u32x4 v = {pack2(x[0], x[1]), pack2(x[2], x[3]), pack2(x[4], x[5]), pack2(x[6], x[7])};
      st<u32x4, NT>(reinterpret_cast<u32x4*>(p), v);
    } else if constexpr (E == 4) {
      u32x2 v = {pack2(x[0], x[1]), pack2(x[2], x[3])};
      st<u32x2, NT>(reinterpret_cast<u32x2*>(p), v);
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) DT::store1(p + i, x[i]);
    }
  }
}

// E fp32 values (already rounded to DT) back into packed raw words
template <class DT, int E>
__device__ __forceinline__ void pack_raw(const float (&x)[E], Raw<DT, E>& r) {
  if constexpr (sizeof(typename DT::S) == 4) {
#pragma unroll
    for (int i = 0; i < E; ++i) r.w[i] = __float_as_uint(x[i]);
  } else if constexpr (E == 1) {
    if constexpr (DT::kCode == 1) r.w[0] = __float_as_uint(x[0]) >> 16;
    else r.w[0] = f32_to_f16_bits(x[0]);
  } else {
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
      if constexpr (DT::kCode == 1) r.w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
      else r.w[i] = f32_to_f16_bits(x[2 * i]) | (f32_to_f16_bits(x[2 * i + 1]) << 16);
    }
  }
}

// two fp32 values rounded to the 16-bit dtype (nearest even), packed into one
// word (low element in the low half)
template <class DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (DT::kCode == 1) return pack_bf16x2(lo, hi);
  else return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
}

// Packed 16-bit arithmetic: lo_pair / hi_pair interleave the low / high
// halves of two words (element i of two sources), and dot2 is one v_dot2
// (a.lo * b.lo + a.hi * b.hi + c; the products of two 16-bit floats are
// exact in fp32).
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

template <class DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT::kCode == 1)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a), __builtin_bit_cast(bf16x2v, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2v, a), __builtin_bit_cast(f16x2v, b), c, false);
}

// 16-bit storage bits of a dtype-rounded value
template <class DT>
__device__ __forceinline__ uint32_t bits16(float x) {
  if constexpr (DT::kCode == 1) return __float_as_uint(x) >> 16;
  else return f32_to_f16_bits(x);
}

// scalar access to a buffer whose dtype is only known at run time
__device__ __forceinline__ float load_any(const void* p, int64_t i, int code) {
  if (code == 0) return ((const float*)p)[i];
  const uint32_t b = ((const uint16_t*)p)[i];
  return code == 1 ? __uint_as_float(b << 16) : f16_bits_to_f32(b);
}
__device__ __forceinline__ float round_any(float x, int code) {
  return code == 0 ? x : code == 1 ? round_bf16(x) : round_f16(x);
}
__device__ __forceinline__ void store_any(void* p, int64_t i, int code, float x) {
  if (code == 0) ((float*)p)[i] = x;
  else if (code == 1) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(x);
  else ((uint16_t*)p)[i] = (uint16_t)f32_to_f16_bits(x);
}

// ---------------------------------------------------------------- reductions


// Cross-lane moves inside rows of 16 lanes through the DPP modifiers of
// ordinary VALU instructions (no LDS round trip): lane i reads lane i ^ 1,
// i ^ 2 (quad permutes), 7 - i within its half row and 15 - i within its row.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

// All-reduce inside aligned groups of `width` lanes (power of two <= 64).
// Within 16 lanes the partners are a quad butterfly and two mirrors (each
// lane's partner holds the sum of the complementary part, so every lane ends
// with the same value); wider groups continue with lane shuffles.  The order
// is fixed, so results are deterministic.
__device__ __forceinline__ float group_sum(float x, int width) {
  if (width > 1) x += dpp_f32<kDppXor1>(x);
  if (width > 2) x += dpp_f32<kDppXor2>(x);
  if (width > 4) x += dpp_f32<kDppHalfMirror>(x);
  if (width > 8) x += dpp_f32<kDppMirror>(x);
  for (int o = 16; o < width; o <<= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

// All-reduce over the 64 lanes of a wave (every lane gets the sum; the
// association order is fixed, so results are deterministic).
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_f32<kDppXor1>(x);
  x += dpp_f32<kDppXor2>(x);
  x += dpp_f32<kDppHalfMirror>(x);
  x += dpp_f32<kDppMirror>(x);
  x += __shfl_xor(x, 16, kWave);
  x += __shfl_xor(x, 32, kWave);
  return x;
}
// Many wave sums at once.  x[0..V) are per-lane partial sums (V a multiple of
// 4).  v_permlane32_swap exchanges the upper 32 lanes of one register with the
// lower 32 lanes of another, so one swap and one add fold two values over
// lane distance 32 into one register (first value in lanes 0-31, second in
// 32-63); v_permlane16_swap does the same for the odd 16-lane rows of one
// register and the even rows of another.  After both folds register k holds,
// in row r, a 16-lane partial of value 4k + {0, 2, 1, 3}[r], and a DPP
// all-reduce inside each row completes it: 2.5 V instructions instead of 6 V
// for V separate butterflies.  The order is fixed (deterministic results).
template <int V>
__device__ __forceinline__ void wave_sums(const float (&x)[V], float (&z)[V / 4]) {
  static_assert(V % 4 == 0, "wave_sums folds groups of four values");
  float h[V / 2];
#pragma unroll
  for (int j = 0; j < V / 2; ++j) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[2 * j]), __float_as_uint(x[2 * j + 1]), false,
                                                    false);
    h[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < V / 4; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(h[2 * k]), __float_as_uint(h[2 * k + 1]), false,
                                                    false);
    float t = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    t += dpp_f32<kDppXor1>(t);
    t += dpp_f32<kDppXor2>(t);
    t += dpp_f32<kDppHalfMirror>(t);
    t += dpp_f32<kDppMirror>(t);
    z[k] = t;
  }
}
// Many sums over the two 32-lane halves of a wave at once (V even): one
// v_permlane16_swap and one add fold two values over lane distance 16 (the
// first value's halves in rows 0 and 2, the second's in rows 1 and 3), and a
// DPP all-reduce inside each row completes them.  Register j then holds, in
// every lane of row r, value 2 j + (r & 1) summed over half r >> 1.  Fixed
// order (deterministic results).
template <int V>
__device__ __forceinline__ void half_sums(const float (&x)[V], float (&z)[V / 2]) {
  static_assert(V % 2 == 0, "half_sums folds pairs of values");
#pragma unroll
  for (int j = 0; j < V / 2; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[2 * j]), __float_as_uint(x[2 * j + 1]), false,
                                                    false);
    float t = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    t += dpp_f32<kDppXor1>(t);
    t += dpp_f32<kDppXor2>(t);
    t += dpp_f32<kDppHalfMirror>(t);
    t += dpp_f32<kDppMirror>(t);
    z[j] = t;
  }
}
// value m of wave_sums' result (wave-uniform): row {0, 2, 1, 3}[m % 4] of z[m / 4]
template <int V>
__device__ __forceinline__ float wave_sums_get(const float (&z)[V / 4], int m) {
  const int row = (m & 3) == 1 ? 2 : (m & 3) == 2 ? 1 : (m & 3);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(z[m >> 2]), 16 * row));
}

// wave_sums' value m in the lanes where `take` holds, `keep` elsewhere.  The
// readlane runs in every lane, outside any lane-dependent branch: under a
// branch such as `if (lane == s)` the compiler may sink the reduction's last
// add into the branch, and the readlane then reads a lane the branch masked
// off (seen as wrong logits with five source slots).
template <int V>
__device__ __forceinline__ float wave_sums_pick(const float (&z)[V / 4], int m, bool take, float keep) {
  const float v = wave_sums_get<V>(z, m);
  return take ? v : keep;
}

__device__ __forceinline__ float group_max(float x, int width) {
  if (width > 1) x = fmaxf(x, dpp_f32<kDppXor1>(x));
  if (width > 2) x = fmaxf(x, dpp_f32<kDppXor2>(x));
  if (width > 4) x = fmaxf(x, dpp_f32<kDppHalfMirror>(x));
  if (width > 8) x = fmaxf(x, dpp_f32<kDppMirror>(x));
  for (int o = 16; o < width; o <<= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
  return x;
}

// ---------------------------------------------------------------- addressing
// Pointers rebuilt from integers (e.g. tables kept in LDS) are generic to the
// compiler, which then emits flat accesses; casting through the global address
// space keeps them on the global_load / global_store path.
template <class S>
__device__ __forceinline__ S* global_ptr(uint64_t a) {
  return (S*)(__attribute__((address_space(1))) S*)(a);
}

// the value of lane i ^ 1 (quad permute [1, 0, 3, 2])
__device__ __forceinline__ float lane_xor1(float x) { return dpp_f32<kDppXor1>(x); }

// Per-element sums of a[j] over each key head of hd columns, for a key row
// held as element lane + 64 j (j < KJ): a group sum for hd < 64, else wave
// sums added over the head's chunks (all lanes get their head's sum).
template <int KJ>
__device__ __forceinline__ void key_head_sums(int hd, const float (&a)[KJ], float (&s)[KJ]) {
  if (hd < kWave) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) s[j] = group_sum(a[j], hd);
  } else {
    float t[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) t[j] = wave_sum(a[j]);
    const int cph = hd / kWave;  // chunks per head
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      const int h0 = (j / cph) * cph;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KJ; ++k)
        if (k >= h0 && k < h0 + cph) acc += t[k];
      s[j] = acc;
    }
  }
}

// orders one wave's LDS writes before its later LDS reads by other lanes
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Staged rows: one 16-byte lane vector loaded straight into LDS
// (global_load_lds_dwordx4; lane i's 16 bytes land at lds_row + 16 i, checked
// on the box), no VGPR held while the load is in flight.  `lds_row` must be
// wave-uniform.  The compiler does not order LDS reads after these loads:
// read the row back only after wait_staged() (vmcnt(0): every vector-memory
// operation of the wave has completed, these loads included).
__device__ __forceinline__ void stage16(const void* src, void* lds_row) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)lds_row, 16, 0, 0);
}
__device__ __forceinline__ void wait_staged() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroups are dispatched round-robin over the GPU's 8 XCDs (workgroup b on
// XCD b % 8), each XCD with its own L2.  xcd_block gives every XCD a contiguous
// range of logical workgroup indices, so that the tokens of neighbouring
// workgroups are handled in one XCD.  A bijection on [0, grid).
__device__ __forceinline__ int xcd_block(int b, int grid) {
  constexpr int kXcd = 8;
  const int per = grid / kXcd, rem = grid - (grid / kXcd) * kXcd;
  const int x = b - (b / kXcd) * kXcd, i = b / kXcd;
  return x * per + (x < rem ? x : rem) + i;
}

// a wave-uniform 64-bit value, moved to scalar registers
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ int uniform_i32(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ float uniform_f32(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

__device__ __forceinline__ float gate_value(float g, int act) {
  return act == 2 ? 1.0f / (1.0f + expf(-g)) : g;
}

}  // namespace attnres
