// Internal launch interface between the C ABI (attnres_capi.hip) and the
// kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "attnres_params.h"

namespace attnres {

struct Launch {
  int vec;      // 16-byte vector path (else one element per access)
  int wpt;      // waves per token (workgroup = wpt * 64 threads)
  int grid;     // workgroups (persistent over tokens)
  size_t lds;   // dynamic LDS bytes
  int nmax;     // base read: register-resident source slots (8/16; more = streaming)
  int teams;    // token teams per workgroup (LR backward; phase 2: waves per workgroup)
  int vb;       // vector bytes (16 or 8) where a kernel family has both layouts
  int feat;     // LR fast path: optional code the kernel carries (kFeat* bits of attnres_lr_fast.h)
};

hipError_t launch_lr_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st);
hipError_t launch_lr_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st);
hipError_t launch_base_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st);
hipError_t launch_base_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st);
hipError_t launch_average_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st);
hipError_t launch_average_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st);
hipError_t launch_reduce_partials(int dtype, const ReduceParams& p, hipStream_t st);
hipError_t launch_key_colsum(const ColsumParams& p, hipStream_t st);
hipError_t launch_value_norm(int dtype, bool bwd, const ValueNormParams& p, int grid, bool vec, hipStream_t st);
// LR fast path (head-aligned one-wave work items): L.wpt = columns per item,
// L.nmax = source slots (8/16/32), L.teams = key chunks per head slot (2/8)
hipError_t launch_lr_fast_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st);
hipError_t launch_lr_fast_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st);
size_t lr_fast_table_bytes();  // LDS bytes of the fast kernels' per-source tables
// base-key fast path (one wave per token, 16-bit rows of 256 / 512 / 768 / 1024):
// L.vb = vector bytes (8/16), L.wpt = columns per lane, L.nmax = source slots
// (4/8/12/16); per-source tables in the first lr_fast_table_bytes() of LDS
hipError_t launch_base_fast_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st);
hipError_t launch_base_fast_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st);
// cached-logit phases: L.wpt = waves per workgroup; phase-1 backward L.nmax =
// register slots for the read sites (4, 8 or 16); phase-2 L.nmax = 1 for LR keys
hipError_t launch_phase1_forward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st);
hipError_t launch_phase1_backward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st);
// phase 1 (forward / backward) for 16-bit rows of 256 / 512 / 768 / 1024, <= 4 sites, <= 8
// sources, no output norm: L.vb = vector bytes, L.wpt = columns per lane,
// L.nmax = source slots (4/8); four token streams per workgroup
hipError_t launch_phase1_fast_forward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st);
hipError_t launch_phase1_fast_backward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st);
// phase 1 split over L.wpt = D / 256 waves per token (one workgroup per token),
// 16-bit rows, no output norm, n_q * np <= 64: L.nmax = np (2/4/8/16)
hipError_t launch_phase1_split_forward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st);
hipError_t launch_phase1_split_backward(int dtype, const Phase1Params& p, const Launch& L, hipStream_t st);
hipError_t launch_phase2_forward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st);
hipError_t launch_phase2_backward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st);
// phase 2 with base keys, 16-bit rows of 256 / 512 / 768 / 1024, no output norm:
// L.vb = vector bytes (8/16), L.wpt = columns per lane, L.feat bit 0 = key norm
hipError_t launch_phase2_fast_forward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st);
hipError_t launch_phase2_fast_backward(int dtype, const Phase2Params& p, const Launch& L, hipStream_t st);
// query-bank logits: L.grid token workgroups of L.wpt waves, L.lds = wpt *
// kKLMaxQ floats; backward L.teams = query-gradient groups
hipError_t launch_keyed_logits_forward(int dtype, const KeyedLogitsParams& p, const Launch& L, hipStream_t st);
hipError_t launch_keyed_logits_backward(int dtype, const KeyedLogitsParams& p, const Launch& L, hipStream_t st);
// key-producer epilogue: one wave per token, L.teams waves per workgroup,
// L.vec = 16-byte vectors for the output columns
hipError_t launch_keyed_split_forward(int dtype, const KeySplitParams& p, const Launch& L, hipStream_t st);
hipError_t launch_keyed_split_backward(int dtype, const KeySplitParams& p, const Launch& L, hipStream_t st);

// one source's site logits: L.nmax = rank slots (32/64/128), L.grid x 4 waves,
// L.lds = n_q * nmax floats (the queries)
hipError_t launch_site_logits_forward(int dtype, const SiteLogitsParams& p, const Launch& L, hipStream_t st);
hipError_t launch_site_logits_backward(int dtype, const SiteLogitsParams& p, const Launch& L, hipStream_t st);

// dtype switch of the launchers
#define ATTNRES_DISPATCH(dtype, fn, ...)                          \
  switch (dtype) {                                                \
    case ATTNRES_DTYPE_F32: return fn<F32>(__VA_ARGS__);          \
    case ATTNRES_DTYPE_BF16: return fn<BF16>(__VA_ARGS__);        \
    default: return fn<F16>(__VA_ARGS__);                         \
  }

}  // namespace attnres
