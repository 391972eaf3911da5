// Base AttnRes read, fast path: forward launches (kernels in attnres_base_fast.h).
#include "attnres_base_fast.h"

namespace attnres {

template <class DT, int VB, int CB, int NB, bool KN>
static hipError_t base_fast_fwd_t(const ReadParams& p, const Launch& L, hipStream_t st) {
  hipLaunchKernelGGL((base_fwd_fast_kernel<DT, VB, CB, NB, KN>), dim3(L.grid), dim3(kFastWaves * kWave), L.lds, st, p);
  return hipGetLastError();
}

template <class DT>
static hipError_t base_fast_fwd_dt(const ReadParams& p, const Launch& L, hipStream_t st) {
  if (p.key_norm) {
    ATTNRES_BASE_FAST_SWITCH(base_fast_fwd_t, p, true)
  }
  ATTNRES_BASE_FAST_SWITCH(base_fast_fwd_t, p, false)
}

// 16-bit types only (the host plan never selects this path for fp32)
hipError_t launch_base_fast_forward(int dtype, const ReadParams& p, const Launch& L, hipStream_t st) {
  if (dtype == ATTNRES_DTYPE_BF16) return base_fast_fwd_dt<BF16>(p, L, st);
  if (dtype == ATTNRES_DTYPE_F16) return base_fast_fwd_dt<F16>(p, L, st);
  return hipErrorInvalidValue;
}

}  // namespace attnres
