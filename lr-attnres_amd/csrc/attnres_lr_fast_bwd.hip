// LR AttnRes read, fast path: backward launches (kernels in attnres_lr_fast.h).
#include "attnres_lr_fast.h"

namespace attnres {

template <class DT, int VB, int CB, int NB, int RHC, int FEAT>
static hipError_t fast_bwd_t(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  hipLaunchKernelGGL((lr_bwd_fast_kernel<DT, VB, CB, NB, RHC, FEAT>), dim3(L.grid), dim3(kFastWaves * kWave), L.lds,
                     st, p);
  return hipGetLastError();
}

template <class DT>
static hipError_t fast_bwd_dt(const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  if (L.feat == 0) {
    ATTNRES_FAST_SWITCH(fast_bwd_t, p, 0)
  }
  if (L.feat == kFeatDyn) {
    ATTNRES_FAST_SWITCH(fast_bwd_t, p, kFeatDyn)
  }
  if (L.feat == (kFeatDyn | kFeatStatic)) {
    ATTNRES_FAST_SWITCH(fast_bwd_t, p, kFeatDyn | kFeatStatic)
  }
  ATTNRES_FAST_SWITCH(fast_bwd_t, p, kFeatAll)
}

size_t lr_fast_table_bytes() { return sizeof(SrcTab); }

hipError_t launch_lr_fast_backward(int dtype, const ReadBwdParams& p, const Launch& L, hipStream_t st) {
  switch (dtype) {
    case ATTNRES_DTYPE_F32: return fast_bwd_dt<F32>(p, L, st);
    case ATTNRES_DTYPE_BF16: return fast_bwd_dt<BF16>(p, L, st);
    default: return fast_bwd_dt<F16>(p, L, st);
  }
}

}  // namespace attnres
