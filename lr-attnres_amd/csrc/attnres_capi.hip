// C ABI of the AttnRes read library: argument checking, kernel selection and
// launch geometry.  Declared in include/attnres_hip.h.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>

#include "attnres_launch.h"
#include "attnres_params.h"

using namespace attnres;

namespace {

thread_local std::string g_last_error;

// Opt-in kernel timing (attnres_kernel_timing): HIP events recorded on the
// call's stream right before and after the read's main kernel, so that a
// benchmark times that kernel alone, without the partial-sum reduction that
// follows it in the backward.  One process-wide set of event pairs, created
// on the device current at enable time; not for concurrent callers.
constexpr int kTimerPairs = 256;
struct KernelTimer {
  bool on = false;
  bool failed = false;  // an event record failed since the last attnres_kernel_times
  int n = 0;
  hipEvent_t ev[2 * kTimerPairs];
};
KernelTimer g_timer;

// Test hook (attnres_test_phase2_block_layout): phase 2 on the workgroup-per-token kernels.
std::atomic<int> g_phase2_block_layout{0};

// Whether a start event was recorded for this call: not while the stream is
// being captured into a graph (the pair would land in the graph).
inline bool timer_begin(hipStream_t st) {
  if (!g_timer.on || g_timer.n >= kTimerPairs) return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  if (hipEventRecord(g_timer.ev[2 * g_timer.n], st) != hipSuccess) {
    g_timer.failed = true;
    return false;
  }
  return true;
}
// A pair counts only around a kernel that launched and when both records succeeded.
inline void timer_end(hipStream_t st, bool began, hipError_t launch) {
  if (!began || launch != hipSuccess) return;
  if (hipEventRecord(g_timer.ev[2 * g_timer.n + 1], st) != hipSuccess) {
    g_timer.failed = true;
    return;
  }
  ++g_timer.n;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int elem_size(int dtype) { return dtype == ATTNRES_DTYPE_F32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest dynamic LDS a workgroup may use on this device.
size_t lds_limit() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
    return 65536;
  return (size_t)v;
}

struct Plan {
  bool lr;
  int vec;        // 16-byte path
  int E;          // elements per vector
  int cb;         // columns per lane
  int ncols;
  int wpt;
  int nmax;
  int key_vec;
  int vb;         // vector bytes of the vector path (16, or 8 for 16-bit base rows of 256 / 768)
};

int check_desc(const attnres_read_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->n_src < 1 || d->n_src > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_EUNSUPPORTED, "n_src=%d outside [1, %d]", d->n_src, ATTNRES_MAX_SOURCES);
  if (d->dtype != ATTNRES_DTYPE_F32 && d->dtype != ATTNRES_DTYPE_BF16 && d->dtype != ATTNRES_DTYPE_F16)
    return fail(ATTNRES_EINVAL, "unknown dtype %d", d->dtype);
  if (d->n_tok < 0) return fail(ATTNRES_EINVAL, "n_tok=%lld < 0", (long long)d->n_tok);
  if (d->dim < 1) return fail(ATTNRES_EINVAL, "dim=%d < 1", d->dim);
  if (d->mode != ATTNRES_MODE_SOFTMAX && d->mode != ATTNRES_MODE_AVERAGE)
    return fail(ATTNRES_EINVAL, "unknown mode %d", d->mode);
  if (!d->values || !d->value_row_stride) return fail(ATTNRES_EINVAL, "values / value_row_stride is NULL");
  const bool live = d->n_tok > 0;  // empty inputs may carry NULL data pointers
  for (int s = 0; s < d->n_src; ++s) {
    if (live && !d->values[s]) return fail(ATTNRES_EINVAL, "values[%d] is NULL", s);
    if (d->value_row_stride[s] < d->dim || d->value_row_stride[s] > INT32_MAX)
      return fail(ATTNRES_EINVAL, "value_row_stride[%d]=%lld must be in [dim, 2^31)", s,
                  (long long)d->value_row_stride[s]);
  }
  if (d->static_keys && (d->mode != ATTNRES_MODE_SOFTMAX || d->rank == 0))
    return fail(ATTNRES_EINVAL, "static_keys apply to LR reads only");
  if (d->static_keys && d->rank > 256)
    return fail(ATTNRES_EUNSUPPORTED, "static_keys need rank <= 256, got %d", d->rank);
  if (d->mode == ATTNRES_MODE_AVERAGE) return ATTNRES_OK;
  if (d->heads < 1) return fail(ATTNRES_EINVAL, "heads=%d < 1", d->heads);
  if (d->rank == 0) {
    if (d->heads != 1) return fail(ATTNRES_EINVAL, "base read (rank 0) needs heads == 1, got %d", d->heads);
    if (!d->query) return fail(ATTNRES_EINVAL, "base read needs a [dim] query");
    if (d->query_dyn || d->gate) return fail(ATTNRES_EUNSUPPORTED, "base read has no per-token query or gate");
  } else {
    if (d->rank < 0) return fail(ATTNRES_EINVAL, "rank=%d < 0", d->rank);
    if (d->dim % d->heads || d->rank % d->heads)
      return fail(ATTNRES_EINVAL, "heads=%d must divide dim=%d and rank=%d", d->heads, d->dim, d->rank);
    if (!d->keys || !d->key_row_stride) return fail(ATTNRES_EINVAL, "LR read needs keys and key_row_stride");
    if (d->key_dtype != ATTNRES_DTYPE_F32 && d->key_dtype != ATTNRES_DTYPE_BF16 && d->key_dtype != ATTNRES_DTYPE_F16)
      return fail(ATTNRES_EINVAL, "unknown key dtype %d", d->key_dtype);
    if (d->key_dtype != d->dtype && d->gate)
      return fail(ATTNRES_EUNSUPPORTED, "a gated query needs keys in the value dtype");
    for (int s = 0; s < d->n_src; ++s) {
      if (live && !d->keys[s]) return fail(ATTNRES_EINVAL, "keys[%d] is NULL", s);
      if (d->key_row_stride[s] < d->rank || d->key_row_stride[s] > INT32_MAX)
        return fail(ATTNRES_EINVAL, "key_row_stride[%d]=%lld must be in [rank, 2^31)", s,
                    (long long)d->key_row_stride[s]);
    }
    if (!d->query && !d->query_dyn && live)
      return fail(ATTNRES_EINVAL, "LR read needs a static and/or per-token query");
    if (d->query_dyn && d->query_dyn_row_stride < d->rank)
      return fail(ATTNRES_EINVAL, "query_dyn_row_stride=%lld < rank", (long long)d->query_dyn_row_stride);
    if (d->gate && !d->query_dyn && live) return fail(ATTNRES_EINVAL, "a gate needs a per-token query");
    if (d->gate && d->gate_act != ATTNRES_GATE_LINEAR && d->gate_act != ATTNRES_GATE_SIGMOID)
      return fail(ATTNRES_EINVAL, "unknown gate activation %d", d->gate_act);
  }
  return ATTNRES_OK;
}

// dtype of the LR logit path: the reference norms keys in fp32 and rounds them
// to the value dtype, so with key_norm the logits are a value-dtype
// contraction; without it they stay in the key dtype (attnres_ops.py:4179-4186)
int logit_dtype(const attnres_read_desc* d) {
  if (d->mode != ATTNRES_MODE_SOFTMAX || d->rank == 0) return d->dtype;
  return d->key_norm ? d->dtype : d->key_dtype;
}

// Geometry shared by forward and backward.  `extra` are the other [n_tok, dim]
// buffers that must be 16-byte aligned for the vector path.
int make_plan(const attnres_read_desc* d, const void* const* extra, int n_extra, void* const* extra_src, Plan* pl) {
  const int es = elem_size(d->dtype);
  const int EV = 16 / es;
  pl->lr = d->mode == ATTNRES_MODE_SOFTMAX && d->rank > 0;
  const int heads = d->mode == ATTNRES_MODE_SOFTMAX ? d->heads : 1;
  const int dh = d->dim / heads;
  bool vec = (d->dim % EV == 0) && (dh % EV == 0);
  for (int s = 0; vec && s < d->n_src; ++s)
    vec = aligned16(d->values[s]) && ((d->value_row_stride[s] * es) % 16 == 0);
  for (int i = 0; vec && i < n_extra; ++i) vec = !extra[i] || aligned16(extra[i]);
  for (int s = 0; vec && extra_src && s < d->n_src; ++s) vec = !extra_src[s] || aligned16(extra_src[s]);
  if (vec && d->mode == ATTNRES_MODE_SOFTMAX && d->rank == 0) vec = aligned16(d->query);
  pl->vec = vec ? 1 : 0;
  pl->E = vec ? EV : 1;
  pl->vb = 16;
  pl->ncols = (d->dim + kWaveSize * pl->E - 1) / (kWaveSize * pl->E);
  pl->nmax = 0;
  if (d->mode == ATTNRES_MODE_SOFTMAX && d->rank == 0) {
    // register-resident kernels for up to 16 sources, streaming beyond
    pl->nmax = d->n_src <= 8 ? 8 : d->n_src <= 16 ? 16 : 64;
    pl->cb = vec ? 2 : 4;
    // 16-bit rows of 256 or 768 elements: 8-byte vectors fill one or three
    // whole columns of a wave (16-byte ones leave half a column idle)
    const int col8 = kWaveSize * (EV / 2);
    if (vec && es == 2 && pl->nmax <= 16 && (d->dim == col8 || d->dim == 3 * col8)) {
      pl->E = EV / 2;
      pl->vb = 8;
      pl->ncols = d->dim / col8;
      pl->cb = pl->ncols;
    }
  } else {
    pl->cb = vec ? 2 : 4;
  }
  pl->wpt = (pl->ncols + pl->cb - 1) / pl->cb;
  if (pl->wpt > 16)
    return fail(ATTNRES_EUNSUPPORTED, "dim=%d needs %d waves per token (max 16) on the %s path", d->dim, pl->wpt,
                vec ? "vector" : "unaligned");
  pl->key_vec = 0;
  if (pl->lr && d->key_dtype == d->dtype) {  // (keys of another dtype take the scalar key path)
    const int rh = d->rank / d->heads;
    bool kv = rh % EV == 0;
    for (int s = 0; kv && s < d->n_src; ++s) kv = aligned16(d->keys[s]) && ((d->key_row_stride[s] * es) % 16 == 0);
    if (kv && d->query) kv = aligned16(d->query);
    if (kv && d->static_keys) kv = aligned16(d->static_keys) && ((d->rank * es) % 16 == 0);
    if (kv && d->query_dyn) kv = aligned16(d->query_dyn) && ((d->query_dyn_row_stride * es) % 16 == 0);
    pl->key_vec = kv ? 1 : 0;
  }
  return ATTNRES_OK;
}

void fill_params(const attnres_read_desc* d, const Plan& pl, ReadParams* p) {
  memset(p, 0, sizeof(*p));
  for (int s = 0; s < d->n_src; ++s) {
    p->val[s] = d->values[s];
    p->vstride[s] = (int32_t)d->value_row_stride[s];
    if (pl.lr) {
      p->key[s] = d->keys[s];
      p->kstride[s] = (int32_t)d->key_row_stride[s];
    }
  }
  const bool softmax = d->mode == ATTNRES_MODE_SOFTMAX;
  p->q_static = softmax ? d->query : nullptr;
  p->q_dyn = softmax ? d->query_dyn : nullptr;
  p->q_dyn_stride = d->query_dyn_row_stride;
  p->gate = softmax ? d->gate : nullptr;
  p->bias = softmax ? d->logit_bias : nullptr;
  p->n_tok = d->n_tok;
  p->n_src = d->n_src;
  p->D = d->dim;
  p->H = softmax ? d->heads : 1;
  p->R = pl.lr ? d->rank : 0;
  p->rh = pl.lr ? d->rank / d->heads : 0;
  p->dh = d->dim / p->H;
  p->ncols = pl.ncols;
  p->wpt = pl.wpt;
  p->key_norm = d->key_norm ? 1 : 0;
  p->norm_out = d->normalize_output ? 1 : 0;
  p->mode = d->mode;
  p->gate_per_token = d->gate_per_token ? 1 : 0;
  p->gate_act = d->gate_act;
  p->key_vec = pl.key_vec;
  p->scale = pl.lr ? d->logit_scale : 1.0f;
  p->eps = d->norm_eps;
  p->kdt = pl.lr ? d->key_dtype : d->dtype;
  p->ldt = logit_dtype(d);
  p->skey = pl.lr ? d->static_keys : nullptr;
}

// The static keys' gradient: per-source token sums of dkeys, partial sums
// per token chunk in the workspace after the cross-token partial rows.
// LDS bytes of the static keys in the fast LR kernels ([n_src, rank] in the
// dtype, rows one 16-byte chunk apart more than rank)
size_t static_keys_lds(const attnres_read_desc* d) {
  return d->static_keys ? (size_t)d->n_src * ((size_t)d->rank * elem_size(d->dtype) + 16) : 0;
}

int colsum_chunks(int64_t n_tok) {
  const int64_t c = (n_tok + kColsumTokens - 1) / kColsumTokens;
  return (int)(c < 1 ? 1 : c < kColsumMaxChunks ? c : kColsumMaxChunks);
}
size_t colsum_bytes(const attnres_read_desc* d) {
  if (!d->static_keys || d->rank <= 0 || d->n_tok == 0) return 0;
  return (size_t)d->n_src * colsum_chunks(d->n_tok) * d->rank * sizeof(float);
}

struct PartLayout {
  int n_part, part_q, n_q, part_gate, n_gate, part_bias, n_bias;
};

PartLayout part_layout(const attnres_read_desc* d, bool want_q, bool want_gate, bool want_bias) {
  PartLayout L{0, -1, 0, -1, 0, -1, 0};
  if (d->mode != ATTNRES_MODE_SOFTMAX) return L;
  const bool lr = d->rank > 0;
  if (want_q && d->query) {
    L.part_q = L.n_part;
    L.n_q = lr ? d->rank : d->dim;
    L.n_part += L.n_q;
  }
  if (want_gate && lr && d->gate && d->query_dyn && !d->gate_per_token) {
    L.part_gate = L.n_part;
    L.n_gate = d->heads;
    L.n_part += L.n_gate;
  }
  if (want_bias && d->logit_bias) {
    L.part_bias = L.n_part;
    L.n_bias = d->n_src;
    L.n_part += L.n_bias;
  }
  return L;
}

// Zeroes `bytes` bytes with a kernel on the caller's stream.  A memset node
// would do the same, but callers may capture these calls in a HIP graph, where
// a kernel node is the safer form.  Used only for the gradients of empty inputs
// (a few KB at most).
__global__ void zero_bytes_kernel(unsigned char* p, size_t bytes) {
  for (size_t i = threadIdx.x; i < bytes; i += blockDim.x) p[i] = 0;
}
void zero_async(void* p, size_t bytes, hipStream_t st) {
  if (p && bytes) hipLaunchKernelGGL(zero_bytes_kernel, dim3(1), dim3(256), 0, st, (unsigned char*)p, bytes);
}

int64_t bwd_groups(int64_t n_tok) { return n_tok < kMaxBwdGroups ? n_tok : kMaxBwdGroups; }

// LR fast path: one wave per (token, head-aligned column group).  Returns false
// when the shape is outside what the fast kernels support.
struct FastPlan {
  int vb, cb, nb, rhc, n_items, nh, kch, np;
};

bool lr_fast_plan(const attnres_read_desc* d, const Plan& pl, bool backward, FastPlan* f) {
  if (!pl.lr || !pl.vec || !pl.key_vec) return false;
  const int es = elem_size(d->dtype);
  f->vb = 16;  // 16-byte lane vectors
  const int E = f->vb / es;
  const int colw = kWaveSize * E;
  const int dh = d->dim / d->heads, rh = d->rank / d->heads;
  if (dh <= colw) {
    if (colw % dh) return false;
    f->cb = 1;
    f->nh = colw / dh;
  } else if (dh == 2 * colw && f->vb == 16) {
    f->cb = 2;
    f->nh = 1;
  } else {
    return false;
  }
  if (f->nh > d->heads) f->nh = d->heads;
  f->n_items = (d->dim + f->cb * colw - 1) / (f->cb * colw);
  if (d->normalize_output && f->n_items != 1) return false;
  const int N = d->n_src;
  if (N > (f->cb == 2 ? 16 : 32)) return false;
  f->np = 2;  // at least two lanes per head: the packed mix reads source pairs
  while (f->np < N) f->np <<= 1;
  // 32-bit token index and byte strides in the fast kernels' address math
  if (d->n_tok > INT32_MAX) return false;
  for (int s = 0; s < N; ++s)
    if ((uint64_t)d->value_row_stride[s] * es > UINT32_MAX || (uint64_t)d->key_row_stride[s] * es > UINT32_MAX)
      return false;
  if (f->np * f->nh > 64 || f->nh * rh > 64) return false;
  // the backward sums the gate gradient over each head's rh lanes (aligned groups)
  if (backward && d->gate && (rh & (rh - 1))) return false;
  if ((rh * es) % 16) return false;
  f->kch = rh * es / 16;
  if (f->kch > 8) return false;
  f->rhc = f->kch <= 2 ? 2 : 8;
  // value slots: the kernels load NB rows per token whatever N is (branch-free
  // unrolled loads; slots past N re-read a real row), so each slot past N is a
  // wasted load instruction.  The common shape (one column per wave, short key
  // slices) is instantiated for slot counts close together.
  f->nb = N <= 8 ? 8 : N <= 16 ? 16 : 32;
  if (f->cb == 1 && f->rhc == 2) {
    static const int kFineSlots[] = {8, 12, 14, 16, 18, 20, 24, 32};
    for (int nb : kFineSlots)
      if (N <= nb) {
        f->nb = nb;
        break;
      }
  }
  if (N < lr_fast_slot_floor(f->cb, f->rhc, f->nb)) return false;  // (the kernels assume the floor)
  if (f->cb == 2 && f->rhc == 8 && f->nb == 16) return false;  // no register room
  if (f->cb == 1 && f->rhc == 8 && f->vb == 16 && f->nb == 32) return false;  // not instantiated
  return true;
}

// Base-key fast path (attnres_base_fast.h): 16-bit rows that one wave covers
// exactly with 8-byte (D = 256, 768) or 16-byte (D = 512, 1024) lane vectors,
// up to 16 sources, no output norm.  vb / cb / nb = vector bytes, columns per
// lane, source slots.
struct BaseFastPlan {
  int vb, cb, nb;
};

// Token streams of the fast base kernels: one resident round of waves (16 per
// CU: four waves on each SIMD, the occupancy both kernels reach at d=768), each
// walking tokens with that stride.  Measured at C2 (8192 tokens): one round
// with two tokens per wave beats 8192 one-token waves (forward 18.8 vs 19.8
// us, backward 52.9 vs 57.7 us with the reduction) and half a round.
int64_t base_fast_streams() {
  static const int64_t v = [] {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    return (int64_t)cus * 16;
  }();
  return v;
}

bool base_fast_plan(const attnres_read_desc* d, const Plan& pl, BaseFastPlan* f) {
  if (d->mode != ATTNRES_MODE_SOFTMAX || pl.lr || !pl.vec || elem_size(d->dtype) != 2) return false;
  if (d->normalize_output || d->n_src > 16 || !d->query) return false;
  switch (d->dim) {
    case 256: f->vb = 8; f->cb = 1; break;
    case 512: f->vb = 16; f->cb = 1; break;
    case 768: f->vb = 8; f->cb = 3; break;
    case 1024: f->vb = 16; f->cb = 2; break;
    default: return false;
  }
  // 32-bit token index and byte strides in the kernels' address math
  if (d->n_tok > INT32_MAX) return false;
  for (int s = 0; s < d->n_src; ++s)
    if ((uint64_t)d->value_row_stride[s] * 2 > UINT32_MAX) return false;
  // source slots: the exact count up to 8 (a slot past n_src is a wasted row
  // load and its arithmetic: C2's N = 7 in 8 slots cost 4% of the backward),
  // then 10 / 12 / 14 / 16
  const int N = d->n_src;
  f->nb = N <= 1 ? 2 : N <= 8 ? N : (N + 1) / 2 * 2;
  return true;
}

// Optional code the fast LR kernels must carry for a read, rounded up to an
// instantiated set: 0 (static query, no output norm), kFeatDyn (per-token query
// / gate), kFeatDyn | kFeatStatic (and static source keys) or kFeatAll.
int lr_fast_features(const attnres_read_desc* d) {
  if (d->normalize_output) return kFeatAll;
  if (d->static_keys) return kFeatDyn | kFeatStatic;
  return (d->query_dyn || d->gate) ? kFeatDyn : 0;
}

// token teams per LR-backward workgroup: four independent one-wave teams when a
// token fits one wave, else one team of wpt waves
int lr_bwd_teams(const Plan& pl) { return pl.wpt == 1 ? 4 : 1; }

size_t lr_bwd_lds(const attnres_read_desc* d, const Plan& pl, int n_part) {
  const int HN = d->heads * d->n_src;
  const int cph_full = (d->dim / d->heads) / pl.E;
  int gl = cph_full & (-cph_full);
  if (gl > kWaveSize) gl = kWaveSize;
  const int gpc = kWaveSize / gl;
  const size_t floats =
      5 * (size_t)HN + (size_t)d->n_src * pl.ncols * gpc + (size_t)d->n_src * d->rank + d->rank + n_part + 32;
  return floats * sizeof(float) * lr_bwd_teams(pl);
}

}  // namespace

extern "C" int attnres_abi_version(void) { return ATTNRES_ABI_VERSION; }

extern "C" const char* attnres_last_error(void) { return g_last_error.c_str(); }

extern "C" int attnres_kernel_timing(int enable) {
  if (enable && !g_timer.on) {
    for (int i = 0; i < 2 * kTimerPairs; ++i) {
      const hipError_t e = hipEventCreate(&g_timer.ev[i]);
      if (e != hipSuccess) {
        for (int j = 0; j < i; ++j) (void)hipEventDestroy(g_timer.ev[j]);
        return fail(ATTNRES_ELAUNCH, "hipEventCreate failed: %s", hipGetErrorString(e));
      }
    }
    g_timer.on = true;
    g_timer.failed = false;
    g_timer.n = 0;
  } else if (!enable && g_timer.on) {
    for (int i = 0; i < 2 * kTimerPairs; ++i) (void)hipEventDestroy(g_timer.ev[i]);
    g_timer.on = false;
    g_timer.failed = false;
    g_timer.n = 0;
  }
  return ATTNRES_OK;
}

extern "C" int attnres_kernel_times(float* ms, int max_n) {
  if (!g_timer.on) return fail(ATTNRES_EINVAL, "kernel timing is not enabled");
  if (max_n < 0 || (max_n > 0 && !ms)) return fail(ATTNRES_EINVAL, "bad output buffer");
  if (g_timer.failed) {
    g_timer.failed = false;
    g_timer.n = 0;
    return fail(ATTNRES_ELAUNCH, "a kernel timing event record failed; the recording is discarded");
  }
  const int n = g_timer.n < max_n ? g_timer.n : max_n;
  for (int i = 0; i < n; ++i) {
    hipError_t e = hipEventSynchronize(g_timer.ev[2 * i + 1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms[i], g_timer.ev[2 * i], g_timer.ev[2 * i + 1]);
    if (e != hipSuccess) return fail(ATTNRES_ELAUNCH, "kernel timing event failed: %s", hipGetErrorString(e));
  }
  const int recorded = g_timer.n;
  g_timer.n = 0;
  return recorded < max_n ? recorded : max_n;
}

extern "C" int attnres_test_phase2_block_layout(int on) {
  if (on != 0 && on != 1) return fail(ATTNRES_EINVAL, "on must be 0 or 1, got %d", on);
  g_phase2_block_layout.store(on, std::memory_order_relaxed);
  return ATTNRES_OK;
}

// bytes of the cross-token partial rows (the largest layout), padded so that
// the static keys' column sums start on a 256-byte boundary after them
size_t partial_rows_bytes(const attnres_read_desc* d) {
  const PartLayout L = part_layout(d, true, true, true);
  if (L.n_part == 0 || d->n_tok == 0) return 0;
  return ((size_t)bwd_groups(d->n_tok) * L.n_part * sizeof(float) + 255) / 256 * 256;
}

extern "C" size_t attnres_read_backward_workspace_size(const attnres_read_desc* d) {
  if (check_desc(d) != ATTNRES_OK) return 0;
  const size_t cs = colsum_bytes(d);
  const PartLayout L = part_layout(d, true, true, true);
  if (d->n_tok == 0) return 0;
  if (cs == 0) return L.n_part == 0 ? 0 : (size_t)bwd_groups(d->n_tok) * L.n_part * sizeof(float);
  return partial_rows_bytes(d) + cs;
}

extern "C" int attnres_read_forward(const attnres_read_desc* d, void* out, void* out_prenorm, float* weights,
                                    float* out_inv_rms, void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!out) return fail(ATTNRES_EINVAL, "out is NULL");
  Plan pl;
  const void* extra[2] = {out, d->normalize_output ? out_prenorm : nullptr};
  rc = make_plan(d, extra, 2, nullptr, &pl);
  if (rc) return rc;
  ReadParams p;
  fill_params(d, pl, &p);
  p.out = out;
  p.out_prenorm = d->normalize_output ? out_prenorm : nullptr;
  p.weights = weights;
  p.out_inv_rms = out_inv_rms;

  Launch L;
  memset(&L, 0, sizeof(L));
  L.vec = pl.vec;
  L.vb = pl.vb;
  L.wpt = pl.wpt;
  L.nmax = pl.nmax;
  L.teams = 1;
  L.grid = (int)(d->n_tok < kMaxFwdGroups ? d->n_tok : kMaxFwdGroups);
  hipStream_t st = (hipStream_t)stream;
  hipError_t err;
  const bool timed = timer_begin(st);
  if (d->mode == ATTNRES_MODE_AVERAGE) {
    L.lds = 32 * sizeof(float);
    err = launch_average_forward(d->dtype, p, L, st);
  } else if (pl.lr) {
    FastPlan f;
    if (lr_fast_plan(d, pl, false, &f)) {
      const int64_t streams = d->n_tok < 16384 / f.n_items ? d->n_tok : 16384 / f.n_items;
      p.n_items = f.n_items;
      p.nh = f.nh;
      p.kch = f.kch;
      p.np = f.np;
      p.streams = (int32_t)(streams > 0 ? streams : 1);
      L.vec = f.vb;
      L.wpt = f.cb;
      L.nmax = f.nb;
      L.teams = f.rhc;
      L.feat = lr_fast_features(d);
      L.grid = (int)((f.n_items * (int64_t)p.streams + 3) / 4);
      L.lds = lr_fast_table_bytes() + ((size_t)d->rank + 4 * 64) * sizeof(float) + static_keys_lds(d) +
              4 * (size_t)lr_fast_staged_rows(f.cb, f.rhc, f.nb, elem_size(d->dtype), lr_fast_features(d)) * 1024;
      if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "LR forward needs %zu bytes of LDS", L.lds);
      err = launch_lr_fast_forward(d->dtype, p, L, st);
    } else {
      L.lds = (2 * (size_t)d->heads * d->n_src + 32) * sizeof(float);
      if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "LDS need %zu bytes", L.lds);
      err = launch_lr_forward(d->dtype, p, L, st);
    }
  } else {
    BaseFastPlan f;
    if (base_fast_plan(d, pl, &f)) {
      const int64_t cap = base_fast_streams();
      p.streams = (int32_t)(d->n_tok < cap ? d->n_tok : cap);
      L.vb = f.vb;
      L.wpt = f.cb;
      L.nmax = f.nb;
      L.grid = (int)((p.streams + 3) / 4);
      L.lds = lr_fast_table_bytes();
      err = launch_base_fast_forward(d->dtype, p, L, st);
    } else {
      L.lds = (pl.nmax <= 16 ? (size_t)pl.wpt * pl.nmax + 32 : (size_t)d->n_src + 32) * sizeof(float);
      err = launch_base_forward(d->dtype, p, L, st);
    }
  }
  timer_end(st, timed, err);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_read_backward(const attnres_read_desc* d, const attnres_read_grads* g, void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!g) return fail(ATTNRES_EINVAL, "grads is NULL");
  const bool softmax = d->mode == ATTNRES_MODE_SOFTMAX;
  const bool lr = softmax && d->rank > 0;
  if (d->n_tok > 0) {
    if (!g->grad_out) return fail(ATTNRES_EINVAL, "grad_out is NULL");
    if (!g->dvalues) return fail(ATTNRES_EINVAL, "dvalues is NULL");
    for (int s = 0; s < d->n_src; ++s)
      if (!g->dvalues[s]) return fail(ATTNRES_EINVAL, "dvalues[%d] is NULL", s);
    if (softmax && !g->weights) return fail(ATTNRES_EINVAL, "the backward needs the saved softmax weights");
    if (d->normalize_output && (!g->out_prenorm || !g->out_inv_rms))
      return fail(ATTNRES_EINVAL, "normalize_output backward needs out_prenorm and out_inv_rms");
    if (lr) {
      if (!g->dkeys) return fail(ATTNRES_EINVAL, "LR backward needs dkeys");
      for (int s = 0; s < d->n_src; ++s)
        if (!g->dkeys[s]) return fail(ATTNRES_EINVAL, "dkeys[%d] is NULL", s);
      if (d->query_dyn && !g->dquery_dyn) return fail(ATTNRES_EINVAL, "per-token query needs dquery_dyn");
      if (g->dstatic_keys && !d->static_keys) return fail(ATTNRES_EINVAL, "dstatic_keys without static_keys");
      if (d->gate && d->gate_per_token && !g->dgate) return fail(ATTNRES_EINVAL, "per-token gate needs dgate");
    }
  }
  if (d->n_tok == 0) {
    // gradients of the cross-token quantities are zero
    hipStream_t st = (hipStream_t)stream;
    const int es = elem_size(d->dtype);
    if (softmax && g->dquery && d->query)
      zero_async(g->dquery, (size_t)(lr ? d->rank : d->dim) * elem_size(logit_dtype(d)), st);
    if (softmax && g->dgate && d->gate && !d->gate_per_token) zero_async(g->dgate, (size_t)d->heads * es, st);
    if (softmax && g->dbias && d->logit_bias) zero_async(g->dbias, (size_t)d->n_src * 4, st);
    if (lr && g->dstatic_keys && d->static_keys)
      zero_async(g->dstatic_keys, (size_t)d->n_src * d->rank * elem_size(d->key_dtype), st);
    return ATTNRES_OK;
  }
  Plan pl;
  const void* extra[2] = {g->grad_out, d->normalize_output ? g->out_prenorm : nullptr};
  rc = make_plan(d, extra, 2, g->dvalues, &pl);
  if (rc) return rc;

  ReadBwdParams bp;
  memset(&bp, 0, sizeof(bp));
  fill_params(d, pl, &bp.f);
  bp.f.out_prenorm = const_cast<void*>(g->out_prenorm);
  bp.gout = g->grad_out;
  bp.saved_w = g->weights;
  bp.saved_inv = g->out_inv_rms;
  for (int s = 0; s < d->n_src; ++s) {
    bp.dval[s] = g->dvalues[s];
    if (lr) bp.dkey[s] = g->dkeys[s];
  }
  bp.dq_dyn = lr ? g->dquery_dyn : nullptr;
  bp.dgate = lr ? g->dgate : nullptr;

  const PartLayout PL = part_layout(d, g->dquery != nullptr, g->dgate != nullptr, g->dbias != nullptr);
  const int64_t groups = bwd_groups(d->n_tok);
  if (PL.n_part > 0) {
    const size_t need = (size_t)groups * PL.n_part * sizeof(float);
    if (!g->workspace || g->workspace_bytes < need)
      return fail(ATTNRES_EWORKSPACE, "workspace of %zu bytes needed, got %zu", need,
                  g->workspace ? g->workspace_bytes : (size_t)0);
    bp.partials = (float*)g->workspace;
  }
  // the static keys' column sums follow the partial rows in the workspace:
  // checked here, before anything is launched, so a too-small workspace leaves
  // every output untouched
  if (lr && g->dstatic_keys) {
    const size_t need = partial_rows_bytes(d) + colsum_bytes(d);
    if (!g->workspace || g->workspace_bytes < need)
      return fail(ATTNRES_EWORKSPACE, "workspace of %zu bytes needed, got %zu", need,
                  g->workspace ? g->workspace_bytes : (size_t)0);
  }
  bp.n_part = PL.n_part;
  bp.part_q = PL.part_q;
  bp.part_gate = PL.part_gate;
  bp.part_bias = PL.part_bias;

  Launch L;
  memset(&L, 0, sizeof(L));
  L.vec = pl.vec;
  L.vb = pl.vb;
  L.wpt = pl.wpt;
  L.nmax = pl.nmax;
  L.teams = 1;
  const int64_t full_groups = groups < kFullBwdGroups ? groups : kFullBwdGroups;
  L.grid = (int)full_groups;
  if (lr) L.teams = lr_bwd_teams(pl);
  else if (softmax && pl.nmax <= 16 && pl.wpt == 1) L.teams = 4;  // resident base read, one wave per token
  if (L.teams > 1) {
    // workgroups carry `teams` tokens at a time; the workspace is sized for
    // `groups` partials and the grid never exceeds it
    const int64_t need = (d->n_tok + L.teams - 1) / L.teams;
    L.grid = (int)(need < full_groups ? need : full_groups);
  }
  hipStream_t st = (hipStream_t)stream;
  int partials_layout = kPartRowMajor;  // fast LR: slot-major; fast base: tiled (slot-major for tiny inputs)
  BaseFastPlan bf;
  hipError_t err;
  const bool timed = timer_begin(st);
  if (d->mode == ATTNRES_MODE_AVERAGE) {
    L.lds = 32 * sizeof(float);
    err = launch_average_backward(d->dtype, bp, L, st);
  } else if (lr) {
    FastPlan f;
    int64_t streams = 0;
    const int feat = lr_fast_features(d);
    if (lr_fast_plan(d, pl, true, &f)) {
      // at most `groups` workgroups of four waves (the workspace rows); the
      // instantiations with all optional code (fewer waves per SIMD) stream
      // best with 2048 workgroups, the leaner ones with twice as many
      // (measured at C3 and C4)
      const int64_t cap = feat != kFeatAll ? groups : (groups < kFullBwdGroups ? groups : kFullBwdGroups);
      streams = 4 * cap / f.n_items;
      if (streams > d->n_tok) streams = d->n_tok;
    }
    if (streams > 0) {
      bp.f.n_items = f.n_items;
      bp.f.nh = f.nh;
      bp.f.kch = f.kch;
      bp.f.np = f.np;
      bp.f.streams = (int32_t)streams;
      L.vec = f.vb;
      L.wpt = f.cb;
      L.nmax = f.nb;
      L.teams = f.rhc;
      L.feat = feat;
      L.grid = (int)((f.n_items * streams + 3) / 4);
      L.lds = lr_fast_table_bytes() +
              ((size_t)d->rank + 4 * (192 + (size_t)f.np * f.nh * (d->rank / d->heads + 1)) +
               (4 * (size_t)PL.n_part + 3) / 4 * 4) *
                  sizeof(float) +
              static_keys_lds(d) + 4 * (size_t)lr_fast_staged_rows(f.cb, f.rhc, f.nb, elem_size(d->dtype), lr_fast_features(d)) * 1024;
      if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "LR backward needs %zu bytes of LDS", L.lds);
      // slot-major partials (R + few slots: one reduction workgroup per slot
      // beats 16-slot tiles here, measured at C3 and C4)
      partials_layout = kPartSlotMajor;
      err = launch_lr_fast_backward(d->dtype, bp, L, st);
    } else {
      L.lds = lr_bwd_lds(d, pl, PL.n_part);
      if (L.lds > lds_limit())
        return fail(ATTNRES_EUNSUPPORTED, "LR backward needs %zu bytes of LDS (limit %zu)", L.lds, lds_limit());
      err = launch_lr_backward(d->dtype, bp, L, st);
    }
  } else if (base_fast_plan(d, pl, &bf)) {
    // four token streams per workgroup, one resident round of waves and at
    // most `groups` workgroups (the workspace rows); partials slot-major like
    // the fast LR backward
    const int64_t cap = groups * 4 < base_fast_streams() ? groups * 4 : base_fast_streams();
    bp.f.streams = (int32_t)(d->n_tok < cap ? d->n_tok : cap);
    L.vb = bf.vb;
    L.wpt = bf.cb;
    L.nmax = bf.nb;
    L.grid = (int)((bp.f.streams + 3) / 4);
    L.lds = lr_fast_table_bytes() + base_bwd_fast_lds(PL.n_part);
    if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "base backward needs %zu bytes of LDS", L.lds);
    // D query slots per workgroup: tiles of 16 (64-byte runs) rather than
    // slot-major rows, whose 4-byte writes to a new line per slot cost a
    // partial-line write each (a fifth of the backward's bytes at D=768);
    // slot-major when the padded tiles would not fit the workspace (tiny inputs)
    partials_layout =
        (size_t)L.grid * part_stride(PL.n_part) <= (size_t)groups * PL.n_part ? kPartTiled : kPartSlotMajor;
    bp.part_layout = partials_layout;
    err = launch_base_fast_backward(d->dtype, bp, L, st);
  } else {
    size_t fl = pl.nmax <= 16 ? (size_t)pl.wpt * pl.nmax + 32 : 2 * (size_t)d->n_src + 32;
    if ((size_t)L.teams * PL.n_part > fl) fl = (size_t)L.teams * PL.n_part;
    L.lds = fl * sizeof(float);
    if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "base backward needs %zu bytes of LDS", L.lds);
    err = launch_base_backward(d->dtype, bp, L, st);
  }
  timer_end(st, timed, err);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "backward launch failed: %s", hipGetErrorString(err));

  if (PL.n_part > 0) {
    ReduceParams rp;
    memset(&rp, 0, sizeof(rp));
    rp.partials = bp.partials;
    rp.n_groups = L.grid;
    rp.n_part = PL.n_part;
    rp.layout = partials_layout;
    rp.part_q = PL.part_q;
    rp.n_q = PL.n_q;
    rp.part_gate = PL.part_gate;
    rp.n_gate = PL.n_gate;
    rp.part_bias = PL.part_bias;
    rp.n_bias = PL.n_bias;
    rp.dquery = g->dquery;
    rp.dgate = g->dgate;
    rp.dbias = g->dbias;
    rp.part_extra = -1;
    rp.n_extra = 0;
    rp.dextra = nullptr;
    err = launch_reduce_partials(logit_dtype(d), rp, st);  // the query gradient is in the logit dtype
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "reduce launch failed: %s", hipGetErrorString(err));
  }
  if (lr && g->dstatic_keys) {  // (workspace size checked above)
    ColsumParams cp;
    memset(&cp, 0, sizeof(cp));
    for (int s = 0; s < d->n_src; ++s) cp.dk[s] = g->dkeys[s];
    cp.partials = (float*)((char*)g->workspace + partial_rows_bytes(d));
    cp.out = g->dstatic_keys;
    cp.n_tok = d->n_tok;
    cp.n_src = d->n_src;
    cp.R = d->rank;
    cp.chunks = colsum_chunks(d->n_tok);
    cp.kdt = d->key_dtype;
    err = launch_key_colsum(cp, st);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "static-key gradient launch failed: %s", hipGetErrorString(err));
  }
  return ATTNRES_OK;
}

// ------------------------------------------------------- no-allocation backward
// The backward's cross-token partial sums in a fixed array inside the library
// instead of a caller workspace.  Each GPU holds its own copy from the first
// call on it until the process ends.  In host code `scratch` is only a stand-in
// for the device symbol: its device address comes from hipGetSymbolAddress,
// looked up once per device with that device current.  No call clears it:
// every partial-sum slot the reduction reads is written by the same call.
static __device__ __align__(256) unsigned char scratch[ATTNRES_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(ATTNRES_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(ATTNRES_EUNSUPPORTED, "device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(ATTNRES_ELAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ATTNRES_OK;
}

}  // namespace

extern "C" int attnres_read_backward_noalloc(const attnres_read_desc* d, const attnres_read_grads* g, void* stream) {
  int rc = check_desc(d);
  if (rc) return rc;
  if (!g) return fail(ATTNRES_EINVAL, "grads is NULL");
  const size_t need = attnres_read_backward_workspace_size(d);
  if (need > (size_t)ATTNRES_NOALLOC_SCRATCH_BYTES)
    return fail(ATTNRES_EWORKSPACE, "this backward needs %zu bytes of partial sums; the no-allocation entry point "
                "holds %zu (use attnres_read_backward with a workspace)", need, (size_t)ATTNRES_NOALLOC_SCRATCH_BYTES);
  attnres_read_grads g2 = *g;
  g2.workspace = nullptr;
  g2.workspace_bytes = 0;
  if (need > 0) {
    rc = scratch_address(&g2.workspace);
    if (rc) return rc;
    g2.workspace_bytes = ATTNRES_NOALLOC_SCRATCH_BYTES;
  }
  return attnres_read_backward(d, &g2, stream);
}

// ====================================================================== phases
namespace {

struct PhasePlan {
  int vec, E, cb, ncols, wpt;
  int vb;  // vector bytes of the vector path
};

// Row geometry of the phase kernels: one 16-byte vector per column when every
// row is aligned (fp32: two columns per lane), else eight single-element
// columns per lane; at most 8 waves per token.  With `rows8`, 16-bit rows of
// 256 or 768 elements take one wave of 8-byte vectors (one or three columns
// per lane, every lane busy) instead of one or two waves of 16-byte vectors
// with idle lanes; `rows8` is the largest column count allowed (0: off).
int phase_plan(int dtype, int dim, const void* const* rows, const int64_t* strides, int n_rows, PhasePlan* pl,
               int rows8 = 0) {
  const int es = elem_size(dtype);
  const int EV = 16 / es;
  bool vec = dim % EV == 0;
  for (int i = 0; vec && i < n_rows; ++i)
    vec = (!rows[i] || aligned16(rows[i])) && ((strides[i] * es) % 16 == 0);
  pl->vec = vec ? 1 : 0;
  pl->vb = 16;
  pl->E = vec ? EV : 1;
  pl->cb = vec ? (es == 4 ? 2 : 1) : 8;
  pl->ncols = (dim + kWaveSize * pl->E - 1) / (kWaveSize * pl->E);
  const int col8 = kWaveSize * (EV / 2);
  if (vec && es == 2 && ((dim == col8 && rows8 >= 1) || (dim == 3 * col8 && rows8 >= 3))) {
    pl->vb = 8;
    pl->E = EV / 2;
    pl->ncols = dim / col8;
    pl->cb = pl->ncols;
  }
  pl->wpt = (pl->ncols + pl->cb - 1) / pl->cb;
  if (pl->wpt > 8) return fail(ATTNRES_EUNSUPPORTED, "dim=%d exceeds the phase kernels' row width", dim);
  return ATTNRES_OK;
}

int check_phase1(const attnres_phase1_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->n_src < 1 || d->n_src > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_EUNSUPPORTED, "n_src=%d outside [1, %d]", d->n_src, ATTNRES_MAX_SOURCES);
  if (d->n_q < 1 || d->n_q > ATTNRES_PHASE1_MAX_QUERIES)
    return fail(ATTNRES_EUNSUPPORTED, "n_q=%d outside [1, %d]", d->n_q, ATTNRES_PHASE1_MAX_QUERIES);
  if (d->dtype < 0 || d->dtype > 2 || d->logits_dtype < 0 || d->logits_dtype > 2)
    return fail(ATTNRES_EINVAL, "unknown dtype %d / logits dtype %d", d->dtype, d->logits_dtype);
  if (d->n_tok < 0) return fail(ATTNRES_EINVAL, "n_tok=%lld < 0", (long long)d->n_tok);
  if (d->dim < 1 || d->dim > ATTNRES_PHASE_MAX_DIM)
    return fail(ATTNRES_EUNSUPPORTED, "dim=%d outside [1, %d]", d->dim, ATTNRES_PHASE_MAX_DIM);
  if (!d->values || !d->value_row_stride) return fail(ATTNRES_EINVAL, "values / value_row_stride is NULL");
  const bool live = d->n_tok > 0;
  for (int s = 0; s < d->n_src; ++s) {
    if (live && !d->values[s]) return fail(ATTNRES_EINVAL, "values[%d] is NULL", s);
    if (d->value_row_stride[s] < d->dim || d->value_row_stride[s] > INT32_MAX)
      return fail(ATTNRES_EINVAL, "value_row_stride[%d]=%lld must be in [dim, 2^31)", s,
                  (long long)d->value_row_stride[s]);
  }
  if (d->source_logits) {
    for (int s = 0; s < d->n_src; ++s)
      if (live && !d->source_logits[s]) return fail(ATTNRES_EINVAL, "source_logits[%d] is NULL", s);
    if (d->logit_q_stride < d->n_tok)
      return fail(ATTNRES_EINVAL, "logit_q_stride %lld < n_tok=%lld", (long long)d->logit_q_stride,
                  (long long)d->n_tok);
    return ATTNRES_OK;
  }
  if (live && !d->logits) return fail(ATTNRES_EINVAL, "logits is NULL");
  if (d->logit_s_stride < d->n_tok || d->logit_q_stride < (int64_t)d->n_src * d->n_tok)
    return fail(ATTNRES_EINVAL, "logit strides (%lld, %lld) overlap for n_tok=%lld, S=%d", (long long)d->logit_q_stride,
                (long long)d->logit_s_stride, (long long)d->n_tok, d->n_src);
  return ATTNRES_OK;
}

// true when ptr[i] = ptr[0] + i * stride for one stride in elements of es bytes
// (returned in *stride); a single pointer is trivially uniform
bool uniform_stride(const void* const* ptr, int n, size_t es, int64_t* stride) {
  *stride = 0;
  if (n <= 1) return true;
  const int64_t d = (int64_t)((intptr_t)ptr[1] - (intptr_t)ptr[0]);
  if (d % (int64_t)es) return false;
  for (int i = 2; i < n; ++i)
    if ((int64_t)((intptr_t)ptr[i] - (intptr_t)ptr[0]) != d * i) return false;
  *stride = d / (int64_t)es;
  return true;
}

void fill_phase1(const attnres_phase1_desc* d, const PhasePlan& pl, Phase1Params* p) {
  memset(p, 0, sizeof(*p));
  for (int s = 0; s < d->n_src; ++s) {
    p->val[s] = d->values[s];
    p->vstride[s] = (int32_t)d->value_row_stride[s];
  }
  const size_t les = elem_size(d->logits_dtype);
  for (int s = 0; s < d->n_src; ++s)
    p->lsrc[s] = d->source_logits ? d->source_logits[s]
                                  : (const void*)((const char*)d->logits + (size_t)s * d->logit_s_stride * les);
  p->lq = d->logit_q_stride;
  p->stacked = uniform_stride(p->lsrc, d->n_src, les, &p->ls) ? 1 : 0;  // the backward refines it
  p->n_tok = d->n_tok;
  p->n_src = d->n_src;
  p->n_q = d->n_q;
  p->D = d->dim;
  p->ncols = pl.ncols;
  p->ldt = d->logits_dtype;
  p->norm_out = d->normalize_output ? 1 : 0;
  p->np = 1;
  while (p->np < d->n_src) p->np <<= 1;
  p->eps = d->norm_eps;
}

int check_phase2(const attnres_phase2_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->dtype < 0 || d->dtype > 2) return fail(ATTNRES_EINVAL, "unknown dtype %d", d->dtype);
  if (d->n_tok < 0) return fail(ATTNRES_EINVAL, "n_tok=%lld < 0", (long long)d->n_tok);
  if (d->dim < 1 || d->dim > ATTNRES_PHASE_MAX_DIM)
    return fail(ATTNRES_EUNSUPPORTED, "dim=%d outside [1, %d]", d->dim, ATTNRES_PHASE_MAX_DIM);
  if (d->merge != ATTNRES_MERGE_ADDCMUL && d->merge != ATTNRES_MERGE_LERP)
    return fail(ATTNRES_EINVAL, "unknown merge %d", d->merge);
  if (d->rank < 0 || d->rank > 4 * 64 * 8) return fail(ATTNRES_EUNSUPPORTED, "rank=%d outside [0, 2048]", d->rank);
  const bool live = d->n_tok > 0;
  if (live && (!d->partial_value || !d->interblock_output || !d->interblock_lse))
    return fail(ATTNRES_EINVAL, "partial_value / interblock_output / interblock_lse is NULL");
  if (d->partial_value_row_stride < d->dim || d->partial_value_row_stride > INT32_MAX ||
      d->interblock_row_stride < d->dim || d->interblock_row_stride > INT32_MAX)
    return fail(ATTNRES_EINVAL, "row strides must be in [dim, 2^31)");
  if (d->logit_given) {
    if (live && !d->partial_logit) return fail(ATTNRES_EINVAL, "logit_given needs partial_logit");
    if (d->partial_logit_dtype < 0 || d->partial_logit_dtype > 2)
      return fail(ATTNRES_EINVAL, "unknown partial_logit dtype %d", d->partial_logit_dtype);
  } else {
    if (live && !d->query) return fail(ATTNRES_EINVAL, "query is NULL");
    if (d->rank > 0) {
      if (live && !d->partial_key) return fail(ATTNRES_EINVAL, "LR merge needs partial_key");
      if (d->partial_key_row_stride < d->rank) return fail(ATTNRES_EINVAL, "partial_key_row_stride < rank");
    }
  }
  return ATTNRES_OK;
}

struct P2Layout {
  int n_part, part_q, n_q, part_bias, part_scale;
};

P2Layout phase2_layout(const attnres_phase2_desc* d, bool want_q, bool want_bias, bool want_scale) {
  P2Layout L{0, -1, 0, -1, -1};
  if (want_q && !d->logit_given) {
    L.part_q = 0;
    L.n_q = d->rank > 0 ? d->rank : d->dim;
    L.n_part = L.n_q;
  }
  if (want_bias) L.part_bias = L.n_part++;
  if (want_scale) {
    L.part_scale = L.n_part;
    L.n_part += (d->rank > 0 && d->scale_key && !d->logit_given) ? 2 : 1;
  }
  return L;
}

void fill_phase2(const attnres_phase2_desc* d, const PhasePlan& pl, Phase2Params* p) {
  memset(p, 0, sizeof(*p));
  p->pv = d->partial_value;
  p->pk = d->rank > 0 ? d->partial_key : nullptr;
  p->q = d->logit_given ? nullptr : d->query;
  p->plogit = d->logit_given ? d->partial_logit : nullptr;
  p->inter = d->interblock_output;
  p->lse = d->interblock_lse;
  p->bias_dev = d->logit_bias_dev;
  p->scale_dev = d->value_scale_dev;
  p->n_tok = d->n_tok;
  p->pv_stride = d->partial_value_row_stride;
  p->pk_stride = d->partial_key_row_stride;
  p->inter_stride = d->interblock_row_stride;
  p->part_q = p->part_bias = p->part_scale = -1;
  p->D = d->dim;
  p->R = d->rank;
  p->ncols = pl.ncols;
  p->logit_given = d->logit_given ? 1 : 0;
  p->merge = d->merge;
  p->key_norm = d->key_norm ? 1 : 0;
  p->norm_out = d->normalize_output ? 1 : 0;
  p->scale_key = (d->rank > 0 && d->scale_key && !d->logit_given) ? 1 : 0;
  p->pl_dt = d->partial_logit_dtype;
  p->scale = d->logit_scale;
  p->eps = d->norm_eps;
  p->bias = d->logit_bias;
  p->vscale = d->value_scale;
}

// waves per phase-2 workgroup: the row's columns, and enough threads for the
// LR key (four elements per thread)
int phase2_waves(const attnres_phase2_desc* d, const PhasePlan& pl) {
  int w = pl.wpt;
  const int kw = (d->rank + 4 * kWaveSize - 1) / (4 * kWaveSize);
  return kw > w ? kw : w;
}

// One wave per token when a wave covers the row with at most 16 elements per
// lane and the LR key with at most 4: fp32 rows in 16-byte vectors (1-4 per
// lane), 16-bit rows in 16-byte vectors (1-2 per lane) or, where those would
// leave lanes idle (D <= 256, 512 < D <= 768), in 8-byte vectors (1 or 3).
// attnres_test_phase2_block_layout(1) keeps the workgroup-per-token kernels
// instead: the two layouts give the same per-token results, which a test checks.
constexpr int kPhase2Teams = 4;  // tokens (waves) per workgroup
struct P2Wave {
  int vb, cb, ncols;
};
bool phase2_wave_plan(const attnres_phase2_desc* d, const PhasePlan& pl, P2Wave* w) {
  if (g_phase2_block_layout.load(std::memory_order_relaxed)) return false;
  if (!pl.vec || d->rank > 4 * kWaveSize) return false;
  const int D = d->dim;
  if (elem_size(d->dtype) == 4) {
    w->vb = 16;
    w->ncols = (D + 255) / 256;
    w->cb = w->ncols;
    return w->ncols <= 4;
  }
  if (D <= 256 || (D > 512 && D <= 768)) {
    w->vb = 8;
    w->ncols = (D + 255) / 256;
    w->cb = w->ncols == 1 ? 1 : 3;
    return true;
  }
  if (D > 1024) return false;
  w->vb = 16;
  w->ncols = (D + 511) / 512;
  w->cb = w->ncols;
  return true;
}

// The packed-arithmetic kernels of attnres_phase2_fast.hip, on 16-bit rows one
// wave covers exactly (D = 256, 512, 768, 1024): base keys with the addcmul
// merge and no output norm, or LR keys (r <= 256) with either merge and the
// optional output norm.
bool phase2_fast(const attnres_phase2_desc* d, const P2Wave& w) {
  if (elem_size(d->dtype) != 2 || d->logit_given) return false;
  if (d->dim != kWaveSize * (w.vb / 2) * w.cb) return false;
  if (d->rank > 0) return d->rank <= 4 * kWaveSize;
  return !d->normalize_output && d->merge == ATTNRES_MERGE_ADDCMUL;
}

// Phase 1 with one wave per token and packed arithmetic
// (attnres_phase1_fast.hip): 16-bit rows one wave covers exactly, <= 4 sites,
// <= 8 sources, no output norm.  Fills the launch geometry.
bool phase1_fast(const attnres_phase1_desc* d, const PhasePlan& pl, Launch* L) {
  if (!pl.vec || elem_size(d->dtype) != 2 || d->normalize_output || d->n_q > 4 || d->n_src > 8) return false;
  if (d->dim != 256 && d->dim != 512 && d->dim != 768 && d->dim != 1024) return false;
  L->vb = (d->dim == 256 || d->dim == 768) ? 8 : 16;
  L->wpt = d->dim / (kWaveSize * (L->vb / 2));
  // source slots: the count rounded up to a pair (the forward mixes sources
  // in pairs); a slot past n_src is a wasted row load and its dot products
  // (p5's six sources in eight slots cost the backward 3 waves per SIMD)
  L->nmax = d->n_src <= 2 ? 2 : (d->n_src + 1) / 2 * 2;
  // one token per wave: no cross-token sums here, and fresh waves balance the
  // CUs better than a resident round walking four tokens each (p5: forward
  // 50.5 -> 49.2 us, backward 79.9 -> 77.2 us at 16384 tokens)
  // (the kernels stride over tokens, so the grid may stop short: at most 2^22
  // workgroups keep the launch's work-item count within 32 bits)
  const int64_t groups = (d->n_tok + 3) / 4;
  L->grid = (int)(groups < (1 << 22) ? groups : (1 << 22));
  return true;
}

// Phase 1 split over D / 256 waves per token (attnres_phase1_fast.hip, column
// split): 16-bit rows of a multiple of 256 elements up to 2048, no output norm,
// n_q * np <= 64 -- the reference model's block widths (up to 16 read sites)
// that the one-wave kernels do not cover.  Sets the lane count np (>= 2) and
// the launch geometry.
bool phase1_split(const attnres_phase1_desc* d, const PhasePlan& pl, Phase1Params* p, Launch* L) {
  if (!pl.vec || elem_size(d->dtype) != 2 || d->normalize_output) return false;
  if (d->dim % 256 || d->dim / 256 > 8) return false;
  int np = 2;
  while (np < d->n_src) np <<= 1;
  if (np > 16 || d->n_q * np > 64) return false;
  p->np = np;
  L->wpt = d->dim / 256;
  L->nmax = np;
  // site slots: a site past n_q loads an upstream row and computes S row dot
  // products for nothing (the published block's 12 sites in 16 slots cost the
  // backward a quarter of its upstream loads and dot products)
  const int q = d->n_q;
  L->teams = q <= 4 ? 4 : q <= 6 ? 6 : q <= 8 ? 8 : q <= 12 ? 12 : 16;
  L->grid = (int)(d->n_tok < kPhase1SplitGroups ? d->n_tok : kPhase1SplitGroups);
  return true;
}

}  // namespace

extern "C" int attnres_phase1_forward(const attnres_phase1_desc* d, void* out, void* out_prenorm, float* lse,
                                      float* out_inv_rms, void* stream) {
  int rc = check_phase1(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!out || !lse) return fail(ATTNRES_EINVAL, "out / lse is NULL");
  PhasePlan pl;
  const void* rows[ATTNRES_MAX_SOURCES + 2];
  int64_t strides[ATTNRES_MAX_SOURCES + 2];
  for (int s = 0; s < d->n_src; ++s) {
    rows[s] = d->values[s];
    strides[s] = d->value_row_stride[s];
  }
  rows[d->n_src] = out;
  rows[d->n_src + 1] = d->normalize_output ? out_prenorm : nullptr;
  strides[d->n_src] = strides[d->n_src + 1] = d->dim;
  rc = phase_plan(d->dtype, d->dim, rows, strides, d->n_src + 2, &pl, 3);
  if (rc) return rc;
  Phase1Params p;
  fill_phase1(d, pl, &p);
  p.out = out;
  p.out_prenorm = d->normalize_output ? out_prenorm : nullptr;
  p.lse = lse;
  p.out_inv_rms = d->normalize_output ? out_inv_rms : nullptr;
  Launch L;
  memset(&L, 0, sizeof(L));
  if (phase1_fast(d, pl, &L)) {
    hipError_t err = launch_phase1_fast_forward(d->dtype, p, L, (hipStream_t)stream);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-1 forward launch failed: %s", hipGetErrorString(err));
    return ATTNRES_OK;
  }
  if (phase1_split(d, pl, &p, &L)) {
    hipError_t err = launch_phase1_split_forward(d->dtype, p, L, (hipStream_t)stream);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-1 forward launch failed: %s", hipGetErrorString(err));
    return ATTNRES_OK;
  }
  L.vec = pl.vec;
  L.vb = pl.vb;
  L.wpt = pl.wpt;
  L.grid = (int)(d->n_tok < kMaxFwdGroups ? d->n_tok : kMaxFwdGroups);
  L.lds = ((size_t)pl.wpt * d->n_q * d->n_src + 8 * (size_t)pl.wpt) * sizeof(float);
  if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "phase-1 forward needs %zu bytes of LDS", L.lds);
  hipError_t err = launch_phase1_forward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-1 forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_phase1_backward_sites(const attnres_phase1_desc* d, const void* const* grad_out,
                                             const float* const* grad_lse, const void* out_prenorm,
                                             const float* out_inv_rms, void* const* dvalues,
                                             void* const* dlogits, int64_t dlogit_q_stride, void* stream) {
  int rc = check_phase1(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!grad_out || !dvalues || !dlogits) return fail(ATTNRES_EINVAL, "grad_out / dvalues / dlogits is NULL");
  if (d->normalize_output && (!out_prenorm || !out_inv_rms))
    return fail(ATTNRES_EINVAL, "normalize_output backward needs out_prenorm and out_inv_rms");
  if (dlogit_q_stride < d->n_tok)
    return fail(ATTNRES_EINVAL, "dlogit_q_stride %lld < n_tok=%lld", (long long)dlogit_q_stride, (long long)d->n_tok);
  PhasePlan pl;
  const void* rows[2 * ATTNRES_MAX_SOURCES + ATTNRES_PHASE1_MAX_QUERIES + 1];
  int64_t strides[2 * ATTNRES_MAX_SOURCES + ATTNRES_PHASE1_MAX_QUERIES + 1];
  int n = 0;
  for (int s = 0; s < d->n_src; ++s) {
    if (!dvalues[s]) return fail(ATTNRES_EINVAL, "dvalues[%d] is NULL", s);
    if (!dlogits[s]) return fail(ATTNRES_EINVAL, "dlogits[%d] is NULL", s);
    rows[n] = d->values[s];
    strides[n++] = d->value_row_stride[s];
    rows[n] = dvalues[s];
    strides[n++] = d->dim;
  }
  for (int q = 0; q < d->n_q; ++q) {
    if (!grad_out[q]) return fail(ATTNRES_EINVAL, "grad_out[%d] is NULL", q);
    rows[n] = grad_out[q];
    strides[n++] = d->dim;
  }
  rows[n] = d->normalize_output ? out_prenorm : nullptr;
  strides[n++] = d->dim;
  // three 8-byte columns hold the upstream rows of at most 4 sites in registers
  rc = phase_plan(d->dtype, d->dim, rows, strides, n, &pl, d->n_q <= 4 ? 3 : 1);
  if (rc) return rc;
  Phase1Params p;
  fill_phase1(d, pl, &p);
  for (int s = 0; s < d->n_src; ++s) {
    p.dval[s] = dvalues[s];
    p.dlsrc[s] = dlogits[s];
  }
  p.dlq = dlogit_q_stride;
  int n_glse = 0;
  for (int q = 0; q < d->n_q; ++q) {
    p.gout[q] = grad_out[q];
    p.glse[q] = grad_lse ? grad_lse[q] : nullptr;
    n_glse += p.glse[q] != nullptr;
  }
  // one base and uniform strides for every table (e.g. the stacked layouts of
  // attnres_phase1_backward): the column-split kernels then address rows from
  // the first entry
  if (p.stacked) {
    const size_t les = elem_size(d->logits_dtype);
    const bool ok = uniform_stride((const void* const*)p.dlsrc, d->n_src, les, &p.dls) &&
                    uniform_stride(p.gout, d->n_q, elem_size(d->dtype), &p.gq) &&
                    (n_glse == 0 || (n_glse == d->n_q && uniform_stride((const void* const*)p.glse, d->n_q, 4, &p.glq)));
    p.stacked = ok ? 1 : 0;
  }
  p.out_prenorm = d->normalize_output ? const_cast<void*>(out_prenorm) : nullptr;
  p.out_inv_rms = d->normalize_output ? const_cast<float*>(out_inv_rms) : nullptr;
  Launch L;
  memset(&L, 0, sizeof(L));
  if (phase1_fast(d, pl, &L)) {
    hipError_t err = launch_phase1_fast_backward(d->dtype, p, L, (hipStream_t)stream);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-1 backward launch failed: %s", hipGetErrorString(err));
    return ATTNRES_OK;
  }
  if (phase1_split(d, pl, &p, &L)) {
    hipError_t err = launch_phase1_split_backward(d->dtype, p, L, (hipStream_t)stream);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-1 backward launch failed: %s", hipGetErrorString(err));
    return ATTNRES_OK;
  }
  L.vec = pl.vec;
  L.vb = pl.vb;
  L.wpt = pl.wpt;
  L.nmax = d->n_q <= 4 ? 4 : d->n_q <= 8 ? 8 : ATTNRES_PHASE1_MAX_QUERIES;
  L.grid = (int)(d->n_tok < kMaxFwdGroups ? d->n_tok : kMaxFwdGroups);
  const size_t qn = (size_t)d->n_q * d->n_src;
  L.lds = (2 * qn + 2 * (size_t)pl.wpt * qn + (size_t)pl.wpt * L.nmax) * sizeof(float);
  if (L.lds > lds_limit()) return fail(ATTNRES_EUNSUPPORTED, "phase-1 backward needs %zu bytes of LDS", L.lds);
  hipError_t err = launch_phase1_backward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-1 backward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_phase1_backward(const attnres_phase1_desc* d, const void* grad_out, const float* grad_lse,
                                       const void* out_prenorm, const float* out_inv_rms, void* const* dvalues,
                                       void* dlogits, void* stream) {
  int rc = check_phase1(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!grad_out || !dvalues || !dlogits) return fail(ATTNRES_EINVAL, "grad_out / dvalues / dlogits is NULL");
  // the stacked layouts as per-site and per-source pointers: grad_out [Q, n_tok,
  // dim], grad_lse [Q, n_tok], dlogits [Q, S, n_tok]
  const void* go[ATTNRES_PHASE1_MAX_QUERIES];
  const float* gl[ATTNRES_PHASE1_MAX_QUERIES];
  void* dl[ATTNRES_MAX_SOURCES];
  const size_t es = elem_size(d->dtype), les = elem_size(d->logits_dtype);
  for (int q = 0; q < d->n_q; ++q) {
    go[q] = (const char*)grad_out + (size_t)q * d->n_tok * d->dim * es;
    gl[q] = grad_lse ? grad_lse + (size_t)q * d->n_tok : nullptr;
  }
  for (int s = 0; s < d->n_src; ++s) dl[s] = (char*)dlogits + (size_t)s * d->n_tok * les;
  return attnres_phase1_backward_sites(d, go, grad_lse ? gl : nullptr, out_prenorm, out_inv_rms, dvalues, dl,
                                       (int64_t)d->n_src * d->n_tok, stream);
}

extern "C" size_t attnres_phase2_backward_workspace_size(const attnres_phase2_desc* d) {
  if (check_phase2(d) != ATTNRES_OK || d->n_tok == 0) return 0;
  const P2Layout PL = phase2_layout(d, true, true, true);
  if (PL.n_part == 0) return 0;
  return (size_t)bwd_groups(d->n_tok) * part_stride(PL.n_part) * sizeof(float);
}

namespace {

// The block accumulation fused in front of an LR merge
// (attnres_accum_read_*): the accumulation's description and buffers.
struct AccRead {
  const attnres_block_accum_desc* a;
  void* value_out;          // forward: the grown block
  void* key_out;
  float* key_inv_rms;       // forward writes, backward reads ([n_tok, heads] with key norm)
  const void* grad_value;   // backward: the grown block's other gradients, or NULL
  int64_t grad_value_stride;
  const void* grad_key;
  void* grad_projected;     // backward: [n_tok, proj_cols]
  void* grad_partial_key;   // backward: the old partial key's gradient, or NULL
};

// phase-2 parameters of the fused accumulation (the merge reads the grown block)
void fill_accum(const AccRead& acc, Phase2Params* p) {
  const attnres_keyed_split_desc& s = acc.a->split;
  p->acc_y = s.projected;
  p->acc_y_stride = s.row_stride;
  p->acc_P = s.proj_cols;
  p->acc_H = s.heads;
  p->acc_hd = s.rank / s.heads;
  p->acc_key_norm = s.key_norm ? 1 : 0;
  p->acc_eps = s.norm_eps;
  p->acc_pv_old = acc.a->partial_value;
  p->acc_pk_old = acc.a->partial_key;
  p->acc_pv_out = acc.value_out;
  p->acc_pk_out = acc.key_out;
  p->acc_inv = acc.key_inv_rms;
  p->acc_gv = acc.grad_value;
  p->acc_gv_stride = acc.grad_value_stride;
  p->acc_gk = acc.grad_key;
  p->acc_gy = acc.grad_projected;
  p->acc_dpk_old = acc.grad_partial_key;
}

int phase2_forward_impl(const attnres_phase2_desc* d, void* out, void* stream, const AccRead* acc) {
  int rc = check_phase2(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!out) return fail(ATTNRES_EINVAL, "out is NULL");
  PhasePlan pl;
  const void* rows[6] = {d->partial_value, d->interblock_output, out,
                         (d->rank == 0 && !d->logit_given) ? d->query : nullptr,
                         acc ? acc->a->split.projected : nullptr, acc ? acc->a->partial_value : nullptr};
  const int64_t strides[6] = {d->partial_value_row_stride, d->interblock_row_stride, d->dim, d->dim,
                              acc ? acc->a->split.row_stride : d->dim, d->dim};
  rc = phase_plan(d->dtype, d->dim, rows, strides, 6, &pl);
  if (rc) return rc;
  Phase2Params p;
  fill_phase2(d, pl, &p);
  p.out = out;
  Launch L;
  memset(&L, 0, sizeof(L));
  L.vec = pl.vec;
  L.nmax = (d->rank > 0 && !d->logit_given) ? 1 : 0;
  P2Wave wv;
  if (phase2_wave_plan(d, pl, &wv)) {
    p.ncols = wv.ncols;
    L.teams = kPhase2Teams;
    L.vb = wv.vb;
    L.wpt = wv.cb;
    // one resident round of the fast kernels' waves (8 per SIMD), each walking
    // tokens with that stride: the per-wave setup (query, scale, bias) is paid
    // once per few tokens (measured at p5lr: 16.4 -> 15.3 us per LR merge,
    // 17.1 us with four tokens per wave)
    const int64_t wgs = (d->n_tok + kPhase2Teams - 1) / kPhase2Teams;
    const int64_t cap = phase2_fast(d, wv) ? 2 * base_fast_streams() / kPhase2Teams : kMaxFwdGroups;
    L.grid = (int)(wgs < cap ? wgs : cap);
    L.lds = 0;
    L.feat = (d->key_norm ? 1 : 0) | (d->merge == ATTNRES_MERGE_LERP ? 2 : 0);
  } else {
    L.wpt = phase2_waves(d, pl);
    L.grid = (int)(d->n_tok < kMaxFwdGroups ? d->n_tok : kMaxFwdGroups);
    L.lds = (2 * (size_t)L.wpt + 8) * sizeof(float);
  }
  const bool fast = L.teams > 0 && phase2_fast(d, wv);
  if (acc) {
    if (!fast || L.nmax != 1 || d->rank > 4 * kWaveSize)
      return fail(ATTNRES_EUNSUPPORTED, "the fused accumulation needs the one-wave LR merge (16-bit rows of "
                  "256/512/768/1024 aligned to 16 bytes, rank <= 256)");
    fill_accum(*acc, &p);
    L.feat |= 4;
  }
  hipError_t err = fast ? launch_phase2_fast_forward(d->dtype, p, L, (hipStream_t)stream)
                        : launch_phase2_forward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-2 forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

}  // namespace

extern "C" int attnres_phase2_forward(const attnres_phase2_desc* d, void* out, void* stream) {
  return phase2_forward_impl(d, out, stream, nullptr);
}

namespace {

int phase2_backward_impl(const attnres_phase2_desc* d, const attnres_phase2_grads* g, void* stream,
                         const AccRead* acc) {
  int rc = check_phase2(d);
  if (rc) return rc;
  if (!g) return fail(ATTNRES_EINVAL, "grads is NULL");
  const bool lr = d->rank > 0 && !d->logit_given;
  hipStream_t st = (hipStream_t)stream;
  const int q_rows = g->dquery_rows > 1 ? g->dquery_rows : 1;
  if (g->dquery_rows > 1 && (g->dquery_row < 0 || g->dquery_row >= g->dquery_rows))
    return fail(ATTNRES_EINVAL, "dquery_row=%d outside [0, %d)", g->dquery_row, g->dquery_rows);
  if (d->n_tok == 0) {
    if (g->dquery && !d->logit_given)
      zero_async(g->dquery, (size_t)q_rows * (lr ? d->rank : d->dim) * elem_size(d->dtype), st);
    if (g->dlogit_bias) zero_async(g->dlogit_bias, sizeof(float), st);
    if (g->dvalue_scale) zero_async(g->dvalue_scale, sizeof(float), st);
    return ATTNRES_OK;
  }
  if (!g->grad_out || !(acc || g->dpartial_value) || !g->dinterblock_output || !g->dinterblock_lse)
    return fail(ATTNRES_EINVAL, "grad_out / dpartial_value / dinterblock_output / dinterblock_lse is NULL");
  if (lr && !acc && !g->dpartial_key) return fail(ATTNRES_EINVAL, "LR merge backward needs dpartial_key");
  PhasePlan pl;
  const void* rows[9] = {d->partial_value, d->interblock_output, g->grad_out, acc ? nullptr : g->dpartial_value,
                         g->dinterblock_output, (d->rank == 0 && !d->logit_given) ? d->query : nullptr,
                         acc ? acc->grad_projected : nullptr, acc ? acc->grad_value : nullptr,
                         acc ? acc->a->split.projected : nullptr};
  const int64_t strides[9] = {d->partial_value_row_stride, d->interblock_row_stride, d->dim, d->dim, d->dim, d->dim,
                              acc ? acc->a->split.proj_cols : d->dim, acc ? acc->grad_value_stride : d->dim,
                              acc ? acc->a->split.row_stride : d->dim};
  rc = phase_plan(d->dtype, d->dim, rows, strides, 9, &pl);
  if (rc) return rc;
  Phase2Params p;
  fill_phase2(d, pl, &p);
  p.gout = g->grad_out;
  p.dpv = g->dpartial_value;
  p.dpk = lr ? g->dpartial_key : nullptr;
  p.dinter = g->dinterblock_output;
  p.dlse = g->dinterblock_lse;
  p.dplogit = d->logit_given ? g->dpartial_logit : nullptr;
  const P2Layout PL = phase2_layout(d, g->dquery != nullptr, g->dlogit_bias != nullptr, g->dvalue_scale != nullptr);
  const int64_t groups = bwd_groups(d->n_tok);
  if (PL.n_part > 0) {
    const size_t need = (size_t)groups * part_stride(PL.n_part) * sizeof(float);
    if (!g->workspace || g->workspace_bytes < need)
      return fail(ATTNRES_EWORKSPACE, "workspace of %zu bytes needed, got %zu", need,
                  g->workspace ? g->workspace_bytes : (size_t)0);
    p.partials = (float*)g->workspace;
  }
  p.n_part = PL.n_part;
  p.part_q = PL.part_q;
  p.part_bias = PL.part_bias;
  p.part_scale = PL.part_scale;
  Launch L;
  memset(&L, 0, sizeof(L));
  L.vec = pl.vec;
  L.nmax = lr ? 1 : 0;
  P2Wave wv;
  if (phase2_wave_plan(d, pl, &wv)) {
    // at most bwd_groups(n_tok) workgroups, so the workspace size above holds
    p.ncols = wv.ncols;
    L.teams = kPhase2Teams;
    L.vb = wv.vb;
    L.wpt = wv.cb;
    const int64_t wgs = (d->n_tok + kPhase2Teams - 1) / kPhase2Teams;
    int64_t cap = groups < kFullBwdGroups ? groups : kFullBwdGroups;
    // one resident round of waves: half the partial rows of 2048 workgroups,
    // and the reduction's chains of dependent loads half as long (measured at
    // p5: packed kernels 33.0 -> 29.9 us per call)
    if (cap > base_fast_streams() / kPhase2Teams) cap = base_fast_streams() / kPhase2Teams;
    // the fused accumulation's backward holds 3 waves per SIMD (its registers
    // at d768 / d1024, one key element per lane), not the 4 the resident round
    // above assumes: one round of those (the narrower instantiations, which fit
    // 4-5 waves, run one wave per SIMD short of a full round)
    if (acc && cap > 3 * base_fast_streams() / (4 * kPhase2Teams)) cap = 3 * base_fast_streams() / (4 * kPhase2Teams);
    L.grid = (int)(wgs < cap ? wgs : cap);
    L.lds = (size_t)kPhase2Teams * (PL.n_part > 0 ? PL.n_part : 1) * sizeof(float);
    L.feat = (d->key_norm ? 1 : 0) | (d->merge == ATTNRES_MERGE_LERP ? 2 : 0);
  } else {
    L.wpt = phase2_waves(d, pl);
    L.grid = (int)(groups < kFullBwdGroups ? groups : kFullBwdGroups);
    L.lds = (2 * (size_t)L.wpt + 8) * sizeof(float);
  }
  const bool fast = L.teams > 0 && phase2_fast(d, wv);
  if (acc) {
    if (!fast || L.nmax != 1 || d->rank > 4 * kWaveSize)
      return fail(ATTNRES_EUNSUPPORTED, "the fused accumulation needs the one-wave LR merge (16-bit rows of "
                  "256/512/768/1024 aligned to 16 bytes, rank <= 256)");
    fill_accum(*acc, &p);
    L.feat |= 4;
  }
  hipError_t err = fast ? launch_phase2_fast_backward(d->dtype, p, L, st) : launch_phase2_backward(d->dtype, p, L, st);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "phase-2 backward launch failed: %s", hipGetErrorString(err));
  if (PL.n_part > 0) {
    ReduceParams rp;
    memset(&rp, 0, sizeof(rp));
    rp.partials = p.partials;
    rp.n_groups = L.grid;
    rp.n_part = PL.n_part;
    rp.layout = L.teams > 0 ? kPartTiled : kPartRowMajor;  // wave kernels write tiles
    rp.part_q = PL.part_q;
    rp.n_q = PL.n_q;
    rp.part_gate = -1;
    rp.part_bias = PL.part_bias;
    rp.n_bias = PL.part_bias >= 0 ? 1 : 0;
    rp.part_extra = PL.part_scale;
    rp.n_extra = PL.part_scale >= 0 ? PL.n_part - PL.part_scale : 0;
    rp.dquery = g->dquery;
    rp.q_rows = q_rows;
    rp.q_row = q_rows > 1 ? g->dquery_row : 0;
    rp.dbias = g->dlogit_bias;
    rp.dextra = g->dvalue_scale;
    err = launch_reduce_partials(d->dtype, rp, st);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "reduce launch failed: %s", hipGetErrorString(err));
  }
  return ATTNRES_OK;
}

int check_block_accum(const attnres_block_accum_desc* d);  // the block accumulation's checks (below)

// the fused accumulation's description against its merge's
int check_accum_read(const attnres_accum_read_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  int rc = check_block_accum(&d->accum);
  if (rc) return rc;
  const attnres_keyed_split_desc& s = d->accum.split;
  const attnres_phase2_desc& r = d->read;
  if (d->accum.complete) return fail(ATTNRES_EINVAL, "the fused accumulation grows a live block (complete = 0)");
  if (r.logit_given || r.rank < 1) return fail(ATTNRES_EINVAL, "the fused accumulation feeds an LR merge");
  if (r.dtype != s.dtype || r.n_tok != s.n_tok || r.dim != s.dim || r.rank != s.rank)
    return fail(ATTNRES_EINVAL, "accum and read disagree on dtype / n_tok / dim / rank");
  return ATTNRES_OK;
}

}  // namespace

extern "C" int attnres_phase2_backward(const attnres_phase2_desc* d, const attnres_phase2_grads* g, void* stream) {
  return phase2_backward_impl(d, g, stream, nullptr);
}

extern "C" int attnres_accum_read_forward(const attnres_accum_read_desc* d, void* value_out, void* key_out,
                                          float* key_inv_rms, void* out, void* stream) {
  int rc = check_accum_read(d);
  if (rc) return rc;
  if (d->read.n_tok == 0) return ATTNRES_OK;
  if (!value_out || !key_out) return fail(ATTNRES_EINVAL, "value_out / key_out is NULL");
  if (d->accum.split.key_norm && !key_inv_rms) return fail(ATTNRES_EINVAL, "key_norm needs key_inv_rms");
  // the merge reads the grown block this call writes
  attnres_phase2_desc r = d->read;
  r.partial_value = value_out;
  r.partial_value_row_stride = r.dim;
  r.partial_key = key_out;
  r.partial_key_row_stride = r.rank;
  AccRead acc{&d->accum, value_out, key_out, key_inv_rms, nullptr, 0, nullptr, nullptr, nullptr};
  return phase2_forward_impl(&r, out, stream, &acc);
}

extern "C" int attnres_accum_read_backward(const attnres_accum_read_desc* d, const attnres_phase2_grads* g,
                                           const void* grad_value, int64_t grad_value_row_stride,
                                           const void* grad_key, const float* key_inv_rms, void* grad_projected,
                                           void* grad_partial_key, void* stream) {
  int rc = check_accum_read(d);
  if (rc) return rc;
  if (!g) return fail(ATTNRES_EINVAL, "grads is NULL");
  if (grad_value && (grad_value_row_stride < d->read.dim || grad_value_row_stride > INT32_MAX))
    return fail(ATTNRES_EINVAL, "grad_value_row_stride=%lld must be in [dim, 2^31)", (long long)grad_value_row_stride);
  if (d->read.n_tok > 0) {
    if (!grad_projected) return fail(ATTNRES_EINVAL, "grad_projected is NULL");
    if (d->accum.split.key_norm && !key_inv_rms) return fail(ATTNRES_EINVAL, "key_norm backward needs key_inv_rms");
  }
  AccRead acc{&d->accum, nullptr, nullptr, const_cast<float*>(key_inv_rms), grad_value, grad_value_row_stride,
              grad_key, grad_projected,
              d->accum.partial_key ? grad_partial_key : nullptr};
  return phase2_backward_impl(&d->read, g, stream, &acc);
}

// ---------------------------------------------------------------- query-bank logits
namespace {

constexpr int kKeyedLogitsGroups = 128;  // query-gradient partial rows (token strides)

int check_keyed_logits(const attnres_keyed_logits_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->n_src < 1 || d->n_src > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_EUNSUPPORTED, "n_src=%d outside [1, %d]", d->n_src, ATTNRES_MAX_SOURCES);
  if (d->n_q < 1 || d->n_q > ATTNRES_PHASE1_MAX_QUERIES)
    return fail(ATTNRES_EUNSUPPORTED, "n_q=%d outside [1, %d]", d->n_q, ATTNRES_PHASE1_MAX_QUERIES);
  if (d->dtype != ATTNRES_DTYPE_F32 && d->dtype != ATTNRES_DTYPE_BF16 && d->dtype != ATTNRES_DTYPE_F16)
    return fail(ATTNRES_EINVAL, "unknown dtype %d", d->dtype);
  if (d->n_tok < 0) return fail(ATTNRES_EINVAL, "n_tok=%lld < 0", (long long)d->n_tok);
  if (d->dim < 1 || d->dim > ATTNRES_PHASE_MAX_DIM)
    return fail(ATTNRES_EUNSUPPORTED, "dim=%d outside [1, %d]", d->dim, ATTNRES_PHASE_MAX_DIM);
  if (!d->values || !d->value_row_stride) return fail(ATTNRES_EINVAL, "values / value_row_stride is NULL");
  const bool live = d->n_tok > 0;
  for (int s = 0; s < d->n_src; ++s) {
    if (live && !d->values[s]) return fail(ATTNRES_EINVAL, "values[%d] is NULL", s);
    if (d->value_row_stride[s] < d->dim || d->value_row_stride[s] > INT32_MAX)
      return fail(ATTNRES_EINVAL, "value_row_stride[%d]=%lld must be in [dim, 2^31)", s,
                  (long long)d->value_row_stride[s]);
  }
  if (live && !d->queries) return fail(ATTNRES_EINVAL, "queries is NULL");
  return ATTNRES_OK;
}

void fill_keyed_logits(const attnres_keyed_logits_desc* d, KeyedLogitsParams* p, Launch* L) {
  memset(p, 0, sizeof(*p));
  for (int s = 0; s < d->n_src; ++s) {
    p->val[s] = d->values[s];
    p->vstride[s] = (int32_t)d->value_row_stride[s];
  }
  p->queries = d->queries;
  p->n_tok = d->n_tok;
  p->n_src = d->n_src;
  p->n_q = d->n_q;
  p->D = d->dim;
  p->key_norm = d->key_norm ? 1 : 0;
  p->eps = d->norm_eps;
  memset(L, 0, sizeof(*L));
  L->wpt = (d->dim + 8 * kWaveSize - 1) / (8 * kWaveSize);  // eight elements per lane
  L->grid = (int)(d->n_tok < kMaxFwdGroups ? d->n_tok : kMaxFwdGroups);
  L->lds = (size_t)L->wpt * kKLMaxQ * sizeof(float);
}

int64_t keyed_logits_groups(int64_t n_tok) { return n_tok < kKeyedLogitsGroups ? n_tok : kKeyedLogitsGroups; }

}  // namespace

namespace {

int check_site_logits(const attnres_site_logits_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->dtype < 0 || d->dtype > 2) return fail(ATTNRES_EINVAL, "unknown dtype %d", d->dtype);
  if (d->logits_dtype != d->dtype && d->logits_dtype != ATTNRES_DTYPE_F32)
    return fail(ATTNRES_EINVAL, "logits_dtype %d must be the dtype %d or fp32", d->logits_dtype, d->dtype);
  if (d->n_tok < 0) return fail(ATTNRES_EINVAL, "n_tok=%lld < 0", (long long)d->n_tok);
  if (d->rank < 1 || d->rank > ATTNRES_SITE_LOGITS_MAX_RANK)
    return fail(ATTNRES_EUNSUPPORTED, "rank=%d outside [1, %d]", d->rank, ATTNRES_SITE_LOGITS_MAX_RANK);
  if (d->n_q < 1 || d->n_q > ATTNRES_SITE_LOGITS_MAX_QUERIES)
    return fail(ATTNRES_EUNSUPPORTED, "n_q=%d outside [1, %d]", d->n_q, ATTNRES_SITE_LOGITS_MAX_QUERIES);
  if (d->key_row_stride < d->rank) return fail(ATTNRES_EINVAL, "key_row_stride %lld < rank", (long long)d->key_row_stride);
  if (d->n_tok > 0 && (!d->key || !d->queries)) return fail(ATTNRES_EINVAL, "key / queries is NULL");
  return ATTNRES_OK;
}

// rank slots of the kernel (32 / 64 / 128), LDS for the queries, 16-byte key loads
int plan_site_logits(const attnres_site_logits_desc* d, SiteLogitsParams* p, Launch* L) {
  memset(p, 0, sizeof(*p));
  memset(L, 0, sizeof(*L));
  L->nmax = d->rank <= 32 ? 32 : d->rank <= 64 ? 64 : 128;
  L->lds = (size_t)d->n_q * L->nmax * sizeof(float);
  if (L->lds > lds_limit())
    return fail(ATTNRES_EUNSUPPORTED, "site logits need %zu bytes of LDS for %d queries", L->lds, d->n_q);
  const int64_t groups = (d->n_tok + 31) / 32;  // 32 tokens per workgroup (8 lanes each)
  L->grid = (int)(groups < kMaxFwdGroups ? groups : kMaxFwdGroups);
  const size_t es = elem_size(d->dtype);
  p->key = d->key;
  p->kstride = d->key_row_stride;
  p->queries = d->queries;
  p->n_tok = d->n_tok;
  p->R = d->rank;
  p->n_q = d->n_q;
  p->key_norm = d->key_norm ? 1 : 0;
  p->odt = d->logits_dtype;
  p->vec = ((uintptr_t)d->key % 16 == 0 && (d->key_row_stride * es) % 16 == 0 && (d->rank * es) % 16 == 0) ? 1 : 0;
  p->eps = d->norm_eps;
  p->scale = d->logit_scale;
  p->bias = d->logits_dtype == ATTNRES_DTYPE_F32 ? d->logit_bias : 0.f;
  return ATTNRES_OK;
}

}  // namespace

extern "C" int attnres_site_logits_forward(const attnres_site_logits_desc* d, void* logits, void* stream) {
  int rc = check_site_logits(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!logits) return fail(ATTNRES_EINVAL, "logits is NULL");
  SiteLogitsParams p;
  Launch L;
  rc = plan_site_logits(d, &p, &L);
  if (rc) return rc;
  p.out = logits;
  hipError_t err = launch_site_logits_forward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "site-logits forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_site_logits_backward(const attnres_site_logits_desc* d, const void* const* grad_logits,
                                            void* dkey, void* grad_scaled, void* key_hat, void* stream) {
  int rc = check_site_logits(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!grad_logits || !dkey || !grad_scaled || !key_hat)
    return fail(ATTNRES_EINVAL, "grad_logits / dkey / grad_scaled / key_hat is NULL");
  SiteLogitsParams p;
  Launch L;
  rc = plan_site_logits(d, &p, &L);
  if (rc) return rc;
  for (int q = 0; q < d->n_q; ++q) {
    if (!grad_logits[q]) return fail(ATTNRES_EINVAL, "grad_logits[%d] is NULL", q);
    p.dout[q] = grad_logits[q];
  }
  p.dkey = dkey;
  p.du = grad_scaled;
  p.khat = key_hat;
  hipError_t err = launch_site_logits_backward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "site-logits backward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_keyed_logits_forward(const attnres_keyed_logits_desc* d, void* logits, float* inv_rms,
                                            void* stream) {
  int rc = check_keyed_logits(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!logits) return fail(ATTNRES_EINVAL, "logits is NULL");
  KeyedLogitsParams p;
  Launch L;
  fill_keyed_logits(d, &p, &L);
  p.logits = logits;
  p.inv = d->key_norm ? inv_rms : nullptr;
  hipError_t err = launch_keyed_logits_forward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "keyed-logits forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" size_t attnres_keyed_logits_backward_workspace_size(const attnres_keyed_logits_desc* d) {
  if (check_keyed_logits(d) != ATTNRES_OK || d->n_tok == 0) return 0;
  return (size_t)keyed_logits_groups(d->n_tok) * d->n_q * d->dim * sizeof(float);
}

extern "C" int attnres_keyed_logits_backward(const attnres_keyed_logits_desc* d, const void* dlogits,
                                             const float* inv_rms, void* const* dvalues, void* dqueries,
                                             void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_keyed_logits(d);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (d->n_tok == 0) {
    if (dqueries) zero_async(dqueries, (size_t)d->n_q * d->dim * elem_size(d->dtype), st);
    return ATTNRES_OK;
  }
  if (!dlogits || !dvalues) return fail(ATTNRES_EINVAL, "dlogits / dvalues is NULL");
  for (int s = 0; s < d->n_src; ++s)
    if (!dvalues[s]) return fail(ATTNRES_EINVAL, "dvalues[%d] is NULL", s);
  if (d->key_norm && !inv_rms) return fail(ATTNRES_EINVAL, "key_norm backward needs the forward's inv_rms");
  KeyedLogitsParams p;
  Launch L;
  fill_keyed_logits(d, &p, &L);
  for (int s = 0; s < d->n_src; ++s) p.dval[s] = dvalues[s];
  p.dlogits = dlogits;
  p.inv = const_cast<float*>(inv_rms);
  const int64_t groups = keyed_logits_groups(d->n_tok);
  if (dqueries) {
    const size_t need = (size_t)groups * d->n_q * d->dim * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(ATTNRES_EWORKSPACE, "workspace of %zu bytes needed, got %zu", need,
                  workspace ? workspace_bytes : (size_t)0);
    p.partials = (float*)workspace;
    p.n_part = d->n_q * d->dim;
    L.teams = (int)groups;
  }
  hipError_t err = launch_keyed_logits_backward(d->dtype, p, L, st);
  if (err != hipSuccess)
    return fail(ATTNRES_ELAUNCH, "keyed-logits backward launch failed: %s", hipGetErrorString(err));
  if (dqueries) {
    ReduceParams rp;
    memset(&rp, 0, sizeof(rp));
    rp.partials = p.partials;
    rp.n_groups = (int)groups;
    rp.n_part = p.n_part;
    rp.layout = kPartRowMajor;
    rp.part_q = 0;
    rp.n_q = p.n_part;
    rp.part_gate = -1;
    rp.part_bias = -1;
    rp.part_extra = -1;
    rp.dquery = dqueries;
    err = launch_reduce_partials(d->dtype, rp, st);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "reduce launch failed: %s", hipGetErrorString(err));
  }
  return ATTNRES_OK;
}

// ---------------------------------------------------------------- key-producer epilogue
namespace {

constexpr int kKeySplitTeams = 4;  // tokens (waves) per workgroup

int check_keyed_split(const attnres_keyed_split_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->dtype < 0 || d->dtype > 2) return fail(ATTNRES_EINVAL, "unknown dtype %d", d->dtype);
  if (d->n_tok < 0 || d->n_tok > INT32_MAX) return fail(ATTNRES_EINVAL, "n_tok=%lld outside [0, 2^31)", (long long)d->n_tok);
  if (d->dim < 1 || d->rank < 1) return fail(ATTNRES_EINVAL, "dim=%d / rank=%d must be positive", d->dim, d->rank);
  if (d->rank > 4 * kWaveSize)
    return fail(ATTNRES_EUNSUPPORTED, "rank=%d exceeds %d", d->rank, 4 * kWaveSize);
  if (d->heads < 1 || d->rank % d->heads != 0)
    return fail(ATTNRES_EINVAL, "heads=%d must divide rank=%d", d->heads, d->rank);
  const int hd = d->rank / d->heads;
  const bool pow2 = (hd & (hd - 1)) == 0;
  if (d->key_norm && !((hd < kWaveSize && pow2) || hd % kWaveSize == 0))
    return fail(ATTNRES_EUNSUPPORTED, "key head width %d must be a power of two below 64 or a multiple of 64", hd);
  if (d->proj_cols < d->dim + d->rank)
    return fail(ATTNRES_EINVAL, "proj_cols=%d < dim + rank = %d", d->proj_cols, d->dim + d->rank);
  if (d->row_stride < d->proj_cols)
    return fail(ATTNRES_EINVAL, "row_stride=%lld < proj_cols=%d", (long long)d->row_stride, d->proj_cols);
  return ATTNRES_OK;
}

void fill_keyed_split(const attnres_keyed_split_desc* d, KeySplitParams* p, Launch* L, bool vec) {
  memset(p, 0, sizeof(*p));
  p->y = d->projected;
  p->n_tok = d->n_tok;
  p->y_stride = d->row_stride;
  p->D = d->dim;
  p->R = d->rank;
  p->P = d->proj_cols;
  p->H = d->heads;
  p->hd = d->rank / d->heads;
  p->key_norm = d->key_norm ? 1 : 0;
  p->eps = d->norm_eps;
  memset(L, 0, sizeof(*L));
  L->vec = vec ? 1 : 0;
  L->teams = kKeySplitTeams;
  const int64_t wgs = (d->n_tok + kKeySplitTeams - 1) / kKeySplitTeams;
  L->grid = (int)(wgs < kMaxFwdGroups ? wgs : kMaxFwdGroups);
}

}  // namespace

extern "C" int attnres_keyed_split_forward(const attnres_keyed_split_desc* d, void* out, void* key,
                                           float* key_inv_rms, void* stream) {
  int rc = check_keyed_split(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!d->projected || !out || !key) return fail(ATTNRES_EINVAL, "projected / out / key is NULL");
  if (d->key_norm && !key_inv_rms) return fail(ATTNRES_EINVAL, "key_norm needs key_inv_rms");
  const int es = elem_size(d->dtype);
  const bool vec = (d->dim * es) % 16 == 0 && (d->row_stride * es) % 16 == 0 && aligned16(d->projected) &&
                   aligned16(out);
  KeySplitParams p;
  Launch L;
  fill_keyed_split(d, &p, &L, vec);
  p.out = out;
  p.key = key;
  p.inv = key_inv_rms;
  hipError_t err = launch_keyed_split_forward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "keyed split forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_keyed_split_backward(const attnres_keyed_split_desc* d, const void* grad_out,
                                            const void* grad_key, const float* key_inv_rms, void* grad_projected,
                                            void* stream) {
  int rc = check_keyed_split(d);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!grad_projected) return fail(ATTNRES_EINVAL, "grad_projected is NULL");
  if (d->key_norm && grad_key && (!key_inv_rms || !d->projected))
    return fail(ATTNRES_EINVAL, "key_norm backward needs projected and key_inv_rms");
  const int es = elem_size(d->dtype);
  const bool vec = (d->dim * es) % 16 == 0 && (d->proj_cols * es) % 16 == 0 && aligned16(grad_projected) &&
                   (!grad_out || aligned16(grad_out));
  KeySplitParams p;
  Launch L;
  fill_keyed_split(d, &p, &L, vec);
  p.gout = grad_out;
  p.gout_stride = d->dim;
  p.gkey = grad_key;
  p.inv = const_cast<float*>(key_inv_rms);
  p.gy = grad_projected;
  hipError_t err = launch_keyed_split_backward(d->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "keyed split backward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

// ---------------------------------------------------------------- block accumulation
namespace {

constexpr int kAccumBwdGroups = 1024;  // backward workgroups at most (the learned-scale partial rows)

int check_block_accum(const attnres_block_accum_desc* d) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  int rc = check_keyed_split(&d->split);
  if (rc) return rc;
  if (d->complete != 0 && d->complete != 1) return fail(ATTNRES_EINVAL, "complete must be 0 or 1, got %d", d->complete);
  if (!d->complete && (d->value_norm || d->scale_key || d->value_scale_dev))
    return fail(ATTNRES_EINVAL, "value_norm / scale_key / value_scale_dev apply to the completed block source only");
  if (d->value_norm && (d->scale_key || d->value_scale_dev))
    return fail(ATTNRES_EINVAL, "value_norm takes no scale (the key stays as it is)");
  return ATTNRES_OK;
}

bool accum_wants_scale_grad(const attnres_block_accum_desc* d) {
  return d->complete && !d->value_norm && d->value_scale_dev;
}

int64_t accum_bwd_groups(int64_t n_tok) {
  const int64_t wgs = (n_tok + kKeySplitTeams - 1) / kKeySplitTeams;
  return wgs < kAccumBwdGroups ? wgs : kAccumBwdGroups;
}

void fill_block_accum(const attnres_block_accum_desc* d, KeySplitParams* p) {
  p->accum = d->complete ? 2 : 1;
  p->pv = d->partial_value;
  p->pk = d->partial_key;
  p->value_norm = d->complete && d->value_norm ? 1 : 0;
  p->scale_key = d->complete && d->scale_key ? 1 : 0;
  p->vscale = d->value_scale;
  p->scale_dev = d->complete ? d->value_scale_dev : nullptr;
}

}  // namespace

extern "C" size_t attnres_block_accum_backward_workspace_size(const attnres_block_accum_desc* d) {
  if (check_block_accum(d) != ATTNRES_OK || d->split.n_tok == 0 || !accum_wants_scale_grad(d)) return 0;
  return (size_t)accum_bwd_groups(d->split.n_tok) * 2 * sizeof(float);
}

extern "C" int attnres_block_accum_forward(const attnres_block_accum_desc* d, void* value_out, void* key_out,
                                           float* key_inv_rms, float* value_inv_rms, void* stream) {
  int rc = check_block_accum(d);
  if (rc) return rc;
  const attnres_keyed_split_desc* sd = &d->split;
  if (sd->n_tok == 0) return ATTNRES_OK;
  if (!sd->projected || !value_out || !key_out) return fail(ATTNRES_EINVAL, "projected / value_out / key_out is NULL");
  const int es = elem_size(sd->dtype);
  const bool vec = (sd->dim * es) % 16 == 0 && (sd->row_stride * es) % 16 == 0 && aligned16(sd->projected) &&
                   aligned16(value_out) && (!d->partial_value || aligned16(d->partial_value));
  KeySplitParams p;
  Launch L;
  fill_keyed_split(sd, &p, &L, vec);
  fill_block_accum(d, &p);
  p.out = value_out;
  p.key = key_out;
  p.inv = sd->key_norm ? key_inv_rms : nullptr;
  p.vinv = p.value_norm ? value_inv_rms : nullptr;
  hipError_t err = launch_keyed_split_forward(sd->dtype, p, L, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "block accumulation forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_block_accum_backward(const attnres_block_accum_desc* d, const void* grad_value,
                                            int64_t grad_value_row_stride, const void* grad_key,
                                            const float* key_inv_rms, const float* value_inv_rms,
                                            void* grad_projected, void* grad_partial_key, float* grad_value_scale,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_block_accum(d);
  if (rc) return rc;
  const attnres_keyed_split_desc* sd = &d->split;
  hipStream_t st = (hipStream_t)stream;
  const bool want_ds = grad_value_scale && accum_wants_scale_grad(d);
  if (sd->n_tok == 0) {
    if (want_ds) zero_async(grad_value_scale, sizeof(float), st);
    return ATTNRES_OK;
  }
  if (!sd->projected || !grad_projected) return fail(ATTNRES_EINVAL, "projected / grad_projected is NULL");
  if (sd->key_norm && !key_inv_rms) return fail(ATTNRES_EINVAL, "key_norm backward needs the forward's key_inv_rms");
  if (d->complete && d->value_norm && grad_value && !value_inv_rms)
    return fail(ATTNRES_EINVAL, "value_norm backward needs the forward's value_inv_rms");
  if (grad_value && grad_value_row_stride < sd->dim)
    return fail(ATTNRES_EINVAL, "grad_value_row_stride=%lld < dim", (long long)grad_value_row_stride);
  const int es = elem_size(sd->dtype);
  const bool vec = (sd->dim * es) % 16 == 0 && (sd->proj_cols * es) % 16 == 0 && (sd->row_stride * es) % 16 == 0 &&
                   aligned16(sd->projected) && aligned16(grad_projected) && (!d->partial_value || aligned16(d->partial_value)) &&
                   (!grad_value || (aligned16(grad_value) && (grad_value_row_stride * es) % 16 == 0));
  KeySplitParams p;
  Launch L;
  fill_keyed_split(sd, &p, &L, vec);
  fill_block_accum(d, &p);
  p.gout = grad_value;
  p.gout_stride = grad_value_row_stride;
  p.gkey = grad_key;
  p.inv = const_cast<float*>(key_inv_rms);
  p.vinv = const_cast<float*>(value_inv_rms);
  p.gy = grad_projected;
  p.dpk = (p.scale_key && !p.value_norm) ? grad_partial_key : nullptr;
  if (want_ds) {
    L.grid = (int)accum_bwd_groups(sd->n_tok);
    const size_t need = (size_t)L.grid * 2 * sizeof(float);
    if (!workspace || workspace_bytes < need)
      return fail(ATTNRES_EWORKSPACE, "workspace of %zu bytes needed, got %zu", need, workspace ? workspace_bytes : (size_t)0);
    p.partials = (float*)workspace;
  }
  hipError_t err = launch_keyed_split_backward(sd->dtype, p, L, st);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "block accumulation backward launch failed: %s", hipGetErrorString(err));
  if (want_ds) {
    // the value and key edges' sums, each rounded to the dtype, then added
    ReduceParams rp;
    memset(&rp, 0, sizeof(rp));
    rp.partials = p.partials;
    rp.n_groups = L.grid;
    rp.n_part = 2;
    rp.layout = kPartRowMajor;
    rp.part_q = rp.part_gate = rp.part_bias = -1;
    rp.part_extra = 0;
    rp.n_extra = p.scale_key ? 2 : 1;
    rp.dextra = grad_value_scale;
    err = launch_reduce_partials(sd->dtype, rp, st);
    if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "reduce launch failed: %s", hipGetErrorString(err));
  }
  return ATTNRES_OK;
}

// ---------------------------------------------------------------- value-derived keys
namespace {

int check_value_key(const attnres_value_key_desc* d, bool* vec) {
  if (!d) return fail(ATTNRES_EINVAL, "desc is NULL");
  if (d->n_src < 1 || d->n_src > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_EUNSUPPORTED, "n_src=%d outside [1, %d]", d->n_src, ATTNRES_MAX_SOURCES);
  if (d->dtype != ATTNRES_DTYPE_F32 && d->dtype != ATTNRES_DTYPE_BF16 && d->dtype != ATTNRES_DTYPE_F16)
    return fail(ATTNRES_EINVAL, "unknown dtype %d", d->dtype);
  if (d->n_tok < 0) return fail(ATTNRES_EINVAL, "n_tok=%lld < 0", (long long)d->n_tok);
  if (d->dim < 1) return fail(ATTNRES_EINVAL, "dim=%d < 1", d->dim);
  if (!d->values || !d->value_row_stride) return fail(ATTNRES_EINVAL, "values / value_row_stride is NULL");
  const int es = elem_size(d->dtype);
  bool v = (d->dim * es) % 16 == 0;
  for (int s = 0; s < d->n_src; ++s) {
    if (d->n_tok > 0 && !d->values[s]) return fail(ATTNRES_EINVAL, "values[%d] is NULL", s);
    if (d->value_row_stride[s] < d->dim || d->value_row_stride[s] > INT32_MAX)
      return fail(ATTNRES_EINVAL, "value_row_stride[%d]=%lld must be in [dim, 2^31)", s,
                  (long long)d->value_row_stride[s]);
    v = v && aligned16(d->values[s]) && (d->value_row_stride[s] * es) % 16 == 0;
  }
  // a row is held in registers: 8 vectors per lane of 64
  const int max_dim = 64 * 8 * (v ? 16 / es : 1);
  if (d->dim > max_dim)
    return fail(ATTNRES_EUNSUPPORTED, "dim=%d exceeds %d on the %s path", d->dim, max_dim, v ? "vector" : "unaligned");
  *vec = v;
  return ATTNRES_OK;
}

void fill_value_norm(const attnres_value_key_desc* d, ValueNormParams* p) {
  memset(p, 0, sizeof(*p));
  for (int s = 0; s < d->n_src; ++s) {
    p->val[s] = d->values[s];
    p->vstride[s] = (int32_t)d->value_row_stride[s];
  }
  p->n_tok = d->n_tok;
  p->n_src = d->n_src;
  p->D = d->dim;
  p->eps = d->norm_eps;
}

int value_norm_grid(const attnres_value_key_desc* d) {
  const int64_t rows = (int64_t)d->n_src * d->n_tok;
  const int64_t wgs = (rows + 3) / 4;
  return (int)(wgs < kMaxFwdGroups ? wgs : kMaxFwdGroups);
}

}  // namespace

extern "C" int attnres_value_norm_forward(const attnres_value_key_desc* d, void* normed, float* inv_rms,
                                          void* stream) {
  bool vec = false;
  int rc = check_value_key(d, &vec);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!normed || !inv_rms) return fail(ATTNRES_EINVAL, "normed / inv_rms is NULL");
  vec = vec && aligned16(normed);
  ValueNormParams p;
  fill_value_norm(d, &p);
  p.normed = normed;
  p.inv = inv_rms;
  hipError_t err = launch_value_norm(d->dtype, false, p, value_norm_grid(d), vec, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "value norm forward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}

extern "C" int attnres_value_norm_backward(const attnres_value_key_desc* d, const void* grad_normed,
                                           const float* inv_rms, void* const* grad_values, void* stream) {
  bool vec = false;
  int rc = check_value_key(d, &vec);
  if (rc) return rc;
  if (d->n_tok == 0) return ATTNRES_OK;
  if (!grad_normed || !inv_rms || !grad_values) return fail(ATTNRES_EINVAL, "grad_normed / inv_rms / grad_values is NULL");
  vec = vec && aligned16(grad_normed);
  ValueNormParams p;
  fill_value_norm(d, &p);
  for (int s = 0; s < d->n_src; ++s) {
    if (!grad_values[s]) return fail(ATTNRES_EINVAL, "grad_values[%d] is NULL", s);
    vec = vec && aligned16(grad_values[s]);
    p.dval[s] = grad_values[s];
  }
  p.gnormed = grad_normed;
  p.inv = const_cast<float*>(inv_rms);
  hipError_t err = launch_value_norm(d->dtype, true, p, value_norm_grid(d), vec, (hipStream_t)stream);
  if (err != hipSuccess) return fail(ATTNRES_ELAUNCH, "value norm backward launch failed: %s", hipGetErrorString(err));
  return ATTNRES_OK;
}
