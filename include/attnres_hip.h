/*
 * attnres_hip.h -- C ABI of the MI355X (gfx950) Attention-Residual read library.
 *
 * The reference (jon123boss/LR-AttnRes) has no native library: its fused read
 * is a set of Triton kernels launched from Python.  Each entry point below
 * replaces one of those host launchers; the citation names the reference
 * function (file:line in attnres_ops.py) whose job it takes over.  The Python
 * drop-in module (lr-attnres_amd/attnres_ops.py) binds these symbols with
 * ctypes; INTEGRATION.md shows the binding.
 *
 * Conventions
 *  - Plain C types only.  Device buffers are passed as device pointers;
 *    per-source pointer / stride tables are HOST arrays of length n_src.
 *  - The library never allocates: the caller owns every buffer, including the
 *    backward workspace (size from attnres_read_backward_workspace_size()).
 *  - Every launch is asynchronous on the caller's stream (hipStream_t passed
 *    as void*; NULL = the default stream).  No host synchronisation.
 *  - Return 0 on success, a negative ATTNRES_E* code otherwise; the message of
 *    the last failure on the calling thread is attnres_last_error().
 *  - Tensor layout: token t = b*T + tt.  Source s's row for token t starts at
 *    values[s] + t * value_row_stride[s] (elements); the last dimension is
 *    contiguous.  Outputs and gradients are dense [n_tok, width].
 */
#ifndef ATTNRES_HIP_H
#define ATTNRES_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATTNRES_ABI_VERSION 2
#define ATTNRES_MAX_SOURCES 64

/* element type of values / keys / queries / gate / out / gradients */
#define ATTNRES_DTYPE_F32 0
#define ATTNRES_DTYPE_BF16 1
#define ATTNRES_DTYPE_F16 2

/* read mode */
#define ATTNRES_MODE_SOFTMAX 0 /* depth softmax read (base or LR) */
#define ATTNRES_MODE_AVERAGE 1 /* uniform mean over sources (values only) */

/* gate on the input-dependent query: q = q_static + act(gate) * q_dyn */
#define ATTNRES_GATE_NONE 0    /* q = q_static + q_dyn */
#define ATTNRES_GATE_LINEAR 1  /* act(g) = g        (model.py:2109-2110) */
#define ATTNRES_GATE_SIGMOID 2 /* act(g) = sigmoid(g) (benchmark config 4) */

/* error codes */
#define ATTNRES_OK 0
#define ATTNRES_EINVAL (-1)      /* bad argument (null pointer, bad size, mismatch) */
#define ATTNRES_EUNSUPPORTED (-2) /* shape outside what the kernels support */
#define ATTNRES_ELAUNCH (-3)     /* HIP reported an error at launch */
#define ATTNRES_EWORKSPACE (-4)  /* workspace missing or too small */

/*
 * Description of one read.  rank == 0 selects the base read, whose keys are
 * the values themselves (rms-normed when key_norm), with a [dim] query and a
 * single head; rank > 0 selects the LR read with low-rank keys [n_tok, rank]
 * split into `heads` contiguous chunks of rank/heads, and value heads of
 * dim/heads.
 */
typedef struct attnres_read_desc {
  int32_t n_src;          /* N sources, 1..ATTNRES_MAX_SOURCES */
  int32_t dtype;          /* ATTNRES_DTYPE_* */
  int64_t n_tok;          /* B*T (0 is allowed: nothing is launched) */
  int32_t dim;            /* D */
  int32_t rank;           /* R (LR) or 0 (base) */
  int32_t heads;          /* H; 1 for base; must divide dim and rank */
  int32_t mode;           /* ATTNRES_MODE_* */
  int32_t key_norm;       /* rms-norm keys (per head for LR) before scoring */
  int32_t normalize_output; /* rms-norm the [dim] output of each token */
  float logit_scale;      /* LR logit multiplier; base ignores it (1) */
  float norm_eps;         /* eps of every rms-norm (torch default: FLT_EPSILON) */
  const void* const* values;       /* [n_src] device pointers */
  const int64_t* value_row_stride; /* [n_src] elements */
  const void* const* keys;         /* [n_src] device pointers (LR) or NULL (base) */
  const int64_t* key_row_stride;   /* [n_src] elements (LR) */
  const void* query;               /* static query: base [dim], LR [heads, rank/heads]; may be NULL for LR when query_dyn is set */
  const void* query_dyn;           /* LR per-token query rows [n_tok, rank] or NULL */
  int64_t query_dyn_row_stride;    /* elements */
  const void* gate;                /* NULL, [heads] (per read site) or [n_tok, heads] */
  int32_t gate_per_token;
  int32_t gate_act;                /* ATTNRES_GATE_* */
  const float* logit_bias;         /* [n_src] fp32 added to every logit of a source, or NULL */
} attnres_read_desc;

/* Gradient buffers for attnres_read_backward. */
typedef struct attnres_read_grads {
  const void* grad_out;      /* [n_tok, dim] dense */
  const void* out_prenorm;   /* forward output before its rms-norm [n_tok, dim] (when normalize_output) */
  const float* out_inv_rms;  /* [n_tok] from the forward (when normalize_output) */
  const float* weights;      /* [n_tok, heads, n_src] softmax weights saved by the forward */
  void* const* dvalues;      /* [n_src] device pointers, each [n_tok, dim] dense */
  void* const* dkeys;        /* [n_src] device pointers, each [n_tok, rank] dense (LR); NULL base */
  void* dquery;              /* static query gradient (dtype, same shape as query) or NULL */
  void* dquery_dyn;          /* [n_tok, rank] dense or NULL */
  void* dgate;               /* gradient of gate (same shape as gate) or NULL */
  float* dbias;              /* [n_src] fp32 or NULL */
  void* workspace;           /* device scratch for deterministic cross-token reductions */
  size_t workspace_bytes;
} attnres_read_grads;

/* ABI version compiled into the library (ATTNRES_ABI_VERSION). */
int attnres_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* attnres_last_error(void);

/*
 * Forward read.  Writes out [n_tok, dim] (dtype); when `weights` is not NULL
 * also the fp32 softmax weights [n_tok, heads, n_src] (the backward needs
 * them); when normalize_output, out is rms-normed, out_prenorm [n_tok, dim]
 * (dtype) receives the read before the norm and out_inv_rms [n_tok] (fp32)
 * receives 1/rms -- both may be NULL when no backward follows.
 *
 * Replaces: _lrid_read_list_triton / attnres::lrid_read_list
 *   (attnres_ops.py:4533-4629, 4636-4722), _attnres_read_list_triton
 *   (attnres_ops.py:2297-2339), _attnres_read_triton (attnres_ops.py:2271-2294)
 *   and the average-read launcher (attnres_ops.py:2568-2617).
 */
int attnres_read_forward(const attnres_read_desc* desc, void* out, void* out_prenorm, float* weights,
                         float* out_inv_rms, void* stream);

/*
 * Backward of attnres_read_forward from the saved weights.  Writes every
 * non-NULL gradient buffer; cross-token sums (static query, per-site gate,
 * bias) are reduced deterministically through the workspace (no atomics).
 *
 * Replaces: _lrid_read_list_backward_triton / attnres::lrid_read_list_backward
 *   (attnres_ops.py:4373-4456, 4725-4802), _attnres_read_list_backward_triton
 *   (attnres_ops.py:2373-2421), _attnres_read_backward_triton
 *   (attnres_ops.py:2342-2370).
 */
int attnres_read_backward(const attnres_read_desc* desc, const attnres_read_grads* grads, void* stream);

/* Bytes of workspace attnres_read_backward needs for this description
 * (0 when no cross-token reduction is required).  Host-only; no GPU call. */
size_t attnres_read_backward_workspace_size(const attnres_read_desc* desc);

#ifdef __cplusplus
}
#endif

#endif /* ATTNRES_HIP_H */
