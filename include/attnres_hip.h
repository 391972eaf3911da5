/*
 * attnres_hip.h -- C ABI of the MI355X (gfx950) Attention-Residual read library.
 *
 * The reference (jon123boss/LR-AttnRes) has no native library: its fused read
 * is a set of Triton kernels launched from Python.  Each entry point below
 * replaces one of those host launchers; the citation names the reference
 * function (file:line in attnres_ops.py) whose job it takes over.  The Python
 * drop-in module (lr-attnres_amd/attnres_ops.py) binds these symbols with
 * ctypes (lr-attnres_amd/_attnres_hip.py holds the ctypes structures).
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

#define ATTNRES_ABI_VERSION 9
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
  int32_t key_dtype;               /* ATTNRES_DTYPE_* of the LR keys (and of their gradients); the
                                      reference's eager read (attnres_ops.py:4163-4192) norms keys of
                                      any dtype in fp32 and rounds them to the value dtype, so with a
                                      key dtype other than the value dtype the logits are computed in
                                      the value dtype when key_norm and in the key dtype without it;
                                      the query (static or per-token) must be in that logit dtype and
                                      its gradient is written in it.  No gate with mixed dtypes.  Base
                                      and average reads ignore it. */
  const void* static_keys;         /* LR: [n_src, rank] dense in key_dtype, or NULL.  Row s is added to
                                      every key of source s before it is scored, rounded to the key
                                      dtype, fused here instead of materialising key + static per
                                      source.  Config 4 defines one [N, 128] key per source.  The
                                      reference model has ONE shared [rank] parameter
                                      (LRIDStaticKey, model.py:275-289, fp32) that
                                      _add_static_lrid_source_key (:2046-2049) adds to every source
                                      key except the embedding's (:2062-2063, 2070-2078): express it
                                      as row 0 = zero and rows 1..n_src-1 = the parameter cast to
                                      key_dtype.  dstatic_keys then holds one gradient per row; the
                                      parameter's gradient is the fp32 sum of rows 1..n_src-1, as
                                      the model's autograd adds one cast per source. */
} attnres_read_desc;

/* Gradient buffers for attnres_read_backward. */
typedef struct attnres_read_grads {
  const void* grad_out;      /* [n_tok, dim] dense */
  const void* out_prenorm;   /* forward output before its rms-norm [n_tok, dim] (when normalize_output) */
  const float* out_inv_rms;  /* [n_tok] from the forward (when normalize_output) */
  const float* weights;      /* [n_tok, heads, n_src] softmax weights saved by the forward */
  void* const* dvalues;      /* [n_src] device pointers, each [n_tok, dim] dense */
  void* const* dkeys;        /* [n_src] device pointers, each [n_tok, rank] dense in key_dtype (LR); NULL base */
  void* dquery;              /* static query gradient (the query's dtype and shape) or NULL */
  void* dquery_dyn;          /* [n_tok, rank] dense (the query's dtype) or NULL */
  void* dgate;               /* gradient of gate (same shape as gate) or NULL */
  float* dbias;              /* [n_src] fp32 or NULL */
  void* workspace;           /* device scratch for deterministic cross-token reductions */
  size_t workspace_bytes;
  void* dstatic_keys;        /* LR with static_keys: [n_src, rank] key_dtype, per row (see static_keys), the token sums of dkeys
                                (each rounded to the key dtype once, as the reference's expand
                                backward sums them), or NULL; needs dkeys */
} attnres_read_grads;

/* ABI version compiled into the library (ATTNRES_ABI_VERSION). */
int attnres_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* attnres_last_error(void);

/* Opt-in kernel timing for benchmarks.  No counterpart in the reference (its
 * benchmarks time the Triton launches with CUDA events from Python); it lets
 * a caller time the read's main kernel alone.  While enabled,
 * attnres_read_forward and attnres_read_backward record a pair of HIP events
 * on the call's stream around their main kernel (the backward's partial-sum
 * reduction stays outside), up to 256 pairs.  Enabling creates the events on
 * the current device; disabling destroys them.  Process-wide state: not for
 * concurrent callers.  Returns ATTNRES_OK or an error code. */
int attnres_kernel_timing(int enable);

/* Waits for the recorded pairs, writes up to max_n durations (ms, in call
 * order) to ms, and starts a new recording.  Returns the number written, or
 * a negative error code (timing not enabled, bad buffer, HIP error). */
int attnres_kernel_times(float* ms, int max_n);

/* Test hook, no counterpart in the reference.  on = 1 makes the phase-2 entry
 * points run the workgroup-per-token kernels for every shape (process-wide),
 * so that a test can compare them with the one-wave-per-token kernels the
 * library otherwise picks from the shape; on = 0 restores that choice.  The
 * two give the same per-token results.  Returns ATTNRES_OK or ATTNRES_EINVAL. */
int attnres_test_phase2_block_layout(int on);

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

/*
 * attnres_read_backward without a workspace and without allocating.  No
 * counterpart in the reference (its backward allocates through PyTorch); it
 * is for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same kernels
 * and results as attnres_read_backward; grads->workspace is ignored and the
 * cross-token partial sums go to a fixed array inside the library of
 * ATTNRES_NOALLOC_SCRATCH_BYTES per GPU, which each GPU holds from the first
 * call on it until the process ends.  A description whose partial sums need
 * more (attnres_read_backward_workspace_size) fails with ATTNRES_EWORKSPACE.
 * Calls no allocator.  Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (from other streams or threads) race.  No state
 * carries from one call to the next.
 */
#define ATTNRES_NOALLOC_SCRATCH_BYTES (32u << 20)
int attnres_read_backward_noalloc(const attnres_read_desc* desc, const attnres_read_grads* grads, void* stream);

/* ------------------------------------------------------------------------
 * Cached-logit block-training schedule (two phases).
 *
 * Phase 1 reads the S completed block summaries once for Q upcoming read
 * sites whose logits were computed ahead (logits[q, s, t]); it returns each
 * site's partial read and the log-sum-exp of its logits.  Phase 2 merges a
 * site's phase-1 result with the still-growing partial block:
 *   prob = sigmoid(logit_partial + bias - lse),  out = merge(inter, partial, prob)
 * where the partial block's logit comes from its key and the site's query
 * (base: key = rms_norm(partial value); LR: key = rms_norm(partial key) and
 * `* logit_scale`) or is given.
 * ------------------------------------------------------------------------ */

#define ATTNRES_PHASE1_MAX_QUERIES 16
#define ATTNRES_PHASE_MAX_DIM 4096

typedef struct attnres_phase1_desc {
  int32_t n_src;            /* S completed sources, 1..ATTNRES_MAX_SOURCES */
  int32_t n_q;              /* Q read sites, 1..ATTNRES_PHASE1_MAX_QUERIES */
  int32_t dtype;            /* values and outputs (ATTNRES_DTYPE_*) */
  int32_t logits_dtype;     /* logits and their gradient (ATTNRES_DTYPE_*) */
  int64_t n_tok;            /* B*T */
  int32_t dim;              /* D <= ATTNRES_PHASE_MAX_DIM */
  int32_t normalize_output; /* rms-norm every [dim] output row */
  float norm_eps;
  const void* const* values;       /* [S] device pointers, rows of dim elements */
  const int64_t* value_row_stride; /* [S] elements */
  const void* logits;              /* device; (q, s, t) at q*logit_q_stride + s*logit_s_stride + t */
  int64_t logit_q_stride;
  int64_t logit_s_stride;
  const void* const* source_logits; /* optional [S] device pointers (ABI 7): when set, source s's logit
                                       for site q, token t is at source_logits[s] + q*logit_q_stride + t
                                       and logits / logit_s_stride are unused -- each source's logits may
                                       live in its own tensor (the block decoder keeps one [Q, n_tok] tensor
                                       per source and block, model.py:1843-1865 builds them per source) */
} attnres_phase1_desc;

/*
 * Phase 1 forward.  out [Q, n_tok, dim] (dtype), lse [Q, n_tok] (fp32).  With
 * normalize_output, out is rms-normed per row and out_prenorm [Q, n_tok, dim]
 * / out_inv_rms [Q, n_tok] receive what the backward needs (may be NULL when
 * no backward follows).
 *
 * Replaces: _attnres_phase1_logits_read_triton (attnres_ops.py:2742-2777) and
 *   _attnres_phase1_logits_read_list_triton (:2931-2969), behind
 *   attention_residual_phase1_from_logits (:3910-3961).
 */
int attnres_phase1_forward(const attnres_phase1_desc* desc, void* out, void* out_prenorm, float* lse,
                           float* out_inv_rms, void* stream);

/*
 * Phase 1 backward.  grad_out [Q, n_tok, dim] dense; grad_lse [Q, n_tok] fp32
 * or NULL (zero).  Writes dvalues[s] [n_tok, dim] dense and dlogits
 * [Q, S, n_tok] dense in logits_dtype.  Needs no workspace.
 *
 * Replaces: _attnres_phase1_logits_backward_weights_triton
 *   (attnres_ops.py:2882-2928) and _attnres_phase1_logits_backward_list_weights_triton
 *   (:2972-3022).
 */
int attnres_phase1_backward(const attnres_phase1_desc* desc, const void* grad_out, const float* grad_lse,
                            const void* out_prenorm, const float* out_inv_rms, void* const* dvalues,
                            void* dlogits, void* stream);

/*
 * Phase 1 backward with per-site upstream gradients and per-source logit
 * gradients (ABI 7): grad_out_sites[q] [n_tok, dim] dense; grad_lse_sites NULL
 * or [Q] pointers of [n_tok] fp32, each NULL for a site whose lse has no
 * gradient; dlogits_sources[s] receives source s's logit gradient for site q,
 * token t at + q*dlogit_q_stride + t (logits_dtype).  Same results as
 * attnres_phase1_backward on the same values.  Lets a caller hand over the
 * per-site gradients its autograd graph produced, and receive one gradient per
 * source, without stacking or slicing [Q, ...] tensors.
 * Replaces the same reference kernels as attnres_phase1_backward (the
 * reference stacks the per-site tensors first, model.py:1931-1933).
 */
int attnres_phase1_backward_sites(const attnres_phase1_desc* desc, const void* const* grad_out_sites,
                                  const float* const* grad_lse_sites, const void* out_prenorm,
                                  const float* out_inv_rms, void* const* dvalues, void* const* dlogits_sources,
                                  int64_t dlogit_q_stride, void* stream);

/*
 * Logits of one completed LR source against the read sites that will read it
 * (the block decoder's per-source logit cache; replaces the eager chain of
 * make_source_logits, model.py:1843-1865: key rms-norm, F.linear with the site
 * queries, permute, `* lrid_logit_scale`, `+ logit biases`):
 *   khat[t]     = rms_norm(key[t]) rounded to dtype (or the key with key_norm off)
 *   logit[q, t] = rnd(rnd(<khat[t], queries[q]>) * logit_scale)  (+ logit_bias, fp32 logits only)
 * logits_dtype is dtype, or fp32 when the caller adds a count-prior bias (the
 * eager chain's bf16 + fp32 add promotes to fp32).
 */
#define ATTNRES_SITE_LOGITS_MAX_QUERIES 256
#define ATTNRES_SITE_LOGITS_MAX_RANK 128

typedef struct attnres_site_logits_desc {
  int32_t dtype;          /* key and queries (ATTNRES_DTYPE_*) */
  int32_t logits_dtype;   /* dtype, or ATTNRES_DTYPE_F32 */
  int64_t n_tok;          /* B*T */
  int32_t rank;           /* R, 1..ATTNRES_SITE_LOGITS_MAX_RANK */
  int32_t n_q;            /* read sites, 1..ATTNRES_SITE_LOGITS_MAX_QUERIES; n_q * 4 * (R rounded up to
                             32 / 64 / 128) bytes of LDS */
  int32_t key_norm;
  float norm_eps;
  float logit_scale;
  float logit_bias;       /* added after the scale when logits_dtype is fp32 */
  const void* key;        /* device, [n_tok] rows of rank elements */
  int64_t key_row_stride; /* elements, >= rank */
  const void* queries;    /* device [n_q, rank] dense, dtype */
} attnres_site_logits_desc;

/* logits [n_q, n_tok] dense (logits_dtype). */
int attnres_site_logits_forward(const attnres_site_logits_desc* desc, void* logits, void* stream);

/*
 * grad_logits: [n_q] device pointers of [n_tok] gradients (logits_dtype).
 * Writes dkey [n_tok, rank] dense, and grad_scaled [n_q, n_tok] / key_hat
 * [n_tok, rank] (dtype, dense): the queries' gradient is grad_scaled @ key_hat
 * (one GEMM, as the reference's linear backward).
 */
int attnres_site_logits_backward(const attnres_site_logits_desc* desc, const void* const* grad_logits, void* dkey,
                                 void* grad_scaled, void* key_hat, void* stream);

/*
 * Phase 1 from a query bank: the logits of Q queries against the keys of the
 * S sources, after which the read is attnres_phase1_forward / _backward on
 * those logits (logits_dtype = dtype):
 *   key[s, t] = rms_norm(values[s][t]) rounded to dtype (or the value itself),
 *   logits[q, s, t] = <queries[q], key[s, t]> rounded to dtype.
 * Replaces the logits half of _attnres_phase1_forward_kernel /
 *   _attnres_phase1_backward_kernel (attnres_ops.py:785-930) behind
 *   attention_residual_phase1 (:3862-3907; eager form _attnres_phase1_read_torch
 *   :2620-2627).
 */
typedef struct attnres_keyed_logits_desc {
  int32_t n_src;            /* S, 1..ATTNRES_MAX_SOURCES */
  int32_t n_q;              /* Q, 1..ATTNRES_PHASE1_MAX_QUERIES */
  int32_t dtype;            /* values, queries, logits */
  int64_t n_tok;
  int32_t dim;              /* D <= ATTNRES_PHASE_MAX_DIM */
  int32_t key_norm;
  float norm_eps;
  const void* const* values;       /* [S] device pointers, rows of dim elements */
  const int64_t* value_row_stride; /* [S] elements */
  const void* queries;             /* device [Q, dim], dtype, contiguous */
} attnres_keyed_logits_desc;

/* logits [Q, S, n_tok] (dtype); inv_rms [S, n_tok] fp32 (the keys' 1/rms, for
 * the backward; may be NULL when none follows or without key_norm). */
int attnres_keyed_logits_forward(const attnres_keyed_logits_desc* desc, void* logits, float* inv_rms, void* stream);

/* Workspace bytes of attnres_keyed_logits_backward (host computation). */
size_t attnres_keyed_logits_backward_workspace_size(const attnres_keyed_logits_desc* desc);

/* dlogits [Q, S, n_tok] (dtype) -> dvalues[s] [n_tok, dim] dense (overwritten)
 * and dqueries [Q, dim] (dtype; NULL: not computed, no workspace needed).
 * inv_rms: the forward's (required with key_norm). */
int attnres_keyed_logits_backward(const attnres_keyed_logits_desc* desc, const void* dlogits, const float* inv_rms,
                                  void* const* dvalues, void* dqueries, void* workspace, size_t workspace_bytes,
                                  void* stream);

#define ATTNRES_MERGE_ADDCMUL 0 /* inter + (partial - inter) * prob   (attnres_ops.py:2642, 4066) */
#define ATTNRES_MERGE_LERP 1    /* torch.lerp(inter, partial, prob)   (attnres_ops.py:4159) */

typedef struct attnres_phase2_desc {
  int32_t dtype;            /* partial value / key, query, interblock output, out */
  int64_t n_tok;
  int32_t dim;              /* D <= ATTNRES_PHASE_MAX_DIM */
  int32_t rank;             /* 0: key = the partial value (base); > 0: LR partial key width (one head) */
  int32_t logit_given;      /* 1: use partial_logit; 0: score key against query */
  int32_t merge;            /* ATTNRES_MERGE_* */
  int32_t key_norm;
  int32_t normalize_output;
  float logit_scale;        /* LR logit multiplier */
  float norm_eps;
  float logit_bias;               /* constant fp32 logit bias (used when logit_bias_dev is NULL) */
  const float* logit_bias_dev;    /* device fp32 scalar bias (learned), or NULL */
  float value_scale;              /* block-summary multiplier of the partial value (1 = none) */
  const float* value_scale_dev;   /* device fp32 scalar multiplier (learned), or NULL; rounded to
                                     the dtype before it scales (model.py:983-985) */
  int32_t scale_key;              /* LR: multiply the partial key by the same scale */
  const void* partial_value;      /* [n_tok] rows of dim */
  int64_t partial_value_row_stride;
  const void* partial_key;        /* LR: [n_tok] rows of rank */
  int64_t partial_key_row_stride;
  const void* query;              /* [dim] (base) or [rank] (LR), dtype */
  const void* partial_logit;      /* [n_tok] when logit_given */
  int32_t partial_logit_dtype;
  const void* interblock_output;  /* [n_tok] rows of dim */
  int64_t interblock_row_stride;
  const float* interblock_lse;    /* [n_tok] fp32 */
} attnres_phase2_desc;

typedef struct attnres_phase2_grads {
  const void* grad_out;        /* [n_tok, dim] dense */
  void* dpartial_value;        /* [n_tok, dim] dense */
  void* dpartial_key;          /* [n_tok, rank] dense (LR) */
  void* dquery;                /* dtype, or NULL */
  void* dinterblock_output;    /* [n_tok, dim] dense */
  float* dinterblock_lse;      /* [n_tok] */
  void* dpartial_logit;        /* [n_tok] in partial_logit_dtype (logit_given) */
  float* dlogit_bias;          /* fp32 scalar, or NULL */
  float* dvalue_scale;         /* fp32 scalar, or NULL */
  void* workspace;             /* for the cross-token sums */
  size_t workspace_bytes;
  /* dquery as one row of a query bank (ABI 8; zero = the query's own
     gradient): with dquery_rows > 1, dquery points at a [dquery_rows, rank]
     (or [dquery_rows, dim]) table whose row dquery_row receives the query's
     gradient and whose other rows are set to zero -- the gradient a row
     select of the bank would hand back (the block decoder reads site i's
     query as row i - 1 of one table), without a separate fill and copy. */
  int32_t dquery_rows;
  int32_t dquery_row;
} attnres_phase2_grads;

/*
 * Phase 2 forward: out [n_tok, dim] (rms-normed when normalize_output).
 *
 * Replaces: _attnres_phase2_merge_triton (attnres_ops.py:3227-3263),
 *   _attnres_phase2_logits_merge_triton (:3348-3382), _lrid_phase2_merge_triton
 *   (:3429-3474) and the eager merges behind attention_residual_phase2[_torch],
 *   attention_residual_phase2_from_logit and lrid_attention_residual_phase2[_torch]
 *   (:3964-4160, :2630-2642).  value_scale folds the block summary
 *   partial * count^-alpha (model.py:990-1018) into the read.
 */
int attnres_phase2_forward(const attnres_phase2_desc* desc, void* out, void* stream);

/*
 * Phase 2 backward (recomputes the forward's per-token quantities).
 *
 * Replaces: _attnres_phase2_backward_triton (attnres_ops.py:3266-3345),
 *   _attnres_phase2_logits_backward_triton (:3385-3426),
 *   _lrid_phase2_backward_triton (:3477-3532).
 */
int attnres_phase2_backward(const attnres_phase2_desc* desc, const attnres_phase2_grads* grads, void* stream);

/* Workspace bytes attnres_phase2_backward needs (host-only). */
size_t attnres_phase2_backward_workspace_size(const attnres_phase2_desc* desc);

/*
 * Key-producer epilogue: split of a sublayer's fused output projection.
 *
 * The reference's LR sublayers project to dim + projection_rank columns with
 * one GEMM and take the sublayer output and its LR key from the result
 * (LRIDFusedProjection.forward, model.py:363-388; per-head key norm
 * _norm_lrid_key, model.py:34-37):
 *     out = y[:, :dim].contiguous()
 *     key = y[:, dim:dim + rank], rms-normed over each of `heads` groups of
 *           rank/heads columns when key_norm (fp32 math, one rounding)
 * y is [n_tok, row_stride] (row_stride >= proj_cols >= dim + rank), so the
 * GEMM output is consumed in place.  The forward writes out (dense
 * [n_tok, dim]), key (dense [n_tok, rank]) and, when key_norm, the fp32
 * inverse rms of each (token, head) [n_tok, heads].
 */
typedef struct attnres_keyed_split_desc {
  int32_t dtype;
  int64_t n_tok;
  int32_t dim;        /* sublayer output columns */
  int32_t rank;       /* key columns (rank % heads == 0; rank <= 256) */
  int32_t proj_cols;  /* columns of y that carry gradient (dim + projection_rank) */
  int32_t heads;      /* depth heads of the key norm: rank/heads a power of two,
                         or a multiple of 64 */
  int32_t key_norm;
  float norm_eps;     /* torch's default: FLT_EPSILON */
  const void* projected;  /* y, device */
  int64_t row_stride;     /* elements between rows of y */
} attnres_keyed_split_desc;

/* Replaces the slice / .contiguous() / _norm_lrid_key sequence of
 * model.py:374-378 with one pass over y. */
int attnres_keyed_split_forward(const attnres_keyed_split_desc* desc, void* out, void* key, float* key_inv_rms,
                                void* stream);

/* Gradient of y, dense [n_tok, proj_cols]: columns [0, dim) take grad_out,
 * columns [dim, dim + rank) the rms-norm backward of grad_key (or grad_key
 * itself without key_norm; key_inv_rms from the forward), the rest zero.
 * grad_out or grad_key may be NULL (a zero gradient).  Replaces the autograd
 * of the slices and the key norm (two zero-filled [n_tok, proj_cols] buffers,
 * two slice copies and their sum) with one pass. */
int attnres_keyed_split_backward(const attnres_keyed_split_desc* desc, const void* grad_out, const void* grad_key,
                                 const float* key_inv_rms, void* grad_projected, void* stream);

/*
 * Block-summary accumulation fused into the key-producer epilogue.
 *
 * In the block schedule a sublayer's output and LR key are used only to grow
 * the live partial block (model.py:2377-2389, 2451-2463):
 *     partial_value' = partial_value + y[:, :dim]
 *     partial_key'   = partial_key + key(y)          (key as attnres_keyed_split_forward)
 * and at a block end the block becomes a source (model.py:990-1028):
 *     value = partial_value' * scale                 (scale = count^-alpha, or a learned scale)
 *           = rms_norm(partial_value')               (value_norm; the key is then left as is)
 *     key   = partial_key' (* scale when scale_key: keys that are not rms-normed)
 * One pass over y writes partial_value' / partial_key' (complete == 0) or the
 * block source (complete == 1), so the sublayer output is never written out
 * on its own and the partial block is read and written once per sublayer.
 * Every sum and product is rounded to the dtype as the reference's eager ops
 * round it; a NULL partial (the first sublayer of a block) adds nothing.
 */
typedef struct attnres_block_accum_desc {
  attnres_keyed_split_desc split;  /* the sublayer's fused projection y */
  int32_t complete;                /* 1: form the completed block source */
  const void* partial_value;       /* [n_tok, dim] dense, or NULL */
  const void* partial_key;         /* [n_tok, rank] dense, or NULL */
  int32_t value_norm;              /* complete: rms-norm the value instead of scaling it */
  int32_t scale_key;               /* complete (without value_norm): scale the key as well */
  float value_scale;               /* complete: the scale (used when value_scale_dev is NULL) */
  const float* value_scale_dev;    /* complete: learned scale, fp32 device scalar, or NULL;
                                      rounded to the dtype before it scales (model.py:983-985) */
} attnres_block_accum_desc;

/* value_out [n_tok, dim] and key_out [n_tok, rank] (dense, dtype);
 * key_inv_rms [n_tok, heads] fp32 when split.key_norm; value_inv_rms [n_tok]
 * fp32 when complete and value_norm (both for the backward; may be NULL when
 * none follows).  Replaces the slice / key norm of LRIDFusedProjection
 * (model.py:363-388) followed by the partial-block adds and
 * _attnres_block_summary / _lrid_block_source (model.py:990-1028). */
int attnres_block_accum_forward(const attnres_block_accum_desc* desc, void* value_out, void* key_out,
                                float* key_inv_rms, float* value_inv_rms, void* stream);

/* Workspace bytes of attnres_block_accum_backward (nonzero only for a learned
 * scale, whose gradient is a deterministic sum over tokens).  Host-only. */
size_t attnres_block_accum_backward_workspace_size(const attnres_block_accum_desc* desc);

/* Gradients from grad_value (rows grad_value_row_stride elements apart) and
 * grad_key (dense) -- either may be NULL (zero):
 *   grad_projected [n_tok, proj_cols] dense: columns [0, dim) the gradient of
 *     partial_value' (which is also the gradient of partial_value: read it
 *     there), [dim, dim + rank) that of the key through its norm, the rest 0;
 *   grad_partial_key [n_tok, rank]: written only when complete and scale_key
 *     (otherwise the partial key's gradient is grad_key itself);
 *   grad_value_scale: fp32 scalar, the learned scale's gradient (NULL: not wanted).
 * key_inv_rms / value_inv_rms: the forward's. */
int attnres_block_accum_backward(const attnres_block_accum_desc* desc, const void* grad_value,
                                 int64_t grad_value_row_stride, const void* grad_key, const float* key_inv_rms,
                                 const float* value_inv_rms, void* grad_projected, void* grad_partial_key,
                                 float* grad_value_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Block accumulation fused with the next read's LR merge: one pass per token
 * grows the live partial block by this sublayer's projection (as
 * attnres_block_accum_forward with complete = 0) and merges the grown block
 * into the next site's read (as attnres_phase2_forward on it).  No single
 * counterpart in the reference, whose model grows the partial block after the
 * projection split (model.py:363-388, 2377-2389) and then calls
 * lrid_attention_residual_phase2[_torch] (attnres_ops.py:4075-4160); the block
 * decoder calls this after every sublayer that does not end a block.
 *   accum: the sublayer's projection and the live block before it
 *          (complete = 0; partial_value / partial_key NULL for a block's first
 *          sublayer).
 *   read:  the merge at the next read site, rank <= 256, its rows one-wave
 *          16-bit rows of 256/512/768/1024 (else ATTNRES_EUNSUPPORTED: compose
 *          the two calls then).  The forward ignores read.partial_value /
 *          partial_key; the backward takes them as the grown block the
 *          forward wrote.
 * Forward: value_out [n_tok, dim], key_out [n_tok, rank] (the grown block),
 * key_inv_rms [n_tok, heads] with key_norm, out [n_tok, dim] (the read).
 * Backward: grads as for attnres_phase2_backward (workspace from
 * attnres_phase2_backward_workspace_size(&desc->read); dpartial_value and
 * dpartial_key unused); grad_value [n_tok, dim] (rows grad_value_row_stride
 * elements apart) / grad_key [n_tok, rank] dense: the grown block's gradients
 * from its other consumers (NULL: none); writes
 * grad_projected [n_tok, proj_cols] -- value columns the grown value's total
 * gradient, which is also the old partial value's; key columns through the
 * key norm; padding zero -- and grad_partial_key, the old partial key's
 * gradient (the grown key's total; NULL without an old partial key).
 */
typedef struct attnres_accum_read_desc {
  attnres_block_accum_desc accum;
  attnres_phase2_desc read;
} attnres_accum_read_desc;

int attnres_accum_read_forward(const attnres_accum_read_desc* desc, void* value_out, void* key_out,
                               float* key_inv_rms, void* out, void* stream);
int attnres_accum_read_backward(const attnres_accum_read_desc* desc, const attnres_phase2_grads* grads,
                                const void* grad_value, int64_t grad_value_row_stride, const void* grad_key,
                                const float* key_inv_rms, void* grad_projected, void* grad_partial_key,
                                void* stream);

/*
 * Value-derived LR keys (config 4's key producer): the rms-norm on either side
 * of LRIDSourceKeyProjection's projection GEMM (model.py:391-428 with
 * lrid_key_from_value and lrid_key_value_norm):  key_s = rms_norm(v_s) @ W^T.
 * The GEMM itself is the caller's (a library GEMM over all sources at once,
 * [n_src * n_tok, dim] x [dim, rank]); these entry points produce its input and
 * take its input gradient back to the values.
 */
typedef struct attnres_value_key_desc {
  int32_t n_src;                   /* 1..ATTNRES_MAX_SOURCES */
  int32_t dtype;                   /* ATTNRES_DTYPE_* of the values (and the normed rows) */
  int64_t n_tok;                   /* rows per source */
  int32_t dim;                     /* D: <= 4096 (16-bit) / 2048 (fp32) on aligned rows, else <= 512 */
  float norm_eps;                  /* torch's default: FLT_EPSILON */
  const void* const* values;       /* [n_src] device pointers */
  const int64_t* value_row_stride; /* [n_src] elements */
} attnres_value_key_desc;

/* normed [n_src, n_tok, dim] dense (dtype): rms_norm(v) rounded once;
 * inv_rms [n_src, n_tok] fp32 (for the backward). */
int attnres_value_norm_forward(const attnres_value_key_desc* desc, void* normed, float* inv_rms, void* stream);

/* grad_normed [n_src, n_tok, dim] dense: the GEMM's input gradient;
 * grad_values [n_src] device pointers, each [n_tok, dim] dense (written, not
 * accumulated): the rms-norm backward, rounded once. */
int attnres_value_norm_backward(const attnres_value_key_desc* desc, const void* grad_normed, const float* inv_rms,
                                void* const* grad_values, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATTNRES_HIP_H */
