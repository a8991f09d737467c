/*
 * ghost_hip.h -- C ABI of libghost_hip.so, the MI355X (gfx950) kernels behind the
 * per-sample-gradient samplers of GhostSuite.
 *
 * Conventions shared by every entry point
 *   - All tensors are caller-owned device buffers, contiguous, row-major, batch outermost.
 *   - A batch holds N = n_train + n_val rows (samples).  The n_val validation rows are the
 *     contiguous block [val_start, val_start + n_val); the train rows are all other rows in
 *     their original order, and output index i is the i-th train row.  The reference layout
 *     (train first, val last; engine_manager.py:201-202, and every torch.split(A,
 *     [train_bs, val_bs]) in supported_layers_grad_samplers_dotprod.py) is
 *     val_start = N - n_val.
 *   - T is the number of tokens per row (product of the middle dims; 1 for 2-D inputs).
 *   - Outputs are fp32 unless stated.  Nothing is allocated: scratch memory comes from the
 *     caller as (workspace, workspace_bytes), sized by the matching *_workspace() query.
 *     The one exception is gs_linear_dot_noalloc, which takes no workspace and runs on a
 *     fixed scratch array of the library's own (one per GPU that calls it; see there).
 *   - Every call is asynchronous on `stream` (a hipStream_t; NULL = default stream) and
 *     makes no host synchronisation.  The caller keeps inputs alive until the stream
 *     passes.  Functions keep no state between calls and are re-entrant, except that calls
 *     of gs_linear_dot_noalloc that overlap on one GPU share its scratch array.
 *   - Return value: GS_OK or a negative gs_status; gs_last_error() returns a thread-local
 *     message for the last failure on the calling thread.  The library never aborts.
 */
#ifndef GHOST_HIP_H
#define GHOST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_ABI_VERSION 2

typedef enum {
  GS_OK = 0,
  GS_ERR_INVALID = -1,     /* bad shape, size, pointer or enum value */
  GS_ERR_DTYPE = -2,       /* dtype not supported by this entry point */
  GS_ERR_WORKSPACE = -3,   /* workspace missing or smaller than the *_workspace() query */
  GS_ERR_LAUNCH = -4,      /* a kernel launch or HIP runtime call failed */
  GS_ERR_UNSUPPORTED = -5  /* valid request outside this build's limits */
} gs_status;

typedef enum { GS_DTYPE_BF16 = 0, GS_DTYPE_F32 = 1, GS_DTYPE_F16 = 2 } gs_dtype;

/* Val-aggregation semantics of a Linear weight dot product.
 *   PAIRWISE_SUM: dot_i = sum_{j in val} sum_{t,s} <a_it,a_js><b_it,b_js>
 *                 (ghost branch, supported_layers_grad_samplers_dotprod.py:108-130)
 *   PRESUM:       dot_i = sum_{t,s} <a_it,abar_s><b_it,bbar_s>, abar_s = sum_j a_js
 *                 (materialised branch, supported_layers_grad_samplers_dotprod.py:131-135) */
typedef enum { GS_SEM_PAIRWISE_SUM = 0, GS_SEM_PRESUM = 1 } gs_semantics;

/* Algorithm used to evaluate a given semantics (the result is the same quantity).
 *   GHOST:   fused dual-Gram MFMA kernel; the T x T Gram blocks live only in registers.
 *   VALGRAD: V = sum_val B^T A (one GEMM), then dot_i = sum_t <b_it, V a_it> fused into
 *            the epilogue of a second GEMM; per-sample gradients are never stored.
 *   AUTO:    the one with fewer MFMA flops for the shape. */
typedef enum { GS_ALGO_AUTO = 0, GS_ALGO_GHOST = 1, GS_ALGO_VALGRAD = 2 } gs_algo;

/* Rounding of the ghost Gram blocks.
 *   FP32:    Gram entries and their Hadamard product stay fp32, except that with bf16
 *            operands (16-byte aligned rows) the activation Gram block is held as bf16
 *            while the grad Gram block accumulates, the rounding point the reference's
 *            bf16 a_dot also has.
 *   REF_BF16: Gram entries and their product are rounded to bf16 before the fp32 sum, as
 *            the reference's bf16 matmul outputs are (supported_layers_grad_samplers_dotprod.py:125-129). */
typedef enum { GS_ROUND_FP32 = 0, GS_ROUND_REF_BF16 = 1 } gs_rounding;

/* Layout of a Kronecker projection output block per sample.
 *   KO_KI: [k_o, k_i] (nn.Linear, autograd_gradproj.py:155-158)
 *   KI_KO: [k_i, k_o] with P_i applied to the output grads and P_o to the inputs
 *          (transformers Conv1D, autograd_gradproj.py:141-147) */
typedef enum { GS_PROJ_KO_KI = 0, GS_PROJ_KI_KO = 1 } gs_proj_layout;

int gs_abi_version(void);
const char* gs_last_error(void);

/* ---- Linear weight dot product ------------------------------------------------------
 * Replaces the weight part of _compute_linear_dot_product
 * (ghostEngines/supported_layers_grad_samplers_dotprod.py:75-135), and the weight part of
 * _compute_Conv1D_dot_product (:369-447, which is PRESUM in both of its branches).
 * A: [N, T, d_in] layer inputs.  G: [N, T, d_out] output grads (raw grad_output of the loss).
 * dtype: GS_DTYPE_BF16 or GS_DTYPE_F32 for both A and G.
 * out_dot:  [n_train] fp32, dot of each train row's weight grad with the val aggregate.
 * out_pair: NULL, or [n_val, n_train] fp32 with out_pair[j][i] = <grad_i, grad_j> (pairwise
 *           semantics) -- the per-pair matrix; sum over j equals out_dot.  Must be NULL
 *           for PRESUM. */
size_t gs_linear_dot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                               int64_t d_out, int semantics, int algo, int want_pair);
/* The algorithm (GS_ALGO_GHOST or GS_ALGO_VALGRAD) a call with these arguments runs. */
int gs_linear_dot_algo(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                       int64_t d_out, int semantics, int algo, int want_pair);
int gs_linear_dot(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                  int64_t val_start, int64_t T, int64_t d_in, int64_t d_out, int semantics,
                  int algo, int rounding, float* out_dot, float* out_pair, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Allocation-free variant of gs_linear_dot.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, semantics, kernels and results
 * as gs_linear_dot, without (workspace, workspace_bytes): the scratch memory is a fixed
 * device array of GS_LINEAR_NOALLOC_SCRATCH_BYTES inside the library, one copy per GPU,
 * reserved on a GPU by the first call there (the array sits in a code object of its own,
 * which the other entry points never load) and held until the process ends.  The call
 * allocates nothing and frees nothing.
 *   - `stream` must belong to the current device (NULL = its default stream).
 *   - A call that needs more scratch than the array holds returns GS_ERR_UNSUPPORTED
 *     (gs_linear_dot_noalloc_bytes tells the need; use gs_linear_dot with a workspace then).
 *   - Every call on one GPU uses the same array and leaves its contents behind (nothing in
 *     it needs to start at zero).  Calls that overlap on one GPU -- on two streams, or from
 *     two threads without ordering -- race on it: serialise them. */
#define GS_LINEAR_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
size_t gs_linear_dot_noalloc_bytes(const void* A, const void* G, int dtype, int64_t N,
                                   int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
                                   int semantics, int algo, int want_pair);
int gs_linear_dot_noalloc(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                          int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                          int semantics, int algo, int rounding, float* out_dot,
                          float* out_pair, void* stream);

/* The val term of a Linear layer's dot, V [d_out, d_in] (dtype; fp32 accumulation):
 *   GS_SEM_PAIRWISE_SUM: V = sum over the val rows and tokens of g a^T
 *   GS_SEM_PRESUM:       V = gbar^T abar, gbar / abar = the val rows summed over the val
 *                        samples per token position (how the reference's materialised
 *                        branch forms its val term)
 * Reference: the val half of _compute_linear_dot_product
 * (supported_layers_grad_samplers_dotprod.py:75-135); the V gs_linear_rowdot and
 * gs_linear_rowdot_bias take. */
size_t gs_linear_val_gradient_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                        int64_t d_in, int64_t d_out, int semantics);
int gs_linear_val_gradient(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                           int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                           int semantics, void* V, void* workspace, size_t workspace_bytes,
                           void* stream);

/* A Linear layer's weight dots and weight train gradient from one pass over the train rows
 * (and, with out_bias_dot / out_bias_grad, its bias dots and bias train gradient):
 *   out_dot[i]      = sum over train row i's tokens of g^T V a, V the val term of
 *                     gs_linear_val_gradient (semantics as there)
 *   out_grad        = grad_scale * sum over the train rows of g a^T, [d_out, d_in], grad_dtype
 *   out_bias_dot[i] = sum_t <g_it, the val rows' column sum of G>
 *   out_bias_grad   = bias_grad_scale * the train rows' column sum of G, bias_grad_dtype
 * out_grad, out_bias_dot, out_bias_grad may be null.  bf16 operands, 16-byte aligned, T a
 * multiple of 64, d_in and d_out multiples of 8, n_val >= 1, operands below 2 GiB; other
 * cases return GS_ERR_UNSUPPORTED (workspace query: 0).  with_bias: 1 when a bias output is
 * passed.  Reference: _compute_linear_dot_product (supported_layers_grad_samplers_dotprod.py
 * :75-146) and _compute_linear_train_grad (:155-173) with _compute_train_grad_bias
 * (autograd_grad_sample_dotprod.py:199-222). */
size_t gs_linear_dot_train_grad_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                          int64_t d_in, int64_t d_out, int semantics,
                                          int with_bias);
int gs_linear_dot_train_grad(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                             int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                             int semantics, float* out_dot, void* out_grad, int grad_dtype,
                             float grad_scale, float* out_bias_dot, void* out_bias_grad,
                             int bias_grad_dtype, float bias_grad_scale, void* workspace,
                             size_t workspace_bytes, void* stream);

/* The same pass for an HF Conv1D layer (weight [d_in, d_out]): A [N, T, d_in], G [N, T, d_out]
 * as for gs_linear_dot_train_grad, the same out_dot, out_bias_dot and out_bias_grad, and
 *   out_grad = grad_scale * sum over the train rows of a g^T, [d_in, d_out]
 * (the operands go into the pass swapped, and the bias terms are taken from the other side).
 * Reference: _compute_Conv1D_dot_product (supported_layers_grad_samplers_dotprod.py:369-471)
 * and _compute_Conv1D_train_grad (:474-506) with _compute_train_grad_bias
 * (autograd_grad_sample_dotprod.py:199-222). */
size_t gs_conv1d_dot_train_grad_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                          int64_t d_in, int64_t d_out, int semantics,
                                          int with_bias);
int gs_conv1d_dot_train_grad(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                             int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                             int semantics, float* out_dot, void* out_grad, int grad_dtype,
                             float grad_scale, float* out_bias_dot, void* out_bias_grad,
                             int bias_grad_dtype, float bias_grad_scale, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Train gradient of a Linear / HF Conv1D weight from the train rows (the val block
 * [val_start, val_start + n_val) skipped), fp32 accumulation, scale applied before the one
 * rounding to out_dtype (GS_DTYPE_BF16 or GS_DTYPE_F32):
 *   layout 0: out [d_out, d_in] = scale * sum over train rows and tokens of g a^T (Linear)
 *   layout 1: out [d_in, d_out] = scale * sum of a g^T (HF Conv1D)
 * bf16 operands, 16-byte aligned, d_in and d_out multiples of 8, every row of A and G below
 * 2 GiB of offset; other cases return GS_ERR_UNSUPPORTED (workspace query: 0).  Outputs of
 * 256 or more 256 x 256 tiles run one work item per tile over all the train rows; smaller
 * ones on 128 x 128 tiles with the rows split, the fp32 split partials in the workspace.
 * Reference: _compute_linear_train_grad (supported_layers_grad_samplers_dotprod.py:155-173)
 * and _compute_Conv1D_train_grad (:474-506), with scale = 1 / n_train there. */
size_t gs_linear_train_grad_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                      int64_t d_in, int64_t d_out);
int gs_linear_train_grad(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                         int64_t val_start, int64_t T, int64_t d_in, int64_t d_out, float scale,
                         void* out, int out_dtype, int layout, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Row-dot with a caller-formed val gradient V = G_val^T A_val ([d_out, d_in], same dtype):
 *   out_dot[i] = sum_t g_it^T V a_it over the train rows (the second half of the
 *   VALGRAD algorithm of gs_linear_dot, for callers that form V with a library GEMM).
 * Replaces the same reference function as gs_linear_dot
 * (supported_layers_grad_samplers_dotprod.py:75-135); with V from the summed val rows it is
 * the pairwise-sum dot, with V from the presummed val rows the presum dot. */
size_t gs_linear_rowdot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                                  int64_t d_out);
int gs_linear_rowdot(const void* A, const void* G, const void* V, int dtype, int64_t N,
                     int64_t n_val, int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                     float* out_dot, void* workspace, size_t workspace_bytes, void* stream);

/* Row-dot with the layer's bias folded into the same pass (reference: the weight and bias
 * parts of _compute_linear_dot_product, :75-146, and _compute_train_grad_bias,
 * autograd_grad_sample_dotprod.py:199-222):
 *   out_dot[i]      = sum_t g_it^T V a_it                    (as gs_linear_rowdot)
 *   out_bias_dot[i] = sum_t <g_it, vb>,   vb = sum over val rows and tokens of g (fp32)
 *   out_bias_grad   = NULL, or grad_scale * sum over train rows and tokens of g ([d_out],
 *                     grad_dtype)
 * The row-dot epilogue sums each G tile it already holds in LDS over its tokens; those
 * column sums give both bias terms, so the train rows of G are read once.
 * Supported for bf16, 16-byte aligned operands below 2 GiB, T a multiple of 256 and d_out a
 * multiple of 192 or 256: the workspace query returns 0 otherwise (use gs_linear_rowdot +
 * gs_bias_dot then). */
size_t gs_linear_rowdot_bias_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                       int64_t d_in, int64_t d_out);
int gs_linear_rowdot_bias(const void* A, const void* G, const void* V, int dtype, int64_t N,
                          int64_t n_val, int64_t val_start, int64_t T,
                          int64_t d_in, int64_t d_out, float* out_dot, float* out_bias_dot,
                          void* out_bias_grad, int grad_dtype, float grad_scale,
                          void* workspace, size_t workspace_bytes, void* stream);

/* The whole Linear sampler with a bias in one call (weight dot, bias dot, bias train
 * gradient), for the semantics of gs_linear_dot: the K-major GEMM forms V (its workgroups
 * also sum the val rows of G: the val bias gradient), then the row-dot + bias pass of
 * gs_linear_rowdot_bias.  With d_out > d_in the pass contracts over d_out instead
 * (sum_t <a_it, V^T g_it>, V^T formed by the K-major GEMM) and takes the bias column sums of
 * G from its mainloop.  Reference: _compute_linear_dot_product weight and bias parts
 * (supported_layers_grad_samplers_dotprod.py:75-146), Conv1D (:369-471), and
 * _compute_train_grad_bias (autograd_grad_sample_dotprod.py:199-222).  Supported for bf16,
 * 16-byte aligned operands below 2 GiB, T a multiple of 256 and d_out a multiple of 192 or
 * 256, or d_out > d_in with d_in such a multiple (the workspace query returns 0 otherwise; use
 * gs_linear_dot and gs_bias_dot then). */
size_t gs_linear_bias_dot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                    int64_t d_in, int64_t d_out, int semantics);
int gs_linear_bias_dot(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                       int64_t val_start, int64_t T, int64_t d_in, int64_t d_out, int semantics,
                       float* out_dot, float* out_bias_dot, void* out_bias_grad, int grad_dtype,
                       float grad_scale, void* workspace, size_t workspace_bytes, void* stream);

/* ---- Bias dot product and bias train gradient ---------------------------------------
 * Replaces the bias part of _compute_linear_dot_product (:137-146), the bias part of
 * _compute_Conv1D_dot_product (:450-471) and _compute_train_grad_bias
 * (ghostEngines/autograd_grad_sample_dotprod.py:199-222).
 * G: [N, T, d_out].  out_dot: [n_train] = <sum_t g_it, sum_{j,t} g_jt>.
 * out_grad: NULL, or [d_out] (dtype grad_dtype) = grad_scale * sum_{train i,t} g_it. */
size_t gs_bias_dot_workspace(int64_t N, int64_t T, int64_t d_out);
int gs_bias_dot(const void* G, int dtype, int64_t N, int64_t n_val, int64_t val_start,
                int64_t T, int64_t d_out, float* out_dot, void* out_grad, int grad_dtype,
                float grad_scale, void* workspace, size_t workspace_bytes, void* stream);

/* ---- Embedding dot product -----------------------------------------------------------
 * Replaces _compute_embedding_dot_product (:181-211):
 *   dot_i = sum_t <g_it, V[x_it]>,  V[v] = sum_{j in val, s : x_js = v} g_js
 * without a [vocab, d] table: val tokens with equal ids form one segment (keyed by the
 * first such val token through a [vocab] int32 index), segment sums are accumulated in
 * 64-bit fixed point (deterministic), and each train token looks its segment up by id.
 * ids: [N, T] int64 token ids in [0, vocab).  G: [N, T, d]. */
size_t gs_embedding_dot_workspace(int64_t N, int64_t n_val, int64_t T, int64_t d,
                                  int64_t vocab);
int gs_embedding_dot(const int64_t* ids, const void* G, int dtype, int64_t N, int64_t n_val,
                     int64_t val_start, int64_t T, int64_t d, int64_t vocab, float* out_dot,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---- Embedding train gradient -----------------------------------------------------------
 * Replaces _compute_embedding_train_grad (:214-235):
 *   grad[v] = scale * sum over the train tokens t with x_t = v of g_t     grad: [vocab, d]
 * (the reference: index_add_ of the N-scaled train rows into zeros_like(weight), then / n_t;
 * here scale = N / n_t carries both factors).  The train tokens are sorted by (id, token
 * index); each id's rows are summed in fp32 in token order over windows of 16 places of the
 * sorted list, a run that crosses windows by its window parts in window order, and written
 * once, rounded once to grad_dtype: the same bits on every run, and work linear in the
 * number of tokens however often an id repeats.
 * accumulate = 0: every row of grad is written (zeros where no train token has the id).
 * accumulate = 1: the rows of ids present are added to grad's contents, others untouched
 *   (a tied weight's Linear train gradient already there).
 * Ids outside [0, vocab) are skipped.  ids: [N, T] int64, G: [N, T, d] (dtype). */
size_t gs_embedding_train_grad_workspace(int64_t N, int64_t n_val, int64_t T, int64_t d,
                                         int64_t vocab);
int gs_embedding_train_grad(const int64_t* ids, const void* G, int dtype, int64_t N,
                            int64_t n_val, int64_t val_start, int64_t T, int64_t d,
                            int64_t vocab, float scale, void* grad, int grad_dtype,
                            int accumulate, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---- LayerNorm dot products and train gradients -------------------------------------
 * Replaces _compute_layernorm_dot_product (:242-300) and _compute_layernorm_train_grad
 * (:303-366) in one pass over X and G.
 * X: [N, T, F] LayerNorm inputs, G: [N, T, F] output grads, eps as in the layer.
 *   xhat = (x - mean) * rsqrt(var + eps)   (biased variance, no affine)
 *   out_dot_w[i] = <sum_t g_it*xhat_it, sum_{j,t} g_jt*xhat_jt>, out_dot_b likewise with g.
 * out_dot_b may be NULL (no bias).  out_grad_w / out_grad_b: NULL or [F] of grad_dtype,
 *   = grad_scale * sum_{train i,t} (g_it*xhat_it) and grad_scale * sum_{train i,t} g_it. */
size_t gs_layernorm_dot_workspace(int64_t N, int64_t T, int64_t F);
int gs_layernorm_dot(const void* X, const void* G, int dtype, int64_t N, int64_t n_val,
                     int64_t val_start, int64_t T, int64_t F, float eps, float* out_dot_w,
                     float* out_dot_b, void* out_grad_w, void* out_grad_b, int grad_dtype,
                     float grad_scale, void* workspace, size_t workspace_bytes, void* stream);

/* ---- Kronecker gradient projection -----------------------------------------------------
 * Replaces GradProjHooks._compute_dense_proj
 * (ghostEngines/gradProjection/autograd_gradproj.py:120-165):
 *   KO_KI: out[b] = scale * sum_t (P_o g_bt)(P_i a_bt)^T   [k_o, k_i]
 *   KI_KO: out[b] = scale * sum_t (P_i g_bt)(P_o a_bt)^T   [k_i, k_o]  (Conv1D roles)
 * A: [B, T, n_a], G: [B, T, n_g] (dtype), P_i / P_o: row-major projection matrices of
 * p_dtype whose column counts match the operand each multiplies.
 * out: [B, k_rows, k_cols] of out_dtype. */
size_t gs_kron_proj_workspace(int64_t B, int64_t T, int64_t k_i, int64_t k_o);
int gs_kron_proj(const void* A, const void* G, int dtype, int64_t B, int64_t T, int64_t n_a,
                 int64_t n_g, const void* P_i, const void* P_o, int p_dtype, int64_t k_i,
                 int64_t k_o, int layout, float scale, void* out, int out_dtype,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Replaces GradProjHooks._compute_embedding_proj
 * (ghostEngines/gradProjection/autograd_gradproj.py:167-222), whose per-token loop reads
 * every token id back to the host:
 *   out[b] = scale * sum_t (P_o g_bt)(P_i[:, ids_bt])^T        [k_o, k_i]
 * ids: [B, T] int64; G: [B, T, n_g] (dtype); P_iT: P_i transposed, [vocab, k_i] row-major;
 * P_o: [k_o, n_g]; both of p_dtype (= dtype).  Ids outside [0, vocab) contribute nothing
 * (the embedding's own forward rejects them first).  Workspace: gs_kron_proj_workspace. */
int gs_kron_embed_proj(const int64_t* ids, const void* G, int dtype, int64_t B, int64_t T,
                       int64_t n_g, const void* P_iT, const void* P_o, int p_dtype,
                       int64_t vocab, int64_t k_i, int64_t k_o, float scale, void* out,
                       int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ---- Ordered sum of the per-parameter dot products --------------------------------------
 * Replaces the summation loop of GradDotProdEngine._aggregate_and_log_dot_products
 * (ghostEngines/graddotprod_engine.py:198-211: total = the first grad_dot_prod, then
 * total += each later one, in named_parameters order) with one launch per 256 sources:
 *   out[i] = ((s_0[i] + s_1[i]) + s_2[i]) + ...
 * element by element in the order given, in fp32 arithmetic, each partial sum rounded to
 * out_dtype -- the rounding of an in-place add into a total of that dtype; out may be s_0
 * (the reference accumulates into its first tensor, whose dtype out_dtype then is).
 * srcs: host array of `count` device pointers to n elements each; dtypes: host array of their
 * dtypes (bf16 or fp32).  No workspace. */
int gs_ordered_sum(const void* const* srcs, const int* dtypes, int count, int64_t n, void* out,
                   int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GHOST_HIP_H */
