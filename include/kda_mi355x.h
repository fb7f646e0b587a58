/*
 * kda_mi355x.h — C ABI of the MI355X (gfx950) Kimi Delta Attention backend.
 *
 * Plain C: device pointers, sizes, a dtype enum and an opaque HIP stream
 * (`void*`, a `hipStream_t`).  No torch types cross this boundary.  All calls
 * are asynchronous on `stream`; they allocate nothing (the chunked prefill
 * takes a caller-provided workspace) and return a status code.
 *
 * Tensor layouts are the reference's canonical contiguous layouts
 * (pablo-reyes8/kimi-k3-pytorch, src/kda):
 *   q, k, g : [tokens, H, K]   (dense batches are [B, T, H, K] = tokens B*T)
 *   v, out  : [tokens, H, V]
 *   beta    : [tokens, H]
 *   states  : [N, H, K, V]     (the `recurrent_state` of src/kda/state.py:16)
 *
 * Sequences.  `cu_seqlens == NULL` means N dense sequences of `dense_span`
 * tokens each (sequence s owns rows [s*T, (s+1)*T)).  Otherwise
 * `cu_seqlens` is an int32 device array of N+1 monotone offsets (packed
 * documents; the state starts from zero or `initial_state[s]` at each
 * document start), and `dense_span` is then the longest document's length in
 * tokens when the caller knows it, 0 otherwise: a scheduling hint only (the
 * offsets live in device memory), which lets the chunk prefill cut a
 * document far longer than the rest into segments instead of leaving the
 * GPU to its one chain; results do not depend on it beyond rounding.
 * `valid_lens` (int32 device array [N], or NULL) marks a
 * monotone right-padding: tokens at positions >= valid_lens[s] of sequence s
 * neither decay, write nor read the state and their output rows are zero
 * (src/kda/utils.py:82-94).
 *
 * Arithmetic: bf16/f16/f32 inputs compute in f32 with an f32 state; f64
 * inputs compute in f64 with an f64 state (src/kda/utils.py:74-79).
 */
#ifndef KDA_MI355X_H
#define KDA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDA_ABI_VERSION 10

/* status codes */
#define KDA_OK 0
#define KDA_ERR_INVALID_ARGUMENT 1
#define KDA_ERR_UNSUPPORTED 2
#define KDA_ERR_WORKSPACE 3
#define KDA_ERR_LAUNCH 4

/* element types */
#define KDA_DTYPE_F32 0
#define KDA_DTYPE_F16 1
#define KDA_DTYPE_BF16 2
#define KDA_DTYPE_F64 3

/* Version of this ABI (KDA_ABI_VERSION). No reference counterpart. */
int kda_abi_version(void);

/* Human-readable text for a status code, including the last error detail
 * recorded on the calling thread. No reference counterpart. */
const char* kda_status_string(int status);

/*
 * Exact token-by-token KDA recurrence: per token
 *   S <- diag(exp g_t) S;  e = v_t - S^T k_t;  S <- S + beta_t k_t e^T;  o_t = S^T q_t.
 * Replaces `recurrent_kda` (src/kda/recurrent.py:25-80) for T >= 1.
 *   in_dtype        : dtype of q, k, v, g, beta and `out`.
 *   state_dtype     : KDA_DTYPE_F32 for bf16/f16/f32 inputs, KDA_DTYPE_F64 for f64.
 *   initial_state   : [N,H,K,V] or NULL (zero state). May alias final_state.
 *   final_state     : [N,H,K,V] or NULL.
 *   states_per_token: NULL, or [T,N,H,K,V] written after every token
 *                     (`return_states_per_token`, recurrent.py:61,73-74,79);
 *                     dense sequences only (cu_seqlens == NULL).
 */
int kda_recurrent_fwd(const void* q, const void* k, const void* v, const void* g,
                      const void* beta, int in_dtype, const void* initial_state,
                      void* final_state, int state_dtype, void* out, void* states_per_token,
                      const int32_t* cu_seqlens, int64_t dense_span, const int32_t* valid_lens,
                      int64_t num_seqs, int64_t total_tokens, int64_t heads, int64_t key_dim,
                      int64_t value_dim, void* stream);

/*
 * One decode step (T = 1) for `batch` sequences: the memory-bound
 * diagonal-decay, rank-1 delta update of the cached state, read once and
 * written once.  This is what `KimiDeltaAttention.forward(mode="decode")`
 * runs through `recurrent_kda` with T = 1 (src/kda/kda.py:144-145,
 * src/kda/recurrent.py:62-74).  `state_out` may equal `state_in` (in-place
 * update); `state_in == NULL` means a zero state.
 */
int kda_decode_step(const void* q, const void* k, const void* v, const void* g,
                    const void* beta, int in_dtype, const void* state_in, void* state_out,
                    int state_dtype, void* out, int64_t batch, int64_t heads, int64_t key_dim,
                    int64_t value_dim, void* stream);

/*
 * Workspace bytes `kda_chunk_fwd` needs for these sizes (0 if none), for
 * dense sequences of total_tokens / num_seqs tokens (longest_tokens 0) or for
 * packed documents whose longest is longest_tokens tokens (the value the call
 * passes in `dense_span`; 0 when unknown); off the MFMA path packed documents
 * take a zero-padded batch of num_seqs x longest_tokens tokens, and an
 * f32-state call never needs more.  0 for a longest_tokens outside
 * 0..total_tokens.
 * No reference counterpart (the reference allocates per call).
 */
size_t kda_chunk_fwd_workspace_bytes(int64_t num_seqs, int64_t total_tokens, int64_t longest_tokens,
                                     int64_t heads, int64_t key_dim, int64_t value_dim, int in_dtype);

/*
 * The schedule `kda_chunk_fwd` picks for these sizes: *chunks_per_segment is
 * the number of 64-token chunks per segment (0 when every sequence is one
 * segment, -2 when the shape takes the split-bf16 chunk path, -1 when it runs
 * the exact recurrence kernel: f64 inputs, and K > 128) and *segments
 * the bound on segments it sizes its workspace for; longest_tokens as for
 * kda_chunk_fwd_workspace_bytes.  No reference
 * counterpart (the reference has one schedule, a Python loop over chunks,
 * src/kda/chunkwise.py:61-102); benchmarks and tests use it to attribute
 * time and to cover both schedules.
 */
int kda_chunk_fwd_plan(int64_t num_seqs, int64_t total_tokens, int64_t longest_tokens, int64_t heads,
                       int64_t key_dim, int64_t value_dim, int in_dtype, int64_t* chunks_per_segment,
                       int64_t* segments);

/*
 * Overrides the segment length that kda_chunk_fwd and kda_chunk_fwd_decay
 * choose for the MFMA prefill (process-wide, every device): a positive value
 * forces that many chunks per segment, 0 one segment per sequence, -1
 * restores the library's own plan.  Results do not depend on the schedule;
 * tests use it to cover the segmented composition at small sizes.  No
 * reference counterpart (the reference has no schedule).  Returns
 * KDA_ERR_INVALID_ARGUMENT below -1.
 */
int kda_set_segment_chunks(int64_t chunks_per_segment);

/*
 * Chunkwise-parallel KDA prefill (chunk 64): intra-chunk UT transform with a
 * forward-substitution solve, bf16 MFMA chunk products with f32 accumulation
 * and an f32 inter-chunk state scan, cut into segments whose affine state
 * maps are composed when batch * heads alone would not fill the GPU.  Replaces `chunkwise_kda`
 * (src/kda/chunkwise.py:17-107); its result does not depend on the
 * reference's chunk_size / secondary_tile_size (the reference's own
 * invariance, tests/kda/test_kda_chunkwise_equivalence.py:42-57,
 * tests/kda/test_kda_ut_transform.py:94-103).  Packed documents via
 * `cu_seqlens` have no reference counterpart: each document equals an
 * independent `chunkwise_kda` call.
 * The MFMA path covers bf16/f16 inputs with K <= 128 a multiple of 16 (a smaller K is
 * zero-padded to 128 channels inside the kernel) and V a multiple of 16 in
 * 16..256.  Other bf16/f16/f32 inputs with K <= 128 and an f32 state take
 * the split-bf16 chunk path: per-chunk operands in a chunk-parallel kernel,
 * the state scan with every product on split operands (x = hi + lo, two bf16
 * each, relative error about 2^-17) and the outputs in a second
 * chunk-parallel kernel; its workspace is B x H x ceil(T/64) records of
 * 240.5 KiB (K = V = 128: the operands the forward scan and the output
 * kernel read, and each chunk's start state and pseudo-values).  Packed documents on that path are gathered into a
 * zero-padded batch of num_seqs x dense_span tokens (dense_span must be the
 * longest document's length; a smaller one returns KDA_ERR_INVALID_ARGUMENT
 * where the host can tell, and drops tokens past it otherwise) and their
 * outputs scattered back (one document is the dense batch, no copies); value widths past 128 run as
 * slices of at most 128 columns (state and value columns never interact).
 * The rest (K > 128, f64 inputs, a bf16/f16 state, packed documents without
 * their longest length) runs the exact recurrence kernel, which needs no
 * workspace.
 */
int kda_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  int in_dtype, const void* initial_state, void* final_state, int state_dtype,
                  void* out, const int32_t* cu_seqlens, int64_t dense_span,
                  const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens,
                  int64_t heads, int64_t key_dim, int64_t value_dim, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * `kda_chunk_fwd` with the decay formed inside the chunk kernel from the decay
 * logits, so g never makes a round trip through HBM: the loader waves compute
 *   g = g_min * clamp(sigmoid(exp(a_log[h]) * (decay_logits + decay_bias[h])), eps, 1 - eps)
 * (eps of the input type), round it to the input type and take its in-chunk
 * cumulative sum.  Replaces the chain LowerBoundedDecay.forward
 * (src/kda/decay.py:36-43, with the bias of src/kda/projections.py:215) ->
 * chunkwise_kda (src/kda/chunkwise.py:17-107) of KimiDeltaAttention.forward
 * (src/kda/kda.py:131-151).  The result equals kda_gates_fwd followed by
 * kda_chunk_fwd bit for bit.
 *   decay_logits : [tokens, H, K] in in_dtype (in place of g); decay_bias [H, K] or NULL;
 *   a_log        : f32 [H];  g_min < 0.
 * The MFMA shapes only (bf16/f16 inputs, K <= 128 a multiple of 16, V a multiple of 16
 * in 16..256): other shapes return KDA_ERR_UNSUPPORTED.  Workspace as
 * kda_chunk_fwd_workspace_bytes.
 */
int kda_chunk_fwd_decay(const void* q, const void* k, const void* v, const void* decay_logits,
                        const void* decay_bias, const float* a_log, double g_min, const void* beta,
                        int in_dtype, const void* initial_state, void* final_state, int state_dtype,
                        void* out, const int32_t* cu_seqlens, int64_t dense_span,
                        const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens,
                        int64_t heads, int64_t key_dim, int64_t value_dim, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * `kda_chunk_fwd` for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments, checks and kernels as
 * `kda_chunk_fwd`, minus the workspace: it lives in a static device array of
 * KDA_NOALLOC_SCRATCH_BYTES that each GPU the library runs on holds until the
 * process ends.  A prefill whose workspace exceeds it returns
 * KDA_ERR_WORKSPACE before anything is launched (128 MiB covers one
 * 8192-token bf16 sequence at H=16, which needs 72.5 MB; shapes with
 * batch * heads >= 192 need only the small chunk maps; the split-bf16 path's
 * records, 240.5 KiB per 64 tokens and head at K = V = 128 for f32 inputs and
 * 184.5 KiB for bf16/f16 inputs, cover about 390 and 450 of them with their
 * segment records).  The call performs
 * no device allocation.  All calls on one GPU share that GPU's array:
 * calls that overlap on one GPU (two streams, two host threads) race.  The
 * stream must belong to the current device.
 */
#ifndef KDA_NOALLOC_SCRATCH_BYTES
#define KDA_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)
#endif
int kda_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g,
                          const void* beta, int in_dtype, const void* initial_state,
                          void* final_state, int state_dtype, void* out,
                          const int32_t* cu_seqlens, int64_t dense_span,
                          const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens,
                          int64_t heads, int64_t key_dim, int64_t value_dim, void* stream);

/*
 * `kda_chunk_fwd` with a HIP event recorded between its kernels; returns,
 * after synchronising `stream`, the duration of each stage in kernel_ms[0..3]
 * (chunk map, segment summaries, segment combine, chunk outputs; zero for a
 * stage the call did not run) and the number of stages in *num_kernels.  No
 * reference counterpart: it exists so that a benchmark can attribute time
 * per kernel.
 */
int kda_chunk_fwd_profiled(const void* q, const void* k, const void* v, const void* g, const void* beta,
                           int in_dtype, const void* initial_state, void* final_state, int state_dtype,
                           void* out, const int32_t* cu_seqlens, int64_t dense_span,
                           const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens,
                           int64_t heads, int64_t key_dim, int64_t value_dim, void* workspace,
                           size_t workspace_bytes, void* stream, float* kernel_ms, int* num_kernels);

/*
 * UT transform of independent chunks, canonical [B,C,H,*] inputs.
 * Replaces `ut_transform` (src/kda/ut_transform.py:61-92).  Outputs, in
 * `out_dtype` (f32 for bf16/f16/f32 inputs, f64 for f64):
 *   M [B,H,C,C]; U [B,C,H,V]; W, log_gamma, k_gamma [B,C,H,K].
 */
int kda_ut_transform(const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                     void* M, void* U, void* W, void* log_gamma, void* k_gamma, int out_dtype,
                     int64_t batch, int64_t count, int64_t heads, int64_t key_dim,
                     int64_t value_dim, void* stream);

/*
 * Backward of `kda_ut_transform`: the gradients of a loss through (M, U, W,
 * log_gamma, k_gamma) with respect to (k, v, g, beta), as autograd takes them
 * through src/kda/ut_transform.py:23-92 (M = (I + diag(beta) A)^-1 diag(beta)
 * by triangular solve, W = M k_gamma, U = M v).  The upstream gradients are in
 * `out_dtype` (f32 for bf16/f16/f32 inputs, f64 for f64), shaped like the
 * forward outputs, each NULL for zero; dk, dv, dg, dbeta are written in
 * `out_dtype` with the inputs' shapes.  One workgroup per (batch, head);
 * workspace: kda_ut_transform_bwd_workspace_bytes.  count <= 1024.
 */
size_t kda_ut_transform_bwd_workspace_bytes(int64_t batch, int64_t count, int64_t heads,
                                            int64_t key_dim, int out_dtype);

int kda_ut_transform_bwd(const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                         const void* dM, const void* dU, const void* dW, const void* d_log_gamma,
                         const void* d_k_gamma, void* dk, void* dv, void* dg, void* dbeta, int out_dtype,
                         int64_t batch, int64_t count, int64_t heads, int64_t key_dim, int64_t value_dim,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward of the chunkwise operator: the gradients of a loss through
 * (out, final_state) = chunkwise(q, k, v, g, beta, initial_state) with respect
 * to every input.  Replaces the autograd backward of chunkwise_kda
 * (src/kda/chunkwise.py:17-107; its gradients are pinned by
 * tests/kda/test_kda_chunkwise_equivalence.py:92-134).
 *   q, k, g [batch, tokens, heads, key_dim]; v, d_out [batch, tokens, heads, value_dim];
 *   beta [batch, tokens, heads]: dtype bf16, f16, f32 or f64 (inputs already masked);
 *   initial_state, d_final_state : f32 [batch, heads, key_dim, value_dim] or NULL (zero);
 *                                  f64 (passed through these pointers) when dtype is f64
 *   dq, dk, dv, dg, dbeta        : outputs, shaped and typed like the inputs
 *   d_initial_state              : like initial_state, or NULL
 *   key_dim, value_dim <= 128; dense layout.  Packed documents are differentiated as
 *   dense batches of similar-length documents, zero-padded (a zero row is an
 *   identity step), by the caller (the Python wrapper's length buckets); wider
 *   values as column slices whose dq, dk, dg, dbeta add up.
 * Arithmetic is f32 for bf16/f16/f32 inputs and f64 for f64 inputs; the state
 * scans and the gradient slabs multiply split-bf16 operands for f32 inputs and
 * single bf16 operands for bf16/f16 inputs.  The workspace
 * (kda_chunk_bwd_workspace_bytes for the same dtype, 16-byte aligned; 0 for an
 * unknown dtype) holds per-chunk intermediates and is fully rewritten.
 */
size_t kda_chunk_bwd_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim,
                                     int64_t value_dim, int dtype);

int kda_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const void* d_out, int dtype, const float* initial_state, const float* d_final_state,
                  void* dq, void* dk, void* dv, void* dg, void* dbeta, float* d_initial_state,
                  int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Directional derivative of the chunkwise backward, for second derivatives.
 * For f64 values x = (q, k, v, g, beta, initial_state), the output cotangent
 * d_out and the final-state cotangent d_final_state (NULL = zero), and
 * tangents tx of x (same shapes; each NULL = zero), writes
 *   t_d*     = d/de of kda_chunk_bwd's gradients (dq, dk, dv, dg, dbeta,
 *              d_initial_state) at x + e tx,
 *   t_out    = d/de of the output [B,T,H,V] at x + e tx,
 *   t_final  = d/de of the final state [B,H,K,V] at x + e tx
 * (every output pointer may be NULL).  The second derivatives are symmetric,
 * so with tx the cotangent of the gradients these are the double backward:
 * the cotangent of x is t_d*, that of d_out is t_out and that of
 * d_final_state is t_final.  f64 arithmetic (the f64 backward kernel on
 * value-and-derivative pairs), one workgroup per (sequence, head): for
 * second-order gradients and gradient checks, not for speed.  No reference
 * counterpart: the reference differentiates twice through autograd
 * (tests/kda/test_kda_recurrent.py:184-198).
 */
size_t kda_chunk_grad_tangent_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim,
                                              int64_t value_dim);
int kda_chunk_grad_tangent(const double* q, const double* k, const double* v, const double* g,
                           const double* beta, const double* initial_state, const double* d_out,
                           const double* d_final_state, const double* tq, const double* tk, const double* tv,
                           const double* tg, const double* tbeta, const double* t_initial_state, double* t_dq,
                           double* t_dk, double* t_dv, double* t_dg, double* t_dbeta,
                           double* t_d_initial_state, double* t_out, double* t_final_state, int64_t batch,
                           int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Fused stages around the operator.  Tensors are contiguous, of one dtype
 * (`dtype`: f32, f16, bf16 or f64); arithmetic is f32 (f64 for f64) with one
 * rounding to the output type.
 *
 * ShortConv + SiLU, and for q/k the per-head L2 normalisation, of one
 * projection: y = silu(causal_depthwise_conv(x)) [/ max(||y_head||_2, eps)].
 * Replaces, for one of q/k/v, KDAProjections._run_conv + F.silu (+ F.normalize)
 * (src/kda/projections.py:100-140,164-206) over CausalShortConv1D
 * (src/kimi_primitives/short_conv.py:69-98).
 *   x, y         : [batch, tokens, channels]
 *   weight       : [channels, kernel_size] in lag order (weight[c, j] multiplies x[t - j]); kernel_size <= 8
 *   bias         : [channels] or NULL
 *   history_in   : [batch, kernel_size - 1, channels] (the last inputs, oldest first) or NULL (zeros)
 *   history_out  : same shape or NULL; receives the last kernel_size - 1 rows of [history | valid prefix]
 *   valid_lens   : int32 [batch] right-padding lengths or NULL; padded outputs are zero and padding
 *                  never enters the history
 *   normalize    : nonzero for q/k; head_dim must then be a power of two in 16..512
 * channels must be a multiple of 16 bytes' worth of elements; x, y and the histories are
 * 16-byte aligned.  Each HBM row is read once and written once (one wave per 8-token tile).
 */
int kda_conv_silu_fwd(const void* x, const void* weight, const void* bias, const void* history_in,
                      void* y, void* history_out, const int32_t* valid_lens, int64_t batch,
                      int64_t tokens, int64_t channels, int64_t kernel_size, int64_t head_dim,
                      int normalize, double eps, int dtype, void* stream);

/*
 * The lower-bounded decay g = g_min * clamp(sigmoid(exp(a_log[h]) * (z + decay_bias)), eps, 1 - eps),
 * alpha = exp(g), and the beta gate clamp(sigmoid(beta_logits), eps, 1 - eps), with eps the
 * machine epsilon of `dtype`.  Replaces LowerBoundedDecay.forward (src/kda/decay.py:30-43) with
 * the decay-logit bias and the beta gate of KDAProjections.forward (src/kda/projections.py:207-218).
 *   decay_logits, g, alpha : [rows, heads, key_dim], 16-byte aligned (alpha may be NULL); or all NULL;
 *                            key_dim a multiple of 16 bytes' worth of elements
 *   decay_bias             : [heads, key_dim], 16-byte aligned, or NULL;  a_log : f32 [heads]
 *   beta_logits, beta      : [rows, heads] or NULL
 */
int kda_gates_fwd(const void* decay_logits, const void* decay_bias, const float* a_log, double g_min,
                  void* g, void* alpha, const void* beta_logits, void* beta, int64_t rows,
                  int64_t heads, int64_t key_dim, int dtype, void* stream);

/*
 * Head-wise RMSNorm x * rsqrt(mean(x^2) + eps) * weight, times sigmoid(gate_logits) when given:
 * the input of the output projection.  Replaces HeadwiseRMSNorm.forward
 * (src/kimi_primitives/headwise_rmsnorm.py:39-64) followed by the gate product of
 * FullRankOutputGate.forward (src/kimi_primitives/output_gate.py:62-75).
 *   x, y        : [rows, heads, head_dim], head_dim a power of two in 16..512
 *   weight      : [heads, head_dim] (weight_per_head != 0), [head_dim], or NULL
 *   gate_logits : [rows, heads * head_dim] (pre-sigmoid) or NULL
 * All pointers 16-byte aligned.
 */
int kda_rmsnorm_gate_fwd(const void* x, const void* weight, int weight_per_head,
                         const void* gate_logits, void* y, int64_t rows, int64_t heads,
                         int64_t head_dim, double eps, int dtype, void* stream);


/*
 * Backward of the fused stages: the gradients the reference takes from
 * autograd through KDAProjections.forward (src/kda/projections.py:164-218),
 * LowerBoundedDecay.forward (src/kda/decay.py:36-43), HeadwiseRMSNorm.forward
 * (src/kimi_primitives/headwise_rmsnorm.py:39-64) and the gate product of
 * FullRankOutputGate.forward (src/kimi_primitives/output_gate.py:62-75).
 * Arguments mirror the forward entry points; every forward intermediate is
 * recomputed from the inputs.  Activation gradients have the tensors' dtype.
 * Parameter gradients (d_weight, d_bias, d_decay_bias, d_a_log) are
 * ACCUMULATORS in the compute type (f64 for f64 tensors, f32 otherwise) that
 * the caller zeroes first; each may be NULL to skip it.  They are summed with
 * float atomics, so their rounding varies from run to run.
 *
 * kda_conv_silu_bwd: dy [batch, tokens, channels] (the gradient of y) and
 *   d_history_out (the gradient of the returned history, or NULL) give dx,
 *   d_history_in (or NULL), d_weight [channels, kernel_size], d_bias [channels].
 *   normalize: head_dim a power of two in 16..256 (16..128 for f64).
 */
int kda_conv_silu_bwd(const void* x, const void* weight, const void* bias, const void* history_in,
                      const int32_t* valid_lens, const void* dy, const void* d_history_out, void* dx,
                      void* d_history_in, void* d_weight, void* d_bias, int64_t batch, int64_t tokens,
                      int64_t channels, int64_t kernel_size, int64_t head_dim, int normalize, double eps,
                      int dtype, void* stream);

/*
 * kda_gates_bwd: d_g (and d_alpha or NULL) give d_decay_logits, d_decay_bias
 *   [heads, key_dim] and d_a_log [heads]; d_beta gives d_beta_logits.  The
 *   clamps pass gradient inside [eps, 1 - eps], as torch.clamp does.
 */
int kda_gates_bwd(const void* decay_logits, const void* decay_bias, const float* a_log, double g_min,
                  const void* d_g, const void* d_alpha, void* d_decay_logits, void* d_decay_bias,
                  void* d_a_log, const void* beta_logits, const void* d_beta, void* d_beta_logits,
                  int64_t rows, int64_t heads, int64_t key_dim, int dtype, void* stream);

/*
 * kda_rmsnorm_gate_bwd: dy [rows, heads, head_dim] gives dx, d_gate_logits and
 *   d_weight (shaped like weight).
 */
int kda_rmsnorm_gate_bwd(const void* x, const void* weight, int weight_per_head, const void* gate_logits,
                         const void* dy, void* dx, void* d_gate_logits, void* d_weight, int64_t rows,
                         int64_t heads, int64_t head_dim, double eps, int dtype, void* stream);

/*
 * Backward of the token recurrence that returns its per-token states: the
 * autograd of recurrent_kda(..., return_states_per_token=True)
 * (src/kda/recurrent.py:61-79), where every intermediate state may carry a gradient.
 *   q, k, g [batch, tokens, heads, key_dim]; v, d_out [batch, tokens, heads, value_dim];
 *   beta [batch, tokens, heads]: all of dtype f32 or f64 (the work type), masked already
 *   initial_state, d_final_state : [batch, heads, key_dim, value_dim] or NULL (zero)
 *   states, d_states             : the forward's per-token states [tokens, batch, heads,
 *                                  key_dim, value_dim] and their gradient (or NULL)
 *   dq, dk, dv, dg, dbeta        : outputs shaped like the inputs; d_initial_state or NULL
 * One workgroup per (batch, head), serial over the tokens: a debugging path.
 * Workspace: kda_recurrent_bwd_workspace_bytes(batch, heads, key_dim, value_dim, dtype).
 */
size_t kda_recurrent_bwd_workspace_bytes(int64_t batch, int64_t heads, int64_t key_dim, int64_t value_dim,
                                         int dtype);

int kda_recurrent_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                      const void* d_out, const void* initial_state, const void* states, const void* d_states,
                      const void* d_final_state, void* dq, void* dk, void* dv, void* dg, void* dbeta,
                      void* d_initial_state, int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim,
                      int64_t value_dim, int dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Cache plumbing for serving: out_t[i, ...] = src_t[index[i], ...] for every tensor t of a
 * decode cache, in one launch per 64 tensors.  Replaces the per-tensor index_select of
 * KDAState.reorder (src/kda/state.py:50-67) and ShortConvState, taken over every layer by
 * HybridLayerCache/HybridBackboneCache.reorder (src/hybrid_backbone/cache.py:58-61,118-126);
 * with index == NULL it is the copy of KDAState.clone (src/kda/state.py:41-48).
 *   src[t], dst[t] : device pointers to batch-major tensors of n_src and n_out rows of
 *                    row_bytes[t] bytes each (any dtype; 16-byte units when sizes and
 *                    addresses allow); an output may not overlap any source or other output
 *   index          : device int64 [n_out], each in [0, n_src), or NULL (n_out == n_src)
 *   status         : device int32, or NULL; set to 1 (never cleared here) when an index is
 *                    out of range, whose output row is then left unwritten
 * The host arrays src, dst and row_bytes are read before the call returns.
 */
int kda_cache_gather(const void* const* src, void* const* dst, const int64_t* row_bytes, int n_tensors,
                     const int64_t* index, int64_t n_src, int64_t n_out, int* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KDA_MI355X_H */
