// Host-side launchers shared between the kernels' translation units and the
// C-ABI glue in kda_api.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "kda_common.h"

namespace kda_host {

int launch_recurrent(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                     const void* s_in, void* s_out, int state_dtype, void* out, void* s_hist,
                     const kda::SeqDesc& seq, int64_t N, int64_t H, int64_t K, int64_t V, hipStream_t stream,
                     bool streaming_state);

// `longest`: the longest packed document in tokens (0 for dense sequences or
// when unknown), the scheduling hint of make_plan.
size_t chunk_workspace_bytes(int64_t num_seqs, int64_t total_tokens, int64_t longest, int64_t heads,
                             int64_t key_dim, int64_t value_dim, int in_dtype);

// The schedule launch_chunk picks: chunks per segment (0: one segment per
// sequence; -1: the exact recurrence kernel) and the bound on segments.
void chunk_plan(int64_t num_seqs, int64_t total_tokens, int64_t longest, int64_t heads, int64_t key_dim,
                int64_t value_dim, int in_dtype, int64_t* chunks_per_segment, int64_t* segments);

// Optional per-kernel timing: events[i] is recorded before kernel i and
// events[n] after the last one; *n_launched receives n.  Bit i of `empty`
// marks a slot whose kernel the call does not need (its time reads zero).
struct KernelEvents {
  hipEvent_t ev[5];
  int n_launched;
  unsigned empty;
};

// The workspace one launch_chunk call needs: the MFMA path's maps and
// segment records, the split-bf16 chunk path's per-chunk records, or none
// (recurrence kernel).
size_t chunk_call_workspace_bytes(const kda::SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H, int64_t K,
                                  int64_t V, int in_dtype, int state_dtype);

int launch_chunk(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                 const void* s_in, void* s_out, int state_dtype, void* out, const kda::SeqDesc& seq, int64_t N,
                 int64_t total_tokens, int64_t H, int64_t K, int64_t V, void* workspace, size_t workspace_bytes,
                 hipStream_t stream, KernelEvents* events = nullptr);

// The prefill with g formed inside the chunk kernel from decay logits
// (lower-bounded decay of the logits plus bias); MFMA shapes only.
int launch_chunk_decay(const void* q, const void* k, const void* v, const void* z, const void* zbias,
                       const float* a_log, float g_min, const void* beta, int in_dtype, const void* s_in, void* s_out,
                       int state_dtype, void* out, const kda::SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H,
                       int64_t K, int64_t V, void* workspace, size_t workspace_bytes, hipStream_t stream);

int launch_ut_transform(const void* k, const void* v, const void* g, const void* beta, int in_dtype, void* M,
                        void* U, void* W, void* log_gamma, void* k_gamma, int out_dtype, int64_t batch,
                        int64_t count, int64_t heads, int64_t key_dim, int64_t value_dim, hipStream_t stream);

// Backward of the public UT transform (csrc/kda_ut_transform.hip).
size_t ut_transform_bwd_workspace_bytes(int64_t batch, int64_t count, int64_t heads, int64_t key_dim, int out_dtype);

int launch_ut_transform_bwd(const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                            const void* dM, const void* dU, const void* dW, const void* dlg, const void* dkg,
                            void* dk, void* dv, void* dg, void* dbeta, int out_dtype, int64_t batch, int64_t count,
                            int64_t heads, int64_t key_dim, int64_t value_dim, void* ws, size_t ws_bytes,
                            hipStream_t stream);

// Backward of the chunkwise operator (csrc/kda_chunk_bwd.hip).
size_t chunk_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int in_dtype);

int launch_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                     const void* dout, int in_dtype, const float* s0, const float* dsT, void* dq, void* dk, void* dv,
                     void* dg, void* dbeta, float* ds0, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

// The chunkwise forward through the backward's chunk operands (prep, forward
// scan, output kernel; csrc/kda_chunk_bwd.hip): dense sequences with optional
// right padding, f32 state, K and V up to 128.
bool chunk_split_path(int in_dtype, int state_dtype, int64_t K, int64_t V);

size_t chunk_split_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int in_dtype);

int launch_chunk_split(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                       const float* s_in, float* s_out, void* out, const int32_t* valid_lens, int64_t B, int64_t T,
                       int64_t H, int64_t K, int64_t V, void* workspace, size_t workspace_bytes, hipStream_t stream);

// The same path for packed documents (gathered into a zero-padded dense batch
// of T = the longest document's tokens, outputs scattered back) and for any
// value width (slices of at most 128 columns): K up to 128, f32 state.
bool chunk_split_general(int in_dtype, int state_dtype, int64_t K, int64_t V);

size_t chunk_split_general_workspace_bytes(int64_t N, int64_t T, int64_t H, int64_t K, int64_t V, int in_dtype,
                                           bool packed);

int launch_chunk_split_general(const void* q, const void* k, const void* v, const void* g, const void* beta,
                               int in_dtype, const float* s_in, float* s_out, void* out, const int32_t* cu_seqlens,
                               const int32_t* valid_lens, int64_t N, int64_t T, int64_t total_tokens, int64_t H,
                               int64_t K, int64_t V, void* workspace, size_t workspace_bytes, hipStream_t stream);

// The same backward in f64 arithmetic (csrc/kda_chunk_bwd_f64.hip).
size_t chunk_bwd_f64_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V);

int launch_chunk_bwd_f64(const double* q, const double* k, const double* v, const double* g, const double* beta,
                         const double* dout, const double* s0, const double* dsT, double* dq, double* dk, double* dv,
                         double* dg, double* dbeta, double* ds0, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                         double* ws, hipStream_t stream);

// Directional derivative of the chunk backward, of the output and of the
// final state along tangents of the inputs (f64 arithmetic; the f64 kernel on
// dual numbers, csrc/kda_chunk_bwd_f64.hip).  in / tan: q, k, v, g, beta,
// s0 (tangent entries may be null); tgrad: dq, dk, dv, dg, dbeta, ds0
// tangents (entries may be null).
size_t chunk_grad_tangent_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V);

int launch_chunk_grad_tangent(const double* const* in, const double* const* tan, const double* dout,
                              const double* dsT, double* const* tgrad, double* tout, double* tsT, int64_t B, int64_t T,
                              int64_t H, int64_t K, int64_t V, void* ws, hipStream_t stream);

// Backward of the token recurrence with per-token states (csrc/kda_recurrent_bwd.hip).
size_t recurrent_bwd_workspace_bytes(int64_t B, int64_t H, int64_t K, int64_t V, int dtype);

int launch_recurrent_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const void* dout, const void* s0, const void* hist, const void* dhist, const void* dsT,
                         void* dq, void* dk, void* dv, void* dg, void* dbeta, void* ds0, int64_t B, int64_t T,
                         int64_t H, int64_t K, int64_t V, int dtype, void* ws, size_t ws_bytes, hipStream_t stream);

// Fused stages around the operator (csrc/kda_fused.hip).
int launch_conv_silu(const void* x, const void* w, const void* bias, const void* hist_in, void* y, void* hist_out,
                     const int32_t* valid_lens, int64_t B, int64_t T, int64_t C, int64_t K, int64_t head_dim,
                     int normalize, double eps, int dtype, hipStream_t stream);

int launch_gates(const void* z, const void* zbias, const float* a_log, double g_min, void* g, void* alpha,
                 const void* bl, void* beta, int64_t rows, int64_t H, int64_t K, int dtype, hipStream_t stream);

int launch_rmsnorm_gate(const void* x, const void* w, int w_per_head, const void* gl, void* y, int64_t rows,
                        int64_t H, int64_t D, double eps, int dtype, hipStream_t stream);

// Backward of the fused stages (csrc/kda_fused_bwd.hip).  Parameter-gradient
// buffers are accumulators in the compute type (f64 for f64 tensors, f32
// otherwise), zeroed by the caller.
int launch_conv_silu_bwd(const void* x, const void* w, const void* bias, const void* hist_in,
                         const int32_t* valid_lens, const void* dy, const void* dhist_out, void* dx, void* dhist_in,
                         void* dw, void* dbias, int64_t B, int64_t T, int64_t C, int64_t K, int64_t head_dim,
                         int normalize, double eps, int dtype, hipStream_t stream);

int launch_gates_bwd(const void* z, const void* zbias, const float* a_log, double g_min, const void* dg,
                     const void* dalpha, void* dz, void* dzbias, void* da_log, const void* bl, const void* dbeta,
                     void* dbl, int64_t rows, int64_t H, int64_t K, int dtype, hipStream_t stream);

int launch_rmsnorm_gate_bwd(const void* x, const void* w, int w_per_head, const void* gl, const void* dy, void* dx,
                            void* dgl, void* dw, int64_t rows, int64_t H, int64_t D, double eps, int dtype,
                            hipStream_t stream);

// Batch-row gather over many cache tensors (csrc/kda_cache.hip).
int launch_cache_gather(const void* const* src, void* const* dst, const int64_t* row_bytes, int n_tensors,
                        const int64_t* index, int64_t n_src, int64_t n_out, int* status, hipStream_t stream);

}  // namespace kda_host
