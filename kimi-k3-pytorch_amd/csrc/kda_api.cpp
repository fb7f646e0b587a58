// extern "C" entry points of libkda_mi355x.so (declared in include/kda_mi355x.h).
// Argument checks happen here, before any launch, so a bad call returns
// KDA_ERR_INVALID_ARGUMENT instead of launching a kernel whose grid or
// indexing would not match the buffers.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <utility>

#include "kda_common.h"
#include "kda_launch.h"

namespace kda_host {

static thread_local char g_detail[512];
static thread_local char g_status[640];

void set_detail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_detail, sizeof(g_detail), fmt, ap);
  va_end(ap);
}

const char* detail() { return g_detail; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_detail("%s launch failed: %s", what, hipGetErrorString(e));
    return KDA_ERR_LAUNCH;
  }
  return KDA_OK;
}

bool reserve_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;  // (kernel, device ordinal)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kernel, dev}) != 0) return true;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) return false;
  done.insert({kernel, dev});
  return true;
}

static bool is_input_dtype(int d) {
  return d == KDA_DTYPE_F32 || d == KDA_DTYPE_F16 || d == KDA_DTYPE_BF16 || d == KDA_DTYPE_F64;
}

static int expected_state_dtype(int in_dtype) { return in_dtype == KDA_DTYPE_F64 ? KDA_DTYPE_F64 : KDA_DTYPE_F32; }

static int check_common(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                        int state_dtype, const void* out, int64_t num_seqs, int64_t total_tokens, int64_t heads,
                        int64_t key_dim, int64_t value_dim) {
  g_detail[0] = '\0';
  if (!is_input_dtype(in_dtype)) {
    set_detail("unknown input dtype %d", in_dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (state_dtype != expected_state_dtype(in_dtype)) {
    set_detail("state dtype %d does not match input dtype %d", state_dtype, in_dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (num_seqs <= 0 || total_tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("sizes must be positive (N=%lld tokens=%lld H=%lld K=%lld V=%lld)", (long long)num_seqs,
               (long long)total_tokens, (long long)heads, (long long)key_dim, (long long)value_dim);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!q || !k || !v || !g || !beta || !out) {
    set_detail("q, k, v, g, beta and out must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return KDA_OK;
}

static int check_seq(const int32_t* cu_seqlens, int64_t dense_span, int64_t num_seqs, int64_t total_tokens) {
  if (cu_seqlens == nullptr) {
    if (dense_span <= 0 || dense_span * num_seqs != total_tokens) {
      set_detail("dense layout needs dense_span * num_seqs == total_tokens (%lld * %lld != %lld)",
                 (long long)dense_span, (long long)num_seqs, (long long)total_tokens);
      return KDA_ERR_INVALID_ARGUMENT;
    }
  } else if (dense_span < 0 || dense_span > total_tokens) {
    // packed documents: dense_span is the longest document (0 when unknown)
    set_detail("packed documents take the longest document's length (0 if unknown) in dense_span, got %lld of %lld",
               (long long)dense_span, (long long)total_tokens);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (total_tokens > 0x7fffffffLL) {
    set_detail("total_tokens %lld exceeds int32 offsets", (long long)total_tokens);
    return KDA_ERR_UNSUPPORTED;
  }
  return KDA_OK;
}

}  // namespace kda_host

using namespace kda_host;

extern "C" {

int kda_abi_version(void) { return KDA_ABI_VERSION; }

int kda_set_segment_chunks(int64_t chunks_per_segment) {
  if (chunks_per_segment < -1) {
    kda_host::set_detail("chunks_per_segment must be -1 (the library's plan), 0 or positive, got %lld",
                         (long long)chunks_per_segment);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  kda_host::set_segment_override(chunks_per_segment);
  return KDA_OK;
}

const char* kda_status_string(int status) {
  const char* base = "unknown status";
  switch (status) {
    case KDA_OK: base = "ok"; break;
    case KDA_ERR_INVALID_ARGUMENT: base = "invalid argument"; break;
    case KDA_ERR_UNSUPPORTED: base = "unsupported configuration"; break;
    case KDA_ERR_WORKSPACE: base = "workspace too small"; break;
    case KDA_ERR_LAUNCH: base = "kernel launch failed"; break;
    default: break;
  }
  if (g_detail[0] != '\0')
    snprintf(g_status, sizeof(g_status), "%s: %s", base, g_detail);
  else
    snprintf(g_status, sizeof(g_status), "%s", base);
  return g_status;
}

int kda_recurrent_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                      const void* initial_state, void* final_state, int state_dtype, void* out,
                      void* states_per_token, const int32_t* cu_seqlens, int64_t dense_span,
                      const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens, int64_t heads,
                      int64_t key_dim, int64_t value_dim, void* stream) {
  int st = check_common(q, k, v, g, beta, in_dtype, state_dtype, out, num_seqs, total_tokens, heads, key_dim,
                        value_dim);
  if (st != KDA_OK) return st;
  st = check_seq(cu_seqlens, dense_span, num_seqs, total_tokens);
  if (st != KDA_OK) return st;
  if (states_per_token != nullptr && cu_seqlens != nullptr) {
    set_detail("states_per_token needs dense sequences (cu_seqlens == NULL)");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  kda::SeqDesc seq{cu_seqlens, dense_span, valid_lens};
  return launch_recurrent(q, k, v, g, beta, in_dtype, initial_state, final_state, state_dtype, out,
                          states_per_token, seq, num_seqs, heads, key_dim, value_dim,
                          static_cast<hipStream_t>(stream), false);
}

int kda_decode_step(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                    const void* state_in, void* state_out, int state_dtype, void* out, int64_t batch,
                    int64_t heads, int64_t key_dim, int64_t value_dim, void* stream) {
  int st = check_common(q, k, v, g, beta, in_dtype, state_dtype, out, batch, batch, heads, key_dim, value_dim);
  if (st != KDA_OK) return st;
  if (state_out == nullptr) {
    set_detail("decode step needs state_out");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  kda::SeqDesc seq{nullptr, 1, nullptr};
  return launch_recurrent(q, k, v, g, beta, in_dtype, state_in, state_out, state_dtype, out, nullptr, seq, batch,
                          heads, key_dim, value_dim, static_cast<hipStream_t>(stream), true);
}

size_t kda_chunk_fwd_workspace_bytes(int64_t num_seqs, int64_t total_tokens, int64_t longest_tokens, int64_t heads,
                                     int64_t key_dim, int64_t value_dim, int in_dtype) {
  if (longest_tokens < 0 || longest_tokens > total_tokens) return 0;
  return chunk_workspace_bytes(num_seqs, total_tokens, longest_tokens, heads, key_dim, value_dim, in_dtype);
}

int kda_chunk_fwd_plan(int64_t num_seqs, int64_t total_tokens, int64_t longest_tokens, int64_t heads,
                       int64_t key_dim, int64_t value_dim, int in_dtype, int64_t* chunks_per_segment,
                       int64_t* segments) {
  g_detail[0] = '\0';
  if (!chunks_per_segment || !segments) {
    set_detail("chunk_fwd_plan: output pointers must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!is_input_dtype(in_dtype) || num_seqs <= 0 || total_tokens <= 0 || heads <= 0 || key_dim <= 0 ||
      value_dim <= 0 || longest_tokens < 0 || longest_tokens > total_tokens) {
    set_detail("chunk_fwd_plan: bad sizes or dtype");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  chunk_plan(num_seqs, total_tokens, longest_tokens, heads, key_dim, value_dim, in_dtype, chunks_per_segment,
             segments);
  return KDA_OK;
}

int kda_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                  const void* initial_state, void* final_state, int state_dtype, void* out,
                  const int32_t* cu_seqlens, int64_t dense_span, const int32_t* valid_lens, int64_t num_seqs,
                  int64_t total_tokens, int64_t heads, int64_t key_dim, int64_t value_dim, void* workspace,
                  size_t workspace_bytes, void* stream) {
  int st = check_common(q, k, v, g, beta, in_dtype, state_dtype, out, num_seqs, total_tokens, heads, key_dim,
                        value_dim);
  if (st != KDA_OK) return st;
  st = check_seq(cu_seqlens, dense_span, num_seqs, total_tokens);
  if (st != KDA_OK) return st;
  kda::SeqDesc seq{cu_seqlens, dense_span, valid_lens};
  const size_t need = chunk_call_workspace_bytes(seq, num_seqs, total_tokens, heads, key_dim, value_dim, in_dtype,
                                                 state_dtype);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_detail("chunk_fwd needs %zu workspace bytes, got %zu", need, workspace_bytes);
    return KDA_ERR_WORKSPACE;
  }
  return launch_chunk(q, k, v, g, beta, in_dtype, initial_state, final_state, state_dtype, out, seq, num_seqs,
                      total_tokens, heads, key_dim, value_dim, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream));
}

int kda_chunk_fwd_decay(const void* q, const void* k, const void* v, const void* decay_logits, const void* decay_bias,
                        const float* a_log, double g_min, const void* beta, int in_dtype, const void* initial_state,
                        void* final_state, int state_dtype, void* out, const int32_t* cu_seqlens, int64_t dense_span,
                        const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens, int64_t heads,
                        int64_t key_dim, int64_t value_dim, void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_common(q, k, v, decay_logits, beta, in_dtype, state_dtype, out, num_seqs, total_tokens, heads,
                        key_dim, value_dim);
  if (st != KDA_OK) return st;
  st = check_seq(cu_seqlens, dense_span, num_seqs, total_tokens);
  if (st != KDA_OK) return st;
  if (a_log == nullptr) {
    set_detail("chunk_fwd_decay: a_log must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(g_min < 0.0)) {
    set_detail("chunk_fwd_decay: g_min must be negative");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  kda::SeqDesc seq{cu_seqlens, dense_span, valid_lens};
  int64_t per_segment = 0, segments = 0;  // off the MFMA path the launcher reports the shape unsupported
  const int64_t longest = cu_seqlens != nullptr ? dense_span : 0;
  chunk_plan(num_seqs, total_tokens, longest, heads, key_dim, value_dim, in_dtype, &per_segment, &segments);
  const size_t need = per_segment >= 0 ? chunk_workspace_bytes(num_seqs, total_tokens, longest, heads, key_dim,
                                                               value_dim, in_dtype)
                                       : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_detail("chunk_fwd_decay needs %zu workspace bytes, got %zu", need, workspace_bytes);
    return KDA_ERR_WORKSPACE;
  }
  return launch_chunk_decay(q, k, v, decay_logits, decay_bias, a_log, static_cast<float>(g_min), beta, in_dtype,
                            initial_state, final_state, state_dtype, out, seq, num_seqs, total_tokens, heads, key_dim,
                            value_dim, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int kda_chunk_fwd_profiled(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                           const void* initial_state, void* final_state, int state_dtype, void* out,
                           const int32_t* cu_seqlens, int64_t dense_span, const int32_t* valid_lens, int64_t num_seqs,
                           int64_t total_tokens, int64_t heads, int64_t key_dim, int64_t value_dim, void* workspace,
                           size_t workspace_bytes, void* stream, float* kernel_ms, int* num_kernels) {
  if (kernel_ms == nullptr || num_kernels == nullptr) {
    g_detail[0] = '\0';
    set_detail("kernel_ms and num_kernels must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  int st = check_common(q, k, v, g, beta, in_dtype, state_dtype, out, num_seqs, total_tokens, heads, key_dim,
                        value_dim);
  if (st != KDA_OK) return st;
  st = check_seq(cu_seqlens, dense_span, num_seqs, total_tokens);
  if (st != KDA_OK) return st;
  const size_t need = chunk_call_workspace_bytes(kda::SeqDesc{cu_seqlens, dense_span, valid_lens}, num_seqs,
                                                 total_tokens, heads, key_dim, value_dim, in_dtype, state_dtype);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_detail("chunk_fwd needs %zu workspace bytes, got %zu", need, workspace_bytes);
    return KDA_ERR_WORKSPACE;
  }
  KernelEvents ev;
  ev.n_launched = 0;
  ev.empty = 0;
  for (auto& e : ev.ev) {
    if (hipEventCreate(&e) != hipSuccess) {
      set_detail("hipEventCreate failed");
      return KDA_ERR_LAUNCH;
    }
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  kda::SeqDesc seq{cu_seqlens, dense_span, valid_lens};
  st = launch_chunk(q, k, v, g, beta, in_dtype, initial_state, final_state, state_dtype, out, seq, num_seqs,
                    total_tokens, heads, key_dim, value_dim, workspace, workspace_bytes, s, &ev);
  for (int i = 0; i < 4; ++i) kernel_ms[i] = 0.f;
  *num_kernels = 0;
  if (st == KDA_OK && hipStreamSynchronize(s) == hipSuccess) {
    *num_kernels = ev.n_launched;
    for (int i = 0; i < ev.n_launched && i < 4; ++i)
      if (!((ev.empty >> i) & 1u)) (void)hipEventElapsedTime(&kernel_ms[i], ev.ev[i], ev.ev[i + 1]);
  }
  for (auto& e : ev.ev) (void)hipEventDestroy(e);
  return st;
}

int kda_ut_transform(const void* k, const void* v, const void* g, const void* beta, int in_dtype, void* M, void* U,
                     void* W, void* log_gamma, void* k_gamma, int out_dtype, int64_t batch, int64_t count,
                     int64_t heads, int64_t key_dim, int64_t value_dim, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(in_dtype) || out_dtype != expected_state_dtype(in_dtype)) {
    set_detail("ut_transform: bad dtypes (in %d, out %d)", in_dtype, out_dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (batch <= 0 || count <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("ut_transform: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!k || !v || !g || !beta || !M || !U || !W || !log_gamma || !k_gamma) {
    set_detail("ut_transform: all pointers must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_ut_transform(k, v, g, beta, in_dtype, M, U, W, log_gamma, k_gamma, out_dtype, batch, count, heads,
                             key_dim, value_dim, static_cast<hipStream_t>(stream));
}

size_t kda_ut_transform_bwd_workspace_bytes(int64_t batch, int64_t count, int64_t heads, int64_t key_dim,
                                            int out_dtype) {
  if (batch <= 0 || count <= 0 || heads <= 0 || key_dim <= 0) return 0;
  return ut_transform_bwd_workspace_bytes(batch, count, heads, key_dim, out_dtype);
}

int kda_ut_transform_bwd(const void* k, const void* v, const void* g, const void* beta, int in_dtype, const void* dM,
                         const void* dU, const void* dW, const void* d_log_gamma, const void* d_k_gamma, void* dk,
                         void* dv, void* dg, void* dbeta, int out_dtype, int64_t batch, int64_t count, int64_t heads,
                         int64_t key_dim, int64_t value_dim, void* workspace, size_t workspace_bytes, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(in_dtype) || out_dtype != expected_state_dtype(in_dtype)) {
    set_detail("ut_transform_bwd: bad dtypes (in %d, out %d)", in_dtype, out_dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (batch <= 0 || count <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("ut_transform_bwd: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!k || !v || !g || !beta || !dk || !dv || !dg || !dbeta) {
    set_detail("ut_transform_bwd: inputs and gradients must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_ut_transform_bwd(k, v, g, beta, in_dtype, dM, dU, dW, d_log_gamma, d_k_gamma, dk, dv, dg, dbeta,
                                 out_dtype, batch, count, heads, key_dim, value_dim, workspace, workspace_bytes,
                                 static_cast<hipStream_t>(stream));
}

size_t kda_chunk_bwd_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim,
                                     int64_t value_dim, int dtype) {
  if (batch <= 0 || tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) return 0;
  if (dtype != KDA_DTYPE_BF16 && dtype != KDA_DTYPE_F16 && dtype != KDA_DTYPE_F32 && dtype != KDA_DTYPE_F64) return 0;
  return chunk_bwd_workspace_bytes(batch, tokens, heads, key_dim, value_dim, dtype);
}

int kda_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta, const void* d_out,
                  int in_dtype, const float* initial_state, const float* d_final_state, void* dq, void* dk, void* dv,
                  void* dg, void* dbeta, float* d_initial_state, int64_t batch, int64_t tokens, int64_t heads,
                  int64_t key_dim, int64_t value_dim, void* workspace, size_t workspace_bytes, void* stream) {
  g_detail[0] = '\0';
  if (in_dtype != KDA_DTYPE_BF16 && in_dtype != KDA_DTYPE_F16 && in_dtype != KDA_DTYPE_F32 &&
      in_dtype != KDA_DTYPE_F64) {
    set_detail("chunk_bwd: inputs must be bf16, f16, f32 or f64 (dtype %d)", in_dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (batch <= 0 || tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("chunk_bwd: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!q || !k || !v || !g || !beta || !d_out || !dq || !dk || !dv || !dg || !dbeta) {
    set_detail("chunk_bwd: inputs, d_out and the input gradients must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_chunk_bwd(q, k, v, g, beta, d_out, in_dtype, initial_state, d_final_state, dq, dk, dv, dg, dbeta,
                          d_initial_state, batch, tokens, heads, key_dim, value_dim, workspace, workspace_bytes,
                          static_cast<hipStream_t>(stream));
}

size_t kda_chunk_grad_tangent_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim,
                                              int64_t value_dim) {
  if (batch <= 0 || tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) return 0;
  return chunk_grad_tangent_workspace_bytes(batch, tokens, heads, key_dim, value_dim);
}

int kda_chunk_grad_tangent(const double* q, const double* k, const double* v, const double* g, const double* beta,
                           const double* initial_state, const double* d_out, const double* d_final_state,
                           const double* tq, const double* tk, const double* tv, const double* tg, const double* tbeta,
                           const double* t_initial_state, double* t_dq, double* t_dk, double* t_dv, double* t_dg,
                           double* t_dbeta, double* t_d_initial_state, double* t_out, double* t_final_state,
                           int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim, int64_t value_dim,
                           void* workspace, size_t workspace_bytes, void* stream) {
  g_detail[0] = '\0';
  if (batch <= 0 || tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("chunk_grad_tangent: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!q || !k || !v || !g || !beta || !d_out) {
    set_detail("chunk_grad_tangent: q, k, v, g, beta and d_out must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (t_d_initial_state && !initial_state) {
    set_detail("chunk_grad_tangent: the initial-state gradient needs an initial state");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  const size_t need = chunk_grad_tangent_workspace_bytes(batch, tokens, heads, key_dim, value_dim);
  if (workspace == nullptr || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    set_detail("chunk_grad_tangent needs %zu bytes of 16-byte aligned workspace, got %zu", need, workspace_bytes);
    return KDA_ERR_WORKSPACE;
  }
  const double* in[6] = {q, k, v, g, beta, initial_state};
  const double* tan[6] = {tq, tk, tv, tg, tbeta, initial_state ? t_initial_state : nullptr};
  double* tgrad[6] = {t_dq, t_dk, t_dv, t_dg, t_dbeta, t_d_initial_state};
  return launch_chunk_grad_tangent(in, tan, d_out, d_final_state, tgrad, t_out, t_final_state, batch, tokens, heads,
                                   key_dim, value_dim, workspace, static_cast<hipStream_t>(stream));
}

int kda_conv_silu_fwd(const void* x, const void* weight, const void* bias, const void* history_in, void* y,
                      void* history_out, const int32_t* valid_lens, int64_t batch, int64_t tokens, int64_t channels,
                      int64_t kernel_size, int64_t head_dim, int normalize, double eps, int dtype, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(dtype)) {
    set_detail("conv_silu: bad dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (batch <= 0 || tokens <= 0 || channels <= 0 || kernel_size <= 0 || (normalize && head_dim <= 0)) {
    set_detail("conv_silu: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (normalize && channels % head_dim != 0) {
    set_detail("conv_silu: channels %lld not a multiple of head_dim %lld", (long long)channels, (long long)head_dim);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!x || !weight || !y) {
    set_detail("conv_silu: x, weight and y must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(eps > 0.0)) {
    set_detail("conv_silu: eps must be > 0");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_conv_silu(x, weight, bias, history_in, y, history_out, valid_lens, batch, tokens, channels,
                          kernel_size, head_dim, normalize, eps, dtype, static_cast<hipStream_t>(stream));
}

int kda_gates_fwd(const void* decay_logits, const void* decay_bias, const float* a_log, double g_min, void* g,
                  void* alpha, const void* beta_logits, void* beta, int64_t rows, int64_t heads, int64_t key_dim,
                  int dtype, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(dtype)) {
    set_detail("gates: bad dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (rows <= 0 || heads <= 0 || key_dim <= 0) {
    set_detail("gates: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(g_min < 0.0)) {
    set_detail("gates: g_min must be negative");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!decay_logits && !beta_logits) {
    set_detail("gates: nothing to do (both logits null)");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_gates(decay_logits, decay_bias, a_log, g_min, g, alpha, beta_logits, beta, rows, heads, key_dim,
                      dtype, static_cast<hipStream_t>(stream));
}

int kda_rmsnorm_gate_fwd(const void* x, const void* weight, int weight_per_head, const void* gate_logits, void* y,
                         int64_t rows, int64_t heads, int64_t head_dim, double eps, int dtype, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(dtype)) {
    set_detail("rmsnorm_gate: bad dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (rows <= 0 || heads <= 0 || head_dim <= 0) {
    set_detail("rmsnorm_gate: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!x || !y) {
    set_detail("rmsnorm_gate: x and y must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(eps > 0.0)) {
    set_detail("rmsnorm_gate: eps must be > 0");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_rmsnorm_gate(x, weight, weight_per_head, gate_logits, y, rows, heads, head_dim, eps, dtype,
                             static_cast<hipStream_t>(stream));
}

int kda_conv_silu_bwd(const void* x, const void* weight, const void* bias, const void* history_in,
                      const int32_t* valid_lens, const void* dy, const void* d_history_out, void* dx,
                      void* d_history_in, void* d_weight, void* d_bias, int64_t batch, int64_t tokens,
                      int64_t channels, int64_t kernel_size, int64_t head_dim, int normalize, double eps, int dtype,
                      void* stream) {
  g_detail[0] = '\0';
  if (batch <= 0 || tokens <= 0 || channels <= 0 || kernel_size <= 0 || (normalize && head_dim <= 0)) {
    set_detail("conv_silu_bwd: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (normalize && channels % head_dim != 0) {
    set_detail("conv_silu_bwd: channels %lld not a multiple of head_dim %lld", (long long)channels,
               (long long)head_dim);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!x || !weight || !dy || !dx) {
    set_detail("conv_silu_bwd: x, weight, dy and dx must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(eps > 0.0)) {
    set_detail("conv_silu_bwd: eps must be > 0");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_conv_silu_bwd(x, weight, bias, history_in, valid_lens, dy, d_history_out, dx, d_history_in,
                              d_weight, d_bias, batch, tokens, channels, kernel_size, head_dim, normalize, eps, dtype,
                              static_cast<hipStream_t>(stream));
}

int kda_gates_bwd(const void* decay_logits, const void* decay_bias, const float* a_log, double g_min, const void* d_g,
                  const void* d_alpha, void* d_decay_logits, void* d_decay_bias, void* d_a_log,
                  const void* beta_logits, const void* d_beta, void* d_beta_logits, int64_t rows, int64_t heads,
                  int64_t key_dim, int dtype, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(dtype)) {
    set_detail("gates_bwd: bad dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (rows <= 0 || heads <= 0 || key_dim <= 0) {
    set_detail("gates_bwd: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(g_min < 0.0)) {
    set_detail("gates_bwd: g_min must be negative");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!decay_logits && !beta_logits) {
    set_detail("gates_bwd: nothing to do (both logits null)");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_gates_bwd(decay_logits, decay_bias, a_log, g_min, d_g, d_alpha, d_decay_logits, d_decay_bias, d_a_log,
                          beta_logits, d_beta, d_beta_logits, rows, heads, key_dim, dtype,
                          static_cast<hipStream_t>(stream));
}

int kda_rmsnorm_gate_bwd(const void* x, const void* weight, int weight_per_head, const void* gate_logits,
                         const void* dy, void* dx, void* d_gate_logits, void* d_weight, int64_t rows, int64_t heads,
                         int64_t head_dim, double eps, int dtype, void* stream) {
  g_detail[0] = '\0';
  if (!is_input_dtype(dtype)) {
    set_detail("rmsnorm_gate_bwd: bad dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (rows <= 0 || heads <= 0 || head_dim <= 0) {
    set_detail("rmsnorm_gate_bwd: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!x || !dy || !dx || (gate_logits && !d_gate_logits)) {
    set_detail("rmsnorm_gate_bwd: x, dy, dx (and d_gate_logits with gate_logits) must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!(eps > 0.0)) {
    set_detail("rmsnorm_gate_bwd: eps must be > 0");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_rmsnorm_gate_bwd(x, weight, weight_per_head, gate_logits, dy, dx, d_gate_logits, weight ? d_weight : nullptr,
                                 rows, heads, head_dim, eps, dtype, static_cast<hipStream_t>(stream));
}

int kda_cache_gather(const void* const* src, void* const* dst, const int64_t* row_bytes, int n_tensors,
                     const int64_t* index, int64_t n_src, int64_t n_out, int* status, void* stream) {
  g_detail[0] = '\0';
  return launch_cache_gather(src, dst, row_bytes, n_tensors, index, n_src, n_out, status,
                             static_cast<hipStream_t>(stream));
}

size_t kda_recurrent_bwd_workspace_bytes(int64_t batch, int64_t heads, int64_t key_dim, int64_t value_dim,
                                         int dtype) {
  if (batch <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) return 0;
  return recurrent_bwd_workspace_bytes(batch, heads, key_dim, value_dim, dtype);
}

int kda_recurrent_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                      const void* d_out, const void* initial_state, const void* states, const void* d_states,
                      const void* d_final_state, void* dq, void* dk, void* dv, void* dg, void* dbeta,
                      void* d_initial_state, int64_t batch, int64_t tokens, int64_t heads, int64_t key_dim,
                      int64_t value_dim, int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  g_detail[0] = '\0';
  if (batch <= 0 || tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("recurrent_bwd: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!q || !k || !v || !g || !beta || !d_out || !states || !dq || !dk || !dv || !dg || !dbeta) {
    set_detail("recurrent_bwd: inputs, d_out, the states and the input gradients must be non-null");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  return launch_recurrent_bwd(q, k, v, g, beta, d_out, initial_state, states, d_states, d_final_state, dq, dk, dv, dg,
                              dbeta, d_initial_state, batch, tokens, heads, key_dim, value_dim, dtype, workspace,
                              workspace_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
