// Stand-alone UT transform of independent chunks (API parity for
// `ut_transform`, src/kda/ut_transform.py:61-92).  Not on the prefill hot
// path — the chunked prefill computes the same quantities inside its own
// kernels — so this is a plain VALU kernel, one workgroup per (batch, head):
//   log_gamma = cumsum_t g                       (ut_transform.py:38)
//   A_ij = sum_c k_i k_j exp(lg_i - lg_j), j < i (ut_transform.py:39-46, exact pairwise exponent)
//   M = (I + diag(beta) A)^{-1} diag(beta)       (ut_transform.py:47-52, forward substitution)
//   k_gamma = exp(log_gamma) * k ; W = M k_gamma ; U = M v   (ut_transform.py:53-55)
#include "kda_launch.h"

namespace kda {

constexpr int kUtThreads = 256;
constexpr int kUtMaxCount = 1024;

template <class IT, class ST>
__global__ __launch_bounds__(kUtThreads) void ut_transform_kernel(const IT* __restrict__ k, const IT* __restrict__ v,
                                                                  const IT* __restrict__ g,
                                                                  const IT* __restrict__ beta, ST* __restrict__ M,
                                                                  ST* __restrict__ U, ST* __restrict__ W,
                                                                  ST* __restrict__ lg, ST* __restrict__ kg,
                                                                  int64_t C, int64_t H, int64_t K, int64_t V) {
  __shared__ ST arow[kUtMaxCount];
  const int64_t b = blockIdx.x / H;
  const int64_t h = blockIdx.x % H;
  const int tid = threadIdx.x;
  // [B,C,H,*] row index of token t
  auto rowk = [&](int64_t t) { return ((b * C + t) * H + h) * K; };
  auto rowv = [&](int64_t t) { return ((b * C + t) * H + h) * V; };
  ST* Mb = M + (b * H + h) * C * C;

  // 1. inclusive cumsum of g per key channel, k_gamma
  for (int64_t c = tid; c < K; c += kUtThreads) {
    ST run = ST(0);
    for (int64_t t = 0; t < C; ++t) {
      run += to_compute<ST>(g[rowk(t) + c]);
      lg[rowk(t) + c] = run;
      kg[rowk(t) + c] = fast_exp(run) * to_compute<ST>(k[rowk(t) + c]);
    }
  }
  __syncthreads();
  // 2. strictly lower decayed k k^T into M's storage; zeros elsewhere
  for (int64_t p = tid; p < C * C; p += kUtThreads) {
    const int64_t i = p / C, j = p % C;
    ST acc = ST(0);
    if (j < i) {
      for (int64_t c = 0; c < K; ++c) {
        acc += to_compute<ST>(k[rowk(i) + c]) * to_compute<ST>(k[rowk(j) + c]) *
               fast_exp(lg[rowk(i) + c] - lg[rowk(j) + c]);
      }
    }
    Mb[i * C + j] = acc;
  }
  __syncthreads();
  // 3. forward substitution, row by row: M_i = beta_i (e_i - sum_{j<i} A_ij M_j)
  for (int64_t i = 0; i < C; ++i) {
    for (int64_t j = tid; j < i; j += kUtThreads) arow[j] = Mb[i * C + j];
    __syncthreads();
    const ST bi = to_compute<ST>(beta[(b * C + i) * H + h]);
    for (int64_t c = tid; c <= i; c += kUtThreads) {
      ST acc = (c == i) ? ST(1) : ST(0);
      for (int64_t j = c; j < i; ++j) acc -= arow[j] * Mb[j * C + c];
      Mb[i * C + c] = bi * acc;
    }
    __syncthreads();
  }
  // 4. W = M k_gamma, U = M v
  for (int64_t p = tid; p < C * K; p += kUtThreads) {
    const int64_t i = p / K, c = p % K;
    ST acc = ST(0);
    for (int64_t j = 0; j <= i; ++j) acc += Mb[i * C + j] * kg[rowk(j) + c];
    W[rowk(i) + c] = acc;
  }
  for (int64_t p = tid; p < C * V; p += kUtThreads) {
    const int64_t i = p / V, c = p % V;
    ST acc = ST(0);
    for (int64_t j = 0; j <= i; ++j) acc += Mb[i * C + j] * to_compute<ST>(v[rowv(j) + c]);
    U[rowv(i) + c] = acc;
  }
}

template <class IT, class ST>
static int run_ut(const void* k, const void* v, const void* g, const void* beta, void* M, void* U, void* W, void* lg,
                  void* kg, int64_t B, int64_t C, int64_t H, int64_t K, int64_t V, hipStream_t stream) {
  hipLaunchKernelGGL((ut_transform_kernel<IT, ST>), dim3(static_cast<unsigned>(B * H)), dim3(kUtThreads), 0, stream,
                     static_cast<const IT*>(k), static_cast<const IT*>(v), static_cast<const IT*>(g),
                     static_cast<const IT*>(beta), static_cast<ST*>(M), static_cast<ST*>(U), static_cast<ST*>(W),
                     static_cast<ST*>(lg), static_cast<ST*>(kg), C, H, K, V);
  return kda_host::check_launch("ut_transform_kernel");
}

// ---- backward -----------------------------------------------------------------
// The gradients of (M, U, W, log_gamma, k_gamma) with respect to (k, v, g,
// beta), as autograd takes them through src/kda/ut_transform.py:23-58.  With
// L = I + diag(beta) A (unit lower) and M = L^{-1} diag(beta):
//   dv = M^T dU;  dM' = dM + dU v^T + dW kg^T (its lower part: M is lower);
//   G = L^{-T} dM' (back substitution);  dbeta_i = G_ii + sum_{j<i} dL_ij A_ij,
//   dL = -strict_lower(G M^T),  dA = diag(beta) dL;
//   dkg = dk_gamma + M^T dW;  dk = exp(lg) dkg + the pair terms of dA,
//   dlg = dlog_gamma + kg dkg + the pair terms of dA;  dg = reverse cumsum of dlg.
// One workgroup per (batch, head), plain loops; A, M, dM' and G live in the
// caller's workspace (4 C^2 values per (batch, head)), lg in the k-gradient
// output until the end.
template <class IT, class ST>
__global__ __launch_bounds__(kUtThreads) void ut_transform_bwd_kernel(
    const IT* __restrict__ k, const IT* __restrict__ v, const IT* __restrict__ g, const IT* __restrict__ beta,
    const ST* __restrict__ dM, const ST* __restrict__ dU, const ST* __restrict__ dW, const ST* __restrict__ dlg,
    const ST* __restrict__ dkg, ST* __restrict__ dk, ST* __restrict__ dv, ST* __restrict__ dg, ST* __restrict__ dbeta,
    ST* __restrict__ ws, int64_t C, int64_t H, int64_t K, int64_t V) {
  __shared__ ST col[kUtMaxCount];
  const int64_t b = blockIdx.x / H;
  const int64_t h = blockIdx.x % H;
  const int tid = threadIdx.x;
  auto rowk = [&](int64_t t) { return ((b * C + t) * H + h) * K; };
  auto rowv = [&](int64_t t) { return ((b * C + t) * H + h) * V; };
  auto bet = [&](int64_t t) { return to_compute<ST>(beta[(b * C + t) * H + h]); };
  // per (batch, head): A, M, D (C^2 each), then G (C^2, later C * K values of dlg)
  const int64_t per = 4 * C * C > C * K + 3 * C * C ? 4 * C * C : C * K + 3 * C * C;
  ST* A = ws + blockIdx.x * per;
  ST* M = A + C * C;
  ST* D = M + C * C;  // dM', then dL
  ST* G = D + C * C;
  ST* lg = dg;        // log_gamma kept in dg's rows until the reverse cumsum

  // forward quantities: lg, A (strict lower), M by forward substitution
  for (int64_t c = tid; c < K; c += kUtThreads) {
    ST run = ST(0);
    for (int64_t t = 0; t < C; ++t) {
      run += to_compute<ST>(g[rowk(t) + c]);
      lg[rowk(t) + c] = run;
    }
  }
  __syncthreads();
  for (int64_t p = tid; p < C * C; p += kUtThreads) {
    const int64_t i = p / C, j = p % C;
    ST acc = ST(0);
    if (j < i)
      for (int64_t c = 0; c < K; ++c)
        acc += to_compute<ST>(k[rowk(i) + c]) * to_compute<ST>(k[rowk(j) + c]) * fast_exp(lg[rowk(i) + c] - lg[rowk(j) + c]);
    A[p] = acc;
    M[p] = ST(0);
  }
  __syncthreads();
  // M_i = beta_i (e_i - sum_{j<i} A_ij M_j), row by row (the forward kernel's substitution)
  for (int64_t i = 0; i < C; ++i) {
    const ST bi = bet(i);
    for (int64_t c = tid; c <= i; c += kUtThreads) {
      ST acc = (c == i) ? ST(1) : ST(0);
      for (int64_t j = c; j < i; ++j) acc -= A[i * C + j] * M[j * C + c];
      M[i * C + c] = bi * acc;
    }
    __syncthreads();
  }
  // dv = M^T dU
  for (int64_t p = tid; p < C * V; p += kUtThreads) {
    const int64_t j = p / V, c = p % V;
    ST acc = ST(0);
    if (dU != nullptr)
      for (int64_t i = j; i < C; ++i) acc += M[i * C + j] * dU[rowv(i) + c];
    dv[rowv(j) + c] = acc;
  }
  // dM' = dM + dU v^T + dW kg^T on the lower triangle (kg = exp(lg) k)
  for (int64_t p = tid; p < C * C; p += kUtThreads) {
    const int64_t i = p / C, j = p % C;
    ST acc = ST(0);
    if (j <= i) {
      if (dM != nullptr) acc = dM[(blockIdx.x * C + i) * C + j];
      if (dU != nullptr)
        for (int64_t c = 0; c < V; ++c) acc += dU[rowv(i) + c] * to_compute<ST>(v[rowv(j) + c]);
      if (dW != nullptr)
        for (int64_t c = 0; c < K; ++c)
          acc += dW[rowk(i) + c] * fast_exp(lg[rowk(j) + c]) * to_compute<ST>(k[rowk(j) + c]);
    }
    D[p] = acc;
  }
  __syncthreads();
  // G = L^{-T} dM': rows from the last, G_i = dM'_i - sum_{r>i} beta_r A_ri G_r
  for (int64_t i = C - 1; i >= 0; --i) {
    for (int64_t r = tid; r < C; r += kUtThreads) col[r] = r > i ? bet(r) * A[r * C + i] : ST(0);
    __syncthreads();
    for (int64_t c = tid; c < C; c += kUtThreads) {
      ST acc = D[i * C + c];
      for (int64_t r = i + 1; r < C; ++r) acc -= col[r] * G[r * C + c];
      G[i * C + c] = acc;
    }
    __syncthreads();
  }
  // dL = -strict_lower(G M^T) into D; dbeta
  for (int64_t p = tid; p < C * C; p += kUtThreads) {
    const int64_t i = p / C, j = p % C;
    ST acc = ST(0);
    if (j < i)
      for (int64_t s = 0; s <= j; ++s) acc -= G[i * C + s] * M[j * C + s];
    D[p] = acc;
  }
  __syncthreads();
  for (int64_t i = tid; i < C; i += kUtThreads) {
    ST acc = G[i * C + i];
    for (int64_t j = 0; j < i; ++j) acc += D[i * C + j] * A[i * C + j];
    dbeta[(b * C + i) * H + h] = acc;
  }
  __syncthreads();  // G's diagonal is read above; its region is overwritten below
  // dk, dlg per (token, channel): the k_gamma path and the pair terms of dA = diag(beta) dL
  for (int64_t p = tid; p < C * K; p += kUtThreads) {
    const int64_t i = p / K, c = p % K;
    const ST ki = to_compute<ST>(k[rowk(i) + c]);
    const ST li = lg[rowk(i) + c];
    ST dkgi = dkg != nullptr ? dkg[rowk(i) + c] : ST(0);
    if (dW != nullptr)
      for (int64_t r = i; r < C; ++r) dkgi += M[r * C + i] * dW[rowk(r) + c];
    const ST ei = fast_exp(li);
    ST dki = ei * dkgi;
    ST dli = ei * ki * dkgi;
    for (int64_t j = 0; j < i; ++j) {  // A_ij with i as the row
      const ST dA = bet(i) * D[i * C + j];
      const ST kj = to_compute<ST>(k[rowk(j) + c]);
      const ST e = fast_exp(li - lg[rowk(j) + c]);
      dki += dA * kj * e;
      dli += dA * ki * kj * e;
    }
    for (int64_t j = i + 1; j < C; ++j) {  // A_ji with i as the column
      const ST dA = bet(j) * D[j * C + i];
      const ST kj = to_compute<ST>(k[rowk(j) + c]);
      const ST e = fast_exp(lg[rowk(j) + c] - li);
      dki += dA * kj * e;
      dli -= dA * ki * kj * e;
    }
    dk[rowk(i) + c] = dki;
    G[i * K + c] = dli;  // G is read by nobody now: dlg goes there (the region holds C * K values)
  }
  __syncthreads();
  // dg = reverse cumulative sum of dlg
  for (int64_t c = tid; c < K; c += kUtThreads) {
    ST run = ST(0);
    for (int64_t t = C - 1; t >= 0; --t) {
      run += G[t * K + c] + (dlg != nullptr ? dlg[rowk(t) + c] : ST(0));
      dg[rowk(t) + c] = run;
    }
  }
}

template <class IT, class ST>
static int run_ut_bwd(const void* k, const void* v, const void* g, const void* beta, const void* dM, const void* dU,
                      const void* dW, const void* dlg, const void* dkg, void* dk, void* dv, void* dg, void* dbeta,
                      void* ws, int64_t B, int64_t C, int64_t H, int64_t K, int64_t V, hipStream_t stream) {
  hipLaunchKernelGGL((ut_transform_bwd_kernel<IT, ST>), dim3(static_cast<unsigned>(B * H)), dim3(kUtThreads), 0,
                     stream, static_cast<const IT*>(k), static_cast<const IT*>(v), static_cast<const IT*>(g),
                     static_cast<const IT*>(beta), static_cast<const ST*>(dM), static_cast<const ST*>(dU),
                     static_cast<const ST*>(dW), static_cast<const ST*>(dlg), static_cast<const ST*>(dkg),
                     static_cast<ST*>(dk), static_cast<ST*>(dv), static_cast<ST*>(dg), static_cast<ST*>(dbeta),
                     static_cast<ST*>(ws), C, H, K, V);
  return kda_host::check_launch("ut_transform_bwd_kernel");
}

}  // namespace kda

namespace kda_host {

size_t ut_transform_bwd_workspace_bytes(int64_t batch, int64_t count, int64_t heads, int64_t key_dim, int out_dtype) {
  const int64_t per = 4 * count * count > count * key_dim + 3 * count * count ? 4 * count * count
                                                                             : count * key_dim + 3 * count * count;
  return static_cast<size_t>(batch * heads * per) * (out_dtype == KDA_DTYPE_F64 ? 8 : 4);
}

int launch_ut_transform_bwd(const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                            const void* dM, const void* dU, const void* dW, const void* dlg, const void* dkg,
                            void* dk, void* dv, void* dg, void* dbeta, int out_dtype, int64_t batch, int64_t count,
                            int64_t heads, int64_t key_dim, int64_t value_dim, void* ws, size_t ws_bytes,
                            hipStream_t stream) {
  using namespace kda;
  if (count > kUtMaxCount) {
    set_detail("ut_transform_bwd: chunk length %lld > %d is not supported", (long long)count, kUtMaxCount);
    return KDA_ERR_UNSUPPORTED;
  }
  if (batch * heads > 0x7fffffffLL) {
    set_detail("ut_transform_bwd: too many (batch, head) pairs");
    return KDA_ERR_UNSUPPORTED;
  }
  if (ws == nullptr || ws_bytes < ut_transform_bwd_workspace_bytes(batch, count, heads, key_dim, out_dtype)) {
    set_detail("ut_transform_bwd: workspace too small");
    return KDA_ERR_WORKSPACE;
  }
  switch (in_dtype) {
#define KDA_UT_BWD(IT, ST)                                                                                          \
  return run_ut_bwd<IT, ST>(k, v, g, beta, dM, dU, dW, dlg, dkg, dk, dv, dg, dbeta, ws, batch, count, heads, key_dim, \
                            value_dim, stream)
    case KDA_DTYPE_BF16: KDA_UT_BWD(bf16, float);
    case KDA_DTYPE_F16: KDA_UT_BWD(f16, float);
    case KDA_DTYPE_F32: KDA_UT_BWD(float, float);
    case KDA_DTYPE_F64: KDA_UT_BWD(double, double);
#undef KDA_UT_BWD
    default:
      set_detail("ut_transform_bwd: unknown dtype");
      return KDA_ERR_INVALID_ARGUMENT;
  }
}

int launch_ut_transform(const void* k, const void* v, const void* g, const void* beta, int in_dtype, void* M,
                        void* U, void* W, void* log_gamma, void* k_gamma, int out_dtype, int64_t batch,
                        int64_t count, int64_t heads, int64_t key_dim, int64_t value_dim, hipStream_t stream) {
  using namespace kda;
  (void)out_dtype;
  if (count > kUtMaxCount) {
    set_detail("ut_transform: chunk length %lld > %d is not supported", (long long)count, kUtMaxCount);
    return KDA_ERR_UNSUPPORTED;
  }
  if (batch * heads > 0x7fffffffLL) {
    set_detail("ut_transform: too many (batch, head) pairs");
    return KDA_ERR_UNSUPPORTED;
  }
  switch (in_dtype) {
    case KDA_DTYPE_BF16:
      return run_ut<bf16, float>(k, v, g, beta, M, U, W, log_gamma, k_gamma, batch, count, heads, key_dim, value_dim,
                                 stream);
    case KDA_DTYPE_F16:
      return run_ut<f16, float>(k, v, g, beta, M, U, W, log_gamma, k_gamma, batch, count, heads, key_dim, value_dim,
                                stream);
    case KDA_DTYPE_F32:
      return run_ut<float, float>(k, v, g, beta, M, U, W, log_gamma, k_gamma, batch, count, heads, key_dim,
                                  value_dim, stream);
    case KDA_DTYPE_F64:
      return run_ut<double, double>(k, v, g, beta, M, U, W, log_gamma, k_gamma, batch, count, heads, key_dim,
                                    value_dim, stream);
    default:
      set_detail("ut_transform: unknown dtype");
      return KDA_ERR_INVALID_ARGUMENT;
  }
}

}  // namespace kda_host
