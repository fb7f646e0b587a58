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

}  // namespace kda

namespace kda_host {

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
