// Backward of the token recurrence with its per-token states
// (recurrent_kda(..., return_states_per_token=True), src/kda/recurrent.py:61-79),
// the debugging path whose every intermediate state is an output and may
// carry a gradient.  Per token (alpha = e^g, S~ = diag(alpha) S_{t-1}):
//   e = v - S~^T k,  S_t = S~ + b k e^T,  o = S_t^T q.
// Going back from the last token with dS (the gradient of S_t, plus the
// token's own state gradient):
//   dS += q do^T,  dq = S_t do,  u = dS e,  db = k . u,  de = b dS^T k,
//   dk = b u - S~ de,  dv = de,  dS~ = dS - k de^T,
//   dg_i = alpha_i sum_j dS~_ij S_{t-1,ij},  dS_{t-1} = diag(alpha) dS~.
// S_{t-1} comes from the forward's per-token states (the initial state
// before the first token), so nothing is recomputed.  One workgroup per
// (sequence, head); the running dS lives in the workspace.  Arithmetic in the
// work type (f32 or f64): a precision path for a debugging mode, not a fast one.
#include "kda_launch.h"

namespace kda {
namespace rbwd {

constexpr int kNT = 256;

template <class T>
struct RecBwdArgs {
  const T *q, *k, *v, *g, *beta, *dout, *s0, *hist, *dhist, *dsT;  // hist, dhist: [T, B, H, K, V]
  T *dq, *dk, *dv, *dg, *dbeta, *ds0, *ws;
  int64_t B, Tn, H, K, V;
};

template <class T>
__device__ __forceinline__ T ex(T x);
template <>
__device__ __forceinline__ float ex<float>(float x) {
  return expf(x);
}
template <>
__device__ __forceinline__ double ex<double>(double x) {
  return exp(x);
}

template <class T>
__global__ __launch_bounds__(kNT) void recurrent_bwd_kernel(const RecBwdArgs<T> a) {
  const int64_t bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int64_t K = a.K, V = a.V, kv = K * V;
  // workspace of this (sequence, head): dS [K][V], e [V], de [V], u [K]
  T* dS = a.ws + bh * (kv + 2 * V + K + 2);
  T *e = dS + kv, *de = e + V, *u = de + V;
  for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) dS[idx] = a.dsT ? a.dsT[bh * kv + idx] : T(0);
  __syncthreads();
  for (int64_t t = a.Tn - 1; t >= 0; --t) {
    const int64_t row = (b * a.Tn + t) * a.H + h;  // token row of q, k, g: [B, T, H, *]
    const T* qt = a.q + row * K;
    const T* kt = a.k + row * K;
    const T* gt = a.g + row * K;
    const T* vt = a.v + row * V;
    const T* dot = a.dout + row * V;
    const T bt = a.beta[row];
    const T* St = a.hist + (t * a.B * a.H + bh) * kv;                         // S_t
    const T* Sp = t > 0 ? a.hist + ((t - 1) * a.B * a.H + bh) * kv : nullptr;  // S_{t-1}
    const T* S0 = a.s0 ? a.s0 + bh * kv : nullptr;
    auto prev = [&](int64_t idx) -> T { return Sp ? Sp[idx] : (S0 ? S0[idx] : T(0)); };
    // dS += dhist_t + q do^T
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) {
      const int64_t i = idx / V, j = idx % V;
      dS[idx] += (a.dhist ? a.dhist[(t * a.B * a.H + bh) * kv + idx] : T(0)) + qt[i] * dot[j];
    }
    // e = v - S~^T k
    for (int64_t j = threadIdx.x; j < V; j += kNT) {
      T s = T(0);
      for (int64_t i = 0; i < K; ++i) s += ex<T>(gt[i]) * prev(i * V + j) * kt[i];
      e[j] = vt[j] - s;
    }
    __syncthreads();
    // dq = S_t do, u = dS e;  de = b dS^T k
    for (int64_t i = threadIdx.x; i < K; i += kNT) {
      T sq = T(0), su = T(0);
      for (int64_t j = 0; j < V; ++j) {
        sq += St[i * V + j] * dot[j];
        su += dS[i * V + j] * e[j];
      }
      a.dq[row * K + i] = sq;
      u[i] = su;
    }
    for (int64_t j = threadIdx.x; j < V; j += kNT) {
      T s = T(0);
      for (int64_t i = 0; i < K; ++i) s += dS[i * V + j] * kt[i];
      de[j] = bt * s;
      a.dv[row * V + j] = bt * s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      T s = T(0);
      for (int64_t i = 0; i < K; ++i) s += kt[i] * u[i];
      a.dbeta[row] = s;
    }
    // dk = b u - S~ de
    for (int64_t i = threadIdx.x; i < K; i += kNT) {
      T s = T(0);
      for (int64_t j = 0; j < V; ++j) s += prev(i * V + j) * de[j];
      a.dk[row * K + i] = bt * u[i] - ex<T>(gt[i]) * s;
    }
    __syncthreads();
    // dS~ = dS - k de^T; dg_i = alpha_i sum_j dS~_ij S_{t-1,ij}; dS_{t-1} = diag(alpha) dS~
    for (int64_t i = threadIdx.x; i < K; i += kNT) {
      const T al = ex<T>(gt[i]);
      T s = T(0);
      for (int64_t j = 0; j < V; ++j) {
        const T d = dS[i * V + j] - kt[i] * de[j];
        s += d * prev(i * V + j);
        dS[i * V + j] = al * d;
      }
      a.dg[row * K + i] = al * s;
    }
    __syncthreads();
  }
  if (a.ds0)
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) a.ds0[bh * kv + idx] = dS[idx];
}

}  // namespace rbwd
}  // namespace kda

namespace kda_host {

size_t recurrent_bwd_workspace_bytes(int64_t B, int64_t H, int64_t K, int64_t V, int dtype) {
  const size_t el = dtype == KDA_DTYPE_F64 ? sizeof(double) : sizeof(float);
  return static_cast<size_t>(B * H * (K * V + 2 * V + K + 2)) * el;
}

template <class T>
static int run_rbwd(const kda::rbwd::RecBwdArgs<T>& a, hipStream_t stream) {
  if (a.B * a.H > 0x7fffffffLL) {
    set_detail("recurrent backward: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(kda::rbwd::recurrent_bwd_kernel<T>, dim3(static_cast<unsigned>(a.B * a.H)),
                     dim3(kda::rbwd::kNT), 0, stream, a);
  return check_launch("recurrent_bwd_kernel");
}

int launch_recurrent_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const void* dout, const void* s0, const void* hist, const void* dhist, const void* dsT,
                         void* dq, void* dk, void* dv, void* dg, void* dbeta, void* ds0, int64_t B, int64_t T,
                         int64_t H, int64_t K, int64_t V, int dtype, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (dtype != KDA_DTYPE_F32 && dtype != KDA_DTYPE_F64) {
    set_detail("recurrent backward: tensors must be f32 or f64 (dtype %d)", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  const size_t need = recurrent_bwd_workspace_bytes(B, H, K, V, dtype);
  if (ws == nullptr || ws_bytes < need) {
    set_detail("recurrent backward: workspace of %zu bytes needed", need);
    return KDA_ERR_WORKSPACE;
  }
  if (dtype == KDA_DTYPE_F64) {
    using D = double;
    return run_rbwd(kda::rbwd::RecBwdArgs<D>{
                        static_cast<const D*>(q), static_cast<const D*>(k), static_cast<const D*>(v),
                        static_cast<const D*>(g), static_cast<const D*>(beta), static_cast<const D*>(dout),
                        static_cast<const D*>(s0), static_cast<const D*>(hist), static_cast<const D*>(dhist),
                        static_cast<const D*>(dsT), static_cast<D*>(dq), static_cast<D*>(dk), static_cast<D*>(dv),
                        static_cast<D*>(dg), static_cast<D*>(dbeta), static_cast<D*>(ds0), static_cast<D*>(ws), B, T,
                        H, K, V},
                    stream);
  }
  using F = float;
  return run_rbwd(kda::rbwd::RecBwdArgs<F>{
                      static_cast<const F*>(q), static_cast<const F*>(k), static_cast<const F*>(v),
                      static_cast<const F*>(g), static_cast<const F*>(beta), static_cast<const F*>(dout),
                      static_cast<const F*>(s0), static_cast<const F*>(hist), static_cast<const F*>(dhist),
                      static_cast<const F*>(dsT), static_cast<F*>(dq), static_cast<F*>(dk), static_cast<F*>(dv),
                      static_cast<F*>(dg), static_cast<F*>(dbeta), static_cast<F*>(ds0), static_cast<F*>(ws), B, T, H,
                      K, V},
                  stream);
}

}  // namespace kda_host
