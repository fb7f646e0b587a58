// Chunkwise KDA backward for float64 inputs: the same chunk equations as the
// f32 kernels of kda_chunk_bwd.hip (gradients of src/kda/chunkwise.py:34-107
// with the UT transform of src/kda/ut_transform.py:23-58), in f64 arithmetic
// throughout, for callers that differentiate in double precision (the
// reference's gradient tests, tests/kda/test_kda_chunkwise_equivalence.py:92-134
// and tests/kda/test_kda_recurrent.py:184-198, run gradcheck in float64).
//
// One workgroup per (batch, head) runs the chunks in order twice: forward, to
// store every chunk's start state S and Vt = U - W S; then backward from the
// last chunk with dS' (the gradient of the chunk's end state), recomputing the
// chunk's local matrices.  Per chunk (lg = cumsum g, Kg = e^lg k,
// Kt = e^(lg_last - lg) k, Qg = e^lg q, D = e^lg_last, N = (I + diag(b) A)^-1,
// M = N diag(b), W = M Kg, U = M v):
//   dVt = Kt dS' + Aqk^T dO,   dS = D dS' + Qg^T dO - W^T dVt,
//   dQg = dO S^T, dAqk = tril(dO Vt^T), dKt = Vt dS'^T, dD = rowsum(dS' * S),
//   dW = -dVt S^T, dv = M^T dVt, dM = dVt v^T + dW Kg^T, dKg = M^T dW,
//   dbeta_j = sum_i N_ij dM_ij + sum_k dL_jk A_jk, dL = -strict(N^T dM diag(b) N^T),
//   dA = diag(b) dL, and per channel the pair sums of dA and dAqk for dq, dk
//   and d lg, whose reverse cumulative sum is dg.
// Plain loops over the workgroup's threads with every intermediate in the
// workspace: this path is for precision, not speed.
#include "kda_launch.h"

namespace kda {
namespace bwd64 {

constexpr int kC = 64;
constexpr int kNT = 256;

// Offsets (in doubles) of one (batch, head)'s region of the workspace.
struct Layout64 {
  int64_t S, Vt;  // per chunk: [NC][K][V] start states, [NC][C][V] Vt
  int64_t q, k, v, lg, b, Kg, Kt, Qg, D, A, Aqk, N, M, W, U, dO, dS, dSn, dVt, dQg, dKt, dW, dKg, dM, T1, dA, dAqk,
      dD, dlg;
  int64_t per;
};

__host__ __device__ inline Layout64 make_layout64(int64_t NC, int64_t K, int64_t V) {
  Layout64 L;
  const int64_t ck = kC * K, cv = kC * V, cc = kC * kC, kv = K * V;
  int64_t o = 0;
  L.S = o; o += NC * kv;
  L.Vt = o; o += NC * cv;
  L.q = o; o += ck;
  L.k = o; o += ck;
  L.v = o; o += cv;
  L.lg = o; o += ck;
  L.b = o; o += kC;
  L.Kg = o; o += ck;
  L.Kt = o; o += ck;
  L.Qg = o; o += ck;
  L.D = o; o += K;
  L.A = o; o += cc;
  L.Aqk = o; o += cc;
  L.N = o; o += cc;
  L.M = o; o += cc;
  L.W = o; o += ck;
  L.U = o; o += cv;
  L.dO = o; o += cv;
  L.dS = o; o += kv;
  L.dSn = o; o += kv;
  L.dVt = o; o += cv;
  L.dQg = o; o += ck;
  L.dKt = o; o += ck;
  L.dW = o; o += ck;
  L.dKg = o; o += ck;
  L.dM = o; o += cc;
  L.T1 = o; o += cc;
  L.dA = o; o += cc;
  L.dAqk = o; o += cc;
  L.dD = o; o += K;
  L.dlg = o; o += ck;
  L.per = (o + 1) / 2 * 2;  // keep every region 16-byte aligned
  return L;
}

// A value and its derivative along one direction (forward-mode
// differentiation): the kernel below, instantiated on Dual, gives the
// directional derivative of everything it computes.
struct Dual {
  double v, d;
};
__device__ __forceinline__ Dual operator+(Dual a, Dual b) { return {a.v + b.v, a.d + b.d}; }
__device__ __forceinline__ Dual operator-(Dual a, Dual b) { return {a.v - b.v, a.d - b.d}; }
__device__ __forceinline__ Dual operator-(Dual a) { return {-a.v, -a.d}; }
__device__ __forceinline__ Dual operator*(Dual a, Dual b) { return {a.v * b.v, a.d * b.v + a.v * b.d}; }
__device__ __forceinline__ Dual operator*(double a, Dual b) { return {a * b.v, a * b.d}; }
__device__ __forceinline__ Dual operator/(Dual a, Dual b) { return {a.v / b.v, (a.d * b.v - a.v * b.d) / (b.v * b.v)}; }
__device__ __forceinline__ Dual& operator+=(Dual& a, Dual b) { return a = a + b; }
__device__ __forceinline__ Dual& operator-=(Dual& a, Dual b) { return a = a - b; }
__device__ __forceinline__ Dual dexp(Dual a) {
  const double e = exp(a.v);
  return {e, e * a.d};
}
__device__ __forceinline__ double dexp(double a) { return exp(a); }
__device__ __forceinline__ double value(double a) { return a; }
__device__ __forceinline__ double value(Dual a) { return a.v; }
template <class T>
__device__ __forceinline__ T cst(double x) {
  if constexpr (__is_same(T, Dual))
    return Dual{x, 0.0};
  else
    return x;
}

// Inputs and outputs: values, and for the Dual instantiation the direction
// (tangents of the inputs; null = 0) and the derivatives it produces along it
// (null = not wanted): of the gradients, of the output and of the final state.
struct Args64 {
  const double *q, *k, *v, *g, *beta, *dout, *s0, *dsT;
  double *dq, *dk, *dv, *dg, *dbeta, *ds0;
  void* ws;
  int64_t B, T, H, K, V, NC;
  const double *tq, *tk, *tv, *tg, *tbeta, *ts0;
  double *tdq, *tdk, *tdv, *tdg, *tdbeta, *tds0, *tout, *tsT;
};

template <class T>
__device__ __forceinline__ T ld(const double* p, const double* tp, int64_t off) {
  if constexpr (__is_same(T, Dual))
    return Dual{p[off], tp ? tp[off] : 0.0};
  else
    return p[off];
}
template <class T>
__device__ __forceinline__ void st(double* p, double* tp, int64_t off, T x) {
  if (p) p[off] = value(x);
  if constexpr (__is_same(T, Dual))
    if (tp) tp[off] = x.d;
}

__device__ __forceinline__ int64_t tok64(int64_t b, int64_t t, int64_t T, int64_t H, int64_t h) {
  return (b * T + t) * H + h;
}

// C[m][n] (row stride ldc) = sum_k A(m, k) B(k, n) (+ C when acc), with
// A(m, k) = A[m * ars + k * acs] and B(k, n) = B[k * brs + n * bcs].
template <class T>
__device__ void gemm(T* C, int64_t ldc, const T* A, int64_t ars, int64_t acs, const T* B, int64_t brs, int64_t bcs,
                     int64_t M, int64_t N, int64_t Kd, double alpha, bool acc) {
  for (int64_t idx = threadIdx.x; idx < M * N; idx += kNT) {
    const int64_t m = idx / N, n = idx % N;
    T s = cst<T>(0.0);
    for (int64_t kk = 0; kk < Kd; ++kk) s += A[m * ars + kk * acs] * B[kk * brs + n * bcs];
    C[m * ldc + n] = acc ? C[m * ldc + n] + alpha * s : alpha * s;
  }
  __syncthreads();
}

// The chunk's inputs (zero past T), lg, Kg, Kt, Qg, D, A, Aqk, N and M.
template <class T>
__device__ void chunk_locals(const Args64& a, const Layout64& L, T* w, int64_t b, int64_t h, int64_t c) {
  const int64_t K = a.K, V = a.V, t0 = c * kC;
  for (int64_t idx = threadIdx.x; idx < kC * K; idx += kNT) {
    const int64_t r = idx / K, j = idx % K, t = t0 + r;
    const bool in = t < a.T;
    const int64_t off = tok64(b, in ? t : 0, a.T, a.H, h) * K + j;
    w[L.q + idx] = in ? ld<T>(a.q, a.tq, off) : cst<T>(0.0);
    w[L.k + idx] = in ? ld<T>(a.k, a.tk, off) : cst<T>(0.0);
    w[L.lg + idx] = in ? ld<T>(a.g, a.tg, off) : cst<T>(0.0);
  }
  for (int64_t idx = threadIdx.x; idx < kC * V; idx += kNT) {
    const int64_t r = idx / V, j = idx % V, t = t0 + r;
    const bool in = t < a.T;
    const int64_t off = tok64(b, in ? t : 0, a.T, a.H, h) * V + j;
    w[L.v + idx] = in ? ld<T>(a.v, a.tv, off) : cst<T>(0.0);
    w[L.dO + idx] = cst<T>(in ? a.dout[off] : 0.0);
  }
  for (int64_t r = threadIdx.x; r < kC; r += kNT) {
    const int64_t t = t0 + r;
    w[L.b + r] = t < a.T ? ld<T>(a.beta, a.tbeta, tok64(b, t, a.T, a.H, h)) : cst<T>(0.0);
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < K; j += kNT) {  // lg = cumsum(g) down the chunk
    T s = cst<T>(0.0);
    for (int64_t r = 0; r < kC; ++r) {
      s += w[L.lg + r * K + j];
      w[L.lg + r * K + j] = s;
    }
    w[L.D + j] = dexp(s);
  }
  __syncthreads();
  for (int64_t idx = threadIdx.x; idx < kC * K; idx += kNT) {
    const int64_t j = idx % K;
    const T l = w[L.lg + idx], last = w[L.lg + (kC - 1) * K + j];
    w[L.Kg + idx] = dexp(l) * w[L.k + idx];
    w[L.Kt + idx] = dexp(last - l) * w[L.k + idx];
    w[L.Qg + idx] = dexp(l) * w[L.q + idx];
  }
  // A_ij = sum_c k_i k_j e^(lg_i - lg_j) (j < i), Aqk_ij the same with q_i (j <= i)
  for (int64_t idx = threadIdx.x; idx < kC * kC; idx += kNT) {
    const int64_t i = idx / kC, j = idx % kC;
    T sa = cst<T>(0.0), sq = cst<T>(0.0);
    if (j <= i)
      for (int64_t x = 0; x < K; ++x) {
        const T e = dexp(w[L.lg + i * K + x] - w[L.lg + j * K + x]) * w[L.k + j * K + x];
        sa += w[L.k + i * K + x] * e;
        sq += w[L.q + i * K + x] * e;
      }
    w[L.A + idx] = j < i ? sa : cst<T>(0.0);
    w[L.Aqk + idx] = j <= i ? sq : cst<T>(0.0);
  }
  __syncthreads();
  // N = (I + diag(b) A)^-1 by forward substitution, row by row
  for (int64_t i = 0; i < kC; ++i) {
    for (int64_t j = threadIdx.x; j < kC; j += kNT) {
      T s = cst<T>(i == j ? 1.0 : 0.0);
      if (j < i)
        for (int64_t x = j; x < i; ++x) s -= w[L.b + i] * w[L.A + i * kC + x] * w[L.N + x * kC + j];
      w[L.N + i * kC + j] = j <= i ? s : cst<T>(0.0);
    }
    __syncthreads();
  }
  for (int64_t idx = threadIdx.x; idx < kC * kC; idx += kNT) w[L.M + idx] = w[L.N + idx] * w[L.b + idx % kC];
  __syncthreads();
}

template <class T>
__global__ __launch_bounds__(kNT) void chunk_bwd_f64_kernel(const Args64 a) {
  const int64_t bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
  const int64_t K = a.K, V = a.V, kv = K * V;
  const Layout64 L = make_layout64(a.NC, K, V);
  T* w = static_cast<T*>(a.ws) + bh * L.per;
  // ---- forward: start states and Vt of every chunk (and, when asked for,
  // the output O = Qg S + Aqk Vt and the final state)
  for (int64_t idx = threadIdx.x; idx < kv; idx += kNT)
    w[L.dS + idx] = a.s0 ? ld<T>(a.s0, a.ts0, bh * kv + idx) : cst<T>(0.0);
  __syncthreads();
  for (int64_t c = 0; c < a.NC; ++c) {
    chunk_locals(a, L, w, b, h, c);
    T *S = w + L.S + c * kv, *Vt = w + L.Vt + c * kC * V;
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) S[idx] = w[L.dS + idx];  // dS holds the running state
    gemm(w + L.W, K, w + L.M, kC, 1, w + L.Kg, K, 1, kC, K, kC, 1.0, false);  // W = M Kg
    gemm(w + L.U, V, w + L.M, kC, 1, w + L.v, V, 1, kC, V, kC, 1.0, false);   // U = M v
    for (int64_t idx = threadIdx.x; idx < kC * V; idx += kNT) Vt[idx] = w[L.U + idx];
    __syncthreads();
    gemm(Vt, V, w + L.W, K, 1, S, V, 1, kC, V, K, -1.0, true);  // Vt = U - W S
    if (a.tout != nullptr) {  // O = Qg S + Aqk Vt, over U (free now)
      gemm(w + L.U, V, w + L.Qg, K, 1, S, V, 1, kC, V, K, 1.0, false);
      gemm(w + L.U, V, w + L.Aqk, kC, 1, Vt, V, 1, kC, V, kC, 1.0, true);
      for (int64_t idx = threadIdx.x; idx < kC * V; idx += kNT) {
        const int64_t t = c * kC + idx / V;
        if (t < a.T) st<T>(nullptr, a.tout, tok64(b, t, a.T, a.H, h) * V + idx % V, w[L.U + idx]);
      }
    }
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) w[L.dS + idx] = w[L.D + idx / V] * S[idx];
    __syncthreads();
    gemm(w + L.dS, V, w + L.Kt, 1, K, Vt, V, 1, K, V, kC, 1.0, true);  // S' = D S + Kt^T Vt
  }
  if (a.tsT != nullptr)
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) st<T>(nullptr, a.tsT, bh * kv + idx, w[L.dS + idx]);
  // ---- backward from the last chunk
  for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) w[L.dS + idx] = cst<T>(a.dsT ? a.dsT[bh * kv + idx] : 0.0);
  __syncthreads();
  for (int64_t c = a.NC - 1; c >= 0; --c) {
    chunk_locals(a, L, w, b, h, c);
    const T *S = w + L.S + c * kv, *Vt = w + L.Vt + c * kC * V;
    const int64_t t0 = c * kC;
    gemm(w + L.W, K, w + L.M, kC, 1, w + L.Kg, K, 1, kC, K, kC, 1.0, false);          // W = M Kg
    gemm(w + L.dVt, V, w + L.Kt, K, 1, w + L.dS, V, 1, kC, V, K, 1.0, false);         // Kt dS'
    gemm(w + L.dVt, V, w + L.Aqk, 1, kC, w + L.dO, V, 1, kC, V, kC, 1.0, true);       // + Aqk^T dO
    gemm(w + L.dQg, K, w + L.dO, V, 1, S, 1, V, kC, K, V, 1.0, false);                // dQg = dO S^T
    gemm(w + L.dAqk, kC, w + L.dO, V, 1, Vt, 1, V, kC, kC, V, 1.0, false);            // dO Vt^T
    gemm(w + L.dKt, K, Vt, V, 1, w + L.dS, 1, V, kC, K, V, 1.0, false);               // dKt = Vt dS'^T
    gemm(w + L.dW, K, w + L.dVt, V, 1, S, 1, V, kC, K, V, -1.0, false);               // dW = -dVt S^T
    for (int64_t j = threadIdx.x; j < K; j += kNT) {                                  // dD = rowsum(dS' * S)
      T s = cst<T>(0.0);
      for (int64_t x = 0; x < V; ++x) s += w[L.dS + j * V + x] * S[j * V + x];
      w[L.dD + j] = s;
    }
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) w[L.dSn + idx] = w[L.D + idx / V] * w[L.dS + idx];
    __syncthreads();
    gemm(w + L.dSn, V, w + L.Qg, 1, K, w + L.dO, V, 1, K, V, kC, 1.0, true);          // + Qg^T dO
    gemm(w + L.dSn, V, w + L.W, 1, K, w + L.dVt, V, 1, K, V, kC, -1.0, true);         // - W^T dVt
    // dv = M^T dVt
    for (int64_t idx = threadIdx.x; idx < kC * V; idx += kNT) {
      const int64_t i = idx / V, x = idx % V, t = t0 + i;
      T s = cst<T>(0.0);
      for (int64_t r = 0; r < kC; ++r) s += w[L.M + r * kC + i] * w[L.dVt + r * V + x];
      if (t < a.T) st<T>(a.dv, a.tdv, tok64(b, t, a.T, a.H, h) * V + x, s);
    }
    gemm(w + L.dM, kC, w + L.dVt, V, 1, w + L.v, 1, V, kC, kC, V, 1.0, false);        // dM = dVt v^T
    gemm(w + L.dM, kC, w + L.dW, K, 1, w + L.Kg, 1, K, kC, kC, K, 1.0, true);         // + dW Kg^T
    gemm(w + L.dKg, K, w + L.M, 1, kC, w + L.dW, K, 1, kC, K, kC, 1.0, false);        // dKg = M^T dW
    // dL = -strict(N^T (dM diag b) N^T): T1 = N^T (dM diag b), then -T1 N^T
    for (int64_t idx = threadIdx.x; idx < kC * kC; idx += kNT) {
      const int64_t i = idx / kC, j = idx % kC;
      T s = cst<T>(0.0);
      for (int64_t r = 0; r < kC; ++r) s += w[L.N + r * kC + i] * w[L.dM + r * kC + j] * w[L.b + j];
      w[L.T1 + idx] = s;
    }
    __syncthreads();
    for (int64_t idx = threadIdx.x; idx < kC * kC; idx += kNT) {
      const int64_t i = idx / kC, j = idx % kC;
      T s = cst<T>(0.0);
      for (int64_t r = 0; r < kC; ++r) s += w[L.T1 + i * kC + r] * w[L.N + j * kC + r];
      w[L.dA + idx] = j < i ? -s * w[L.b + i] : cst<T>(0.0);  // dA = diag(b) dL
      w[L.dAqk + idx] = j <= i ? w[L.dAqk + idx] : cst<T>(0.0);
    }
    __syncthreads();
    for (int64_t j = threadIdx.x; j < kC; j += kNT) {  // dbeta
      T s = cst<T>(0.0);
      for (int64_t i = 0; i < kC; ++i) s += w[L.N + i * kC + j] * w[L.dM + i * kC + j];
      const T bj = w[L.b + j];
      if (value(bj) != 0.0)  // sum_k dL_jk A_jk with dL = dA / b
        for (int64_t x = 0; x < j; ++x) s += w[L.dA + j * kC + x] / bj * w[L.A + j * kC + x];
      else
        for (int64_t x = 0; x < j; ++x) {
          T t = cst<T>(0.0);
          for (int64_t r = 0; r < kC; ++r) t += w[L.T1 + j * kC + r] * w[L.N + x * kC + r];
          s -= t * w[L.A + j * kC + x];
        }
      const int64_t t = t0 + j;
      if (t < a.T) st<T>(a.dbeta, a.tdbeta, tok64(b, t, a.T, a.H, h), s);
    }
    // per channel: the pair sums, dq, dk and d lg
    for (int64_t idx = threadIdx.x; idx < kC * K; idx += kNT) {
      const int64_t i = idx / K, x = idx % K;
      const T li = w[L.lg + idx], ki = w[L.k + idx], qi = w[L.q + idx];
      T r1 = cst<T>(0.0), r2 = cst<T>(0.0), r3 = cst<T>(0.0), r4 = cst<T>(0.0);
      for (int64_t j = 0; j <= i; ++j) {  // R1, R2 over j <= i
        const T e = dexp(li - w[L.lg + j * K + x]) * w[L.k + j * K + x];
        r1 += w[L.dA + i * kC + j] * e;
        r2 += w[L.dAqk + i * kC + j] * e;
      }
      for (int64_t r = i; r < kC; ++r) {  // R3, R4 over rows r >= i
        const T e = dexp(w[L.lg + r * K + x] - li);
        r3 += w[L.dA + r * kC + i] * w[L.k + r * K + x] * e;
        r4 += w[L.dAqk + r * kC + i] * w[L.q + r * K + x] * e;
      }
      const T el = dexp(li), te = dexp(w[L.lg + (kC - 1) * K + x] - li);
      const T dk = r1 + r3 + r4 + el * w[L.dKg + idx] + te * w[L.dKt + idx];
      const T dq = r2 + el * w[L.dQg + idx];
      w[L.dlg + idx] = ki * (r1 - r3 - r4) + qi * r2 + w[L.Kg + idx] * w[L.dKg + idx] +
                       w[L.Qg + idx] * w[L.dQg + idx] - w[L.Kt + idx] * w[L.dKt + idx];
      const int64_t t = t0 + i;
      if (t < a.T) {
        const int64_t off = tok64(b, t, a.T, a.H, h) * K + x;
        st<T>(a.dq, a.tdq, off, dq);
        st<T>(a.dk, a.tdk, off, dk);
      }
    }
    __syncthreads();
    for (int64_t x = threadIdx.x; x < K; x += kNT) {  // dg = reverse cumsum of d lg (+ the last row's terms)
      T run = w[L.D + x] * w[L.dD + x];
      for (int64_t r = 0; r < kC; ++r) run += w[L.Kt + r * K + x] * w[L.dKt + r * K + x];
      for (int64_t i = kC - 1; i >= 0; --i) {
        run += w[L.dlg + i * K + x];
        const int64_t t = t0 + i;
        if (t < a.T) st<T>(a.dg, a.tdg, tok64(b, t, a.T, a.H, h) * K + x, run);
      }
    }
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) w[L.dS + idx] = w[L.dSn + idx];
    __syncthreads();
  }
  if (a.ds0 || a.tds0)
    for (int64_t idx = threadIdx.x; idx < kv; idx += kNT) st<T>(a.ds0, a.tds0, bh * kv + idx, w[L.dS + idx]);
}

}  // namespace bwd64
}  // namespace kda

namespace kda_host {

size_t chunk_bwd_f64_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V) {
  const int64_t NC = (T + kda::bwd64::kC - 1) / kda::bwd64::kC;
  return static_cast<size_t>(B * H * kda::bwd64::make_layout64(NC, K, V).per) * sizeof(double);
}

int launch_chunk_bwd_f64(const double* q, const double* k, const double* v, const double* g, const double* beta,
                         const double* dout, const double* s0, const double* dsT, double* dq, double* dk, double* dv,
                         double* dg, double* dbeta, double* ds0, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                         double* ws, hipStream_t stream) {
  const int64_t NC = (T + kda::bwd64::kC - 1) / kda::bwd64::kC;
  if (B * H > 0x7fffffffLL) {
    set_detail("chunk backward (f64): grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  kda::bwd64::Args64 a{};
  a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta, a.dout = dout, a.s0 = s0, a.dsT = dsT;
  a.dq = dq, a.dk = dk, a.dv = dv, a.dg = dg, a.dbeta = dbeta, a.ds0 = ds0, a.ws = ws;
  a.B = B, a.T = T, a.H = H, a.K = K, a.V = V, a.NC = NC;
  hipLaunchKernelGGL(kda::bwd64::chunk_bwd_f64_kernel<double>, dim3(static_cast<unsigned>(B * H)),
                     dim3(kda::bwd64::kNT), 0, stream, a);
  return check_launch("chunk_bwd_f64_kernel");
}

size_t chunk_grad_tangent_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V) {
  return 2 * chunk_bwd_f64_workspace_bytes(B, T, H, K, V);
}

int launch_chunk_grad_tangent(const double* const* in, const double* const* tan, const double* dout,
                              const double* dsT, double* const* tgrad, double* tout, double* tsT, int64_t B, int64_t T,
                              int64_t H, int64_t K, int64_t V, void* ws, hipStream_t stream) {
  const int64_t NC = (T + kda::bwd64::kC - 1) / kda::bwd64::kC;
  if (B * H > 0x7fffffffLL) {
    set_detail("chunk gradient tangent: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  kda::bwd64::Args64 a{};
  a.q = in[0], a.k = in[1], a.v = in[2], a.g = in[3], a.beta = in[4], a.s0 = in[5], a.dout = dout, a.dsT = dsT;
  a.tq = tan[0], a.tk = tan[1], a.tv = tan[2], a.tg = tan[3], a.tbeta = tan[4], a.ts0 = tan[5];
  a.tdq = tgrad[0], a.tdk = tgrad[1], a.tdv = tgrad[2], a.tdg = tgrad[3], a.tdbeta = tgrad[4], a.tds0 = tgrad[5];
  a.tout = tout, a.tsT = tsT, a.ws = ws;
  a.B = B, a.T = T, a.H = H, a.K = K, a.V = V, a.NC = NC;
  hipLaunchKernelGGL(kda::bwd64::chunk_bwd_f64_kernel<kda::bwd64::Dual>, dim3(static_cast<unsigned>(B * H)),
                     dim3(kda::bwd64::kNT), 0, stream, a);
  return check_launch("chunk_bwd_f64_kernel<tangent>");
}

}  // namespace kda_host
