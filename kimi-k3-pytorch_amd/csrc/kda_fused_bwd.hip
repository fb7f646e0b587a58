// Backward of the fused stages around the KDA operator on gfx950 (the
// derivatives the reference takes from autograd through
// src/kda/projections.py:164-218, src/kda/decay.py:36-43,
// src/kimi_primitives/short_conv.py:69-98, headwise_rmsnorm.py:39-64 and
// output_gate.py:62-75):
//  * conv_silu_bwd_kernel: ShortConv + SiLU (+ per-head L2 norm), its input,
//    weight, bias and history gradients;
//  * gates_bwd_kernel: the lower-bounded decay (logits, bias, A_log) and the
//    beta gate;
//  * rmsnorm_gate_bwd_kernel: head-wise RMSNorm times the sigmoid gate (input,
//    norm weight and gate logits).
// Each is one HBM stream over the activations and their gradients: the
// forward's intermediates (conv pre-activations, norms, sigmoids) are
// recomputed from the inputs in registers rather than stored.  Arithmetic is
// f32 (f64 for f64 tensors); activation gradients are rounded once to the
// tensors' type.  Parameter gradients (f32, or f64 for f64) are summed over a
// workgroup in LDS and added to a caller-zeroed buffer with one vector float
// atomic per parameter element and workgroup, so their summation order (not
// their value beyond rounding) varies from run to run.
#include <math.h>

#include "kda_launch.h"

namespace kda {
namespace fbwd {

template <class T>
struct ComputeOf {
  using type = float;
};
template <>
struct ComputeOf<double> {
  using type = double;
};

__device__ __forceinline__ void atomic_add(float* p, float v) { atomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(double* p, double v) { atomicAdd(p, v); }

// ---- head-wise RMSNorm x sigmoid gate --------------------------------------------
// Forward (per row and head of D elements): r = rsqrt(mean(x^2) + eps),
// n = x r, y = n * w * sigmoid(z).  Backward with dy:
//   dz = dy n w s (1 - s),  dw += dy n s,  dn = dy w s,
//   dx = r (dn - n * sum(dn n) / D).
// A lane group of G lanes holds one (row, head) pair, VEC elements per lane.
// A block takes one head and 256 / G of its rows at a time, striding over the
// rows with the other blocks of that head; the weight gradient accumulates in
// registers, the block's groups' sums meet in LDS in a fixed order, and each
// element goes out with one atomic per block.
template <class T>
struct NormBwdArgs {
  const T* x;    // [rows, H, D]
  const T* w;    // [H, D], [D] or null
  int w_per_head;
  const T* gl;   // [rows, H*D] or null
  const T* dy;   // [rows, H, D]
  T* dx;         // [rows, H, D]
  T* dgl;        // [rows, H*D] or null
  typename ComputeOf<T>::type* dw;  // [H, D] or [D] accumulators (zeroed by the caller) or null
  int64_t rows, H, row_blocks;      // row_blocks: blocks per head (the grid is H x row_blocks)
  float eps;
};

template <class T, int VEC, int G>
__global__ __launch_bounds__(256) void rmsnorm_gate_bwd_kernel(const NormBwdArgs<T> a) {
  using C = typename ComputeOf<T>::type;
  constexpr int D = G * VEC, PB = 256 / G;  // PB: lane groups (rows) per block
  typedef T vec_t __attribute__((ext_vector_type(VEC)));
  __shared__ C red[PB][D];
  const int k = threadIdx.x % G, gi = threadIdx.x / G;
  const int64_t head = blockIdx.x % a.H, rb = blockIdx.x / a.H;
  vec_t wv = {};
  if (a.w != nullptr) wv = *reinterpret_cast<const vec_t*>(a.w + (a.w_per_head ? head * D : 0) + k * VEC);
  C dw[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) dw[e] = C(0);
  // the lanes of a group share the row, so they run the same steps (the
  // reductions stay inside the group)
  for (int64_t row = rb * PB + gi; row < a.rows; row += a.row_blocks * PB) {
    const int64_t pair = row * a.H + head;
    vec_t gv = {};
    const vec_t xv = *reinterpret_cast<const vec_t*>(a.x + pair * D + k * VEC);
    const vec_t dv = *reinterpret_cast<const vec_t*>(a.dy + pair * D + k * VEC);
    if (a.gl != nullptr) gv = *reinterpret_cast<const vec_t*>(a.gl + pair * D + k * VEC);
    C ss = C(0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += to_compute<C>(xv[e]) * to_compute<C>(xv[e]);
    ss = group_sum<G>(ss);
    const C r = frsqrt(ss / C(D) + C(a.eps));
    C nn[VEC], dn[VEC];
    C dot = C(0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      nn[e] = to_compute<C>(xv[e]) * r;
      const C s = a.gl != nullptr ? sigmoid(to_compute<C>(gv[e])) : C(1);
      const C ww = a.w != nullptr ? to_compute<C>(wv[e]) : C(1);
      const C d = to_compute<C>(dv[e]);
      dw[e] += d * nn[e] * s;
      dn[e] = d * ww * s;
      dot += dn[e] * nn[e];
      if (a.dgl != nullptr) gv[e] = from_compute<T>(d * nn[e] * ww * s * (C(1) - s));
    }
    dot = group_sum<G>(dot);
    vec_t o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = from_compute<T>(r * (dn[e] - nn[e] * dot / C(D)));
    *reinterpret_cast<vec_t*>(a.dx + pair * D + k * VEC) = o;
    if (a.dgl != nullptr) *reinterpret_cast<vec_t*>(a.dgl + pair * D + k * VEC) = gv;
  }
  if (a.dw != nullptr) {  // uniform
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[gi][k * VEC + e] = dw[e];
    __syncthreads();
    C* dst = a.dw + (a.w_per_head ? head * D : 0);
    for (int d = threadIdx.x; d < D; d += 256) {
      C sum = red[0][d];
      for (int u = 1; u < PB; ++u) sum += red[u][d];
      atomic_add(dst + d, sum);
    }
  }
}

// ---- lower-bounded decay and beta gate ---------------------------------------------
// Forward: u = z + b, s = exp(A_log[h]), p = sigmoid(s u), g = g_min clamp(p, lo, hi),
// alpha = exp(g); beta = clamp(sigmoid(l), lo, hi).  Backward (the clamp
// passes gradient for lo <= p <= hi, as torch.clamp does):
//   dg' = dg + dalpha * exp(g),  dq = dg' g_min [lo <= p <= hi] p (1 - p),
//   dz = dq s,  db += dq s,  dA_log[h] += s * sum(dq u);
//   dl = dbeta [lo <= beta' <= hi] beta' (1 - beta'),  beta' = sigmoid(l).
// A thread owns one 16-byte vector position of a row's [H, K] block (fixed
// head and channels) and walks a share of a block's rows: a block holds
// kGateRowGroups groups of kGatePos threads over the same positions, each
// group every kGateRowGroups-th row of the block's range.  The bias and A_log
// gradients accumulate in registers, the groups' sums meet in LDS in a fixed
// order, the bias gradient goes out with one atomic per element and block and
// the A_log gradient with one per head and block (summed over the head's
// positions in the block first): about 32 atomics per address at 8192 rows
// (256 blocks) instead of one per row, the atomics having set the time
// (2.55 ms with one per thread and row, 71 us at 256 positions x 4 row groups,
// 33 at 64 x 16, 27 at 32 x 32 for B=1, T=8192, H=16, K=128, bf16).
constexpr int kGatePos = 32, kGateRowGroups = 32;
template <class T>
struct GateBwdArgs {
  const T* z;          // [rows, H, K] or null
  const T* zbias;      // [H, K] or null
  const float* a_log;  // [H]
  const T* dg;         // [rows, H, K]
  const T* dalpha;     // [rows, H, K] or null
  T* dz;               // [rows, H, K]
  typename ComputeOf<T>::type* dzbias;  // [H, K] accumulators or null
  typename ComputeOf<T>::type* da_log;  // [H] accumulators or null
  const T* bl;         // [rows, H] or null
  const T* dbeta;      // [rows, H]
  T* dbl;              // [rows, H]
  int64_t rows, H, K;
  float g_min, eps;
};

template <class T>
__global__ __launch_bounds__(kGatePos * kGateRowGroups) void gates_bwd_kernel(const GateBwdArgs<T> a) {
  using C = typename ComputeOf<T>::type;
  constexpr int VEC = 16 / sizeof(T);
  typedef T vec_t __attribute__((ext_vector_type(VEC)));
  __shared__ C red[kGateRowGroups][kGatePos][VEC + 1];
  const C lo = C(a.eps), hi = C(1) - C(a.eps);
  if (a.z != nullptr) {  // uniform
    const int64_t hkv = a.H * a.K / VEC;
    const int tv = threadIdx.x % kGatePos, rg = threadIdx.x / kGatePos;
    const int64_t v = static_cast<int64_t>(blockIdx.x) * kGatePos + tv;
    const bool live = v < hkv;
    const int64_t h = live ? v * VEC / a.K : 0;
    const C s = live ? fexp(static_cast<C>(a.a_log[h])) : C(0);
    C db[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) db[e] = C(0);
    C ds = C(0);
    if (live) {
      vec_t bv = {};
      if (a.zbias != nullptr) bv = *reinterpret_cast<const vec_t*>(a.zbias + v * VEC);
      const int64_t per = (a.rows + gridDim.y - 1) / gridDim.y;  // rows per block
      const int64_t r0 = static_cast<int64_t>(blockIdx.y) * per;
      const int64_t r1 = r0 + per < a.rows ? r0 + per : a.rows;
      for (int64_t r = r0 + rg; r < r1; r += kGateRowGroups) {
        const int64_t e0 = (r * hkv + v) * VEC;
        const vec_t zv = *reinterpret_cast<const vec_t*>(a.z + e0);
        const vec_t gv = *reinterpret_cast<const vec_t*>(a.dg + e0);
        vec_t av = {};
        if (a.dalpha != nullptr) av = *reinterpret_cast<const vec_t*>(a.dalpha + e0);
        vec_t o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const C u = to_compute<C>(zv[e]) + to_compute<C>(bv[e]);
          const C p = sigmoid(s * u);
          const bool pass = p >= lo && p <= hi;
          const C pc = p < lo ? lo : (p > hi ? hi : p);
          C dgt = to_compute<C>(gv[e]);
          if (a.dalpha != nullptr) dgt += to_compute<C>(av[e]) * fexp(C(a.g_min) * pc);
          const C dq = pass ? dgt * C(a.g_min) * p * (C(1) - p) : C(0);
          o[e] = from_compute<T>(dq * s);
          db[e] += dq * s;
          ds += dq * u;
        }
        *reinterpret_cast<vec_t*>(a.dz + e0) = o;
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[rg][tv][e] = db[e];
    red[rg][tv][VEC] = ds * s;
    __syncthreads();
    if (rg == 0 && live) {
#pragma unroll
      for (int e = 0; e < VEC + 1; ++e) {
        C sum = red[0][tv][e];
#pragma unroll
        for (int u = 1; u < kGateRowGroups; ++u) sum += red[u][tv][e];
        red[0][tv][e] = sum;
      }
      if (a.dzbias != nullptr)
#pragma unroll
        for (int e = 0; e < VEC; ++e) atomic_add(a.dzbias + v * VEC + e, red[0][tv][e]);
    }
    __syncthreads();
    // A_log: the first of a head's positions in this block sums the head's
    // positions in order and adds them with one atomic
    if (rg == 0 && live && a.da_log != nullptr && (tv == 0 || (v * VEC) % a.K == 0)) {
      C sum = C(0);
      for (int u = tv; u < kGatePos && static_cast<int64_t>(blockIdx.x) * kGatePos + u < hkv &&
                       (static_cast<int64_t>(blockIdx.x) * kGatePos + u) * VEC / a.K == h;
           ++u)
        sum += red[0][u][VEC];
      atomic_add(a.da_log + h, sum);
    }
  }
  if (a.bl != nullptr) {
    const int64_t n = a.rows * a.H;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * gridDim.y * blockDim.x;
    for (int64_t j = (static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; j < n;
         j += stride) {
      const C p = sigmoid(to_compute<C>(a.bl[j]));
      const bool pass = p >= lo && p <= hi;
      a.dbl[j] = from_compute<T>(pass ? to_compute<C>(a.dbeta[j]) * p * (C(1) - p) : C(0));
    }
  }
}

// ---- ShortConv + SiLU (+ per-head L2 norm) -----------------------------------------
// Forward (channel c, position t < len, positions < 0 from the history):
//   pre_t = bias + sum_j w[j] x_{t-j},  a_t = silu(pre_t),  y_t = a_t (or a_t / max(||a_t||_head, eps)),
// zero outputs past len; the next history is the last K-1 rows of [history | valid prefix].
// Backward with dy and the next history's gradient dh':
//   da = (dy - y (y . dy)) / ||a|| (||a|| > eps) or dy / eps;  dpre = da sig (1 + pre (1 - sig));
//   dx_s = sum_j w[j] dpre_{s+j} (+ dh' where x_s went into the next history),
//   dhist_m = sum_j w[j] dpre_{m-(K-1)+j} (+ dh' where the history row went on),
//   dw[c][j] += sum_t dpre_t x_{t-j},  dbias[c] += sum_t dpre_t.
// One lane per (batch row, VEC channels, run of kConvBwdRun positions).  The
// lane walks positions t0 - (KM-1) .. t0 + R + KM - 2 in order with the last
// KM inputs and the last KM values of dpre in registers: at position t it
// loads x_t (and dy_t), forms dpre_t (t >= t0; zero before), adds dpre_t and
// dpre_t x_{t-j} to the bias and weight gradients while t is in the run, and
// completes dx_s = sum_j w[j] dpre_{s+j} for s = t - (KM-1) in the run; the
// run at t0 = 0 also completes the history rows (s < 0).  The K-1 rows on
// either side of a run are read by both neighbouring runs (L2 hits).  A block
// takes conv_bwd_waves<KT>() consecutive runs of one channel block (16 at a
// compile-time kernel size, 8 for any K: its windows of kConvBwdMaxK need the
// registers of two waves per SIMD instead of four); its waves' weight and bias
// gradients are summed in LDS in a fixed order and go out with one atomic per
// element and block.
constexpr int kConvBwdRun = 16;
constexpr int kConvBwdMaxK = 8;
template <int KT>
__host__ __device__ constexpr int conv_bwd_waves() { return KT > 0 ? 16 : 8; }

template <class T>
struct ConvBwdArgs {
  const T* x;         // [B, T, C]
  const T* w;         // [C, K]
  const T* bias;      // [C] or null
  const T* hist_in;   // [B, K-1, C] or null (zeros)
  const int32_t* valid_lens;
  const T* dy;        // [B, T, C]
  const T* dhist_out; // [B, K-1, C] or null
  T* dx;              // [B, T, C]
  T* dhist_in;        // [B, K-1, C] or null
  typename ComputeOf<T>::type* dw;     // [C, K] accumulators or null
  typename ComputeOf<T>::type* dbias;  // [C] accumulators or null
  int64_t nb, nt, nc;
  int K;
  float eps;
};

__host__ __device__ constexpr int64_t conv_bwd_runs(int64_t nt) { return (nt + kConvBwdRun - 1) / kConvBwdRun; }

// VEC: channels per lane; KT: the kernel size, or 0 for any K <= kConvBwdMaxK;
// G: lanes per normalised head (0: no normalisation).
template <class T, int VEC, int KT, int G>
__global__ __launch_bounds__(64 * conv_bwd_waves<KT>()) void conv_silu_bwd_kernel(const ConvBwdArgs<T> a) {
  using C = typename ComputeOf<T>::type;
  typedef T vec_t __attribute__((ext_vector_type(VEC)));
  constexpr int KM = KT > 0 ? KT : kConvBwdMaxK;
  constexpr int R = kConvBwdRun, NW = conv_bwd_waves<KT>();
  constexpr int NSTEP = R + 2 * (KM - 1);  // positions walked per run
  __shared__ C red[NW / 2][64 * VEC * (KM + 1)];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t nblk = (a.nc + 64 * VEC - 1) / (64 * VEC);
  const int64_t runs = conv_bwd_runs(a.nt);
  const int64_t rgroups = (runs + NW - 1) / NW;  // a block takes NW consecutive runs of one channel block
  const int64_t bid = blockIdx.x;
  const int64_t rg = bid % rgroups;
  const int64_t cb = (bid / rgroups) % nblk;
  const int64_t b = bid / (rgroups * nblk);
  const int64_t t0 = (rg * NW + wv) * R;
  const int64_t c0 = (cb * 64 + lane) * VEC;
  const bool on = c0 < a.nc;
  const int K = KT > 0 ? KT : a.K;
  const int H1 = K - 1;
  int64_t len = a.nt;
  if (a.valid_lens != nullptr) {
    const int64_t vl = a.valid_lens[b];
    len = vl < 0 ? 0 : (vl < a.nt ? vl : a.nt);
  }
  auto row = [&](const T* base, int64_t r) -> vec_t { return *reinterpret_cast<const vec_t*>(base + r * a.nc + c0); };
  C wr[KM][VEC], br[VEC], gw[KM][VEC], gb[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      wr[j][e] = (on && j < K) ? to_compute<C>(a.w[(c0 + e) * K + j]) : C(0);
      gw[j][e] = C(0);
    }
    br[e] = (on && a.bias != nullptr) ? to_compute<C>(a.bias[c0 + e]) : C(0);
    gb[e] = C(0);
  }
  if (t0 < a.nt) {  // uniform over the wave
    C xw[KM][VEC], pw[KM][VEC];  // x_{t-KM+1} .. x_t and dpre_{t-KM+1} .. dpre_t
#pragma unroll
    for (int j = 0; j < KM; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) xw[j][e] = pw[j][e] = C(0);
#pragma unroll 1
    for (int i = 0; i < NSTEP; ++i) {
      const int64_t t = t0 - (KM - 1) + i;
      // x_t (the history below 0, zero past len)
      vec_t xv = {};
      if (on) {
        if (t >= 0 && t < len)
          xv = row(a.x, b * a.nt + t);
        else if (t < 0 && t >= -H1 && a.hist_in != nullptr)
          xv = row(a.hist_in, b * H1 + H1 + t);
      }
#pragma unroll
      for (int j = 0; j < KM - 1; ++j)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          xw[j][e] = xw[j + 1][e];
          pw[j][e] = pw[j + 1][e];
        }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        xw[KM - 1][e] = to_compute<C>(xv[e]);
        pw[KM - 1][e] = C(0);
      }
      if (i >= KM - 1) {  // t >= t0: dpre_t
        const bool real = t < len;  // uniform over the wave
        C pre[VEC], act[VEC], sg[VEC], da[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          C acc = br[e];
#pragma unroll
          for (int j = 0; j < KM; ++j) acc += wr[j][e] * xw[KM - 1 - j][e];
          pre[e] = acc;
          sg[e] = sigmoid(acc);
          act[e] = acc * sg[e];
        }
        vec_t dv = {};
        if (on && real) dv = row(a.dy, b * a.nt + t);
        if constexpr (G > 0) {
          C ss = C(0), yd = C(0);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ss += act[e] * act[e];
            yd += act[e] * to_compute<C>(dv[e]);
          }
          ss = group_sum<G>(ss);
          yd = group_sum<G>(yd);
          const C eps = C(a.eps);
          if (ss > eps * eps) {
            const C inv = frsqrt(ss);  // 1 / ||a||
#pragma unroll
            for (int e = 0; e < VEC; ++e) da[e] = (to_compute<C>(dv[e]) - act[e] * yd * inv * inv) * inv;
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) da[e] = to_compute<C>(dv[e]) / eps;
          }
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) da[e] = to_compute<C>(dv[e]);
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) pw[KM - 1][e] = real ? da[e] * sg[e] * (C(1) + pre[e] * (C(1) - sg[e])) : C(0);
        if (i < KM - 1 + R) {  // t in the run
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            gb[e] += pw[KM - 1][e];
#pragma unroll
            for (int j = 0; j < KM; ++j) gw[j][e] += pw[KM - 1][e] * xw[KM - 1 - j][e];
          }
        }
      }
      // s = t - (KM-1): dx_s = sum_j w[j] dpre_{s+j} (+ the next history's gradient)
      const int64_t s = t - (KM - 1);
      if (i >= 2 * (KM - 1)) {  // s >= t0
        if (s < a.nt) {
          vec_t hv = {};
          const bool to_hist = a.dhist_out != nullptr && s < len && s >= len - H1;
          if (on && to_hist) hv = row(a.dhist_out, b * H1 + (s - (len - H1)));
          vec_t o;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            C acc = to_compute<C>(hv[e]);
#pragma unroll
            for (int j = 0; j < KM; ++j) acc += wr[j][e] * pw[j][e];
            o[e] = from_compute<T>(acc);
          }
          if (on) *reinterpret_cast<vec_t*>(a.dx + (b * a.nt + s) * a.nc + c0) = o;
        }
      } else if (t0 == 0 && s >= -H1 && a.dhist_in != nullptr && on) {
        // history row m = s + H1 (position s < 0)
        const int64_t m = s + H1, q = m - len;  // its row in the next history, if it stays there
        vec_t hv = {};
        if (a.dhist_out != nullptr && q >= 0 && q < H1) hv = row(a.dhist_out, b * H1 + q);
        vec_t o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          C acc = to_compute<C>(hv[e]);
#pragma unroll
          for (int j = 0; j < KM; ++j) acc += wr[j][e] * pw[j][e];
          o[e] = from_compute<T>(acc);
        }
        *reinterpret_cast<vec_t*>(a.dhist_in + (b * H1 + m) * a.nc + c0) = o;
      }
    }
  }
  // sum the waves' weight and bias gradients in a fixed order (the upper half
  // onto the lower, then the lower half per element), then one atomic per
  // element and block
  if (a.dw != nullptr || a.dbias != nullptr) {
    if (wv >= NW / 2) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
#pragma unroll
        for (int j = 0; j < KM; ++j) red[wv - NW / 2][(j * 64 + lane) * VEC + e] = gw[j][e];
        red[wv - NW / 2][(KM * 64 + lane) * VEC + e] = gb[e];
      }
    }
    __syncthreads();
    if (wv < NW / 2) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
#pragma unroll
        for (int j = 0; j < KM; ++j) red[wv][(j * 64 + lane) * VEC + e] += gw[j][e];
        red[wv][(KM * 64 + lane) * VEC + e] += gb[e];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < 64 * VEC * (KM + 1); idx += 64 * NW) {
      C sum = red[0][idx];
#pragma unroll
      for (int u = 1; u < NW / 2; ++u) sum += red[u][idx];
      const int j = idx / (64 * VEC);
      const int rem = idx % (64 * VEC);
      const int64_t ch = (cb * 64 + rem / VEC) * VEC + rem % VEC;
      if (ch >= a.nc) continue;
      if (j < KM) {
        if (j < K && a.dw != nullptr) atomic_add(a.dw + ch * K + j, sum);
      } else if (a.dbias != nullptr) {
        atomic_add(a.dbias + ch, sum);
      }
    }
  }
}

}  // namespace fbwd
}  // namespace kda

namespace kda_host {

using namespace kda;
using kda::fbwd::ComputeOf;

static bool aligned16b(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

static int dtype_bytes(int dtype) {
  switch (dtype) {
    case KDA_DTYPE_BF16:
    case KDA_DTYPE_F16: return 2;
    case KDA_DTYPE_F32: return 4;
    case KDA_DTYPE_F64: return 8;
    default: return 0;
  }
}

// ---- conv ----
template <class T, int VEC, int KT>
static bool conv_bwd_g(const fbwd::ConvBwdArgs<T>& a, int g, dim3 grid, hipStream_t s) {
  switch (g) {
#define KDA_CONV_BWD_CASE(GG)                                                                  \
  case GG:                                                                                     \
    hipLaunchKernelGGL((fbwd::conv_silu_bwd_kernel<T, VEC, KT, GG>), grid, dim3(64 * fbwd::conv_bwd_waves<KT>()), 0, s, \
                       a);                                                                                   \
    return true;
    KDA_CONV_BWD_CASE(0)
    KDA_CONV_BWD_CASE(2)
    KDA_CONV_BWD_CASE(4)
    KDA_CONV_BWD_CASE(8)
    KDA_CONV_BWD_CASE(16)
    KDA_CONV_BWD_CASE(32)
    KDA_CONV_BWD_CASE(64)
#undef KDA_CONV_BWD_CASE
    default: return false;
  }
}

template <class T>
static int run_conv_bwd(const fbwd::ConvBwdArgs<T>& a, int g, hipStream_t stream) {
  constexpr int VEC = sizeof(T) == 8 ? 2 : 4;
  const int64_t nblk = (a.nc + 64 * VEC - 1) / (64 * VEC);
  const int nw = a.K == 4 ? fbwd::conv_bwd_waves<4>() : fbwd::conv_bwd_waves<0>();  // waves per block
  const int64_t rgroups = (fbwd::conv_bwd_runs(a.nt) + nw - 1) / nw;
  const int64_t blocks = a.nb * nblk * rgroups;
  if (blocks == 0) return KDA_OK;
  if (blocks > 0x7fffffffLL) {
    set_detail("conv_silu_bwd: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  const dim3 grid(static_cast<unsigned>(blocks));
  const bool ok = a.K == 4 ? conv_bwd_g<T, VEC, 4>(a, g, grid, stream) : conv_bwd_g<T, VEC, 0>(a, g, grid, stream);
  if (!ok) {
    set_detail("conv_silu_bwd: no kernel for %d lanes per head", g);
    return KDA_ERR_UNSUPPORTED;
  }
  return check_launch("conv_silu_bwd_kernel");
}

int launch_conv_silu_bwd(const void* x, const void* w, const void* bias, const void* hist_in,
                         const int32_t* valid_lens, const void* dy, const void* dhist_out, void* dx, void* dhist_in,
                         void* dw, void* dbias, int64_t B, int64_t T, int64_t C, int64_t K, int64_t head_dim,
                         int normalize, double eps, int dtype, hipStream_t stream) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) {
    set_detail("conv_silu_bwd: unknown dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  const int vec = eb == 8 ? 2 : 4;
  int g = 0;
  if (normalize) {
    if (head_dim < 16 || (head_dim & (head_dim - 1)) != 0 || head_dim / vec > 64) {
      set_detail("conv_silu_bwd: normalised head_dim %lld must be a power of two in 16..%d", (long long)head_dim,
                 64 * vec);
      return KDA_ERR_UNSUPPORTED;
    }
    g = static_cast<int>(head_dim / vec);
  }
  if (C % vec != 0) {
    set_detail("conv_silu_bwd: channels %lld must be a multiple of %d", (long long)C, vec);
    return KDA_ERR_UNSUPPORTED;
  }
  if (K < 1 || K > fbwd::kConvBwdMaxK) {
    set_detail("conv_silu_bwd: kernel_size %lld outside 1..%d", (long long)K, fbwd::kConvBwdMaxK);
    return KDA_ERR_UNSUPPORTED;
  }
  for (const void* p : {x, hist_in, dy, dhist_out, static_cast<const void*>(dx), static_cast<const void*>(dhist_in)})
    if (!aligned16b(p)) {
      set_detail("conv_silu_bwd: activations, gradients and histories must be 16-byte aligned");
      return KDA_ERR_INVALID_ARGUMENT;
    }
  const int k = static_cast<int>(K);
  const float e = static_cast<float>(eps);
#define KDA_CONV_BWD_RUN(TT)                                                                                       \
  return run_conv_bwd(                                                                                             \
      fbwd::ConvBwdArgs<TT>{static_cast<const TT*>(x), static_cast<const TT*>(w), static_cast<const TT*>(bias),   \
                            static_cast<const TT*>(hist_in), valid_lens, static_cast<const TT*>(dy),             \
                            static_cast<const TT*>(dhist_out), static_cast<TT*>(dx), static_cast<TT*>(dhist_in),  \
                            static_cast<typename ComputeOf<TT>::type*>(dw),                                      \
                            static_cast<typename ComputeOf<TT>::type*>(dbias), B, T, C, k, e},                   \
      g, stream)
  switch (dtype) {
    case KDA_DTYPE_BF16: KDA_CONV_BWD_RUN(bf16);
    case KDA_DTYPE_F16: KDA_CONV_BWD_RUN(f16);
    case KDA_DTYPE_F32: KDA_CONV_BWD_RUN(float);
    default: KDA_CONV_BWD_RUN(double);
  }
#undef KDA_CONV_BWD_RUN
}

// ---- gates ----
static float gate_eps(int dtype) {
  switch (dtype) {
    case KDA_DTYPE_BF16: return 0.0078125f;
    case KDA_DTYPE_F16: return 0.0009765625f;
    case KDA_DTYPE_F32: return 1.1920928955078125e-07f;
    default: return 2.220446049250313e-16f;
  }
}

template <class T>
static int run_gates_bwd(const fbwd::GateBwdArgs<T>& a, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T);
  dim3 grid(1, 1);
  constexpr int NT = fbwd::kGatePos * fbwd::kGateRowGroups;
  if (a.z != nullptr) {
    // about 256 blocks: one per CU, each over a contiguous range of rows
    const int64_t bx = (a.H * a.K / VEC + fbwd::kGatePos - 1) / fbwd::kGatePos;
    int64_t by = 256 / (bx > 0 ? bx : 1);
    if (by < 1) by = 1;
    if (by > a.rows) by = a.rows;
    if (by > 65535) by = 65535;
    if (bx > 0x7fffffffLL) {
      set_detail("gates_bwd: grid too large");
      return KDA_ERR_UNSUPPORTED;
    }
    grid = dim3(static_cast<unsigned>(bx), static_cast<unsigned>(by));
  } else {
    const int64_t n = a.rows * a.H;
    int64_t bx = (n + NT - 1) / NT;
    if (bx > 1024) bx = 1024;
    grid = dim3(static_cast<unsigned>(bx > 0 ? bx : 1), 1);
  }
  hipLaunchKernelGGL((fbwd::gates_bwd_kernel<T>), grid, dim3(NT), 0, stream, a);
  return check_launch("gates_bwd_kernel");
}

int launch_gates_bwd(const void* z, const void* zbias, const float* a_log, double g_min, const void* dg,
                     const void* dalpha, void* dz, void* dzbias, void* da_log, const void* bl, const void* dbeta,
                     void* dbl, int64_t rows, int64_t H, int64_t K, int dtype, hipStream_t stream) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) {
    set_detail("gates_bwd: unknown dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (z != nullptr) {
    if ((K * eb) % 16 != 0) {
      set_detail("gates_bwd: key_dim %lld must be a multiple of %d", (long long)K, 16 / eb);
      return KDA_ERR_UNSUPPORTED;
    }
    for (const void* p : {z, zbias, dg, dalpha, static_cast<const void*>(dz)})
      if (!aligned16b(p)) {
        set_detail("gates_bwd: logits, bias and gradients must be 16-byte aligned");
        return KDA_ERR_INVALID_ARGUMENT;
      }
    if (dg == nullptr || dz == nullptr || a_log == nullptr) {
      set_detail("gates_bwd: decay logits need d_g, d_decay_logits and a_log");
      return KDA_ERR_INVALID_ARGUMENT;
    }
  }
  if (bl != nullptr && (dbeta == nullptr || dbl == nullptr)) {
    set_detail("gates_bwd: beta logits need d_beta and d_beta_logits");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  const float eps = gate_eps(dtype);
  const float gm = static_cast<float>(g_min);
#define KDA_GATES_BWD_RUN(TT)                                                                                      \
  return run_gates_bwd(                                                                                            \
      fbwd::GateBwdArgs<TT>{static_cast<const TT*>(z), static_cast<const TT*>(zbias), a_log,                      \
                            static_cast<const TT*>(dg), static_cast<const TT*>(dalpha), static_cast<TT*>(dz),     \
                            static_cast<typename ComputeOf<TT>::type*>(dzbias),                                  \
                            static_cast<typename ComputeOf<TT>::type*>(da_log), static_cast<const TT*>(bl),       \
                            static_cast<const TT*>(dbeta), static_cast<TT*>(dbl), rows, H, K, gm, eps},           \
      stream)
  switch (dtype) {
    case KDA_DTYPE_BF16: KDA_GATES_BWD_RUN(bf16);
    case KDA_DTYPE_F16: KDA_GATES_BWD_RUN(f16);
    case KDA_DTYPE_F32: KDA_GATES_BWD_RUN(float);
    default: KDA_GATES_BWD_RUN(double);
  }
#undef KDA_GATES_BWD_RUN
}

// ---- rmsnorm ----

template <class T, int VEC, int G>
static int run_norm_bwd(fbwd::NormBwdArgs<T> a, hipStream_t stream) {
  constexpr int per_block = 256 / G;  // lane groups (rows) per block
  // about 1024 blocks: H heads x row_blocks stripes of rows
  int64_t rb = 1024 / (a.H > 0 ? a.H : 1);
  if (rb < 1) rb = 1;
  const int64_t need = (a.rows + per_block - 1) / per_block;
  if (rb > need) rb = need;
  if (rb < 1) rb = 1;
  a.row_blocks = rb;
  const int64_t blocks = a.H * rb;
  if (blocks > 0x7fffffffLL) {
    set_detail("rmsnorm_gate_bwd: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((fbwd::rmsnorm_gate_bwd_kernel<T, VEC, G>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     stream, a);
  return check_launch("rmsnorm_gate_bwd_kernel");
}

template <class T, int VEC>
static int norm_bwd_g(const fbwd::NormBwdArgs<T>& a, int g, hipStream_t s) {
  switch (g) {
    case 2: return run_norm_bwd<T, VEC, 2>(a, s);
    case 4: return run_norm_bwd<T, VEC, 4>(a, s);
    case 8: return run_norm_bwd<T, VEC, 8>(a, s);
    case 16: return run_norm_bwd<T, VEC, 16>(a, s);
    case 32: return run_norm_bwd<T, VEC, 32>(a, s);
    case 64: return run_norm_bwd<T, VEC, 64>(a, s);
    default:
      set_detail("rmsnorm_gate_bwd: no kernel for %d lanes per head", g);
      return KDA_ERR_UNSUPPORTED;
  }
}

template <class T>
static int norm_bwd_vec(const fbwd::NormBwdArgs<T>& a, int vec, int g, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  if (vec == V) return norm_bwd_g<T, V>(a, g, s);
  if constexpr (sizeof(T) >= 4)
    if (vec == 2 * V) return norm_bwd_g<T, 2 * V>(a, g, s);
  if constexpr (sizeof(T) == 8)
    if (vec == 4 * V) return norm_bwd_g<T, 4 * V>(a, g, s);
  set_detail("rmsnorm_gate_bwd: no kernel for %d elements per lane", vec);
  return KDA_ERR_UNSUPPORTED;
}

int launch_rmsnorm_gate_bwd(const void* x, const void* w, int w_per_head, const void* gl, const void* dy, void* dx,
                            void* dgl, void* dw, int64_t rows, int64_t H, int64_t D, double eps, int dtype,
                            hipStream_t stream) {
  const int eb = dtype_bytes(dtype);
  if (eb == 0) {
    set_detail("rmsnorm_gate_bwd: unknown dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (D < 16 || D > 512 || (D & (D - 1)) != 0) {
    set_detail("rmsnorm_gate_bwd: head_dim %lld must be a power of two in 16..512", (long long)D);
    return KDA_ERR_UNSUPPORTED;
  }
  int vec = 16 / eb;
  if (D / vec > 64) vec = static_cast<int>(D / 64);
  const int g = static_cast<int>(D / vec);
  for (const void* p : {x, w, gl, dy, static_cast<const void*>(dx), static_cast<const void*>(dgl)})
    if (!aligned16b(p)) {
      set_detail("rmsnorm_gate_bwd: tensors must be 16-byte aligned");
      return KDA_ERR_INVALID_ARGUMENT;
    }
  if (rows * H == 0) return KDA_OK;
  const float e = static_cast<float>(eps);
#define KDA_NORM_BWD_RUN(TT)                                                                                      \
  return norm_bwd_vec(                                                                                            \
      fbwd::NormBwdArgs<TT>{static_cast<const TT*>(x), static_cast<const TT*>(w), w_per_head,                    \
                            static_cast<const TT*>(gl), static_cast<const TT*>(dy), static_cast<TT*>(dx),        \
                            static_cast<TT*>(dgl), static_cast<typename ComputeOf<TT>::type*>(dw), rows, H, 0, e}, \
      vec, g, stream)
  switch (dtype) {
    case KDA_DTYPE_BF16: KDA_NORM_BWD_RUN(bf16);
    case KDA_DTYPE_F16: KDA_NORM_BWD_RUN(f16);
    case KDA_DTYPE_F32: KDA_NORM_BWD_RUN(float);
    default: KDA_NORM_BWD_RUN(double);
  }
#undef KDA_NORM_BWD_RUN
}

}  // namespace kda_host
