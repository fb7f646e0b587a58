// Fused elementwise stages around the KDA operator on gfx950: the ShortConv +
// SiLU (+ per-head L2 normalisation) that turns the q/k/v projections into
// operator inputs, the lower-bounded decay and beta gates, and the head-wise
// RMSNorm with the output-gate product.  Each is one HBM stream: every input
// element is read once and every output element written once, arithmetic in
// f32 (f64 for f64 tensors) with one rounding to the output type.
#include <math.h>

#include "kda_launch.h"

namespace kda {

template <class T>
struct ComputeOf {
  using type = float;
};
template <>
struct ComputeOf<double> {
  using type = double;
};

// Blocks b and b + 8 run on the same XCD (the dispatcher deals blocks to the
// eight XCDs in turn); this renumbering gives each XCD one contiguous range
// of logical blocks, so neighbouring tiles share their XCD's L2.
__device__ __forceinline__ int64_t xcd_block(unsigned b, unsigned nb) {
  const unsigned per = nb / 8, rem = nb % 8, x = b % 8;
  return static_cast<int64_t>(x) * per + (x < rem ? x : rem) + b / 8;
}

// A lane moves VEC consecutive elements of a row per load and store: 16
// bytes (VEC = 16 / sizeof(T)) unless a head is wider than 64 such vectors,
// in which case the vector grows to head_dim / 64 elements.
template <class T, int VEC>
struct Vec {
  typedef T type __attribute__((ext_vector_type(VEC)));
};

// ---- ShortConv + SiLU (+ L2 normalisation per head) -------------------------
// Reference: CausalShortConv1D (src/kimi_primitives/short_conv.py:69-98:
// weight[c, j] multiplies x[t - j]; the history holds the last K-1 inputs,
// oldest first), KDAProjections._run_conv (src/kda/projections.py:100-140: a
// right-padded row runs on its valid prefix, its padded outputs are zero and
// the padding never enters the history), then F.silu and, for q and k,
// F.normalize(p=2, dim=-1, eps) per head (projections.py:185-204).
//
// One wave per (batch row, block of 64*VEC channels, tile of 16 tokens).
// Lane l owns the VEC channels blk*64*VEC + VEC*l .. (one 16-byte load per
// token).  The wave streams its tile: eight rows in flight ahead of the one
// it forms, the K-1 rows before it in a register window, one store per row,
// so its loads, arithmetic and stores overlap.  With normalisation a head is
// an aligned group of G = head_dim / VEC lanes, and its sum of squares a
// G-lane reduction.
constexpr int kMaxConvK = 8;

// tokens per wave: 16, or 4 when a lane's vector is wider than 16 bytes
__host__ __device__ constexpr int conv_tile(int vec_bytes) { return vec_bytes > 16 ? 4 : 16; }

template <class T>
struct ConvArgs {
  const T* x;        // [B, T, C]
  const T* w;        // [C, K]
  const T* bias;     // [C] or null
  const T* hist_in;  // [B, K-1, C] or null (zeros)
  T* y;              // [B, T, C]
  T* hist_out;       // [B, K-1, C] or null
  const int32_t* valid_lens;  // [B] or null
  int64_t nb, nt, nc;  // batch, tokens, channels
  int K;
  float eps;
};

// VEC: channels per lane; KT: the kernel size, or 0 for any K <= kMaxConvK;
// G: lanes per normalised head (0: no normalisation).
template <class T, int VEC, int KT, int G>
__global__ __launch_bounds__(256) void conv_silu_kernel(const ConvArgs<T> a) {
  using C = typename ComputeOf<T>::type;
  typedef typename Vec<T, VEC>::type vec_t;
  constexpr int TT = conv_tile(VEC * sizeof(T));
  constexpr int D = TT < 8 ? TT : 8;              // rows in flight ahead of the one being formed
  constexpr int KMAX = KT > 0 ? KT : kMaxConvK;  // taps held in registers
  const int lane = threadIdx.x & 63;
  // the wave's tile, batch row and channel block are scalars (the wave index
  // read through readfirstlane), so row addresses are a scalar base plus the
  // lane's 32-bit channel offset
  const int64_t wave = xcd_block(blockIdx.x, gridDim.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nblk = (a.nc + 64 * VEC - 1) / (64 * VEC);
  const int64_t ntile = (a.nt + TT - 1) / TT;
  if (wave >= a.nb * nblk * ntile) return;  // uniform over the wave
  const int64_t tile = wave % ntile;
  const int64_t blk = (wave / ntile) % nblk;
  const int64_t b = wave / (ntile * nblk);
  const int c0 = static_cast<int>(blk * 64 * VEC) + lane * VEC;
  const bool on = c0 < a.nc;  // lanes past the last channel only join the reductions
  int64_t len = a.nt;
  if (a.valid_lens != nullptr) {
    const int vl = __builtin_amdgcn_readfirstlane(a.valid_lens[b]);
    len = vl < 0 ? 0 : (vl < a.nt ? vl : a.nt);
  }
  const int K = KT > 0 ? KT : a.K;
  const int H1 = K - 1;
  const int64_t t0 = tile * TT;
  const vec_t zero = {};
  const T* xb = a.x + b * a.nt * a.nc;  // uniform
  auto row = [&](const T* base, int64_t r) -> vec_t { return *reinterpret_cast<const vec_t*>(base + r * a.nc + c0); };
  // row t of x for t < nt (the address clamped into the row's span; the
  // caller masks what lies past the valid prefix), so the loads of the ring
  // are unconditional and their waits exact; streamed data, so non-temporal
  auto ld = [&](int64_t t) -> vec_t {
    return __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(xb + (t < a.nt ? t : a.nt - 1) * a.nc + c0));
  };
  C wr[KMAX][VEC];
  C br[VEC];
  if constexpr (KT > 0) {
    // the lane's VEC channels x KT taps are VEC*KT consecutive weights: KT vectors
    vec_t wv[KT];
#pragma unroll
    for (int j = 0; j < KT; ++j) wv[j] = on ? *reinterpret_cast<const vec_t*>(a.w + c0 * KT + j * VEC) : zero;
#pragma unroll
    for (int e = 0; e < VEC; ++e)
#pragma unroll
      for (int j = 0; j < KT; ++j) wr[j][e] = to_compute<C>(wv[(e * KT + j) / VEC][(e * KT + j) % VEC]);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e)
#pragma unroll
      for (int j = 0; j < KMAX; ++j) wr[j][e] = (on && j < K) ? to_compute<C>(a.w[(c0 + e) * K + j]) : C(0);
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) br[e] = (on && a.bias != nullptr) ? to_compute<C>(a.bias[c0 + e]) : C(0);
  // the ring of rows in flight: ring[i % D] holds row t0 + i
  vec_t ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d) ring[d] = on ? ld(t0 + d) : zero;
  // the window: win[j] = x[t - 1 - j] in the compute type, zero past the valid prefix
  C win[KMAX > 1 ? KMAX - 1 : 1][VEC];
#pragma unroll
  for (int j = 0; j < KMAX - 1; ++j) {
    const int64_t p = t0 - 1 - j;
    vec_t v = zero;
    if (on && j < H1) {
      if (p >= 0)
        v = p < len ? row(xb, p) : zero;
      else if (a.hist_in != nullptr)
        v = row(a.hist_in, b * H1 + H1 + p);
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) win[j][e] = to_compute<C>(v[e]);
  }
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    const int64_t t = t0 + i;
    if (t >= a.nt) break;  // uniform
    const vec_t raw = ring[i % D];
    if (i + D < TT) ring[i % D] = on ? ld(t + D) : zero;
    const bool valid = t < len;  // uniform
    C xcur[VEC], out[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) xcur[e] = valid ? to_compute<C>(raw[e]) : C(0);
    if (valid) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        C acc = br[e] + wr[0][e] * xcur[e];
#pragma unroll
        for (int j = 1; j < KMAX; ++j) acc += wr[j][e] * win[j - 1][e];
        out[e] = acc * sigmoid(acc);  // SiLU
      }
    } else {  // zero past the valid prefix
#pragma unroll
      for (int e = 0; e < VEC; ++e) out[e] = C(0);
    }
#pragma unroll
    for (int j = KMAX - 2; j > 0; --j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) win[j][e] = win[j - 1][e];
    if constexpr (KMAX > 1) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) win[0][e] = xcur[e];
    }
    if constexpr (G > 0) {
      C ss = C(0);
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss += out[e] * out[e];
      ss = group_sum<G>(ss);
      const C e = C(a.eps);
      const C inv = ss > e * e ? frsqrt(ss) : C(1) / e;  // 1 / max(||y||, eps)
#pragma unroll
      for (int e = 0; e < VEC; ++e) out[e] *= inv;
    }
    if (on) {
      vec_t o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = from_compute<T>(out[e]);
      T* yrow = a.y + (b * a.nt + t) * a.nc;  // uniform
      __builtin_nontemporal_store(o, reinterpret_cast<vec_t*>(yrow + c0));
    }
  }
  // next history: the last K-1 rows of [history | valid prefix]
  if (a.hist_out != nullptr && tile == 0 && on) {
    for (int j = 0; j < H1; ++j) {
      const int64_t p = len + j - H1;  // position relative to the first token
      vec_t val = zero;
      if (p >= 0)
        val = row(xb, p);
      else if (a.hist_in != nullptr)
        val = row(a.hist_in, b * H1 + H1 + p);
      *reinterpret_cast<vec_t*>(a.hist_out + (b * H1 + j) * a.nc + c0) = val;
    }
  }
}

// ---- lower-bounded decay and beta gates --------------------------------------
// Reference: LowerBoundedDecay.forward (src/kda/decay.py:30-43):
//   g = g_min * clamp(sigmoid(exp(A_log[h]) * z), eps, 1 - eps),  alpha = exp(g),
// with z = decay logits + b_alpha (src/kda/projections.py:211-218); and the
// beta gate clamp(sigmoid(logits), eps, 1 - eps) (projections.py:207-209).
// eps is the machine epsilon of the tensors' type.  A thread takes one
// 16-byte vector of logits per step; key_dim is a multiple of the vector, so
// the vector lies in one head.
template <class T>
struct GateArgs {
  const T* z;         // [rows, H, K] or null
  const T* zbias;     // [H, K] or null
  const float* a_log; // [H]
  T* g;               // [rows, H, K]
  T* alpha;           // [rows, H, K] or null
  const T* bl;        // [rows, H] or null
  T* beta;            // [rows, H]
  int64_t rows, H, K;
  float g_min, eps;
};

constexpr int kGateRows = 4;  // rows of decay logits per thread

template <class T>
__global__ __launch_bounds__(256) void gates_kernel(const GateArgs<T> a) {
  using C = typename ComputeOf<T>::type;
  constexpr int VEC = 16 / sizeof(T);
  typedef typename Vec<T, VEC>::type vec_t;
  const C lo = C(a.eps), hi = C(1) - C(a.eps);
  // decay: thread (blockIdx.x, tid) owns vector v of every row's [H, K]
  // block, so its A_log scale and bias are fixed; blockIdx.y takes
  // kGateRows rows at a time
  if (a.z != nullptr) {
    const int64_t hkv = a.H * a.K / VEC;
    const int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (v < hkv) {
      const C scale = fexp(static_cast<C>(a.a_log[v * VEC / a.K]));
      vec_t bv = {};
      if (a.zbias != nullptr) bv = *reinterpret_cast<const vec_t*>(a.zbias + v * VEC);
      for (int64_t r0 = static_cast<int64_t>(blockIdx.y) * kGateRows; r0 < a.rows;
           r0 += static_cast<int64_t>(gridDim.y) * kGateRows) {
        vec_t zv[kGateRows];
#pragma unroll
        for (int u = 0; u < kGateRows; ++u)  // all loads before the first store
          zv[u] = r0 + u < a.rows
                      ? __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(a.z + ((r0 + u) * hkv + v) * VEC))
                      : vec_t{};
#pragma unroll
        for (int u = 0; u < kGateRows; ++u) {
          if (r0 + u >= a.rows) break;
          const int64_t e0 = ((r0 + u) * hkv + v) * VEC;
          vec_t gv, av;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const C gg = lower_bounded_decay(to_compute<C>(zv[u][e]), to_compute<C>(bv[e]), scale, C(a.g_min), lo, hi);
            gv[e] = from_compute<T>(gg);
            av[e] = from_compute<T>(fexp(gg));
          }
          __builtin_nontemporal_store(gv, reinterpret_cast<vec_t*>(a.g + e0));
          if (a.alpha != nullptr) __builtin_nontemporal_store(av, reinterpret_cast<vec_t*>(a.alpha + e0));
        }
      }
    }
  }
  // beta: a grid-stride loop over all threads of the grid
  if (a.bl != nullptr) {
    const int64_t n = a.rows * a.H;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * gridDim.y * blockDim.x;
    for (int64_t j = (static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; j < n;
         j += stride) {
      C p = sigmoid(to_compute<C>(a.bl[j]));
      p = p < lo ? lo : (p > hi ? hi : p);
      a.beta[j] = from_compute<T>(p);
    }
  }
}

// ---- head-wise RMSNorm with the output-gate product -----------------------------
// Reference: HeadwiseRMSNorm.forward (src/kimi_primitives/headwise_rmsnorm.py:39-64:
// x * rsqrt(mean(x^2 over the head) + eps), accumulated in f32 for 16-bit
// inputs, times the per-head or shared weight) and the product gate * output
// of FullRankOutputGate.forward (src/kimi_primitives/output_gate.py:62-75,
// gate = sigmoid(gate_proj(residual))) that feeds output_proj.  A (row, head)
// is an aligned group of G = head_dim / VEC lanes, each moving VEC elements
// of x, of the gate logits and of y; a group takes kNormPairs pairs, with
// every load issued before the first reduction.
template <class T>
struct NormArgs {
  const T* x;    // [rows, H, D]
  const T* w;    // [H, D], [D] or null
  int w_per_head;
  const T* gl;   // gate logits [rows, H*D] or null
  T* y;          // [rows, H, D]
  int64_t rows, H;
  float eps;
};

constexpr int kNormPairs = 4;  // (row, head) pairs per lane group

template <class T, int VEC, int G>
__global__ __launch_bounds__(256) void rmsnorm_gate_kernel(const NormArgs<T> a) {
  using C = typename ComputeOf<T>::type;
  constexpr int D = G * VEC;
  constexpr int GW = 64 / G;  // lane groups per wave
  typedef typename Vec<T, VEC>::type vec_t;
  const int lane = threadIdx.x & 63;
  const int k = lane % G;
  const int64_t n = a.rows * a.H;
  // the wave's pairs are contiguous: step u takes pairs first + u*GW + lane/G
  const int64_t first = ((static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / 64) * GW * kNormPairs + lane / G;
  vec_t xv[kNormPairs], gv[kNormPairs];
#pragma unroll
  for (int u = 0; u < kNormPairs; ++u) {  // all loads first; streamed data, so non-temporal
    const int64_t pair = first + u * GW;
    xv[u] = pair < n ? __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(a.x + pair * D + k * VEC)) : vec_t{};
    if (a.gl != nullptr)
      gv[u] = pair < n ? __builtin_nontemporal_load(reinterpret_cast<const vec_t*>(a.gl + pair * D + k * VEC)) : vec_t{};
  }
#pragma unroll
  for (int u = 0; u < kNormPairs; ++u) {
    const int64_t pair = first + u * GW;
    C ss = C(0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += to_compute<C>(xv[u][e]) * to_compute<C>(xv[u][e]);
    ss = group_sum<G>(ss);  // every lane takes part; groups past n hold zeros
    if (pair >= n) continue;
    const C r = frsqrt(ss / C(D) + C(a.eps));
    vec_t wv;
    if (a.w != nullptr) wv = *reinterpret_cast<const vec_t*>(a.w + (a.w_per_head ? (pair % a.H) * D : 0) + k * VEC);
    vec_t o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      C v = to_compute<C>(xv[u][e]) * r;
      if (a.w != nullptr) v *= to_compute<C>(wv[e]);
      if (a.gl != nullptr) v *= sigmoid(to_compute<C>(gv[u][e]));
      o[e] = from_compute<T>(v);
    }
    __builtin_nontemporal_store(o, reinterpret_cast<vec_t*>(a.y + pair * D + k * VEC));
  }
}

}  // namespace kda

namespace kda_host {

using namespace kda;

static int elem_bytes(int dtype) {
  switch (dtype) {
    case KDA_DTYPE_BF16:
    case KDA_DTYPE_F16: return 2;
    case KDA_DTYPE_F32: return 4;
    case KDA_DTYPE_F64: return 8;
    default: return 0;
  }
}

static bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

static unsigned waves_to_blocks(int64_t waves) { return static_cast<unsigned>((waves + 3) / 4); }

// Lane layout of a head of D elements: VEC elements per lane (16 bytes, or
// D / 64 when that is larger) and G = D / VEC lanes.  D is a power of two
// in 16..512.
static bool head_layout(int64_t D, int elem_bytes, int* vec, int* g) {
  if (D < 16 || D > 512 || (D & (D - 1)) != 0) return false;
  int v = 16 / elem_bytes;
  if (D / v > 64) v = static_cast<int>(D / 64);
  *vec = v;
  *g = static_cast<int>(D / v);
  return true;
}

template <class T, int VEC, int KT>
static bool conv_launch_g(const ConvArgs<T>& a, int g, dim3 grid, hipStream_t s) {
  switch (g) {
    case 0: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 0>), grid, dim3(256), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 2>), grid, dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 4>), grid, dim3(256), 0, s, a); return true;
    case 8: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 8>), grid, dim3(256), 0, s, a); return true;
    case 16: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 16>), grid, dim3(256), 0, s, a); return true;
    case 32: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 32>), grid, dim3(256), 0, s, a); return true;
    case 64: hipLaunchKernelGGL((conv_silu_kernel<T, VEC, KT, 64>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

template <class T, int KT>
static bool conv_launch_k(const ConvArgs<T>& a, int vec, int g, dim3 grid, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  if (vec == V) return conv_launch_g<T, V, KT>(a, g, grid, s);
  // heads wider than 64 16-byte vectors (f32 512, f64 256 and 512)
  if constexpr (sizeof(T) >= 4)
    if (vec == 2 * V && g == 64) {
      hipLaunchKernelGGL((conv_silu_kernel<T, 2 * V, KT, 64>), grid, dim3(256), 0, s, a);
      return true;
    }
  if constexpr (sizeof(T) == 8)
    if (vec == 4 * V && g == 64) {
      hipLaunchKernelGGL((conv_silu_kernel<T, 4 * V, KT, 64>), grid, dim3(256), 0, s, a);
      return true;
    }
  return false;
}

template <class T>
static int run_conv(const ConvArgs<T>& a, int vec, int g, hipStream_t stream) {
  const int64_t nblk = (a.nc + 64 * vec - 1) / (64 * vec);
  const int tt = conv_tile(vec * static_cast<int>(sizeof(T)));
  const int64_t waves = a.nb * nblk * ((a.nt + tt - 1) / tt);
  if (waves == 0) return KDA_OK;
  if (waves / 4 + 1 > 0x7fffffffLL) {
    set_detail("conv_silu: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  const dim3 grid(waves_to_blocks(waves));
  // kernel size 4 (the usual one) with 16-byte aligned weights loads them as vectors
  const bool ok = a.K == 4 && aligned16(a.w) ? conv_launch_k<T, 4>(a, vec, g, grid, stream)
                                             : conv_launch_k<T, 0>(a, vec, g, grid, stream);
  if (!ok) {
    set_detail("conv_silu: no kernel for %d elements per lane, %d lanes per head", vec, g);
    return KDA_ERR_UNSUPPORTED;
  }
  return check_launch("conv_silu_kernel");
}

int launch_conv_silu(const void* x, const void* w, const void* bias, const void* hist_in, void* y, void* hist_out,
                     const int32_t* valid_lens, int64_t B, int64_t T, int64_t C, int64_t K, int64_t head_dim,
                     int normalize, double eps, int dtype, hipStream_t stream) {
  const int eb = elem_bytes(dtype);
  if (eb == 0) {
    set_detail("conv_silu: unknown dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  int vec = 16 / eb, g = 0;
  if (normalize && !head_layout(head_dim, eb, &vec, &g)) {
    set_detail("conv_silu: normalised head_dim %lld must be a power of two in 16..512", (long long)head_dim);
    return KDA_ERR_UNSUPPORTED;
  }
  if (C % vec != 0) {
    set_detail("conv_silu: channels %lld must be a multiple of %d", (long long)C, vec);
    return KDA_ERR_UNSUPPORTED;
  }
  if (K < 1 || K > kMaxConvK) {
    set_detail("conv_silu: kernel_size %lld outside 1..%d", (long long)K, kMaxConvK);
    return KDA_ERR_UNSUPPORTED;
  }
  // rows of x, y and the histories move as whole vectors
  for (const void* p : {x, hist_in, static_cast<const void*>(y), static_cast<const void*>(hist_out)})
    if (!aligned16(p)) {
      set_detail("conv_silu: x, y and the histories must be 16-byte aligned");
      return KDA_ERR_INVALID_ARGUMENT;
    }
  const int k = static_cast<int>(K);
  const float e = static_cast<float>(eps);
  switch (dtype) {
    case KDA_DTYPE_BF16:
      return run_conv(ConvArgs<bf16>{static_cast<const bf16*>(x), static_cast<const bf16*>(w),
                                     static_cast<const bf16*>(bias), static_cast<const bf16*>(hist_in),
                                     static_cast<bf16*>(y), static_cast<bf16*>(hist_out), valid_lens, B, T, C, k, e},
                      vec, g, stream);
    case KDA_DTYPE_F16:
      return run_conv(ConvArgs<f16>{static_cast<const f16*>(x), static_cast<const f16*>(w),
                                    static_cast<const f16*>(bias), static_cast<const f16*>(hist_in),
                                    static_cast<f16*>(y), static_cast<f16*>(hist_out), valid_lens, B, T, C, k, e},
                      vec, g, stream);
    case KDA_DTYPE_F32:
      return run_conv(ConvArgs<float>{static_cast<const float*>(x), static_cast<const float*>(w),
                                      static_cast<const float*>(bias), static_cast<const float*>(hist_in),
                                      static_cast<float*>(y), static_cast<float*>(hist_out), valid_lens, B, T, C, k, e},
                      vec, g, stream);
    default:
      return run_conv(ConvArgs<double>{static_cast<const double*>(x), static_cast<const double*>(w),
                                       static_cast<const double*>(bias), static_cast<const double*>(hist_in),
                                       static_cast<double*>(y), static_cast<double*>(hist_out), valid_lens, B, T, C,
                                       k, e},
                      vec, g, stream);
  }
}

template <class T>
static int run_gates(const GateArgs<T>& a, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t n_beta = a.bl != nullptr ? a.rows * a.H : 0;
  dim3 grid(1, 1);
  if (a.z != nullptr) {
    if (a.rows == 0) return KDA_OK;
    // x covers one row's [H, K] vectors; y takes kGateRows rows per block
    const int64_t bx = (a.H * a.K / VEC + 255) / 256;
    int64_t by = (a.rows + kGateRows - 1) / kGateRows;
    if (by > 65535) by = 65535;
    if (bx > 0x7fffffffLL) {
      set_detail("gates: grid too large");
      return KDA_ERR_UNSUPPORTED;
    }
    grid = dim3(static_cast<unsigned>(bx), static_cast<unsigned>(by < 1 ? 1 : by));
  } else {
    if (n_beta == 0) return KDA_OK;
    int64_t by = (n_beta + 255) / 256;
    grid = dim3(1, static_cast<unsigned>(by > 65535 ? 65535 : by));
  }
  hipLaunchKernelGGL((gates_kernel<T>), grid, dim3(256), 0, stream, a);
  return check_launch("gates_kernel");
}

static float type_eps(int dtype) {
  switch (dtype) {
    case KDA_DTYPE_BF16: return 0.0078125f;         // 2^-7
    case KDA_DTYPE_F16: return 0.0009765625f;       // 2^-10
    case KDA_DTYPE_F32: return 1.1920928955078125e-07f;  // 2^-23
    default: return 2.220446049250313e-16f;         // 2^-52 (f64)
  }
}

int launch_gates(const void* z, const void* zbias, const float* a_log, double g_min, void* g, void* alpha,
                 const void* bl, void* beta, int64_t rows, int64_t H, int64_t K, int dtype, hipStream_t stream) {
  const int eb = elem_bytes(dtype);
  if (eb == 0) {
    set_detail("gates: unknown dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  const int vec = 16 / eb;
  if (z != nullptr && K % vec != 0) {
    set_detail("gates: key_dim %lld must be a multiple of %d", (long long)K, vec);
    return KDA_ERR_UNSUPPORTED;
  }
  // the decay logits and outputs move as 16-byte vectors
  for (const void* p : {z, zbias, static_cast<const void*>(g), static_cast<const void*>(alpha)})
    if (!aligned16(p)) {
      set_detail("gates: decay logits, their bias, g and alpha must be 16-byte aligned");
      return KDA_ERR_INVALID_ARGUMENT;
    }
  if (z != nullptr && (g == nullptr || a_log == nullptr)) {
    set_detail("gates: decay logits need g and a_log");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (bl != nullptr && beta == nullptr) {
    set_detail("gates: beta logits need beta");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  const float eps = type_eps(dtype);
  const float gm = static_cast<float>(g_min);
  switch (dtype) {
    case KDA_DTYPE_BF16:
      return run_gates(GateArgs<bf16>{static_cast<const bf16*>(z), static_cast<const bf16*>(zbias), a_log,
                                      static_cast<bf16*>(g), static_cast<bf16*>(alpha), static_cast<const bf16*>(bl),
                                      static_cast<bf16*>(beta), rows, H, K, gm, eps},
                       stream);
    case KDA_DTYPE_F16:
      return run_gates(GateArgs<f16>{static_cast<const f16*>(z), static_cast<const f16*>(zbias), a_log,
                                     static_cast<f16*>(g), static_cast<f16*>(alpha), static_cast<const f16*>(bl),
                                     static_cast<f16*>(beta), rows, H, K, gm, eps},
                       stream);
    case KDA_DTYPE_F32:
      return run_gates(GateArgs<float>{static_cast<const float*>(z), static_cast<const float*>(zbias), a_log,
                                       static_cast<float*>(g), static_cast<float*>(alpha),
                                       static_cast<const float*>(bl), static_cast<float*>(beta), rows, H, K, gm, eps},
                       stream);
    case KDA_DTYPE_F64:
      return run_gates(GateArgs<double>{static_cast<const double*>(z), static_cast<const double*>(zbias), a_log,
                                        static_cast<double*>(g), static_cast<double*>(alpha),
                                        static_cast<const double*>(bl), static_cast<double*>(beta), rows, H, K, gm,
                                        eps},
                       stream);
    default:
      set_detail("gates: unknown dtype %d", dtype);
      return KDA_ERR_INVALID_ARGUMENT;
  }
}

template <class T, int VEC>
static bool norm_launch_g(const NormArgs<T>& a, int g, dim3 grid, hipStream_t s) {
  switch (g) {
    case 2: hipLaunchKernelGGL((rmsnorm_gate_kernel<T, VEC, 2>), grid, dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((rmsnorm_gate_kernel<T, VEC, 4>), grid, dim3(256), 0, s, a); return true;
    case 8: hipLaunchKernelGGL((rmsnorm_gate_kernel<T, VEC, 8>), grid, dim3(256), 0, s, a); return true;
    case 16: hipLaunchKernelGGL((rmsnorm_gate_kernel<T, VEC, 16>), grid, dim3(256), 0, s, a); return true;
    case 32: hipLaunchKernelGGL((rmsnorm_gate_kernel<T, VEC, 32>), grid, dim3(256), 0, s, a); return true;
    case 64: hipLaunchKernelGGL((rmsnorm_gate_kernel<T, VEC, 64>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

template <class T>
static int run_norm(const NormArgs<T>& a, int vec, int g, hipStream_t stream) {
  constexpr int V = 16 / sizeof(T);
  const int64_t pairs = a.rows * a.H;
  if (pairs == 0) return KDA_OK;
  const int64_t per_wave = (64 / g) * kNormPairs;
  const int64_t waves = (pairs + per_wave - 1) / per_wave;
  if (waves / 4 + 1 > 0x7fffffffLL) {
    set_detail("rmsnorm_gate: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  const dim3 grid(waves_to_blocks(waves));
  bool ok = false;
  if (vec == V) ok = norm_launch_g<T, V>(a, g, grid, stream);
  if constexpr (sizeof(T) >= 4)
    if (vec == 2 * V && g == 64) {
      hipLaunchKernelGGL((rmsnorm_gate_kernel<T, 2 * V, 64>), grid, dim3(256), 0, stream, a);
      ok = true;
    }
  if constexpr (sizeof(T) == 8)
    if (vec == 4 * V && g == 64) {
      hipLaunchKernelGGL((rmsnorm_gate_kernel<T, 4 * V, 64>), grid, dim3(256), 0, stream, a);
      ok = true;
    }
  if (!ok) {
    set_detail("rmsnorm_gate: no kernel for %d elements per lane, %d lanes per head", vec, g);
    return KDA_ERR_UNSUPPORTED;
  }
  return check_launch("rmsnorm_gate_kernel");
}

int launch_rmsnorm_gate(const void* x, const void* w, int w_per_head, const void* gl, void* y, int64_t rows,
                        int64_t H, int64_t D, double eps, int dtype, hipStream_t stream) {
  const int eb = elem_bytes(dtype);
  if (eb == 0) {
    set_detail("rmsnorm_gate: unknown dtype %d", dtype);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  int vec = 0, g = 0;
  if (!head_layout(D, eb, &vec, &g)) {
    set_detail("rmsnorm_gate: head_dim %lld must be a power of two in 16..512", (long long)D);
    return KDA_ERR_UNSUPPORTED;
  }
  for (const void* p : {x, w, gl, static_cast<const void*>(y)})
    if (!aligned16(p)) {
      set_detail("rmsnorm_gate: x, weight, gate logits and y must be 16-byte aligned");
      return KDA_ERR_INVALID_ARGUMENT;
    }
  const float e = static_cast<float>(eps);
  switch (dtype) {
    case KDA_DTYPE_BF16:
      return run_norm(NormArgs<bf16>{static_cast<const bf16*>(x), static_cast<const bf16*>(w), w_per_head,
                                     static_cast<const bf16*>(gl), static_cast<bf16*>(y), rows, H, e},
                      vec, g, stream);
    case KDA_DTYPE_F16:
      return run_norm(NormArgs<f16>{static_cast<const f16*>(x), static_cast<const f16*>(w), w_per_head,
                                    static_cast<const f16*>(gl), static_cast<f16*>(y), rows, H, e},
                      vec, g, stream);
    case KDA_DTYPE_F32:
      return run_norm(NormArgs<float>{static_cast<const float*>(x), static_cast<const float*>(w), w_per_head,
                                      static_cast<const float*>(gl), static_cast<float*>(y), rows, H, e},
                      vec, g, stream);
    default:
      return run_norm(NormArgs<double>{static_cast<const double*>(x), static_cast<const double*>(w), w_per_head,
                                       static_cast<const double*>(gl), static_cast<double*>(y), rows, H, e},
                      vec, g, stream);
  }
}

}  // namespace kda_host
