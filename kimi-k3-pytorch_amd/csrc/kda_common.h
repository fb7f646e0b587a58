// Shared device helpers for the gfx950 KDA kernels: element types, loads and
// stores with conversion, and the sequence bookkeeping common to all kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kda_mi355x.h"

namespace kda {

using bf16 = __bf16;
using f16 = _Float16;

// ---- element conversion ---------------------------------------------------
template <class T> __device__ __forceinline__ float to_float(T x) { return static_cast<float>(x); }
template <> __device__ __forceinline__ float to_float<bf16>(bf16 x) { return static_cast<float>(x); }

template <class C, class T> __device__ __forceinline__ C to_compute(T x) { return static_cast<C>(to_float(x)); }
template <> __device__ __forceinline__ double to_compute<double, double>(double x) { return x; }
template <> __device__ __forceinline__ float to_compute<float, float>(float x) { return x; }

template <class T, class C> __device__ __forceinline__ T from_compute(C x) { return static_cast<T>(x); }
template <> __device__ __forceinline__ bf16 from_compute<bf16, float>(float x) { return static_cast<bf16>(x); }
template <> __device__ __forceinline__ f16 from_compute<f16, float>(float x) { return static_cast<f16>(x); }

__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }
__device__ __forceinline__ double fast_exp(double x) { return exp(x); }

// exp, reciprocal and reciprocal square root of the gate and norm stages: the
// hardware's f32 instructions (v_exp_f32 on x*log2(e), v_rcp_f32, v_rsq_f32;
// about 1 ulp) and the library's correctly rounded routines in f64.
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ double fexp(double x) { return exp(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ double frcp(double x) { return 1.0 / x; }
__device__ __forceinline__ float frsqrt(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ double frsqrt(double x) { return 1.0 / sqrt(x); }

template <class C>
__device__ __forceinline__ C sigmoid(C x) {
  return frcp(C(1) + fexp(-x));
}

// The lower-bounded decay of one element (src/kda/decay.py:36-43 with the
// decay-logit bias of src/kda/projections.py:215):
//   g = g_min * clamp(sigmoid(scale * (z + b)), lo, hi),  scale = exp(A_log[h]),
// lo = eps, hi = 1 - eps of the output type.  One definition for the gates
// kernel and the chunk kernel that forms g from the logits itself, so both
// produce the same bits.
template <class C>
__device__ __forceinline__ C lower_bounded_decay(C z, C b, C scale, C g_min, C lo, C hi) {
  C p = sigmoid(scale * (z + b));
  p = p < lo ? lo : (p > hi ? hi : p);
  C g = g_min * p;
  // keep the product an f32 value: otherwise the compiler may merge it with
  // the caller's conversion to f16 into one mixed-precision FMA (a single
  // rounding) in one kernel and not in another
  if constexpr (sizeof(C) == 4) asm volatile("" : "+v"(g));
  return g;
}

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64).
// In f32 the steps inside a 16-lane row are DPP moves fused into the adds
// (quad permutations [1,0,3,2] and [2,3,0,1], then the half-row and row
// mirrors, each of which pairs the lane with one holding the other half's
// partial sum); wider groups and f64 use the LDS crossbar (__shfl_xor).
template <int ctrl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xf, 0xf, false));
}

template <int G, class C>
__device__ __forceinline__ C group_sum(C v) {
  int off = 1;
  if constexpr (sizeof(C) == 4) {
    if constexpr (G >= 2) v = dpp_add<0xb1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (G >= 4) v = dpp_add<0x4e>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (G >= 8) v = dpp_add<0x141>(v);  // row_half_mirror: the other quad of the 8
    if constexpr (G >= 16) v = dpp_add<0x140>(v); // row_mirror: the other half of the row
    off = G < 16 ? G : 16;
  }
#pragma unroll
  for (; off < G; off <<= 1) v += __shfl_xor(v, off);
  return v;
}

// ---- sequences ------------------------------------------------------------
// A "sequence" is a run of tokens that share one recurrent state: a batch row
// of a dense [B,T,...] call (start = s*T) or a packed document
// (start = cu_seqlens[s]).  `valid` <= `span` tokens are real; the rest are
// right-padding (zero output, state untouched).
struct SeqDesc {
  const int32_t* cu_seqlens;  // [N+1] or nullptr (dense)
  int64_t dense_span;         // tokens per sequence when dense
  const int32_t* valid_lens;  // [N] or nullptr
};

struct SeqRange {
  int64_t start;
  int64_t span;
  int64_t valid;
};

__device__ __forceinline__ SeqRange seq_range(const SeqDesc& d, int64_t s) {
  SeqRange r;
  if (d.cu_seqlens) {
    r.start = d.cu_seqlens[s];
    r.span = static_cast<int64_t>(d.cu_seqlens[s + 1]) - r.start;
  } else {
    r.start = s * d.dense_span;
    r.span = d.dense_span;
  }
  r.valid = r.span;
  if (d.valid_lens) {
    int64_t v = d.valid_lens[s];
    r.valid = v < r.span ? (v < 0 ? 0 : v) : r.span;
  }
  return r;
}

}  // namespace kda

// ---- host-side error reporting shared by the launchers --------------------
namespace kda_host {
void set_detail(const char* fmt, ...);
const char* detail();
int check_launch(const char* what);
// Raise `kernel`'s dynamic LDS limit to `bytes` on the current device, once
// per (kernel, device): the attribute belongs to the kernel on each device,
// and concurrent first calls from several threads set it under one lock.
bool reserve_lds(const void* kernel, int bytes);
// Segment-length override of the chunk prefill's plan (kda_set_segment_chunks).
void set_segment_override(int64_t chunks);
}  // namespace kda_host
