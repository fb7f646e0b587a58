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
}  // namespace kda_host
