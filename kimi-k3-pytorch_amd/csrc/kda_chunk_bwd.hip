// Backward of the chunkwise KDA operator on gfx950: the gradients of the
// output and final state with respect to q, k, v, g, beta and the initial
// state, for the differentiation of chunkwise_kda (src/kda/chunkwise.py:34-107,
// whose gradients the reference takes from autograd).
//
// Per chunk of 64 tokens (rows i, j; channels along K; columns along V), with
//   lg = cumsum(g), E_ij = exp(lg_i - lg_j), A = strict-lower sum_k k_i k_j E_ij,
//   Aqk = lower sum_k q_i k_j E_ij, N = (I + diag(b) A)^-1, M = N diag(b),
//   Kg = e^lg k, Qg = e^lg q, D = e^lg_last, Kt = e^(lg_last - lg) k,
//   W = M Kg, U = M v, Vt = U - W S,
//   O = Qg S + Aqk Vt,  S' = D S + Kt^T Vt,
// the backward is
//   dVt = Kt dS' + Aqk^T dO,   dS = D dS' + Qg^T dO - W^T dVt,
//   dQg = dO S^T, dAqk = tril(dO Vt^T), dKt = Vt dS'^T, dD = rowsum(dS' * S),
//   dW = -dVt S^T, dv = M^T dVt, dM = dVt v^T + dW Kg^T, dKg = M^T dW,
//   db_j = sum_i N_ij dM_ij + sum_k dL_jk A_jk,  dL = -strict(N^T dM diag(b) N^T),
//   dA = diag(b) dL, then the pair sums of dA and dAqk with exact exponents,
//   the exp factors, and dg = reverse cumulative sum of d lg over the chunk.
//
// f32 accumulation everywhere.  pair and prep's inverse and W, U products
// multiply on the f32 MFMA (v_mfma_f32_16x16x4f32); prep's decay products A
// and Aqk, the state scans and grad's slab products use split-bf16 operands on v_mfma_f32_16x16x32_bf16 (x = hi + lo, hi = bf16(x),
// lo = bf16(x - hi); hi*hi + hi*lo + lo*hi, dropping terms of relative size
// 2^-17), which keeps the f32-input gradients within about 1e-5 of the f64
// oracle.  For bf16 and f16 inputs the scans and grad's slab products take
// single bf16 operands (kSplitOps): their gradients, rounded to the input
// type, stay within about 5e-3 of the oracle.  Decay products use a 16-row block factorisation on the MFMA, with
// an exact pairwise-exponent path for chunks whose decays leave its range
// (any g > 0, or a block decaying past e^-80).
//   prep_kernel         one block per (sequence, head, chunk), two per CU
//                       (the key channels by quarters): A, Aqk, N by
//                       forward substitution, W, U, Kt, Qg, Kg, D;
//   seg_kernel,         the forward scan (chunk start states S, pseudo-values
//   seg_combine_kernel  Vt) and the backward scan (dS', dVt per chunk, dS0),
//                       side by side, each cut into segments whose affine
//                       maps are composed (section "segmented state scans");
//   grad_pair_kernel    one block per chunk: grad_body (dv, dbeta, and the records
//                       dQg, dKt, dKg, dA, dAqk), then pair_body (the pair sums
//                       and the final dq, dk, dg) on the records just written.
// Intermediates live in a caller-owned f32 workspace, one record per
// (sequence, head, chunk), followed by the scans' segment records.
#include <math.h>

#include "kda_launch.h"

namespace kda {
namespace bwd {

constexpr int kC = 64;     // chunk rows
constexpr int kRS = 132;   // LDS row stride of [64][<=128] channel matrices
constexpr int kRC = 68;    // LDS row stride of [64][64] chunk matrices
constexpr int kSW = 32;    // state columns per slab in grad_body
constexpr int kSS = 36;    // LDS row stride of slab matrices
constexpr int kTS = 20;    // LDS row stride of 16-column scan tiles

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Offsets (floats) of one (sequence, head, chunk) record of the workspace.
struct Layout {
  int Kp, Vp;  // K padded to 64 or 128, V to a multiple of 32
  int64_t N, A, Aqkt, Wr, Wt, Ktr, Ktt, Qgt, Kg, U, D, S, Vt, dS, dVt, dQg, dKt, dKg, dA, dAqk, dD, per;
  int hs;  // S, dS and Vt of the backward stored as bf16 (single-operand inputs)
};

// `backward` false: the record of the forward through these kernels (the
// split-bf16 chunk path), which holds only what prep_kernel writes without dO,
// the forward scan and out_kernel read (Aqk^T, W, K~^T, Qg^T, U, D, S, Vt:
// 41% of the backward's record); the offsets of the other records are 0 and
// nothing of the forward touches them.  `split` false (bf16 and f16 inputs,
// kSplitOps): the scans' operand records hold their hi plane alone and, in
// the backward, S, dS and Vt are bf16 (the gradient kernel reads them as bf16
// operands), which takes the backward's record from 593 to 425 KiB at
// K = V = 128.
__host__ __device__ inline Layout make_layout(int64_t K, int64_t V, bool backward = true, bool split = true) {
  Layout L;
  L.Kp = K <= 64 ? 64 : 128;
  L.Vp = static_cast<int>((V + 31) / 32 * 32);
  const int64_t cc = kC * kC, ck = kC * L.Kp, cv = kC * L.Vp, kv = static_cast<int64_t>(L.Kp) * L.Vp;
  const int64_t sc = split ? cc : cc / 2, sk = split ? ck : ck / 2;  // split records in floats
  int64_t o = 0;
  L.hs = 0;
  if (!backward) {
    L.N = L.A = L.Wt = L.Ktr = L.Kg = L.dS = L.dVt = L.dQg = L.dKt = L.dKg = L.dA = L.dAqk = L.dD = 0;
    L.Aqkt = o; o += sc;
    L.Wr = o; o += sk;
    L.Ktt = o; o += sk;
    L.Qgt = o; o += sk;
    L.U = o; o += cv;
    L.D = o; o += L.Kp;
    L.S = o; o += kv;
    L.Vt = o; o += cv;
    L.per = (o + 63) / 64 * 64;
    return L;
  }
  L.hs = split ? 0 : 1;
  const int64_t hv = split ? kv : kv / 2, hc = split ? cv : cv / 2;  // S, dS and Vt in floats
  L.N = o; o += cc;
  L.A = o; o += cc;
  L.Aqkt = o; o += sc;  // split operands of the scans: bf16 hi plane, then lo plane
  L.Wr = o; o += sk;
  L.Wt = o; o += sk;
  L.Ktr = o; o += sk;
  L.Ktt = o; o += sk;
  L.Qgt = o; o += sk;
  L.Kg = o; o += ck;
  L.U = o; o += cv;
  L.D = o; o += L.Kp;
  L.S = o; o += hv;
  L.Vt = o; o += hc;
  L.dS = o; o += hv;
  L.dVt = o; o += cv;
  L.dQg = o; o += ck;
  L.dKt = o; o += ck;
  L.dKg = o; o += ck;
  L.dA = o; o += cc;
  L.dAqk = o; o += cc;
  L.dD = o; o += L.Kp;
  L.per = (o + 63) / 64 * 64;  // 256-byte records
  return L;
}

template <class IT>
struct Args {
  const IT *q, *k, *v, *g, *beta, *dout;  // [B,T,H,*], beta [B,T,H]
  const float* s0;                        // [B,H,K,V] or null
  const float* dsT;                       // [B,H,K,V] or null
  IT *dq, *dk, *dv, *dg, *dbeta;
  float* ds0;                             // [B,H,K,V] or null
  float* ws;
  int64_t B, T, H, K, V, NC;
  Layout L;
  // the forward through these kernels (prep_kernel, fscan_kernel, out_kernel)
  const int32_t* valid;  // [B] right-padding lengths or null (prep_kernel)
  float* sT;             // [B,H,K,V] final state or null (forward scan)
  IT* out;               // [B,T,H,V] (out_kernel)
  // segmented state scans: nseg segments of seglen chunks per sequence,
  // their records (P, Q, start state) at seg, [direction][B*H][nseg]
  float* seg;
  int nseg, seglen;
  int dir0, ndir;  // the scans launched: directions dir0 .. dir0 + ndir - 1
};

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// An LDS matrix: element (r, c) at p[r * rs + c * cs] (a transpose swaps rs, cs).
struct Mat {
  const float* p;
  int rs, cs;
};

// acc += A[r0:r0+16, 0:kd] * B[0:kd, c0:c0+16] on the f32 MFMA.  Lane
// (i = lane % 16, g = lane / 16) supplies A[r0+i][kk+g] and B[kk+g][c0+i];
// the accumulator lane holds D[r0 + 4g + r][c0 + i], r = 0..3.
// kd is a multiple of 16; each group of four products has its eight operand
// reads issued before the first product.
__device__ __forceinline__ f32x4 mma(f32x4 acc, Mat A, int r0, Mat B, int c0, int kd) {
  const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const float* a = A.p + (r0 + i) * A.rs + g * A.cs;
  const float* b = B.p + g * B.rs + (c0 + i) * B.cs;
  for (int k0 = 0; k0 < kd; k0 += 16) {
    float av[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = a[(k0 + 4 * u) * A.cs];
      bv[u] = b[(k0 + 4 * u) * B.rs];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], acc, 0, 0, 0);
  }
  return acc;
}

// The same product for long reductions: alternate groups feed two independent
// accumulation chains, added at the end.
__device__ __forceinline__ f32x4 mma_long(f32x4 acc, Mat A, int r0, Mat B, int c0, int kd) {
  const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const float* a = A.p + (r0 + i) * A.rs + g * A.cs;
  const float* b = B.p + g * B.rs + (c0 + i) * B.cs;
  f32x4 acc2 = zero4();
  for (int k0 = 0; k0 < kd; k0 += 32) {
    float av[8], bv[8];
    const int n = kd - k0 >= 32 ? 8 : 4;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      av[u] = u < n ? a[(k0 + 4 * u) * A.cs] : 0.f;
      bv[u] = u < n ? b[(k0 + 4 * u) * B.rs] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv[u], acc, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u + 4], bv[u + 4], acc2, 0, 0, 0);
    }
  }
  return acc + acc2;
}

// Split-bf16 products for the state scans: x = hi + lo with hi = bf16(x)
// and lo = bf16(x - hi) keeps about 16 bits of x, and hi*hi + hi*lo + lo*hi
// on v_mfma_f32_16x16x32_bf16 (three products per 32-deep slice, against
// eight f32 MFMAs) loses terms of relative size 2^-17.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split_bf16(float x, __bf16& hi, __bf16& lo) {
  hi = static_cast<__bf16>(x);
  lo = static_cast<__bf16>(x - static_cast<float>(hi));
}

// bf16 and f16 inputs, held to 2e-2 of the f32 oracle, take the scans' and
// the gradient slabs' products on single bf16 operands (hi*hi, one MFMA per
// 32-deep slice, the records' lo planes neither written nor read); f32
// inputs keep the split pairs.  prep's decay products A and Aqk stay split
// for every input type.
template <class IT>
constexpr bool kSplitOps = sizeof(IT) == 4;

template <bool B, class T, class F>
struct Pick {
  typedef T type;
};
template <class T, class F>
struct Pick<false, T, F> {
  typedef F type;
};

// A split matrix in LDS with its reduction index contiguous: element (r, k)
// at p[r * rs + k] (hi) and p[plane + r * rs + k] (lo); a right operand is
// held as its transpose (row = output column).
struct SMat {
  const __bf16* p;
  int plane, rs;
};

// acc += A[r0:r0+16, 0:kd] B[0:kd, c0:c0+16]; lane (i, g) carries k = k0 + 8g ..
// k0 + 8g + 7 of row r0 + i of A and of column c0 + i of B; kd % 32 == 0.
// SPLIT false: hi*hi alone (the lo planes are not read).
template <bool SPLIT = true>
__device__ __forceinline__ f32x4 mma3(f32x4 acc, SMat A, int r0, SMat B, int c0, int kd) {
  const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const __bf16* pa = A.p + (r0 + i) * A.rs + 8 * g;
  const __bf16* pb = B.p + (c0 + i) * B.rs + 8 * g;
  for (int k0 = 0; k0 < kd; k0 += 32) {
    const bf16x8 ah = *reinterpret_cast<const bf16x8*>(pa + k0);
    const bf16x8 bh = *reinterpret_cast<const bf16x8*>(pb + k0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    if constexpr (SPLIT) {
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(pa + A.plane + k0);
      const bf16x8 bl = *reinterpret_cast<const bf16x8*>(pb + B.plane + k0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    }
  }
  return acc;
}

// Split record in the workspace: n bf16 hi values, then n lo values.  Eight
// consecutive values from element idx (a multiple of 8) as two 16-byte stores
// (SPLIT false: the hi store alone).
template <bool SPLIT = true>
__device__ __forceinline__ void put_split8(float* rec, int n, int idx, const float* x) {
  bf16x8 hi, lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    __bf16 h, l;
    split_bf16(x[e], h, l);
    hi[e] = h;
    lo[e] = l;
  }
  __bf16* p = reinterpret_cast<__bf16*>(rec);
  *reinterpret_cast<bf16x8*>(p + idx) = hi;
  if constexpr (SPLIT) *reinterpret_cast<bf16x8*>(p + n + idx) = lo;
}

// The lane index counted from an all-ones mask (v_mbcnt: independent of the
// execution mask), formed where it is used instead of kept live across a
// kernel.
__device__ __forceinline__ int lane_id() {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
}

// acc += A[r0:r0+16, 0:kd] B[0:kd, c0:c0+16] for f32 matrices in LDS (see
// Mat), on split-bf16 operands formed in registers: lane (i, g) takes
// A[r0+i][k0+8g+e] and B[k0+8g+e][c0+i], e = 0..7, per 32-deep step (three
// bf16 MFMAs against the eight f32 ones of mma_long; kd a multiple of 32).
__device__ __forceinline__ f32x4 mma_sb(f32x4 acc, Mat A, int r0, Mat B, int c0, int kd) {
  const int lane = lane_id(), i = lane & 15, g = lane >> 4;
  const float* a = A.p + (r0 + i) * A.rs + 8 * g * A.cs;
  const float* b = B.p + 8 * g * B.rs + (c0 + i) * B.cs;
  f32x4 acc2 = zero4();
  for (int k0 = 0; k0 < kd; k0 += 32) {
    float av[8], bv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      av[e] = a[(k0 + e) * A.cs];
      bv[e] = b[(k0 + e) * B.rs];
    }
    bf16x8 ah, al, bh, bl;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      __bf16 h, l;
      split_bf16(av[e], h, l);
      ah[e] = h;
      al[e] = l;
      split_bf16(bv[e], h, l);
      bh[e] = h;
      bl[e] = l;
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc2, 0, 0, 0);
    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc2, 0, 0, 0);
  }
  return acc + acc2;
}

__device__ __forceinline__ int64_t tok(const int64_t b, const int64_t t, const int64_t T, const int64_t H,
                                       const int64_t h) {
  return (b * T + t) * H + h;
}

// Four consecutive elements of an input row: loaded raw, converted later, so
// that a batch of loads is in flight before the first conversion waits.
template <class IT>
struct Raw4 {
  typedef IT type __attribute__((ext_vector_type(4)));
};

template <class IT>
__device__ __forceinline__ f32x4 widen(typename Raw4<IT>::type x) {
  return f32x4{to_float(x[0]), to_float(x[1]), to_float(x[2]), to_float(x[3])};
}

// Columns col0 .. col0+NCOL-1 of the chunk's 64 rows of an input [B,T,H,X]
// into LDS rows of stride RS, zero past T and X.  When the columns lie inside
// X in whole 4-element groups (the usual case) every load of a thread is
// issued, from a row clamped into the sequence, before its first conversion.
// Rows at or past Tv (default T: right padding) read as zero too.
template <class IT, int NCOL, int RS, int NT>
__device__ __forceinline__ void load_rows(float* dst, const IT* src, int64_t b, int64_t t0, int64_t T, int64_t H,
                                          int64_t h, int64_t X, int col0, int tid, int64_t Tv = -1) {
  constexpr int G = NCOL / 4, PER = kC * G / NT;
  if (Tv < 0) Tv = T;
  static_assert(PER * NT == kC * G, "the tile must split evenly over the threads");
  typedef typename Raw4<IT>::type raw_t;
  if ((X & 3) == 0 && col0 + NCOL <= X) {
    raw_t v[PER];
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      const int64_t t = t0 + r < T ? t0 + r : T - 1;
      v[it] = *reinterpret_cast<const raw_t*>(src + tok(b, t, T, H, h) * X + col0 + c4);
    }
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      *reinterpret_cast<f32x4*>(&dst[r * RS + c4]) = t0 + r < Tv ? widen<IT>(v[it]) : zero4();
    }
  } else {
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      const int64_t t = t0 + r;
      f32x4 x = zero4();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t col = col0 + c4 + u;
        x[u] = (t < Tv && col < X) ? to_float(src[tok(b, t, T, H, h) * X + col]) : 0.f;
      }
      *reinterpret_cast<f32x4*>(&dst[r * RS + c4]) = x;
    }
  }
}

// load_rows split in two: `fetch` issues the loads of the whole-group case
// (rows_fast) into registers and `store` widens them into LDS, so that the
// loads of several tiles go out together and their latency is paid once (a
// load_rows call waits for its own loads before the next call's are issued).
__device__ __forceinline__ bool rows_fast(int64_t X, int col0, int ncol) {
  return (X & 3) == 0 && col0 + ncol <= X;
}
template <class IT, int NCOL, int NT>
struct RowTile {
  static constexpr int G = NCOL / 4, PER = kC * G / NT;
  static_assert(PER * NT == kC * G, "the tile must split evenly over the threads");
  typename Raw4<IT>::type v[PER];
  __device__ __forceinline__ void fetch(const IT* src, int64_t b, int64_t t0, int64_t T, int64_t H, int64_t h,
                                        int64_t X, int col0, int tid) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      const int64_t t = t0 + r < T ? t0 + r : T - 1;
      v[it] = *reinterpret_cast<const typename Raw4<IT>::type*>(src + tok(b, t, T, H, h) * X + col0 + c4);
    }
  }
  template <int RS>
  __device__ __forceinline__ void store(float* dst, int64_t t0, int64_t Tv, int tid) const {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      *reinterpret_cast<f32x4*>(&dst[r * RS + c4]) = t0 + r < Tv ? widen<IT>(v[it]) : zero4();
    }
  }
};

// k, q and g rows of a chunk into LDS with one round trip to memory
template <class IT, int KP, int NT>
__device__ __forceinline__ void load_kqg(float* kS, float* qS, float* lgS, const Args<IT>& a, int64_t b, int64_t t0,
                                         int64_t h, int tid, int64_t Tv) {
  if (rows_fast(a.K, 0, KP)) {
    RowTile<IT, KP, NT> rk, rq, rg;
    rk.fetch(a.k, b, t0, a.T, a.H, h, a.K, 0, tid);
    rq.fetch(a.q, b, t0, a.T, a.H, h, a.K, 0, tid);
    rg.fetch(a.g, b, t0, a.T, a.H, h, a.K, 0, tid);
    rk.template store<kRS>(kS, t0, Tv, tid);
    rq.template store<kRS>(qS, t0, Tv, tid);
    rg.template store<kRS>(lgS, t0, Tv, tid);
  } else {
    load_rows<IT, KP, kRS, NT>(kS, a.k, b, t0, a.T, a.H, h, a.K, 0, tid, Tv);
    load_rows<IT, KP, kRS, NT>(qS, a.q, b, t0, a.T, a.H, h, a.K, 0, tid, Tv);
    load_rows<IT, KP, kRS, NT>(lgS, a.g, b, t0, a.T, a.H, h, a.K, 0, tid, Tv);
  }
}

// load_ws split in two (fetch into registers, store into LDS rows of stride
// RS), so that the loads can go out ahead of the point where the tile is needed.
template <int NROW, int NCOL, int NT>
struct WsTile {
  static constexpr int G = NCOL / 4, PER = NROW * G / NT;
  static_assert(PER * NT == NROW * G, "the tile must split evenly over the threads");
  f32x4 v[PER];
  __device__ __forceinline__ void fetch(const float* src, int ld, int col0, int tid) {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      v[it] = *reinterpret_cast<const f32x4*>(src + r * ld + col0 + c4);
    }
  }
  template <int RS>
  __device__ __forceinline__ void store(float* dst, int tid) const {
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
      *reinterpret_cast<f32x4*>(&dst[r * RS + c4]) = v[it];
    }
  }
};

// NROW x NCOL f32 from a workspace matrix (row stride ld, from column col0)
// into LDS rows of stride RS.
template <int NROW, int NCOL, int RS, int NT>
__device__ __forceinline__ void load_ws(float* dst, const float* src, int ld, int col0, int tid) {
  constexpr int G = NCOL / 4, PER = NROW * G / NT;
  static_assert(PER * NT == NROW * G, "the tile must split evenly over the threads");
  f32x4 v[PER];
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
    v[it] = *reinterpret_cast<const f32x4*>(src + r * ld + col0 + c4);
  }
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int item = tid + NT * it, r = item / G, c4 = (item % G) * 4;
    *reinterpret_cast<f32x4*>(&dst[r * RS + c4]) = v[it];
  }
}

// Decay products e^(lg_i - lg_j) (j <= i) are formed on the MFMA as
// (x_i e^(lg_i - r)) (y_j e^(r - lg_j)) with r = lg at the first row of i's
// 16-row block: for a chunk whose g are all <= 0 (lg falls down the chunk) and
// whose decay across any 16-row block stays within kMaxBlockDecay, the first
// factor lies in [e^-80, 1] and the second is <= 1 off the diagonal block (it
// underflows only where the product itself is negligible) and <= e^80 on it.
// Other chunks take the exact pairwise path.
constexpr float kMaxBlockDecay = 80.f;

// lg = cumsum(g) down the chunk's 64 rows for each of the KP channels, in
// place in lgS (row stride RS).  Thread (channel tid % KP, quarter tid / KP)
// sums its quarter's 16 rows in registers, the quarter totals meet in `tmp`
// (4 x KP floats), and each quarter adds the totals above it: a chain of 16
// additions instead of 64 dependent LDS round trips.  Returns whether one of
// the thread's own g values is positive; ends with the block synchronised.
template <int KP, int RS = kRS>
__device__ __forceinline__ bool chunk_cumsum(float* lgS, float* tmp, int tid) {
  bool rising = false;
  float v[16];
  const int c = tid % KP, p = tid / KP;
  if (p < 4) {
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = lgS[(16 * p + r) * RS + c];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      rising |= v[r] > 0.f;
      if (r > 0) v[r] += v[r - 1];
    }
    tmp[p * KP + c] = v[15];
  }
  __syncthreads();
  if (p < 4) {
    float off = 0.f;
    for (int q = 0; q < p; ++q) off += tmp[q * KP + c];
#pragma unroll
    for (int r = 0; r < 16; ++r) lgS[(16 * p + r) * RS + c] = v[r] + off;
  }
  __syncthreads();
  return rising;
}

// Whether one of the thread's (16-row block, channel) pairs of lg (KP
// channels, row stride RS) decays by more than kMaxBlockDecay; no barrier.
template <int KP, int NT, int RS = kRS>
__device__ __forceinline__ bool decay_risk(const float* lgS, int tid) {
  bool risky = false;
  for (int idx = tid; idx < 4 * KP; idx += NT) {
    const int I = idx / KP, c = idx % KP;
    risky |= lgS[16 * I * RS + c] - lgS[(16 * I + 15) * RS + c] > kMaxBlockDecay;
  }
  return risky;
}

// True when the chunk needs the exact path; lg in LDS rows of stride kRS,
// the raw g's sign having been folded into `nonneg` by the caller.
template <int KP, int NT>
__device__ __forceinline__ bool needs_exact(const float* lgS, bool nonneg, int tid) {
  return __syncthreads_or(nonneg || decay_risk<KP, NT>(lgS, tid));
}

// accK += sum_c (k_i e^(lg_i - r)) (k_j e^(r - lg_j)) and accQ the same with
// q_i, for rows i in [r0, r0+16), columns j in [c0, c0+16) and r = lg[rr];
// the reduction runs over the kd channels from kb (kd a multiple of 16).  The
// decayed operands are split into bf16 hi + lo and multiplied on
// v_mfma_f32_16x16x32_bf16 (hi*hi + hi*lo + lo*hi, three products per 32
// channels against eight f32 MFMAs per 16); lane (i, g) carries channels
// k0 + 8g .. k0 + 8g + 7 of row r0 + i and of column c0 + i, and with 16
// channels left the lane groups g >= 2 carry zeros.  Channel matrices in LDS
// rows of stride RS.
template <int RS = kRS>
__device__ __forceinline__ void decay_product(f32x4& accK, f32x4& accQ, const float* kS, const float* qS,
                                              const float* lgS, int r0, int c0, int rr, int kd, int kb = 0) {
  const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  for (int k0 = kb; k0 < kb + kd; k0 += 32) {
    const bool live = 8 * g < kb + kd - k0;
    bf16x8 kah, kal, qah, qal, kbh, kbl;
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const int ch = k0 + 8 * g + e;
      f32x4 r4 = zero4(), la = zero4(), lb = zero4(), ka = zero4(), qa = zero4(), kv = zero4();
      if (live) {
        r4 = *reinterpret_cast<const f32x4*>(&lgS[rr * RS + ch]);
        la = *reinterpret_cast<const f32x4*>(&lgS[(r0 + i) * RS + ch]);
        lb = *reinterpret_cast<const f32x4*>(&lgS[(c0 + i) * RS + ch]);
        ka = *reinterpret_cast<const f32x4*>(&kS[(r0 + i) * RS + ch]);
        qa = *reinterpret_cast<const f32x4*>(&qS[(r0 + i) * RS + ch]);
        kv = *reinterpret_cast<const f32x4*>(&kS[(c0 + i) * RS + ch]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float ea = fast_exp(la[u] - r4[u]), eb = fast_exp(r4[u] - lb[u]);
        __bf16 h, l;
        split_bf16(ka[u] * ea, h, l);
        kah[e + u] = h;
        kal[e + u] = l;
        split_bf16(qa[u] * ea, h, l);
        qah[e + u] = h;
        qal[e + u] = l;
        split_bf16(kv[u] * eb, h, l);
        kbh[e + u] = h;
        kbl[e + u] = l;
      }
    }
    accK = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kah, kbh, accK, 0, 0, 0);
    accQ = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qah, kbh, accQ, 0, 0, 0);
    accK = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kah, kbl, accK, 0, 0, 0);
    accQ = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qah, kbl, accQ, 0, 0, 0);
    accK = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kal, kbh, accK, 0, 0, 0);
    accQ = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qal, kbh, accQ, 0, 0, 0);
  }
}

// The ten 16x16 block pairs (I, J <= I) of a chunk.
__device__ __forceinline__ void block_pair(int p, int& I, int& J) {
  I = p < 1 ? 0 : (p < 3 ? 1 : (p < 6 ? 2 : 3));
  J = p - I * (I + 1) / 2;
}

// A per-lane offset the compiler may not hoist out of a loop: keeps the many
// invariant per-lane addresses of the loop from occupying registers (or
// scratch, whose reloads wait for every earlier load and store).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// ---- prep_kernel: per-chunk intermediates ----------------------------------
// The chunk's k, q and g pass through LDS kQC key channels (a quarter of 128)
// at a time, so that the kernel's LDS (79 KB) lets two workgroups share a CU
// and one block's loads and record stores overlap the other's work.  For each
// quarter, its loads issued while the previous quarter is worked on:
//   lg = cumsum(g) over the quarter's channels;
//   the MFMA decay products of A and Aqk, accumulated in registers (each
//   block pair's channel sum runs in the same 32-channel steps as it would
//   over the whole chunk);
//   Kt = e^(lg_last - lg) k and Qg = e^lg q in place of q and lg, and
//   Kg = e^lg k into a [64][KP] tile that stays for W = M Kg, with their
//   records (D, Kg and Kt row-major, Kt^T, Qg^T).
// A chunk whose decays fall outside the factorisation's bounds repeats the
// quarters for A and Aqk with exact pair exponents.  Then N = L^-1,
// M = N diag(b), W = M Kg and U = M v.
constexpr int kPT = 512;  // threads of prep_kernel
constexpr int kQC = 32;   // key channels per quarter
constexpr int kQS = 36;   // LDS row stride of the quarter tiles

// k, q and g of kQC key channels from column c0: fetched into registers ahead
// of use when the rows allow 16-byte loads, read straight into LDS otherwise
template <class IT>
struct QuarterTiles {
  RowTile<IT, kQC, kPT> k, q, g;
  __device__ __forceinline__ void fetch(const Args<IT>& a, int64_t b, int64_t t0, int64_t h, int c0, int tid) {
    if (!rows_fast(a.K, c0, kQC)) return;
    k.fetch(a.k, b, t0, a.T, a.H, h, a.K, c0, tid);
    q.fetch(a.q, b, t0, a.T, a.H, h, a.K, c0, tid);
    g.fetch(a.g, b, t0, a.T, a.H, h, a.K, c0, tid);
  }
  __device__ __forceinline__ void store(float* kS, float* qS, float* lgS, const Args<IT>& a, int64_t b, int64_t t0,
                                        int64_t h, int c0, int tid, int64_t Tv) const {
    if (rows_fast(a.K, c0, kQC)) {
      k.template store<kQS>(kS, t0, Tv, tid);
      q.template store<kQS>(qS, t0, Tv, tid);
      g.template store<kQS>(lgS, t0, Tv, tid);
    } else {
      load_rows<IT, kQC, kQS, kPT>(kS, a.k, b, t0, a.T, a.H, h, a.K, c0, tid, Tv);
      load_rows<IT, kQC, kQS, kPT>(qS, a.q, b, t0, a.T, a.H, h, a.K, c0, tid, Tv);
      load_rows<IT, kQC, kQS, kPT>(lgS, a.g, b, t0, a.T, a.H, h, a.K, c0, tid, Tv);
    }
  }
};

template <class IT, int KP>
__global__ __launch_bounds__(kPT, 4) void prep_kernel(const Args<IT> a) {
  constexpr int NQ = KP / kQC;  // quarters
  constexpr int NW = KP / 32;   // W tiles per wave
  static_assert(KP % kQC == 0, "whole quarters");
  // LDS: the quarter tiles k, q, lg [64][kQS], later Aqk, then N and the
  // inverse's scratch tiles; Kg [64][kRS] (later W, then v); A (later M)
  constexpr int QREG = 3 * kC * kQS;
  __shared__ __attribute__((aligned(16))) float pool[QREG + kC * kRS + kC * kRC];
  __shared__ __attribute__((aligned(16))) float bS[kC];
  __shared__ __attribute__((aligned(16))) float lastS[kQC];  // lg of the chunk's last row, quarter's channels
  __shared__ __attribute__((aligned(16))) float tmpS[4 * kQC];
  static_assert(kC * kRC + 8 * 16 * kTS <= QREG, "N and the scratch tiles fit over the quarter tiles");
  float* const kS = pool;
  float* const qS = pool + kC * kQS;
  float* const lgS = pool + 2 * kC * kQS;
  float* const AqkS = pool;          // after the quarters
  float* const NS = pool;            // after Aqk's record
  float* const KgS = pool + QREG;    // Kg, then W, then v
  float* const AS = KgS + kC * kRS;
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg4 = lane >> 4;
  // the wave index scalar: the block pairs and tiles derived from it stay in
  // scalar registers instead of vector registers (or scratch)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t ch = blockIdx.x;
  const int64_t c = ch % a.NC, bh = ch / a.NC, b = bh / a.H, h = bh % a.H;
  const int64_t t0 = c * kC;
  const int Vp = a.L.Vp;
  float* ws = a.ws + ch * a.L.per;
  // padded tokens (t >= Tv) enter as zero rows: no decay, no write, no output
  int64_t Tv = a.T;
  if (a.valid != nullptr) {
    const int64_t n = a.valid[b];
    Tv = n < 0 ? 0 : (n < a.T ? n : a.T);
  }
  // the records only the gradient kernels read (A, N, Kg, Kt row-major, W^T)
  // are skipped when the kernels serve the forward alone (no dO)
  const bool bwd_records = a.dout != nullptr;

  QuarterTiles<IT> in;
  in.fetch(a, b, t0, h, 0, tid);
  if (tid < kC) {
    const int64_t t = t0 + tid;
    bS[tid] = t < Tv ? to_float(a.beta[tok(b, t, a.T, a.H, h)]) : 0.f;
  }
  for (int idx = tid; idx < kC * kRC; idx += kPT) AS[idx] = 0.f;
  // wave w: block pair w, and waves 0 and 1 pairs 8 and 9 as well
  int I, J, I8, J8;
  block_pair(w, I, J);
  block_pair(8 + (w & 1), I8, J8);
  const bool two = w < 2;
  f32x4 ak = zero4(), aq = zero4(), ak8 = zero4(), aq8 = zero4();
  bool risky = false;
  for (int p = 0; p < NQ; ++p) {
    const int c0 = p * kQC;
    const int tq = opaque(tid);  // per-lane addresses formed in the loop
    in.store(kS, qS, lgS, a, b, t0, h, c0, tq, Tv);
    __syncthreads();
    if (p + 1 < NQ) in.fetch(a, b, t0, h, c0 + kQC, tq);
    risky |= chunk_cumsum<kQC, kQS>(lgS, tmpS, tid);
    risky |= decay_risk<kQC, kPT, kQS>(lgS, tid);
    decay_product<kQS>(ak, aq, kS, qS, lgS, 16 * I, 16 * J, 16 * I, kQC);
    if (two) decay_product<kQS>(ak8, aq8, kS, qS, lgS, 16 * I8, 16 * J8, 16 * I8, kQC);
    if (tq < kQC) {
      const float last = lgS[(kC - 1) * kQS + tq];
      lastS[tq] = last;
      ws[a.L.D + c0 + tq] = fast_exp(last);
    }
    __syncthreads();
    // each element's factors once: Kt and Qg in place of q and lg, Kg into
    // its tile, and the row-major Kg and Kt records written on the way
    for (int i8 = tq; i8 < kC * kQC / 8; i8 += kPT) {
      const int r = (8 * i8) / kQC, cl = (8 * i8) % kQC;
      const float* kp = &kS[r * kQS + cl];
      float* qp = &qS[r * kQS + cl];
      float* lp = &lgS[r * kQS + cl];
      float kg[8], kt[8], qg[8];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f32x4 kk = *reinterpret_cast<const f32x4*>(kp + 4 * u), qq = *reinterpret_cast<const f32x4*>(qp + 4 * u);
        const f32x4 ll = *reinterpret_cast<const f32x4*>(lp + 4 * u);
        const f32x4 la = *reinterpret_cast<const f32x4*>(&lastS[cl + 4 * u]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ex = fast_exp(ll[e]);
          kg[4 * u + e] = ex * kk[e];
          kt[4 * u + e] = fast_exp(la[e] - ll[e]) * kk[e];
          qg[4 * u + e] = ex * qq[e];
        }
      }
      if (bwd_records) {  // Kg (f32) and Kt split, row-major
        const int idx = r * KP + c0 + cl;
#pragma unroll
        for (int u = 0; u < 2; ++u)
          *reinterpret_cast<f32x4*>(ws + a.L.Kg + idx + 4 * u) =
              f32x4{kg[4 * u], kg[4 * u + 1], kg[4 * u + 2], kg[4 * u + 3]};
        put_split8<kSplitOps<IT>>(ws + a.L.Ktr, kC * KP, idx, kt);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        *reinterpret_cast<f32x4*>(&KgS[r * kRS + c0 + cl + 4 * u]) =
            f32x4{kg[4 * u], kg[4 * u + 1], kg[4 * u + 2], kg[4 * u + 3]};
        *reinterpret_cast<f32x4*>(qp + 4 * u) = f32x4{kt[4 * u], kt[4 * u + 1], kt[4 * u + 2], kt[4 * u + 3]};
        *reinterpret_cast<f32x4*>(lp + 4 * u) = f32x4{qg[4 * u], qg[4 * u + 1], qg[4 * u + 2], qg[4 * u + 3]};
      }
    }
    __syncthreads();
    for (int i8 = tq; i8 < kC * kQC / 8; i8 += kPT) {  // Kt^T and Qg^T split, eight positions at a time
      const int col = (8 * i8) / kC, r0 = (8 * i8) % kC;
      float xk[8], xq[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xk[e] = qS[(r0 + e) * kQS + col];
        xq[e] = lgS[(r0 + e) * kQS + col];
      }
      put_split8<kSplitOps<IT>>(ws + a.L.Ktt, kC * KP, c0 * kC + 8 * i8, xk);
      put_split8<kSplitOps<IT>>(ws + a.L.Qgt, kC * KP, c0 * kC + 8 * i8, xq);
    }
    __syncthreads();
  }
  const bool exact = __syncthreads_or(risky);
  if (exact) {
    // A and Aqk with exact pair exponents, 2x2 blocks of (i, j <= i): thread
    // tid takes blocks tid and tid + kPT of the 528, over the quarters again
    float ea[2][2][2], eq[2][2][2];
    int bi[2], bj[2];
    bool off_diag[2], live[2];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const int blk = tid + sl * kPT;
      int I2 = static_cast<int>((sqrtf(8.f * blk + 1.f) - 1.f) * 0.5f);
      while (I2 * (I2 + 1) / 2 > blk) --I2;
      while ((I2 + 1) * (I2 + 2) / 2 <= blk) ++I2;
      const int J2 = blk - I2 * (I2 + 1) / 2;
      live[sl] = blk < 528;
      bi[sl] = 2 * I2;
      bj[sl] = 2 * J2;
      off_diag[sl] = I2 != J2;  // pair (i0, j0 + 1) lies above the diagonal on the diagonal block
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) ea[sl][x][y] = eq[sl][x][y] = 0.f;
    }
    for (int p = 0; p < NQ; ++p) {
      const int c0 = p * kQC;
      in.fetch(a, b, t0, h, c0, tid);
      in.store(kS, qS, lgS, a, b, t0, h, c0, tid, Tv);
      __syncthreads();
      chunk_cumsum<kQC, kQS>(lgS, tmpS, tid);
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        if (!live[sl]) continue;
        const int i0 = bi[sl], j0 = bj[sl];
#pragma unroll 2
        for (int kc = 0; kc < kQC; kc += 4) {
          f32x4 ki[2], qi[2], lI[2], kj[2], lj[2];
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            ki[x] = *reinterpret_cast<const f32x4*>(&kS[(i0 + x) * kQS + kc]);
            qi[x] = *reinterpret_cast<const f32x4*>(&qS[(i0 + x) * kQS + kc]);
            lI[x] = *reinterpret_cast<const f32x4*>(&lgS[(i0 + x) * kQS + kc]);
            kj[x] = *reinterpret_cast<const f32x4*>(&kS[(j0 + x) * kQS + kc]);
            lj[x] = *reinterpret_cast<const f32x4*>(&lgS[(j0 + x) * kQS + kc]);
          }
#pragma unroll
          for (int x = 0; x < 2; ++x)
#pragma unroll
            for (int y = 0; y < 2; ++y) {
              const bool ok = !(x == 0 && y == 1) || off_diag[sl];
              const float e0 = ok ? fast_exp(lI[x].x - lj[y].x) : 0.f;
              const float e1 = ok ? fast_exp(lI[x].y - lj[y].y) : 0.f;
              const float e2 = ok ? fast_exp(lI[x].z - lj[y].z) : 0.f;
              const float e3 = ok ? fast_exp(lI[x].w - lj[y].w) : 0.f;
              ea[sl][x][y] += ki[x].x * kj[y].x * e0 + ki[x].y * kj[y].y * e1 + ki[x].z * kj[y].z * e2 +
                              ki[x].w * kj[y].w * e3;
              eq[sl][x][y] += qi[x].x * kj[y].x * e0 + qi[x].y * kj[y].y * e1 + qi[x].z * kj[y].z * e2 +
                              qi[x].w * kj[y].w * e3;
            }
        }
      }
      __syncthreads();
    }
    for (int idx = tid; idx < kC * kRC; idx += kPT) AqkS[idx] = 0.f;
    __syncthreads();
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      if (!live[sl]) continue;
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) {
          const int i = bi[sl] + x, j = bj[sl] + y;
          if (j < i) AS[i * kRC + j] = ea[sl][x][y];
          if (j <= i) AqkS[i * kRC + j] = eq[sl][x][y];
        }
    }
  } else {
    // the pairs from registers (Aqk's tile, over the quarter tiles, written
    // whole: the six blocks above the diagonal as zeros)
    const int li = lane_id() & 15, lg4 = lane_id() >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * I + 4 * lg4 + r, col = 16 * J + li;
      if (col < row) AS[row * kRC + col] = ak[r];
      AqkS[row * kRC + col] = col <= row ? aq[r] : 0.f;
    }
    if (two) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * I8 + 4 * lg4 + r, col = 16 * J8 + li;
        if (col < row) AS[row * kRC + col] = ak8[r];
        AqkS[row * kRC + col] = col <= row ? aq8[r] : 0.f;
      }
    }
    for (int e = tid; e < 6 * 256; e += kPT) {  // blocks (I, J > I)
      const int p6 = e >> 8, I2 = p6 < 3 ? 0 : (p6 < 5 ? 1 : 2), J2 = p6 < 3 ? p6 + 1 : (p6 < 5 ? p6 - 1 : 3);
      AqkS[(16 * I2 + ((e & 255) >> 4)) * kRC + 16 * J2 + (e & 15)] = 0.f;
    }
  }
  __syncthreads();
  // per-lane addresses of the record stores formed here, not at the top
  const int tr = opaque(tid);
  for (int i4 = tr; bwd_records && i4 < kC * kC / 4; i4 += kPT) {  // A, four at a time
    const int r = (4 * i4) >> 6, cc = (4 * i4) & 63;
    *reinterpret_cast<f32x4*>(ws + a.L.A + 4 * i4) = *reinterpret_cast<const f32x4*>(&AS[r * kRC + cc]);
  }
  for (int i8 = tr; i8 < kC * kC / 8; i8 += kPT) {  // Aqk^T split, eight positions at a time
    const int r = (8 * i8) >> 6, c0 = (8 * i8) & 63;
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = AqkS[(c0 + e) * kRC + r];
    put_split8<kSplitOps<IT>>(ws + a.L.Aqkt, kC * kC, 8 * i8, x);
  }
  __syncthreads();
  for (int i4 = tid; i4 < kC * kC / 4; i4 += kPT) {  // L's strict part b_i A_ij over A; N cleared over Aqk
    const int r = (4 * i4) >> 6, cc = (4 * i4) & 63;
    f32x4* ap = reinterpret_cast<f32x4*>(&AS[r * kRC + cc]);
    *ap = *ap * bS[r];
    *reinterpret_cast<f32x4*>(&NS[r * kRC + cc]) = zero4();
  }
  __syncthreads();
  // v (over Kg's tile once W's records are out): its loads go out now and
  // land while N, M and W are formed
  const bool v_early = (Vp & 31) == 0 && rows_fast(a.V, 0, Vp);
  RowTile<IT, 32, kPT> rv[4];  // Vp <= 128
  if (v_early) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (32 * j < Vp) rv[j].fetch(a.v, b, t0, a.T, a.H, h, a.V, 32 * j, tid);
  }
  // N = L^-1 by 16x16 blocks: wave w inverts diagonal block w by forward
  // substitution (lane c < 16 solves column c), then block rows I = 1..3 follow
  // N_IJ = -N_II sum_{K=J}^{I-1} L_IK N_KJ on the MFMA.
  if (w < 4 && lane < 16) {
    const int base = 16 * w;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sacc = 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) sacc += AS[(base + i) * kRC + base + j] * x[j];
      x[i] = i == lane ? 1.f : (i > lane ? -sacc : 0.f);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) NS[(base + i) * kRC + base + lane] = x[i];
  }
  __syncthreads();
  float* TS = NS + kC * kRC + w * 16 * kTS;  // 16x16 scratch per wave
  for (int Ib = 1; Ib < 4; ++Ib) {
    if (w < Ib) {
      const f32x4 t = mma(zero4(), Mat{AS + 16 * w, kRC, 1}, 16 * Ib, Mat{NS + 16 * w * kRC, kRC, 1}, 16 * w,
                          16 * (Ib - w));
#pragma unroll
      for (int r = 0; r < 4; ++r) TS[(4 * lg4 + r) * kTS + li] = t[r];
    }
    __syncthreads();
    if (w < Ib) {
      const f32x4 n = mma(zero4(), Mat{NS + 16 * Ib, kRC, 1}, 16 * Ib, Mat{TS, kTS, 1}, 0, 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) NS[(16 * Ib + 4 * lg4 + r) * kRC + 16 * w + li] = -n[r];
    }
    __syncthreads();
  }
  for (int i4 = tr; i4 < kC * kC / 4; i4 += kPT) {  // M = N diag(b) over A, four at a time
    const int r = (4 * i4) >> 6, cc = (4 * i4) & 63;
    const f32x4 n = *reinterpret_cast<const f32x4*>(&NS[r * kRC + cc]);
    if (bwd_records) *reinterpret_cast<f32x4*>(ws + a.L.N + 4 * i4) = n;
    *reinterpret_cast<f32x4*>(&AS[r * kRC + cc]) = n * *reinterpret_cast<const f32x4*>(&bS[cc]);
  }
  __syncthreads();
  // W = M Kg, staged in f32 over Kg once every tile is formed
  f32x4 wt[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int tt = w + 8 * j, rt = tt & 3, ct = tt >> 2;
    wt[j] = mma_sb(zero4(), Mat{AS, kRC, 1}, 16 * rt, Mat{KgS, kRS, 1}, 16 * ct, kC);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int tt = w + 8 * j, rt = tt & 3, ct = tt >> 2;
#pragma unroll
    for (int r = 0; r < 4; ++r) KgS[(16 * rt + 4 * (lane_id() >> 4) + r) * kRS + 16 * ct + (lane_id() & 15)] = wt[j][r];
  }
  __syncthreads();
  for (int i8 = tr; i8 < kC * KP / 8; i8 += kPT) {  // W and W^T split
    float x[8], y[8];
    const int r = (8 * i8) / KP, c0 = (8 * i8) % KP;
    const int c2 = (8 * i8) / kC, r2 = (8 * i8) % kC;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = KgS[r * kRS + c0 + e];
      y[e] = KgS[(r2 + e) * kRS + c2];
    }
    put_split8<kSplitOps<IT>>(ws + a.L.Wr, kC * KP, 8 * i8, x);
    if (bwd_records) put_split8<kSplitOps<IT>>(ws + a.L.Wt, kC * KP, 8 * i8, y);
  }
  __syncthreads();
  if (v_early) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (32 * j < Vp) rv[j].template store<kRS>(KgS + 32 * j, t0, Tv, tid);
  } else {
    for (int s0 = 0; s0 < Vp; s0 += 32)
      load_rows<IT, 32, kRS, kPT>(KgS + s0, a.v, b, t0, a.T, a.H, h, a.V, s0, tid, Tv);
  }
  __syncthreads();
  const int nvt = Vp / 16;
  for (int tt = w; tt < 4 * nvt; tt += kPT / 64) {  // U = M v
    const int rt = tt & 3, ct = tt >> 2;
    const f32x4 acc = mma_sb(zero4(), Mat{AS, kRC, 1}, 16 * rt, Mat{KgS, kRS, 1}, 16 * ct, kC);
#pragma unroll
    for (int r = 0; r < 4; ++r) ws[a.L.U + (16 * rt + 4 * (lane_id() >> 4) + r) * Vp + 16 * ct + (lane_id() & 15)] = acc[r];
  }
}

// ---- segmented state scans ------------------------------------------------------
// Both scans are affine maps of a K x N state X per chunk:
//   forward  (chunks 0 .. NC-1):  R = U - W X,               X' = D X + Kt^T R
//   backward (chunks NC-1 .. 0):  R = -(Kt X + Aqk^T dO),    X' = D X + W^T R + Qg^T dO
// (forward X = S and R = Vt; backward X = dS', the gradient of the chunk's end
// state, and R = -dVt).  The chunk chain of each sequence is cut into nseg
// segments of seglen chunks, the same chunks in both directions:
//   seg_kernel<kSumV>, <kSumT>  the segment's affine map X_out = P X_in + Q, by
//                               running the chunk maps on X = [0 | I]: Q from
//                               the V value columns (per direction), P from
//                               the K transition columns (forward only: the
//                               backward's chunk transition D - W^T Kt is the
//                               transpose of the forward's D - Kt^T W, so its
//                               segment map is the forward map of the same
//                               chunks, transposed);
//   seg_combine_kernel          X_{g+1} = P_g X_g + Q_g along the segments (f32 MFMA);
//   seg_kernel<kRun>            each segment again from its true start state,
//                               writing each chunk's X and R (and the final
//                               state after the last chunk).
// The state lives in f32 MFMA accumulators, one 16-column tile per wave.
// Every product uses split-bf16 operands for f32 inputs
// (x = hi + lo; hi*hi + hi*lo + lo*hi) and single bf16 operands otherwise
// (kSplitOps: the records' lo planes are then neither written nor read).  An accumulator pair (row tiles 2s,
// 2s+1) is the B operand of reduction step s with the reduction index
// permuted as perm_k; the A operands are stored in LDS with the same
// permutation: fragment (J, s) holds, for lane (i, g), elements
// M[16 J + i][32 s + perm_k(g, e)], e = 0..7, hi lanes then lo lanes (2 KB).
constexpr int kSC = 512;  // threads of seg_kernel

__device__ __forceinline__ int perm_k(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

template <int KP>
struct SegLds {
  static constexpr int nrow = 4 * (KP / 32);   // fragments of a [64][KP] record
  static constexpr int ncol = (KP / 16) * 2;   // fragments of a [KP][64] record
  static constexpr int fa = 0;                  // forward W, backward Kt        [64][KP]
  static constexpr int fb = fa + nrow * 2048;   // forward Kt^T, backward W^T    [KP][64]
  static constexpr int fq = fb + ncol * 2048;   // backward Qg^T                 [KP][64]
  static constexpr int faq = fq + ncol * 2048;  // backward Aqk^T                [64][64]
  static constexpr int d = faq + 8 * 2048;      // D f32 [KP]
  static constexpr int bytes = d + KP * 4;
};

// A split record [R][NC] of the workspace (R x NC bf16 hi, then lo; the hi
// plane alone when SPLIT is false) held in registers as 8-byte groups; thread
// tid takes the n consecutive groups from tid * n (8, 16 or 32 columns of one
// row), so its loads and LDS stores share one base address with immediate
// offsets.
template <int R, int NC, bool SPLIT = true>
struct Rec {
  static constexpr int planes = SPLIT ? 2 : 1;
  static constexpr int n = R * NC * planes / 4 / kSC;
  static_assert(n * kSC * 4 == R * NC * planes && (n == 8 || n == 4 || n == 2),
                "the record must split into runs of 2, 4 or 8 groups");
  uint2 v[n];
  __device__ __forceinline__ void fetch(const float* rec, int tid) {
    const uint4* p = reinterpret_cast<const uint4*>(rec) + tid * (n / 2);
#pragma unroll
    for (int j = 0; j < n / 2; ++j) {
      const uint4 x = p[j];
      v[2 * j] = uint2{x.x, x.y};
      v[2 * j + 1] = uint2{x.z, x.w};
    }
  }
  // into fragment layout at byte offset base of the LDS: the group at column
  // c of a 32-column slice is group (c % 16) / 4 of half c / 16
  __device__ __forceinline__ void store(unsigned char* sm, int base, int tid) const {
    constexpr int per_plane = R * NC / 4;
    const int q0 = tid * n, plane = q0 / per_plane, el = (q0 % per_plane) * 4;
    const int r = el / NC, c0 = el % NC;
    const int f = (r >> 4) * (NC / 32) + (c0 >> 5);
    unsigned char* dst = sm + base + f * 2048 + plane * 1024 + (r & 15) * 16;
#pragma unroll
    for (int j = 0; j < n; ++j) {
      const int c = (c0 & 31) + 4 * j;
      *reinterpret_cast<uint2*>(dst + ((c & 15) >> 2) * 256 + (c >> 4) * 8) = v[j];
    }
  }
};

__device__ __forceinline__ bf16x8 frag_ld(const unsigned char* sm, int base, int f, int plane, int lane) {
  return *reinterpret_cast<const bf16x8*>(sm + base + f * 2048 + plane * 1024 + lane * 16);
}

// rows 4g..4g+3 of two accumulator tiles as one split B operand (SPLIT
// false: hi alone, lo left unset)
template <bool SPLIT = true>
__device__ __forceinline__ void split_pair(const f32x4& a, const f32x4& b, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if constexpr (SPLIT) {
      __bf16 h, l;
      split_bf16(a[r], h, l);
      hi[r] = h;
      lo[r] = l;
      split_bf16(b[r], h, l);
      hi[4 + r] = h;
      lo[4 + r] = l;
    } else {
      hi[r] = static_cast<__bf16>(a[r]);
      hi[4 + r] = static_cast<__bf16>(b[r]);
    }
  }
}

// SPLIT false: hi*hi alone (the lo parts are not read)
template <bool SPLIT = true>
__device__ __forceinline__ f32x4 mfma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl,
                                       f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
  if constexpr (!SPLIT) return acc;
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
}

// dO of a chunk as the split B operand of the two position steps: lane (i, g)
// element e of step s holds dO[t0 + 32 s + perm_k(g, e)][col]
template <class IT>
struct DoFrag {
  IT x[2][8];
  __device__ __forceinline__ void fetch(const Args<IT>& a, int64_t b, int64_t h, int64_t t0, int col, int g) {
    const int cc = opaque(col < a.V ? col : static_cast<int>(a.V) - 1);
    const IT* row0 = a.dout + tok(b, 0, a.T, a.H, h) * a.V + cc;
    const int64_t step = a.H * a.V;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        int64_t t = t0 + 32 * st + perm_k(g, e);
        t = t < a.T ? t : a.T - 1;
        x[st][e] = row0[t * step];
      }
  }
  template <bool SPLIT>
  __device__ __forceinline__ void split(int64_t t0, int64_t T, int col, int64_t V, int g, bf16x8 (&hi)[2],
                                        bf16x8 (&lo)[2]) const {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool real = t0 + 32 * st + perm_k(g, e) < T && col < V;
        __bf16 hh, ll;
        split_bf16(real ? to_float(x[st][e]) : 0.f, hh, ll);
        hi[st][e] = hh;
        if constexpr (SPLIT) lo[st][e] = ll;
      }
  }
};

// Block kinds of seg_kernel: the value columns of a segment's map (Q), its
// transition columns (P), or the rerun of a segment from its start state.
constexpr int kSumV = 0, kSumT = 1, kRun = 2;

// Segments per (sequence, head) that a launch of kind MODE runs: every
// segment for the reruns; all but the last for the value maps; for the
// transition maps (forward direction only) all but the last when the forward
// runs alone, and all of them when the backward, which takes their
// transposes in reverse order, runs too.
template <class IT>
__host__ __device__ inline int seg_blocks(const Args<IT>& a, int mode) {
  if (mode == kRun) return a.nseg;
  if (mode == kSumT) return a.ndir == 2 ? a.nseg : a.nseg - 1;
  return a.nseg - 1;
}

template <class IT, int KP, int MODE, int DIR>
__device__ __forceinline__ void seg_body(const Args<IT>& a, int64_t id, unsigned char* sm) {
  using SL = SegLds<KP>;
  constexpr int NKT = KP / 16, NKS = KP / 32;
  constexpr bool BWD = DIR == 1, TRANS = MODE == kSumT;
  constexpr bool DO_TERMS = BWD && !TRANS;                            // Aqk^T dO and Qg^T dO
  constexpr bool EXACT_DO = sizeof(IT) == 2 && !__is_same(IT, f16);  // bf16 dO: its lo part is zero
  constexpr bool SPLIT = kSplitOps<IT>;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g4 = lane >> 4;
  const int nsb = seg_blocks(a, MODE);
  const int64_t bhn = a.B * a.H;
  const int64_t bh = id / nsb, b = bh / a.H, h = bh % a.H;
  const int gseg = static_cast<int>(id % nsb);
  const int Vp = a.L.Vp;
  const bool has = w < (TRANS ? NKT : Vp / 16);  // this wave's 16-column tile exists
  const int col = 16 * w + li;                     // this lane's column (value or transition)
  float* rec = a.seg + ((static_cast<int64_t>(DIR) * bhn + bh) * a.nseg + gseg) *
                           (static_cast<int64_t>(KP) * KP + 2 * static_cast<int64_t>(KP) * Vp);
  // segment g of the backward scan is the forward's segment nseg - 1 - g, run
  // from its last chunk down, so that the two directions cut the chain at the
  // same chunks (the backward's transition maps are then the forward's, transposed)
  const int fg = BWD ? a.nseg - 1 - gseg : gseg;
  const int lo = fg * a.seglen;
  const int hi = lo + a.seglen < a.NC ? lo + a.seglen : static_cast<int>(a.NC);
  const int p0 = 0, p1 = hi - lo;

  f32x4 X[NKT];
#pragma unroll
  for (int ct = 0; ct < NKT; ++ct) {
    X[ct] = zero4();
    if constexpr (TRANS) {
#pragma unroll
      for (int r = 0; r < 4; ++r) X[ct][r] = (16 * ct + 4 * g4 + r == col) ? 1.f : 0.f;
    } else if constexpr (MODE == kRun) {
      if (has) {
        const float* x0 = rec + KP * KP + KP * Vp + opaque(4 * g4 * Vp + col);  // start state from the combine
#pragma unroll
        for (int r = 0; r < 4; ++r) X[ct][r] = x0[(16 * ct + r) * Vp];
      }
    }
  }

  Rec<kC, KP, SPLIT> ra;   // forward W, backward Kt        [64][KP]
  Rec<KP, kC, SPLIT> rb;   // forward Kt^T, backward W^T    [KP][64]
  Rec<KP, kC, SPLIT> rq;   // backward Qg^T
  Rec<kC, kC, SPLIT> raq;  // backward Aqk^T
  float dval = 0.f;
  float u[4][4];    // forward value columns: U of the next chunk, accumulator layout
  DoFrag<IT> dof;   // backward value columns: dO of the next chunk
  auto chunk_of = [&](int p) -> int64_t { return BWD ? hi - 1 - p : lo + p; };
  // the next chunk's records in three parts, issued between the product
  // phases of this chunk so that each part's requests drain while the MFMAs
  // of the following phase run
  auto fetch_part = [&](int p, int part) {
    const int64_t c = chunk_of(p);
    const float* ws = a.ws + (bh * a.NC + c) * a.L.per;
    if constexpr (!BWD) {
      if (part == 0) ra.fetch(ws + a.L.Wr, tid);
      if (part == 1) {
        rb.fetch(ws + a.L.Ktt, tid);
        if (tid < KP) dval = ws[a.L.D + tid];
      }
      if (part == 2 && !TRANS && has) {
        const float* up = ws + a.L.U + opaque(4 * g4 * Vp + col);
#pragma unroll
        for (int I = 0; I < 4; ++I)
#pragma unroll
          for (int r = 0; r < 4; ++r) u[I][r] = up[(16 * I + r) * Vp];
      }
    } else {
      if (part == 0) ra.fetch(ws + a.L.Ktr, tid);
      if (part == 1) {
        rb.fetch(ws + a.L.Wt, tid);
        if constexpr (DO_TERMS) raq.fetch(ws + a.L.Aqkt, tid);
        if (tid < KP) dval = ws[a.L.D + tid];
      }
      if constexpr (DO_TERMS) {
        if (part == 2) {
          rq.fetch(ws + a.L.Qgt, tid);
          if (has) dof.fetch(a, b, h, c * kC, col, g4);
        }
      }
    }
  };
  auto fetch = [&](int p) {
    fetch_part(p, 0);
    fetch_part(p, 1);
    fetch_part(p, 2);
  };
  if (p0 < p1) fetch(p0);
  for (int p = p0; p < p1; ++p) {
    const int64_t c = chunk_of(p), t0 = c * kC;
    float* ws = a.ws + (bh * a.NC + c) * a.L.per;
    __syncthreads();  // the previous chunk's fragments are no longer read
    ra.store(sm, SL::fa, tid);
    rb.store(sm, SL::fb, tid);
    if constexpr (DO_TERMS) {
      rq.store(sm, SL::fq, tid);
      raq.store(sm, SL::faq, tid);
    }
    if (tid < KP) reinterpret_cast<float*>(sm + SL::d)[tid] = dval;
    float uc[4][4];
    bf16x8 doh[2], dol[2];
    if (!TRANS && has) {
      if constexpr (!BWD) {
#pragma unroll
        for (int I = 0; I < 4; ++I)
#pragma unroll
          for (int r = 0; r < 4; ++r) uc[I][r] = u[I][r];
      } else {
        dof.template split<SPLIT>(t0, a.T, col, a.V, g4, doh, dol);
      }
    }
    __syncthreads();
    const bool more = p + 1 < p1;
    if (!has) {  // no barrier below: idle waves go straight to the next chunk's barrier
      if (more) fetch(p + 1);
      continue;
    }
    if (more) fetch_part(p + 1, 0);

    // P = B X (forward B = W, backward B = Kt), plus Aqk^T dO (backward value
    // columns); one fragment pair ahead
    f32x4 P[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) P[I] = zero4();
    {
      bf16x8 xh[NKS], xl[NKS];
#pragma unroll
      for (int st = 0; st < NKS; ++st) split_pair<SPLIT>(X[2 * st], X[2 * st + 1], xh[st], xl[st]);
      bf16x8 fh[2], fl[2];
      fh[0] = frag_ld(sm, SL::fa, 0, 0, lane);
      if constexpr (SPLIT) fl[0] = frag_ld(sm, SL::fa, 0, 1, lane);
#pragma unroll
      for (int k = 0; k < 4 * NKS; ++k) {  // k = I * NKS + st: fragment (I, st)
        if (k + 1 < 4 * NKS) {
          fh[(k + 1) & 1] = frag_ld(sm, SL::fa, k + 1, 0, lane);
          if constexpr (SPLIT) fl[(k + 1) & 1] = frag_ld(sm, SL::fa, k + 1, 1, lane);
        }
        P[k / NKS] = mfma3<SPLIT>(fh[k & 1], fl[k & 1], xh[k % NKS], xl[k % NKS], P[k / NKS]);
      }
    }
    if constexpr (DO_TERMS) {
      bf16x8 fh[2], fl[2];
      fh[0] = frag_ld(sm, SL::faq, 0, 0, lane);
      if constexpr (SPLIT) fl[0] = frag_ld(sm, SL::faq, 0, 1, lane);
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // k = I * 2 + st
        if (k + 1 < 8) {
          fh[(k + 1) & 1] = frag_ld(sm, SL::faq, k + 1, 0, lane);
          if constexpr (SPLIT) fl[(k + 1) & 1] = frag_ld(sm, SL::faq, k + 1, 1, lane);
        }
        if constexpr (EXACT_DO) {
          P[k / 2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fh[k & 1], doh[k & 1], P[k / 2], 0, 0, 0);
          if constexpr (SPLIT)
            P[k / 2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fl[k & 1], doh[k & 1], P[k / 2], 0, 0, 0);
        } else {
          P[k / 2] = mfma3<SPLIT>(fh[k & 1], fl[k & 1], doh[k & 1], dol[k & 1], P[k / 2]);
        }
      }
    }
    if (more) fetch_part(p + 1, 1);
    // R = U - P (forward value columns) or -P
#pragma unroll
    for (int I = 0; I < 4; ++I)
#pragma unroll
      for (int r = 0; r < 4; ++r) P[I][r] = (!BWD && !TRANS ? uc[I][r] : 0.f) - P[I][r];
    if constexpr (MODE == kRun) {  // this chunk's X and R (the backward stores dVt = -R)
      const int lo = opaque(4 * g4 * Vp + col);
      if (!SPLIT && a.L.hs) {  // S, dS and Vt as bf16 (dVt stays f32)
        __bf16* xo = reinterpret_cast<__bf16*>(ws + (BWD ? a.L.dS : a.L.S)) + lo;
#pragma unroll
        for (int ct = 0; ct < NKT; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r) xo[(16 * ct + r) * Vp] = static_cast<__bf16>(X[ct][r]);
        if constexpr (BWD) {
          float* ro = ws + a.L.dVt + lo;
#pragma unroll
          for (int I = 0; I < 4; ++I)
#pragma unroll
            for (int r = 0; r < 4; ++r) ro[(16 * I + r) * Vp] = -P[I][r];
        } else {
          __bf16* ro = reinterpret_cast<__bf16*>(ws + a.L.Vt) + lo;
#pragma unroll
          for (int I = 0; I < 4; ++I)
#pragma unroll
            for (int r = 0; r < 4; ++r) ro[(16 * I + r) * Vp] = static_cast<__bf16>(P[I][r]);
        }
      } else {
        float* xo = ws + (BWD ? a.L.dS : a.L.S) + lo;
        float* ro = ws + (BWD ? a.L.dVt : a.L.Vt) + lo;
#pragma unroll
        for (int ct = 0; ct < NKT; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r) xo[(16 * ct + r) * Vp] = X[ct][r];
#pragma unroll
        for (int I = 0; I < 4; ++I)
#pragma unroll
          for (int r = 0; r < 4; ++r) ro[(16 * I + r) * Vp] = BWD ? -P[I][r] : P[I][r];
      }
    }
    // X' = D X + A^T R (forward A = Kt, backward A = W), plus Qg^T dO
    // (backward value columns); one fragment pair ahead
    bf16x8 rh[2], rl[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) split_pair<SPLIT>(P[2 * st], P[2 * st + 1], rh[st], rl[st]);
    if (more) fetch_part(p + 1, 2);
    const float* Ds = reinterpret_cast<const float*>(sm + SL::d);
#pragma unroll
    for (int ct = 0; ct < NKT; ++ct) X[ct] *= *reinterpret_cast<const f32x4*>(Ds + 16 * ct + 4 * g4);
    {
      bf16x8 fh[2], fl[2];
      fh[0] = frag_ld(sm, SL::fb, 0, 0, lane);
      if constexpr (SPLIT) fl[0] = frag_ld(sm, SL::fb, 0, 1, lane);
#pragma unroll
      for (int k = 0; k < 2 * NKT; ++k) {  // k = ct * 2 + st
        if (k + 1 < 2 * NKT) {
          fh[(k + 1) & 1] = frag_ld(sm, SL::fb, k + 1, 0, lane);
          if constexpr (SPLIT) fl[(k + 1) & 1] = frag_ld(sm, SL::fb, k + 1, 1, lane);
        }
        X[k / 2] = mfma3<SPLIT>(fh[k & 1], fl[k & 1], rh[k & 1], rl[k & 1], X[k / 2]);
      }
    }
    if constexpr (DO_TERMS) {
      bf16x8 fh[2], fl[2];
      fh[0] = frag_ld(sm, SL::fq, 0, 0, lane);
      if constexpr (SPLIT) fl[0] = frag_ld(sm, SL::fq, 0, 1, lane);
#pragma unroll
      for (int k = 0; k < 2 * NKT; ++k) {
        if (k + 1 < 2 * NKT) {
          fh[(k + 1) & 1] = frag_ld(sm, SL::fq, k + 1, 0, lane);
          if constexpr (SPLIT) fl[(k + 1) & 1] = frag_ld(sm, SL::fq, k + 1, 1, lane);
        }
        if constexpr (EXACT_DO) {
          X[k / 2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fh[k & 1], doh[k & 1], X[k / 2], 0, 0, 0);
          if constexpr (SPLIT)
            X[k / 2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fl[k & 1], doh[k & 1], X[k / 2], 0, 0, 0);
        } else {
          X[k / 2] = mfma3<SPLIT>(fh[k & 1], fl[k & 1], doh[k & 1], dol[k & 1], X[k / 2]);
        }
      }
    }
  }
  if (!has) return;
  if constexpr (MODE != kRun) {  // the segment's map: P (transition columns) or Q (value columns)
    float* dst = TRANS ? rec + opaque(4 * g4 * KP + col) : rec + KP * KP + opaque(4 * g4 * Vp + col);
    const int ld = TRANS ? KP : Vp;
#pragma unroll
    for (int ct = 0; ct < NKT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(16 * ct + r) * ld] = X[ct][r];
  } else if (gseg == a.nseg - 1 && col < a.V) {  // the final state
    float* fin = BWD ? a.ds0 : a.sT;
    if (fin != nullptr) {
#pragma unroll
      for (int ct = 0; ct < NKT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * ct + 4 * g4 + r;
          if (row < a.K) fin[((b * a.H + h) * a.K + row) * a.V + col] = X[ct][r];
        }
    }
  }
}

// Blocks [0, n) run direction dir0, blocks [n, 2n) (when ndir == 2) the
// backward direction: the two directions are independent and share the launch,
// each in its own inlined body (registers are those of the larger one).
template <class IT, int KP, int MODE>
__global__ __launch_bounds__(kSC) void seg_kernel(const Args<IT> a) {
  __shared__ __attribute__((aligned(16))) unsigned char sm[SegLds<KP>::bytes];
  const int64_t n = a.B * a.H * seg_blocks(a, MODE);
  const int64_t id = blockIdx.x;
  if constexpr (MODE == kSumT) {  // the forward's transition maps serve both directions
    seg_body<IT, KP, MODE, 0>(a, id, sm);
  } else {
    if (a.dir0 == 0 && id < n)
      seg_body<IT, KP, MODE, 0>(a, id, sm);
    else
      seg_body<IT, KP, MODE, 1>(a, id - (a.dir0 == 0 ? n : 0), sm);
  }
}

// The maps of both directions in one launch (the backward's scans): blocks
// [0, n) the backward direction's value maps (the longest: they also carry
// the dO terms), [n, 2n) the forward direction's, then the transition maps,
// which start on the CUs that the forward value maps free first (one block
// per CU; the transition maps alone would fill half the GPU).
template <class IT, int KP>
__global__ __launch_bounds__(kSC) void seg_maps_kernel(const Args<IT> a) {
  __shared__ __attribute__((aligned(16))) unsigned char sm[SegLds<KP>::bytes];
  const int64_t n = a.B * a.H * seg_blocks(a, kSumV);
  const int64_t id = blockIdx.x;
  if (id < n)
    seg_body<IT, KP, kSumV, 1>(a, id, sm);
  else if (id < 2 * n)
    seg_body<IT, KP, kSumV, 0>(a, id - n, sm);
  else
    seg_body<IT, KP, kSumT, 0>(a, id - 2 * n, sm);
}

// X_0 = the initial value (forward S0, backward dS_T; zero when absent), then
// X_{g+1} = P_g X_g + Q_g for each segment in scan order, one block per
// (direction, sequence x head, 16 value columns), f32 MFMA; the next
// segment's P and Q are loaded while the current one multiplies.  Every
// column block reads the whole P_g, so the blocks of one (sequence, head)
// take block indices equal mod 8: they run on one XCD, whose L2 serves P_g to
// all but the first (blocks go to the XCDs round-robin by index; the grid is
// padded to whole groups of 8 sequence x heads).
constexpr int kCT = 512;
constexpr int kCW = kCT / 64;  // waves; wave w takes row tiles w, w + kCW, ..
template <class IT>
__host__ __device__ inline int64_t combine_blocks(const Args<IT>& a) {
  return (a.B * a.H + 7) / 8 * 8 * (a.L.Vp / 16);
}
template <class IT, int KP, int DIR>
__device__ __forceinline__ void combine_body(const Args<IT>& a, int64_t id, float* Ps, float* Xs) {
  constexpr int PS = KP + 4, XS = 20, NP = KP * KP / 4 / kCT;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, g4 = lane >> 4;
  const int Vp = a.L.Vp, nv = Vp / 16;
  const int64_t bhn = a.B * a.H;
  const int64_t bh = (id / 8 / nv) * 8 + id % 8, b = bh / a.H, h = bh % a.H;
  if (bh >= bhn) return;  // padding of the last group
  const int col0 = 16 * static_cast<int>(id / 8 % nv);
  const int64_t segf = static_cast<int64_t>(KP) * KP + 2 * static_cast<int64_t>(KP) * Vp;
  float* base = a.seg + (static_cast<int64_t>(DIR) * bhn + bh) * a.nseg * segf;
  const float* init = DIR == 1 ? a.dsT : a.s0;
  for (int idx = tid; idx < KP * 16; idx += kCT) {
    const int r = idx >> 4, cc = idx & 15;
    const float x = (init != nullptr && r < a.K && col0 + cc < a.V) ? init[((b * a.H + h) * a.K + r) * a.V + col0 + cc]
                                                                     : 0.f;
    Xs[r * XS + cc] = x;
    base[KP * KP + KP * Vp + r * Vp + col0 + cc] = x;
  }
  f32x4 pf[NP];
  constexpr int RT = (KP / 16 + kCW - 1) / kCW;  // row tiles per wave
  float qf[RT][4];
  // the backward's transition map of its segment g is the transpose of the
  // forward's map of segment nseg - 1 - g (the same chunks): staged as it is
  // and read with the strides swapped
  const float* fwd = a.seg + bh * a.nseg * segf;
  auto fetch = [&](int gs) {
    const float* P = DIR == 1 ? fwd + (a.nseg - 1 - gs) * segf : base + gs * segf;
    const float* Q = base + gs * segf + KP * KP;
#pragma unroll
    for (int j = 0; j < NP; ++j) pf[j] = *reinterpret_cast<const f32x4*>(P + 4 * (tid + kCT * j));
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int rt = w + kCW * j;
      if (rt < KP / 16) {
#pragma unroll
        for (int r = 0; r < 4; ++r) qf[j][r] = Q[(16 * rt + 4 * g4 + r) * Vp + col0 + li];
      }
    }
  };
  if (a.nseg > 1) fetch(0);
  for (int gs = 0; gs + 1 < a.nseg; ++gs) {
    float* Xn = base + (gs + 1) * segf + KP * KP + KP * Vp;
    __syncthreads();  // the previous step's reads of P are done
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int e = 4 * (tid + kCT * j);
      *reinterpret_cast<f32x4*>(&Ps[(e / KP) * PS + e % KP]) = pf[j];
    }
    f32x4 acc[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[j][r] = qf[j][r];
    __syncthreads();
    if (gs + 2 < a.nseg) fetch(gs + 1);
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int rt = w + kCW * j;
      if (rt < KP / 16)
        acc[j] = mma_long(acc[j], DIR == 1 ? Mat{Ps, 1, PS} : Mat{Ps, PS, 1}, 16 * rt, Mat{Xs, XS, 1}, 0, KP);
    }
    __syncthreads();  // every read of X_g is done
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int rt = w + kCW * j;
      if (rt < KP / 16) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * rt + 4 * g4 + r;
          Xs[row * XS + li] = acc[j][r];
          Xn[row * Vp + col0 + li] = acc[j][r];
        }
      }
    }
  }
}

template <class IT, int KP>
__global__ __launch_bounds__(kCT) void seg_combine_kernel(const Args<IT> a) {
  __shared__ __attribute__((aligned(16))) float Ps[KP * (KP + 4)];
  __shared__ __attribute__((aligned(16))) float Xs[KP * 20];
  const int64_t n = combine_blocks(a);
  const int64_t id = blockIdx.x;
  if (a.dir0 == 0 && id < n)
    combine_body<IT, KP, 0>(a, id, Ps, Xs);
  else
    combine_body<IT, KP, 1>(a, id - (a.dir0 == 0 ? n : 0), Ps, Xs);
}

// Chunks per segment and segments per sequence: enough blocks (over the
// ndir directions that share a launch) to cover the GPU's 256 CUs.
__host__ __device__ inline int64_t seg_len(int64_t bh, int64_t NC, int ndir) {
  int64_t want = (256 + ndir * bh - 1) / (ndir * bh);
  if (want < 1) want = 1;
  if (want > NC) want = NC;
  return NC > 0 ? (NC + want - 1) / want : 1;
}
__host__ __device__ inline int seg_count(int64_t bh, int64_t NC, int ndir) {
  const int64_t len = seg_len(bh, NC, ndir);
  return static_cast<int>((NC + len - 1) / len);
}

// Segment records of ndir directions: P [KP][KP], Q and the start state [KP][Vp].
__host__ __device__ inline int64_t seg_floats(int64_t K, int64_t V, int64_t bh, int64_t NC, int ndir) {
  const Layout L = make_layout(K, V);
  return static_cast<int64_t>(ndir) * bh * seg_count(bh, NC, ndir) *
         (static_cast<int64_t>(L.Kp) * L.Kp + 2 * static_cast<int64_t>(L.Kp) * L.Vp);
}

// ---- the forward through the same chunk operands ------------------------------
// prep_kernel, then the forward scan alone (which leaves each chunk's start
// state S and pseudo-values Vt in the workspace and writes the final state),
// then out_kernel: O = Qg S + Aqk Vt per chunk, all chunks in parallel.  This
// is the chunkwise prefill for inputs the bf16 MFMA path does not take (f32
// inputs, key or value dims off its grid), at the split-bf16 accuracy of the
// scans.
constexpr int kOT = 512;  // threads of out_kernel: one 16 x 16 output tile per wave and slab
template <class IT, int KP>
__global__ __launch_bounds__(kOT) void out_kernel(const Args<IT> a) {
  __shared__ __attribute__((aligned(16))) float QgT[KP * kRC];  // Qg^T: channel-major, positions contiguous
  __shared__ __attribute__((aligned(16))) float AqT[kC * kRC];  // Aqk^T
  __shared__ __attribute__((aligned(16))) float Ss[KP * kSS];   // S slab [channel][32 columns]
  __shared__ __attribute__((aligned(16))) float Vs[kC * kSS];   // Vt slab [position][32 columns]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, lg4 = lane >> 4;
  const int64_t ch = blockIdx.x;
  const int64_t c = ch % a.NC, bh = ch / a.NC, b = bh / a.H, h = bh % a.H;
  const int64_t t0 = c * kC;
  const float* ws = a.ws + ch * a.L.per;
  // each slab's S and Vt loads go out one slab ahead (the first before the records)
  WsTile<KP, 32, kOT> ts;
  WsTile<kC, 32, kOT> tv;
  ts.fetch(ws + a.L.S, a.L.Vp, 0, tid);
  tv.fetch(ws + a.L.Vt, a.L.Vp, 0, tid);
  {  // the split records back to f32, eight elements at a time: Qgt[col * 64 + r] = Qg[r][col],
     // Aqkt[j * 64 + i] = Aqk[i][j]
    const __bf16* qg = reinterpret_cast<const __bf16*>(ws + a.L.Qgt);
    const __bf16* aq = reinterpret_cast<const __bf16*>(ws + a.L.Aqkt);
    auto unsplit = [&](const __bf16* rec, int n, float* dst) {
      constexpr int PER = kC * KP / 8 / kOT;  // the larger record (Qg); Aqk takes the first n / 8 items
      bf16x8 h[PER], l[PER];
#pragma unroll
      for (int it = 0; it < PER; ++it) {
        const int idx = 8 * (tid + kOT * it);
        if (idx < n) {
          h[it] = *reinterpret_cast<const bf16x8*>(rec + idx);
          if constexpr (kSplitOps<IT>) l[it] = *reinterpret_cast<const bf16x8*>(rec + n + idx);
        }
      }
#pragma unroll
      for (int it = 0; it < PER; ++it) {
        const int idx = 8 * (tid + kOT * it);
        if (idx < n) {
          f32x4 x0, x1;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x0[e] = static_cast<float>(h[it][e]) + (kSplitOps<IT> ? static_cast<float>(l[it][e]) : 0.f);
            x1[e] = static_cast<float>(h[it][4 + e]) + (kSplitOps<IT> ? static_cast<float>(l[it][4 + e]) : 0.f);
          }
          float* d = dst + (idx >> 6) * kRC + (idx & 63);
          *reinterpret_cast<f32x4*>(d) = x0;
          *reinterpret_cast<f32x4*>(d + 4) = x1;
        }
      }
    };
    unsplit(qg, kC * KP, QgT);
    unsplit(aq, kC * kC, AqT);
  }
  const int rt = w & 3, ct = w >> 2;
  for (int s0 = 0; s0 < a.L.Vp; s0 += 32) {
    __syncthreads();  // the previous slab's reads are done
    ts.template store<kSS>(Ss, tid);
    tv.template store<kSS>(Vs, tid);
    if (s0 + 32 < a.L.Vp) {
      ts.fetch(ws + a.L.S, a.L.Vp, s0 + 32, tid);
      tv.fetch(ws + a.L.Vt, a.L.Vp, s0 + 32, tid);
    }
    __syncthreads();
    f32x4 acc = mma_long(zero4(), Mat{QgT, 1, kRC}, 16 * rt, Mat{Ss, kSS, 1}, 16 * ct, KP);
    acc = mma_long(acc, Mat{AqT, 1, kRC}, 16 * rt, Mat{Vs, kSS, 1}, 16 * ct, kC);
    const int col = s0 + 16 * ct + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = t0 + 16 * rt + 4 * lg4 + r;
      if (t < a.T && col < a.V) a.out[tok(b, t, a.T, a.H, h) * a.V + col] = from_compute<IT>(acc[r]);
    }
  }
}

// ---- grad_body: products that reduce over the state columns --------------------
// Eight waves; slabs of 32 state columns accumulate dQg, dKt, dW (wave w:
// row tile w % 4, half w / 4 of the column tiles),
// dAqk and dM in MFMA accumulators and write dv; then dKg = M^T dW,
// dM += dW Kg^T, dbeta and dA follow from N.
constexpr int kSR = kSW + 8;                    // bf16 row stride of the split slab tiles
constexpr int kOffM = 0;                        // [64][68] f32 M = N diag(b)
constexpr int kOffSs = kOffM + kC * kRC;        // S slab split [128][kSR] x 2 planes (bf16; offsets in floats)
constexpr int kOffdSn = kOffSs + 128 * kSR;     // dS' slab split
constexpr int kOffdOs = kOffdSn + 128 * kSR;    // dO slab split [64][kSR] x 2
constexpr int kOffVts = kOffdOs + kC * kSR;     // Vt slab split
constexpr int kOffdVts = kOffVts + kC * kSR;    // dVt slab split
constexpr int kOffvs = kOffdVts + kC * kSR;     // v slab split
constexpr int kOffdVf = kOffvs + kC * kSR;      // dVt slab f32 [64][36] (the B operand of dv = M^T dVt)
constexpr int kGradFloats = kOffdVf + kC * kSS;
// second stage, over the slabs
constexpr int kOffX = kOffSs;                   // [64][132] dW
constexpr int kOffY = kOffX + kC * kRS;         // [64][132] Kg
constexpr int kOffN = kOffSs;                   // [64][68]
constexpr int kOffDM = kOffN + kC * kRC;        // [64][68] dM, then T1 = N^T dN
constexpr int kOffDN = kOffDM + kC * kRC;       // [64][68] dN, then dL
constexpr int kOffA = kOffDN + kC * kRC;        // [64][68]
static_assert(kOffY + kC * kRS <= kGradFloats, "dW and Kg must fit");
static_assert(kOffA + kC * kRC <= kGradFloats, "second-stage tiles must fit");

// One slab tile (rows x 32 columns, f32 values v for columns c4..c4+3 of row r)
// into a split tile of row stride kSR (bf16) and plane `plane` (SPLIT false:
// the hi values alone).
template <bool SPLIT = true>
__device__ __forceinline__ void put_split4(__bf16* dst, int plane, int r, int c4, f32x4 v) {
  bf16x4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    __bf16 x, y;
    split_bf16(v[e], x, y);
    hi[e] = x;
    lo[e] = y;
  }
  *reinterpret_cast<bf16x4*>(dst + r * kSR + c4) = hi;
  if constexpr (SPLIT) *reinterpret_cast<bf16x4*>(dst + plane + r * kSR + c4) = lo;
}

// A NROW x 32 workspace slab (row stride ld, from column col0), split into LDS.
template <int NROW, int NT, bool SPLIT>
__device__ __forceinline__ void load_ws_split(__bf16* dst, const float* src, int ld, int col0, int tid) {
  constexpr int PER = NROW * 8 / NT;
  static_assert(PER * NT == NROW * 8, "the tile must split evenly over the threads");
  f32x4 v[PER];
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
    v[it] = *reinterpret_cast<const f32x4*>(src + r * ld + col0 + c4);
  }
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
    put_split4<SPLIT>(dst, NROW * kSR, r, c4, v[it]);
  }
}

// A NROW x 32 bf16 workspace slab (row stride ld, from column col0) into the
// hi plane of a split tile.
template <int NROW, int NT>
__device__ __forceinline__ void load_ws_half(__bf16* dst, const float* src, int ld, int col0, int tid) {
  constexpr int PER = NROW * 8 / NT;
  static_assert(PER * NT == NROW * 8, "the tile must split evenly over the threads");
  const __bf16* p = reinterpret_cast<const __bf16*>(src);
  bf16x4 v[PER];
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
    v[it] = *reinterpret_cast<const bf16x4*>(p + r * ld + col0 + c4);
  }
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
    *reinterpret_cast<bf16x4*>(dst + r * kSR + c4) = v[it];
  }
}

// One 32-column slab of grad_body's operands in registers: the S and dS
// rows (KP x 32), Vt and dVt (64 x 32, f32 from the workspace) and dO and v
// (64 x 32 from the inputs; the whole-group case of load_rows_split).  The
// next slab's loads go out while the current one is multiplied.
template <class IT, int KP, int NT>
struct GradSlab {
  static constexpr int PS = KP * 8 / NT, PC = kC * 8 / NT;
  static_assert(PS * NT == KP * 8 && PC * NT == kC * 8, "the slab must split evenly over the threads");
  // S, dS and Vt as the workspace holds them: f32 for f32 inputs, bf16 otherwise
  // (the backward's layout for single-operand inputs, Layout::hs)
  static constexpr bool W32 = kSplitOps<IT>;
  typedef typename Pick<W32, f32x4, bf16x4>::type st_t;
  st_t s[PS], ds[PS], vt[PC];
  f32x4 dvt[PC];
  typename Raw4<IT>::type dout[PC], v[PC];
  __device__ __forceinline__ static st_t ld(const float* base, int idx) {
    if constexpr (W32) return *reinterpret_cast<const f32x4*>(base + idx);
    else return *reinterpret_cast<const bf16x4*>(reinterpret_cast<const __bf16*>(base) + idx);
  }
  __device__ __forceinline__ static void put(__bf16* dst, int plane, int r, int c4, const st_t& x) {
    if constexpr (W32) put_split4<true>(dst, plane, r, c4, x);
    else *reinterpret_cast<bf16x4*>(dst + r * kSR + c4) = x;
  }
  __device__ __forceinline__ void fetch(const Args<IT>& a, const float* ws, int64_t b, int64_t t0, int64_t h, int s0,
                                        int tid) {
    const int Vp = a.L.Vp;
#pragma unroll
    for (int it = 0; it < PS; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      s[it] = ld(ws + a.L.S, r * Vp + s0 + c4);
      ds[it] = ld(ws + a.L.dS, r * Vp + s0 + c4);
    }
#pragma unroll
    for (int it = 0; it < PC; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      vt[it] = ld(ws + a.L.Vt, r * Vp + s0 + c4);
      dvt[it] = *reinterpret_cast<const f32x4*>(ws + a.L.dVt + r * Vp + s0 + c4);
      const int64_t t = t0 + r < a.T ? t0 + r : a.T - 1;
      const int64_t row = tok(b, t, a.T, a.H, h) * a.V + s0 + c4;
      dout[it] = *reinterpret_cast<const typename Raw4<IT>::type*>(a.dout + row);
      v[it] = *reinterpret_cast<const typename Raw4<IT>::type*>(a.v + row);
    }
  }
  __device__ __forceinline__ void store(__bf16* Ss, __bf16* dSn, __bf16* Vts, __bf16* dVts, float* dVf, __bf16* dOs,
                                        __bf16* vs, int64_t t0, int64_t T, int tid) const {
#pragma unroll
    for (int it = 0; it < PS; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      put(Ss, KP * kSR, r, c4, s[it]);
      put(dSn, KP * kSR, r, c4, ds[it]);
    }
#pragma unroll
    for (int it = 0; it < PC; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      put(Vts, kC * kSR, r, c4, vt[it]);
      put_split4<W32>(dVts, kC * kSR, r, c4, dvt[it]);
      *reinterpret_cast<f32x4*>(&dVf[r * kSS + c4]) = dvt[it];
      const bool real = t0 + r < T;
      put_split4<W32>(dOs, kC * kSR, r, c4, real ? widen<IT>(dout[it]) : zero4());
      put_split4<W32>(vs, kC * kSR, r, c4, real ? widen<IT>(v[it]) : zero4());
    }
  }
};

// Columns col0 .. col0+31 of the chunk's rows of an input [B,T,H,X], split into
// LDS (zero past T and X); see load_rows.
template <class IT, int NT>
__device__ __forceinline__ void load_rows_split(__bf16* dst, const IT* src, int64_t b, int64_t t0, int64_t T,
                                                int64_t H, int64_t h, int64_t X, int col0, int tid) {
  constexpr int PER = kC * 8 / NT;
  typedef typename Raw4<IT>::type raw_t;
  if ((X & 3) == 0 && col0 + 32 <= X) {
    raw_t v[PER];
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      const int64_t t = t0 + r < T ? t0 + r : T - 1;
      v[it] = *reinterpret_cast<const raw_t*>(src + tok(b, t, T, H, h) * X + col0 + c4);
    }
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      put_split4<kSplitOps<IT>>(dst, kC * kSR, r, c4, t0 + r < T ? widen<IT>(v[it]) : zero4());
    }
  } else {
    for (int it = 0; it < PER; ++it) {
      const int item = tid + NT * it, r = item >> 3, c4 = (item & 7) * 4;
      const int64_t t = t0 + r;
      f32x4 x = zero4();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t col = col0 + c4 + u;
        x[u] = (t < T && col < X) ? to_float(src[tok(b, t, T, H, h) * X + col]) : 0.f;
      }
      put_split4<kSplitOps<IT>>(dst, kC * kSR, r, c4, x);
    }
  }
}

// sm: kGradFloats floats of LDS, bS: kC more; `early` runs when the slab
// products are done (the pair stage's input loads go out there)
struct NoOp {
  __device__ void operator()() const {}
};
template <class IT, int KP, class F = NoOp>
__device__ __forceinline__ void grad_body(const Args<IT>& a, float* sm, float* bS, const F& early = F{}) {
  constexpr int NT = 512;
  constexpr int Kp = KP, CH = KP / 32;  // K-wide column tiles per wave
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, lg4 = lane >> 4;
  const int rt = w & 3, hf = w >> 2;  // wave w: row tile rt, half hf of the column tiles
  const int64_t ch = blockIdx.x;
  const int64_t c = ch % a.NC, bh = ch / a.NC, b = bh / a.H, h = bh % a.H;
  const int64_t t0 = c * kC;
  const int Vp = a.L.Vp;
  float* ws = a.ws + ch * a.L.per;
  float* MS = sm + kOffM;
  // V a multiple of the slab width: each slab's loads are issued one slab
  // ahead, into registers; otherwise slab by slab with the edge checks.  The
  // first slab's loads go out with beta's and N's, in one round trip.
  const bool ahead = rows_fast(a.V, 0, Vp);
  GradSlab<IT, KP, NT> gs;
  if (ahead) gs.fetch(a, ws, b, t0, h, 0, tid);
  constexpr int PN = kC * kC / 4 / NT;
  f32x4 nv[PN];
#pragma unroll
  for (int it = 0; it < PN; ++it) nv[it] = *reinterpret_cast<const f32x4*>(ws + a.L.N + 4 * (tid + NT * it));
  if (tid < kC) {
    const int64_t t = t0 + tid;
    bS[tid] = t < a.T ? to_float(a.beta[tok(b, t, a.T, a.H, h)]) : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < PN; ++it) {  // M = N diag(b)
    const int idx = 4 * (tid + NT * it);
    *reinterpret_cast<f32x4*>(&MS[(idx >> 6) * kRC + (idx & 63)]) =
        nv[it] * *reinterpret_cast<const f32x4*>(&bS[idx & 63]);
  }

  f32x4 aQ[CH], aT[CH], aW[CH], aA[2], aM[2];
#pragma unroll
  for (int m = 0; m < CH; ++m) aQ[m] = aT[m] = aW[m] = zero4();
#pragma unroll
  for (int m = 0; m < 2; ++m) aA[m] = aM[m] = zero4();
  float dd = 0.f;
  __bf16 *Ss = reinterpret_cast<__bf16*>(sm + kOffSs), *dSn = reinterpret_cast<__bf16*>(sm + kOffdSn),
         *dOs = reinterpret_cast<__bf16*>(sm + kOffdOs), *Vts = reinterpret_cast<__bf16*>(sm + kOffVts),
         *dVts = reinterpret_cast<__bf16*>(sm + kOffdVts), *vs = reinterpret_cast<__bf16*>(sm + kOffvs);
  float* dVf = sm + kOffdVf;
  const SMat mS{Ss, KP * kSR, kSR}, mdS{dSn, KP * kSR, kSR}, mdO{dOs, kC * kSR, kSR}, mVt{Vts, kC * kSR, kSR},
      mdVt{dVts, kC * kSR, kSR}, mv{vs, kC * kSR, kSR};
  WsTile<kC, KP, NT> kg;
  for (int s0 = 0; s0 < Vp; s0 += kSW) {  // Vp is a multiple of the slab width
    if (ahead) {
      gs.store(Ss, dSn, Vts, dVts, dVf, dOs, vs, t0, a.T, tid);
    } else {
      if constexpr (kSplitOps<IT>) {
        load_ws_split<KP, NT, true>(Ss, ws + a.L.S, Vp, s0, tid);
        load_ws_split<KP, NT, true>(dSn, ws + a.L.dS, Vp, s0, tid);
        load_ws_split<kC, NT, true>(Vts, ws + a.L.Vt, Vp, s0, tid);
      } else {  // bf16 S, dS and Vt
        load_ws_half<KP, NT>(Ss, ws + a.L.S, Vp, s0, tid);
        load_ws_half<KP, NT>(dSn, ws + a.L.dS, Vp, s0, tid);
        load_ws_half<kC, NT>(Vts, ws + a.L.Vt, Vp, s0, tid);
      }
      load_ws_split<kC, NT, kSplitOps<IT>>(dVts, ws + a.L.dVt, Vp, s0, tid);
      load_ws<kC, kSW, kSS, NT>(dVf, ws + a.L.dVt, Vp, s0, tid);
      load_rows_split<IT, NT>(dOs, a.dout, b, t0, a.T, a.H, h, a.V, s0, tid);
      load_rows_split<IT, NT>(vs, a.v, b, t0, a.T, a.H, h, a.V, s0, tid);
    }
    if (ahead && s0 + kSW < Vp) gs.fetch(a, ws, b, t0, h, s0 + kSW, tid);
    if (s0 + kSW >= Vp) kg.fetch(ws + a.L.Kg, KP, 0, tid);  // for dM += dW Kg^T after the slabs
    __syncthreads();
    {  // dv = M^T dVt, tile (rt, hf) of the slab
      const f32x4 acc = mma(zero4(), Mat{MS, 1, kRC}, 16 * rt, Mat{dVf, kSS, 1}, 16 * hf, kC);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * rt + 4 * lg4 + r, col = s0 + 16 * hf + li;
        const int64_t t = t0 + row;
        if (t < a.T && col < a.V) a.dv[tok(b, t, a.T, a.H, h) * a.V + col] = from_compute<IT>(acc[r]);
      }
    }
    // products over the slab's 32 state columns on split-bf16 operands
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int ct = hf * CH + j;
      aQ[j] = mma3<kSplitOps<IT>>(aQ[j], mdO, 16 * rt, mS, 16 * ct, kSW);
      aT[j] = mma3<kSplitOps<IT>>(aT[j], mVt, 16 * rt, mdS, 16 * ct, kSW);
      aW[j] = mma3<kSplitOps<IT>>(aW[j], mdVt, 16 * rt, mS, 16 * ct, kSW);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ct = hf * 2 + j;
      aA[j] = mma3<kSplitOps<IT>>(aA[j], mdO, 16 * rt, mVt, 16 * ct, kSW);
      aM[j] = mma3<kSplitOps<IT>>(aM[j], mdVt, 16 * rt, mv, 16 * ct, kSW);
    }
    if (tid < Kp)
      for (int cc = 0; cc < kSW; ++cc) {
        float sv = static_cast<float>(Ss[tid * kSR + cc]), dv = static_cast<float>(dSn[tid * kSR + cc]);
        if constexpr (kSplitOps<IT>) {
          sv += static_cast<float>(Ss[KP * kSR + tid * kSR + cc]);
          dv += static_cast<float>(dSn[KP * kSR + tid * kSR + cc]);
        }
        dd += dv * sv;
      }
    __syncthreads();
  }

  // dW = -(dVt S^T) over the slabs, Kg, and the finished dQg, dKt, dAqk, dD
  float *X = sm + kOffX, *Y = sm + kOffY;
#pragma unroll
  for (int j = 0; j < CH; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * rt + 4 * lg4 + r, col = 16 * (hf * CH + j) + li;
      X[row * kRS + col] = -aW[j][r];
      ws[a.L.dQg + row * Kp + col] = aQ[j][r];
      ws[a.L.dKt + row * Kp + col] = aT[j][r];
    }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * rt + 4 * lg4 + r, col = 16 * (hf * 2 + j) + li;
      ws[a.L.dAqk + row * kC + col] = col <= row ? aA[j][r] : 0.f;
    }
  kg.template store<kRS>(Y, tid);
  if (tid < Kp) ws[a.L.dD + tid] = dd;
  __syncthreads();
  early();
  // N and A for dbeta and dA: loaded while dKg and dM are formed
  WsTile<kC, kC, NT> wn, wa;
  wn.fetch(ws + a.L.N, kC, 0, tid);
  wa.fetch(ws + a.L.A, kC, 0, tid);
#pragma unroll
  for (int j = 0; j < CH; ++j) {  // dKg = M^T dW (this stage's products on split-bf16 operands)
    const int ct = hf * CH + j;
    const f32x4 acc = mma_sb(zero4(), Mat{MS, 1, kRC}, 16 * rt, Mat{X, kRS, 1}, 16 * ct, kC);
#pragma unroll
    for (int r = 0; r < 4; ++r) ws[a.L.dKg + (16 * rt + 4 * lg4 + r) * Kp + 16 * ct + li] = acc[r];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)  // dM += dW Kg^T
    aM[j] = mma_sb(aM[j], Mat{X, kRS, 1}, 16 * rt, Mat{Y, 1, kRS}, 16 * (hf * 2 + j), Kp);
  __syncthreads();

  // dbeta and dA from N: dN = dM diag(b), T1 = N^T dN, dL = -strict(T1 N^T)
  float *NS = sm + kOffN, *DM = sm + kOffDM, *DN = sm + kOffDN, *AS = sm + kOffA;
  wn.template store<kRC>(NS, tid);
  wa.template store<kRC>(AS, tid);
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * rt + 4 * lg4 + r, col = 16 * (hf * 2 + j) + li;
      DM[row * kRC + col] = aM[j][r];
      DN[row * kRC + col] = aM[j][r] * bS[col];
    }
  __syncthreads();
  // dbeta_j = sum_i N_ij dM_ij + sum_k dL_jk A_jk: thread (j = tid / 8, p = tid % 8)
  // takes rows i = p, p + 8, .. of the first sum and columns 8p .. 8p + 7 of
  // the second; the eight parts of j are neighbouring lanes of one wave
  const int bj = tid >> 3, bp = tid & 7;
  float db = 0.f;
#pragma unroll
  for (int i = bp; i < kC; i += 8) db += NS[i * kRC + bj] * DM[i * kRC + bj];
  f32x4 t1[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    t1[j] = mma_long(zero4(), Mat{NS, 1, kRC}, 16 * rt, Mat{DN, kRC, 1}, 16 * (hf * 2 + j), kC);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) DM[(16 * rt + 4 * lg4 + r) * kRC + 16 * (hf * 2 + j) + li] = t1[j][r];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ct = hf * 2 + j;
    const f32x4 acc = mma_long(zero4(), Mat{DM, kRC, 1}, 16 * rt, Mat{NS, 1, kRC}, 16 * ct, kC);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * rt + 4 * lg4 + r, col = 16 * ct + li;
      const float dl = col < row ? -acc[r] : 0.f;
      DN[row * kRC + col] = dl;
      ws[a.L.dA + row * kC + col] = bS[row] * dl;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(&DN[bj * kRC + 8 * bp + 4 * u]);
    const f32x4 y = *reinterpret_cast<const f32x4*>(&AS[bj * kRC + 8 * bp + 4 * u]);
    db += x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) db += __shfl_xor(db, m);
  if (bp == 0) {
    const int64_t t = t0 + bj;
    if (t < a.T) a.dbeta[tok(b, t, a.T, a.H, h)] = from_compute<IT>(db);
  }
}

// ---- pair_body: pair sums with exact exponents and the final dq, dk, dg ------
// Thread (column col, part p) owns rows i = p + P m of its column (P = NT / Kp,
// RP = 64 / P rows) and forms
//   R1_i = sum_j dA_ij k_j E_ij,  R2_i = sum_j dAqk_ij k_j E_ij   (j <= i)
//   R3_j = sum_i dA_ij k_i E_ij,  R4_j = sum_i dAqk_ij q_i E_ij   (i >= j)
// then dk = R1 + R3 + R4 + e^lg dKg + e^(lg_last - lg) dKt, dq = R2 + e^lg dQg,
// d lg = k R1 - k R3 + q R2 - k R4 + Kg dKg + Qg dQg - Kt dKt (+ the last row's
// sum(Kt dKt) + D dD), and dg as its reverse cumulative sum.
// The sums run over blocks of 4P positions; a block only visits the owned rows
// it can reach (a compile-time range), and a select drops the pairs on the
// wrong side of the diagonal inside it, so no branch separates the operand
// reads.  dA and dAqk are read four positions at a time along their rows, then
// transposed in place for the second sum.
// Exact path: thread (column col, part p) owns rows i = p + P m of its column.
// Leaves d lg in qS and each thread's sum(Kt dKt) in red[p][col].
template <class IT, int KP, int NT>
__device__ __forceinline__ void pair_exact(const Args<IT>& a, const float* ws, float* kS, float* qS, float* lgS,
                                           float* dAS, float* dQS, float* red, int64_t b, int64_t h, int64_t t0,
                                           int tid) {
  constexpr int RP = kC * KP / NT;  // rows per thread
  constexpr int P = kC / RP;        // parts per column
  constexpr int JB = 4 * P;         // positions per block
  constexpr int NB = kC / JB;       // blocks
  static_assert(RP % 4 == 0 && NB * JB == kC, "rows per thread must be a multiple of 4");
  constexpr int Kp = KP;
  const int col = tid % Kp, part = tid / Kp;
  float li[RP], R1[RP], R2[RP], R3[RP], R4[RP];
#pragma unroll
  for (int m = 0; m < RP; ++m) {
    li[m] = lgS[(part + P * m) * kRS + col];
    R1[m] = R2[m] = R3[m] = R4[m] = 0.f;
  }
#pragma unroll
  for (int jb = 0; jb < NB; ++jb) {  // j-sums: rows i >= j
#pragma unroll 1
    for (int j4 = jb * JB; j4 < (jb + 1) * JB; j4 += 4) {
      f32x4 kj, lj;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kj[u] = kS[(j4 + u) * kRS + col];
        lj[u] = lgS[(j4 + u) * kRS + col];
      }
#pragma unroll
      for (int m0 = 4 * jb; m0 < RP; m0 += 4) {  // four rows at a time: reads first
        f32x4 da[4], dq[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int i = part + P * (m0 + x);
          da[x] = *reinterpret_cast<const f32x4*>(&dAS[i * kRC + j4]);
          dq[x] = *reinterpret_cast<const f32x4*>(&dQS[i * kRC + j4]);
        }
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int m = m0 + x, i = part + P * m;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float e = fast_exp(li[m] - lj[u]);
            const float ke = j4 + u <= i ? kj[u] * e : 0.f;
            R1[m] += da[x][u] * ke;
            R2[m] += dq[x][u] * ke;
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // bounds the live operands
      }
    }
  }
  __syncthreads();
  for (int idx = tid; idx < kC * kC; idx += NT) {  // transpose dA and dAqk in place
    const int r = idx >> 6, cc = idx & 63;
    if (r < cc) {
      const float x = dAS[r * kRC + cc], y = dQS[r * kRC + cc];
      dAS[r * kRC + cc] = dAS[cc * kRC + r];
      dQS[r * kRC + cc] = dQS[cc * kRC + r];
      dAS[cc * kRC + r] = x;
      dQS[cc * kRC + r] = y;
    }
  }
  __syncthreads();
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {  // i-sums: rows j <= i
#pragma unroll 1
    for (int i4 = ib * JB; i4 < (ib + 1) * JB; i4 += 4) {
      f32x4 ki4, qi4, li4;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        ki4[u] = kS[(i4 + u) * kRS + col];
        qi4[u] = qS[(i4 + u) * kRS + col];
        li4[u] = lgS[(i4 + u) * kRS + col];
      }
#pragma unroll
      for (int m0 = 0; m0 < 4 * (ib + 1) && m0 < RP; m0 += 4) {
        f32x4 da[4], dq[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int j = part + P * (m0 + x);
          da[x] = *reinterpret_cast<const f32x4*>(&dAS[j * kRC + i4]);
          dq[x] = *reinterpret_cast<const f32x4*>(&dQS[j * kRC + i4]);
        }
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int m = m0 + x, j = part + P * m;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float e = fast_exp(li4[u] - li[m]);
            const float w = i4 + u >= j ? e : 0.f;
            R3[m] += da[x][u] * ki4[u] * w;
            R4[m] += dq[x][u] * qi4[u] * w;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  const float last = lgS[(kC - 1) * kRS + col];
  __syncthreads();  // every read of q ends before d lg overwrites it
  float lastsum = 0.f;
  float gKg[RP], gKt[RP], gQg[RP];
#pragma unroll
  for (int m = 0; m < RP; ++m) {  // every load before the first store
    const int64_t rec = static_cast<int64_t>(part + P * m) * Kp + col;
    gKg[m] = ws[a.L.dKg + rec];
    gKt[m] = ws[a.L.dKt + rec];
    gQg[m] = ws[a.L.dQg + rec];
  }
#pragma unroll
  for (int m = 0; m < RP; ++m) {
    const int i = part + P * m;
    const float kv = kS[i * kRS + col], qv = qS[i * kRS + col];
    const float e = fast_exp(li[m]), te = fast_exp(last - li[m]);
    const float dKg = gKg[m], dKt = gKt[m], dQg = gQg[m];
    const float dk = R1[m] + R3[m] + R4[m] + e * dKg + te * dKt;
    const float dq = R2[m] + e * dQg;
    const float ktd = te * kv * dKt;
    qS[i * kRS + col] = kv * (R1[m] - R3[m] - R4[m]) + qv * R2[m] + e * kv * dKg + e * qv * dQg - ktd;
    lastsum += ktd;
    const int64_t t = t0 + i;
    if (t < a.T && col < a.K) {
      const int64_t off = tok(b, t, a.T, a.H, h) * a.K + col;
      a.dq[off] = from_compute<IT>(dq);
      a.dk[off] = from_compute<IT>(dk);
    }
  }
  red[part * 128 + col] = lastsum;
}

// MFMA path (NT = 512, eight waves): wave w owns rows 16J.. (J = w / 2) and
// half of the column tiles.  With r_I = lg at row 16I and i in block I,
//   R1_I = e^(lg - r_I) (dA_I,: (k e^(r_I - lg))),  R2 the same with dAqk,
//   R3_J = sum_{I >= J} e^(r_I - lg) (dA_IJ^T (k e^(lg - r_I))_I),  R4 with dAqk, q.
// Leaves d lg in qS and partial sums of Kt dKt in red[4J + g][col].
template <class IT, int KP>
__device__ __forceinline__ void pair_mfma(const Args<IT>& a, const float* ws, float* kS, float* qS, float* lgS,
                                          float* dAS, float* dQS, float* red, int64_t b, int64_t h, int64_t t0,
                                          int tid) {
  constexpr int CW = KP / 32;  // column tiles per wave
  const int w = tid >> 6, lane = tid & 63, li = lane & 15, lg4 = lane >> 4;
  const int J = w >> 1, ct0 = (w & 1) * CW;
  f32x4 R1[CW], R2[CW], R3[CW], R4[CW];
#pragma unroll
  for (int ct = 0; ct < CW; ++ct) R1[ct] = R2[ct] = R3[ct] = R4[ct] = zero4();
  {  // R1, R2 over j < 16 (J + 1): the column tiles inside the reduction loop,
     // so 2 CW independent accumulation chains keep the MFMA pipe full
    float rI[CW];
#pragma unroll
    for (int ct = 0; ct < CW; ++ct) rI[ct] = lgS[16 * J * kRS + 16 * (ct0 + ct) + li];
    for (int k0 = 0; k0 < 16 * (J + 1); k0 += 4) {
      const int j = k0 + lg4;
      const float ak = dAS[(16 * J + li) * kRC + j], aq = dQS[(16 * J + li) * kRC + j];
#pragma unroll
      for (int ct = 0; ct < CW; ++ct) {
        const int cc = 16 * (ct0 + ct) + li;
        const float bk = kS[j * kRS + cc] * fast_exp(rI[ct] - lgS[j * kRS + cc]);
        R1[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(ak, bk, R1[ct], 0, 0, 0);
        R2[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq, bk, R2[ct], 0, 0, 0);
      }
    }
  }
  // the element's gradient pieces from the grad kernel: their loads go out
  // now and land while R3 and R4 are formed
  float gKg[CW][4], gKt[CW][4], gQg[CW][4];
#pragma unroll
  for (int ct = 0; ct < CW; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t rec = static_cast<int64_t>(16 * J + 4 * lg4 + r) * KP + 16 * (ct0 + ct) + li;
      gKg[ct][r] = ws[a.L.dKg + rec];
      gKt[ct][r] = ws[a.L.dKt + rec];
      gQg[ct][r] = ws[a.L.dQg + rec];
    }
  for (int I = J; I < 4; ++I) {  // R3, R4 over rows i of block I >= J
#pragma unroll
    for (int ct = 0; ct < CW; ++ct) {
      const int cc = 16 * (ct0 + ct) + li;
      const float rI = lgS[16 * I * kRS + cc];
      f32x4 t3 = zero4(), t4 = zero4();
#pragma unroll
      for (int k0 = 0; k0 < 16; k0 += 4) {
        const int i = 16 * I + k0 + lg4;
        const float e = fast_exp(lgS[i * kRS + cc] - rI);
        t3 = __builtin_amdgcn_mfma_f32_16x16x4f32(dAS[i * kRC + 16 * J + li], kS[i * kRS + cc] * e, t3, 0, 0, 0);
        t4 = __builtin_amdgcn_mfma_f32_16x16x4f32(dQS[i * kRC + 16 * J + li], qS[i * kRS + cc] * e, t4, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sc = fast_exp(rI - lgS[(16 * J + 4 * lg4 + r) * kRS + cc]);
        R3[ct][r] += t3[r] * sc;
        R4[ct][r] += t4[r] * sc;
      }
    }
  }
  // the element's own inputs, all read before any store
  float kv[CW][4], qv[CW][4], lv[CW][4];
#pragma unroll
  for (int ct = 0; ct < CW; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * J + 4 * lg4 + r, cc = 16 * (ct0 + ct) + li;
      kv[ct][r] = kS[row * kRS + cc];
      qv[ct][r] = qS[row * kRS + cc];
      lv[ct][r] = lgS[row * kRS + cc];
    }
  __syncthreads();  // every read of q ends before d lg overwrites it
#pragma unroll
  for (int ct = 0; ct < CW; ++ct) {
    const int cc = 16 * (ct0 + ct) + li;
    const float rJ = lgS[16 * J * kRS + cc], last = lgS[(kC - 1) * kRS + cc];
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * J + 4 * lg4 + r;
      const float f1 = fast_exp(lv[ct][r] - rJ);
      const float r1 = R1[ct][r] * f1, r2 = R2[ct][r] * f1, r3 = R3[ct][r], r4 = R4[ct][r];
      const float e = fast_exp(lv[ct][r]), te = fast_exp(last - lv[ct][r]);
      const float k_ = kv[ct][r], q_ = qv[ct][r];
      const float dk = r1 + r3 + r4 + e * gKg[ct][r] + te * gKt[ct][r];
      const float dq = r2 + e * gQg[ct][r];
      const float ktd = te * k_ * gKt[ct][r];
      qS[row * kRS + cc] = k_ * (r1 - r3 - r4) + q_ * r2 + e * k_ * gKg[ct][r] + e * q_ * gQg[ct][r] - ktd;
      part += ktd;
      const int64_t t = t0 + row;
      if (t < a.T && cc < a.K) {
        const int64_t off = tok(b, t, a.T, a.H, h) * a.K + cc;
        a.dq[off] = from_compute<IT>(dq);
        a.dk[off] = from_compute<IT>(dk);
      }
    }
    red[(4 * J + lg4) * 128 + cc] = part;
  }
}

// ---- pair_body: the pair sums and the final dq, dk, dg ------------------------
//   R1_i = sum_j dA_ij k_j E_ij,  R2_i = sum_j dAqk_ij k_j E_ij   (j <= i)
//   R3_j = sum_i dA_ij k_i E_ij,  R4_j = sum_i dAqk_ij q_i E_ij   (i >= j)
// then dk = R1 + R3 + R4 + e^lg dKg + e^(lg_last - lg) dKt, dq = R2 + e^lg dQg,
// d lg = k R1 - k R3 + q R2 - k R4 + Kg dKg + Qg dQg - Kt dKt (+ the last row's
// sum(Kt dKt) + D dD), and dg as its reverse cumulative sum.  The sums run on
// the MFMA with the block factorisation of the decay unless the chunk needs
// the exact pairwise path.
// The pair kernel's LDS: k, q and lg tiles [64][kRS], dA and dAqk [64][kRC],
// and the partial sums `red` [16][128], kPairFloats floats in this order.
constexpr int kPairFloats = 3 * kC * kRS + 2 * kC * kRC + 16 * 128;
// PRE: k, q and g of the chunk arrive in rk, rq, rg (fetched during the
// gradient stage) when their rows take the whole-group path
template <class IT, int KP, int NT, bool PRE>
__device__ __forceinline__ void pair_body(const Args<IT>& a, float* lds, const RowTile<IT, KP, NT>& rk,
                                          const RowTile<IT, KP, NT>& rq, const RowTile<IT, KP, NT>& rg) {
  static_assert(NT == 512, "the MFMA path uses eight waves");
  float *kS = lds, *qS = kS + kC * kRS, *lgS = qS + kC * kRS, *dAS = lgS + kC * kRS, *dQS = dAS + kC * kRC;
  float* red = dQS + kC * kRC;
  const int tid = threadIdx.x;
  const int64_t ch = blockIdx.x;
  const int64_t c = ch % a.NC, bh = ch / a.NC, b = bh / a.H, h = bh % a.H;
  const int64_t t0 = c * kC;
  const float* ws = a.ws + ch * a.L.per;
  {
    // dA and dAqk go out first (no branch), then k, q, g: one round trip
    constexpr int PW = kC * (kC / 4) / NT;
    f32x4 wa[PW], wq[PW];
#pragma unroll
    for (int it = 0; it < PW; ++it) {
      const int item = tid + NT * it, r = item / (kC / 4), c4 = (item % (kC / 4)) * 4;
      wa[it] = *reinterpret_cast<const f32x4*>(ws + a.L.dA + r * kC + c4);
      wq[it] = *reinterpret_cast<const f32x4*>(ws + a.L.dAqk + r * kC + c4);
    }
    if (PRE && rows_fast(a.K, 0, KP)) {
      rk.template store<kRS>(kS, t0, a.T, tid);
      rq.template store<kRS>(qS, t0, a.T, tid);
      rg.template store<kRS>(lgS, t0, a.T, tid);
    } else {
      load_kqg<IT, KP, NT>(kS, qS, lgS, a, b, t0, h, tid, a.T);
    }
#pragma unroll
    for (int it = 0; it < PW; ++it) {
      const int item = tid + NT * it, r = item / (kC / 4), c4 = (item % (kC / 4)) * 4;
      *reinterpret_cast<f32x4*>(&dAS[r * kRC + c4]) = wa[it];
      *reinterpret_cast<f32x4*>(&dQS[r * kRC + c4]) = wq[it];
    }
  }
  __syncthreads();
  const bool rising = chunk_cumsum<KP>(lgS, red, tid);  // red is written later
  int nred;
  if (!needs_exact<KP, NT>(lgS, rising, tid)) {
    pair_mfma<IT, KP>(a, ws, kS, qS, lgS, dAS, dQS, red, b, h, t0, tid);
    nred = 16;
  } else {
    pair_exact<IT, KP, NT>(a, ws, kS, qS, lgS, dAS, dQS, red, b, h, t0, tid);
    nred = kC / (kC * KP / NT);
  }
  __syncthreads();
  {  // dg = reverse cumulative sum of d lg, by quarters of 16 rows (totals through kS)
    const int cc = tid % KP, p = tid / KP;
    float v[16];
    if (p < 4) {
#pragma unroll
      for (int r = 15; r >= 0; --r) v[r] = qS[(16 * p + r) * kRS + cc] + (r < 15 ? v[r + 1] : 0.f);
      kS[p * 128 + cc] = v[0];
    }
    __syncthreads();
    if (p < 4) {
      float run = fast_exp(lgS[(kC - 1) * kRS + cc]) * ws[a.L.dD + cc];
      for (int q = 0; q < nred; ++q) run += red[q * 128 + cc];
      for (int q = p + 1; q < 4; ++q) run += kS[q * 128 + cc];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t t = t0 + 16 * p + r;
        if (t < a.T && cc < a.K) a.dg[tok(b, t, a.T, a.H, h) * a.K + cc] = from_compute<IT>(v[r] + run);
      }
    }
  }
}

// ---- grad_pair_kernel: grad_body, then pair_body on the same chunk ------------
// The gradient records grad_body writes (dQg, dKt, dKg, dA, dAqk, dD: 128 KB
// per chunk at K=V=128) are read back by pair_body in the same workgroup right
// after, while they are still in this XCD's L2, instead of by a second kernel
// from HBM.  The two bodies use one LDS buffer in turn.
constexpr int kGradPairFloats = kGradFloats + kC > kPairFloats ? kGradFloats + kC : kPairFloats;
template <class IT, int KP>
__global__ __launch_bounds__(512) void grad_pair_kernel(const Args<IT> a) {
  __shared__ __attribute__((aligned(16))) float lds[kGradPairFloats];
  // single-operand inputs fetch the pair stage's k, q, g while the gradient
  // stage forms dKg, dM, dbeta and dA (registers allow it; f32 inputs load
  // them in the pair stage)
  constexpr bool kPre = !kSplitOps<IT>;
  RowTile<IT, KP, 512> rk, rq, rg;
  const int64_t ch = blockIdx.x, c = ch % a.NC, bh = ch / a.NC, b = bh / a.H, h = bh % a.H;
  auto early = [&] {
    if (kPre && rows_fast(a.K, 0, KP)) {
      rk.fetch(a.k, b, c * kC, a.T, a.H, h, a.K, 0, threadIdx.x);
      rq.fetch(a.q, b, c * kC, a.T, a.H, h, a.K, 0, threadIdx.x);
      rg.fetch(a.g, b, c * kC, a.T, a.H, h, a.K, 0, threadIdx.x);
    }
  };
  grad_body<IT, KP>(a, lds, lds + kGradFloats, early);
  __syncthreads();  // every record written and every LDS read of grad_body done
  pair_body<IT, KP, 512, kPre>(a, lds, rk, rq, rg);
}


// ---- rows moved between a caller's tensor and a dense zero-padded batch ------
// The split-bf16 chunk path runs dense batches [N, T, H, *].  Packed
// documents are gathered into one (each document a row of T = the longest
// document's tokens, zero past its length), and value widths past 128 run as
// independent column slices of at most 128 (state and value columns never
// interact).  Row d of the dense side is token p = d / R (R rows per token),
// sub-row j = d % R; with packed offsets, p is (document b = p / T, token
// t = p % T) and maps to the caller's row (cu[b] + t) R + j, dropped
// (zero-filled on a gather, skipped on a scatter) when t passes the
// document's length; without offsets the dense row is the caller's row.
struct RowMove {
  const char* src;
  char* dst;
  int64_t src_stride, dst_stride;  // bytes between consecutive rows
  int64_t n_rows;                  // rows of the dense side
  int64_t T, R;
  const int32_t* cu;               // [N+1] packed offsets, or null
  int64_t upr;                     // units per row
  int scatter;                     // 0: caller -> dense, 1: dense -> caller
};

template <class U>
__global__ __launch_bounds__(256) void move_rows_kernel(const RowMove m) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= m.n_rows * m.upr) return;
  const int64_t d = i / m.upr;
  const int64_t u = i - d * m.upr;
  int64_t r = d;
  bool live = true;
  if (m.cu != nullptr) {
    const int64_t p = d / m.R, j = d - p * m.R;
    const int64_t b = p / m.T, t = p - b * m.T;
    const int64_t start = m.cu[b];
    live = t < static_cast<int64_t>(m.cu[b + 1]) - start;
    r = (start + t) * m.R + j;
  }
  if (!m.scatter) {
    U x{};
    if (live) x = reinterpret_cast<const U*>(m.src + r * m.src_stride)[u];
    reinterpret_cast<U*>(m.dst + d * m.dst_stride)[u] = x;
  } else if (live) {
    reinterpret_cast<U*>(m.dst + r * m.dst_stride)[u] = reinterpret_cast<const U*>(m.src + d * m.src_stride)[u];
  }
}

// Document lengths from packed offsets.
__global__ __launch_bounds__(256) void doc_lengths_kernel(const int32_t* cu, int64_t N, int32_t* len) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b < N) len[b] = cu[b + 1] - cu[b];
}

}  // namespace bwd
}  // namespace kda

namespace kda_host {

using namespace kda;

size_t chunk_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int in_dtype) {
  if (in_dtype == KDA_DTYPE_F64) return chunk_bwd_f64_workspace_bytes(B, T, H, K, V);
  // bf16 and f16 inputs keep the single-operand records (bwd::kSplitOps)
  const bwd::Layout L = bwd::make_layout(K, V, true, in_dtype == KDA_DTYPE_F32);
  const int64_t nc = (T + bwd::kC - 1) / bwd::kC;
  return static_cast<size_t>(B * H * nc * L.per + bwd::seg_floats(K, V, B * H, nc, 2)) * sizeof(float);
}

size_t chunk_split_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int in_dtype) {
  const bwd::Layout L = bwd::make_layout(K, V, false, in_dtype == KDA_DTYPE_F32);
  const int64_t nc = (T + bwd::kC - 1) / bwd::kC;
  return static_cast<size_t>(B * H * nc * L.per + bwd::seg_floats(K, V, B * H, nc, 1)) * sizeof(float);
}

// The segment geometry and records of the scans (after the chunk records).
// The scans of directions 0 .. ndir - 1 (forward, then backward) share
// their launches.
template <class IT>
static void set_segments(bwd::Args<IT>& a, int ndir) {
  a.dir0 = 0;
  a.ndir = ndir;
  a.seglen = static_cast<int>(bwd::seg_len(a.B * a.H, a.NC, ndir));
  a.nseg = bwd::seg_count(a.B * a.H, a.NC, ndir);
  a.seg = a.ws + a.B * a.H * a.NC * a.L.per;
}

// Both phases and the combine of the segmented scans.
template <class IT, int KP>
static void launch_scans(const bwd::Args<IT>& a, hipStream_t s) {
  const int64_t bh = a.B * a.H * a.ndir;
  if (a.nseg > 1 && a.ndir == 2) {  // value maps of both directions and the transition maps together
    hipLaunchKernelGGL((bwd::seg_maps_kernel<IT, KP>),
                       dim3(static_cast<unsigned>(bh * (a.nseg - 1) + a.B * a.H * bwd::seg_blocks(a, bwd::kSumT))),
                       dim3(bwd::kSC), 0, s, a);
  } else if (a.nseg > 1) {
    hipLaunchKernelGGL((bwd::seg_kernel<IT, KP, bwd::kSumV>), dim3(static_cast<unsigned>(bh * (a.nseg - 1))),
                       dim3(bwd::kSC), 0, s, a);
    // transition maps: the forward direction's, which the backward reads transposed
    hipLaunchKernelGGL((bwd::seg_kernel<IT, KP, bwd::kSumT>),
                       dim3(static_cast<unsigned>(a.B * a.H * bwd::seg_blocks(a, bwd::kSumT))), dim3(bwd::kSC), 0, s,
                       a);
  }
  hipLaunchKernelGGL((bwd::seg_combine_kernel<IT, KP>), dim3(static_cast<unsigned>(a.ndir * bwd::combine_blocks(a))),
                     dim3(bwd::kCT), 0, s, a);
  hipLaunchKernelGGL((bwd::seg_kernel<IT, KP, bwd::kRun>), dim3(static_cast<unsigned>(bh * a.nseg)), dim3(bwd::kSC),
                     0, s, a);
}

bool chunk_split_path(int in_dtype, int state_dtype, int64_t K, int64_t V) {
  return (in_dtype == KDA_DTYPE_BF16 || in_dtype == KDA_DTYPE_F16 || in_dtype == KDA_DTYPE_F32) &&
         state_dtype == KDA_DTYPE_F32 && K >= 1 && K <= 128 && V >= 1 && V <= 128;
}

template <class IT, int KP>
static void launch_split(const bwd::Args<IT>& a, dim3 chunks, hipStream_t s) {
  hipLaunchKernelGGL((bwd::prep_kernel<IT, KP>), chunks, dim3(bwd::kPT), 0, s, a);
  launch_scans<IT, KP>(a, s);
  hipLaunchKernelGGL((bwd::out_kernel<IT, KP>), chunks, dim3(bwd::kOT), 0, s, a);
}

template <class IT>
static int run_split(const IT* q, const IT* k, const IT* v, const IT* g, const IT* beta, const float* s0, float* sT,
                     IT* out, const int32_t* valid, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, float* ws,
                     hipStream_t s) {
  bwd::Args<IT> a{};
  a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta, a.s0 = s0;
  a.ws = ws, a.B = B, a.T = T, a.H = H, a.K = K, a.V = V, a.NC = (T + bwd::kC - 1) / bwd::kC;
  a.L = bwd::make_layout(K, V, false, bwd::kSplitOps<IT>);  // the forward's records only (no dO)
  a.valid = valid, a.sT = sT, a.out = out;
  set_segments(a, 1);
  const int64_t chunks = B * H * a.NC;
  if (chunks > 0x7fffffffLL || B * H * a.nseg > 0x7fffffffLL || bwd::combine_blocks(a) > 0x7fffffffLL) {
    set_detail("chunk_fwd: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  const dim3 gc(static_cast<unsigned>(chunks));
  if (a.L.Kp == 64)
    launch_split<IT, 64>(a, gc, s);
  else
    launch_split<IT, 128>(a, gc, s);
  return check_launch("chunk_fwd (split-bf16 chunk path)");
}

int launch_chunk_split(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                       const float* s_in, float* s_out, void* out, const int32_t* valid_lens, int64_t B, int64_t T,
                       int64_t H, int64_t K, int64_t V, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!chunk_split_path(in_dtype, KDA_DTYPE_F32, K, V) || B <= 0 || T <= 0 || H <= 0) {
    set_detail("chunk_fwd: the split-bf16 chunk path needs bf16/f16/f32 inputs, K and V in 1..128 and T > 0");
    return KDA_ERR_UNSUPPORTED;
  }
  if (workspace == nullptr || workspace_bytes < chunk_split_workspace_bytes(B, T, H, K, V, in_dtype)) {
    set_detail("chunk_fwd: workspace of %zu bytes needed", chunk_split_workspace_bytes(B, T, H, K, V, in_dtype));
    return KDA_ERR_WORKSPACE;
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    set_detail("chunk_fwd: workspace must be 16-byte aligned");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  float* ws = static_cast<float*>(workspace);
  switch (in_dtype) {
    case KDA_DTYPE_BF16:
      return run_split(static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                       static_cast<const bf16*>(g), static_cast<const bf16*>(beta), s_in, s_out, static_cast<bf16*>(out),
                       valid_lens, B, T, H, K, V, ws, stream);
    case KDA_DTYPE_F16:
      return run_split(static_cast<const f16*>(q), static_cast<const f16*>(k), static_cast<const f16*>(v),
                       static_cast<const f16*>(g), static_cast<const f16*>(beta), s_in, s_out, static_cast<f16*>(out),
                       valid_lens, B, T, H, K, V, ws, stream);
    default:
      return run_split(static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
                       static_cast<const float*>(g), static_cast<const float*>(beta), s_in, s_out,
                       static_cast<float*>(out), valid_lens, B, T, H, K, V, ws, stream);
  }
}

template <class IT, int KP>
static void launch_all(const bwd::Args<IT>& a, dim3 chunks, hipStream_t s) {
  hipLaunchKernelGGL((bwd::prep_kernel<IT, KP>), chunks, dim3(bwd::kPT), 0, s, a);
  launch_scans<IT, KP>(a, s);
  hipLaunchKernelGGL((bwd::grad_pair_kernel<IT, KP>), chunks, dim3(512), 0, s, a);
}

template <class IT>
static int run_bwd(bwd::Args<IT> a, hipStream_t s) {
  set_segments(a, 2);
  const int64_t chunks = a.B * a.H * a.NC;
  if (chunks > 0x7fffffffLL || 2 * a.B * a.H * a.nseg > 0x7fffffffLL || 2 * bwd::combine_blocks(a) > 0x7fffffffLL) {
    set_detail("chunk backward: grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  const dim3 gc(static_cast<unsigned>(chunks));
  if (a.L.Kp == 64)
    launch_all<IT, 64>(a, gc, s);
  else
    launch_all<IT, 128>(a, gc, s);
  return check_launch("chunk backward");
}

int launch_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                     const void* dout, int in_dtype, const float* s0, const float* dsT, void* dq, void* dk, void* dv,
                     void* dg, void* dbeta, float* ds0, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (K > 128 || V > 128) {
    set_detail("chunk backward: key_dim and value_dim must be <= 128 (got %lld, %lld)", (long long)K, (long long)V);
    return KDA_ERR_UNSUPPORTED;
  }
  const size_t need = chunk_bwd_workspace_bytes(B, T, H, K, V, in_dtype);
  if (workspace == nullptr || workspace_bytes < need) {
    set_detail("chunk backward: workspace of %zu bytes needed", need);
    return KDA_ERR_WORKSPACE;
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    set_detail("chunk backward: workspace must be 16-byte aligned");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (in_dtype == KDA_DTYPE_F64)  // f64 arithmetic throughout (kda_chunk_bwd_f64.hip); states are f64 too
    return launch_chunk_bwd_f64(static_cast<const double*>(q), static_cast<const double*>(k),
                                static_cast<const double*>(v), static_cast<const double*>(g),
                                static_cast<const double*>(beta), static_cast<const double*>(dout),
                                reinterpret_cast<const double*>(s0), reinterpret_cast<const double*>(dsT),
                                static_cast<double*>(dq), static_cast<double*>(dk), static_cast<double*>(dv),
                                static_cast<double*>(dg), static_cast<double*>(dbeta), reinterpret_cast<double*>(ds0),
                                B, T, H, K, V, static_cast<double*>(workspace), stream);
  // single-operand records for bf16 and f16 inputs
  const bwd::Layout L = bwd::make_layout(K, V, true, in_dtype == KDA_DTYPE_F32);
  const int64_t NC = (T + bwd::kC - 1) / bwd::kC;
  float* ws = static_cast<float*>(workspace);
  switch (in_dtype) {
    case KDA_DTYPE_BF16:
      return run_bwd(bwd::Args<bf16>{static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                                     static_cast<const bf16*>(v), static_cast<const bf16*>(g),
                                     static_cast<const bf16*>(beta), static_cast<const bf16*>(dout), s0, dsT,
                                     static_cast<bf16*>(dq), static_cast<bf16*>(dk), static_cast<bf16*>(dv),
                                     static_cast<bf16*>(dg), static_cast<bf16*>(dbeta), ds0, ws, B, T, H, K, V, NC, L},
                     stream);
    case KDA_DTYPE_F16:
      return run_bwd(bwd::Args<f16>{static_cast<const f16*>(q), static_cast<const f16*>(k),
                                    static_cast<const f16*>(v), static_cast<const f16*>(g),
                                    static_cast<const f16*>(beta), static_cast<const f16*>(dout), s0, dsT,
                                    static_cast<f16*>(dq), static_cast<f16*>(dk), static_cast<f16*>(dv),
                                    static_cast<f16*>(dg), static_cast<f16*>(dbeta), ds0, ws, B, T, H, K, V, NC, L},
                     stream);
    case KDA_DTYPE_F32:
      return run_bwd(bwd::Args<float>{static_cast<const float*>(q), static_cast<const float*>(k),
                                      static_cast<const float*>(v), static_cast<const float*>(g),
                                      static_cast<const float*>(beta), static_cast<const float*>(dout), s0, dsT,
                                      static_cast<float*>(dq), static_cast<float*>(dk), static_cast<float*>(dv),
                                      static_cast<float*>(dg), static_cast<float*>(dbeta), ds0, ws, B, T, H, K, V,
                                      NC, L},
                     stream);
    default:
      set_detail("chunk backward: inputs must be bf16, f16 or f32 (dtype %d)", in_dtype);
      return KDA_ERR_UNSUPPORTED;
  }
}


// ---- the split path over packed documents and value slices -----------------
static int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }
static int64_t elem_bytes(int in_dtype) { return in_dtype == KDA_DTYPE_F32 ? 4 : 2; }
static constexpr int64_t kSliceCols = 128;  // value columns per slice of the split path

bool chunk_split_general(int in_dtype, int state_dtype, int64_t K, int64_t V) {
  return (in_dtype == KDA_DTYPE_BF16 || in_dtype == KDA_DTYPE_F16 || in_dtype == KDA_DTYPE_F32) &&
         state_dtype == KDA_DTYPE_F32 && K >= 1 && K <= 128 && V >= 1;
}

size_t chunk_split_general_workspace_bytes(int64_t N, int64_t T, int64_t H, int64_t K, int64_t V, int in_dtype,
                                           bool packed) {
  const int64_t e = elem_bytes(in_dtype);
  const bool sliced = V > kSliceCols;
  const int64_t w = sliced ? kSliceCols : V;
  int64_t bytes = static_cast<int64_t>(chunk_split_workspace_bytes(N, T, H, K, w, in_dtype));
  if (packed) bytes += 3 * align256(N * T * H * K * e) + align256(N * T * H * e) + align256(N * 4);
  if (packed || sliced) bytes += 2 * align256(N * T * H * w * e);
  if (sliced) bytes += 2 * align256(N * H * K * w * 4);
  return static_cast<size_t>(bytes);
}

// Moves n_rows rows of row_bytes bytes (see bwd::RowMove), in the widest unit
// that divides the row, both strides and both addresses.
static int move_rows(const void* src, int64_t src_stride, void* dst, int64_t dst_stride, int64_t row_bytes,
                     int64_t n_rows, int64_t T, int64_t R, const int32_t* cu, bool scatter, hipStream_t s) {
  if (n_rows <= 0 || row_bytes <= 0) return KDA_OK;
  const uintptr_t all = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) |
                        static_cast<uintptr_t>(src_stride) | static_cast<uintptr_t>(dst_stride) |
                        static_cast<uintptr_t>(row_bytes);
  const int unit = all % 16 == 0 ? 16 : all % 4 == 0 ? 4 : 2;
  bwd::RowMove m{static_cast<const char*>(src), static_cast<char*>(dst), src_stride, dst_stride, n_rows, T, R, cu,
                 row_bytes / unit, scatter ? 1 : 0};
  const int64_t blocks = (n_rows * m.upr + 255) / 256;
  if (blocks > 0x7fffffffLL) {
    set_detail("chunk_fwd: gather grid too large");
    return KDA_ERR_UNSUPPORTED;
  }
  const dim3 grid(static_cast<unsigned>(blocks));
  if (unit == 16)
    hipLaunchKernelGGL(bwd::move_rows_kernel<uint4>, grid, dim3(256), 0, s, m);
  else if (unit == 4)
    hipLaunchKernelGGL(bwd::move_rows_kernel<uint32_t>, grid, dim3(256), 0, s, m);
  else
    hipLaunchKernelGGL(bwd::move_rows_kernel<uint16_t>, grid, dim3(256), 0, s, m);
  return check_launch("move_rows_kernel");
}

int launch_chunk_split_general(const void* q, const void* k, const void* v, const void* g, const void* beta,
                               int in_dtype, const float* s_in, float* s_out, void* out, const int32_t* cu_seqlens,
                               const int32_t* valid_lens, int64_t N, int64_t T, int64_t total_tokens, int64_t H,
                               int64_t K, int64_t V, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (cu_seqlens != nullptr && (T * N < total_tokens || (N == 1 && T != total_tokens))) {
    // the padded batch holds N x T tokens: T must be the longest document
    set_detail("chunk_fwd: packed documents off the MFMA path need the longest document's length in dense_span "
               "(got %lld for %lld documents of %lld tokens)", (long long)T, (long long)N, (long long)total_tokens);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  // one packed document spanning every token is the dense batch itself
  if (cu_seqlens != nullptr && N == 1) cu_seqlens = nullptr;
  const bool packed = cu_seqlens != nullptr;
  const bool sliced = V > kSliceCols;
  if (!packed && !sliced)
    return launch_chunk_split(q, k, v, g, beta, in_dtype, s_in, s_out, out, valid_lens, N, T, H, K, V, workspace,
                              workspace_bytes, stream);
  if (!chunk_split_general(in_dtype, KDA_DTYPE_F32, K, V) || N <= 0 || T <= 0 || H <= 0) {
    set_detail("chunk_fwd: the split-bf16 chunk path needs bf16/f16/f32 inputs, K in 1..128 and T > 0");
    return KDA_ERR_UNSUPPORTED;
  }
  if (packed && valid_lens != nullptr) {
    set_detail("chunk_fwd: packed documents take no right-padding lengths");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (workspace == nullptr || workspace_bytes < chunk_split_general_workspace_bytes(N, T, H, K, V, in_dtype, packed)) {
    set_detail("chunk_fwd: workspace of %zu bytes needed",
               chunk_split_general_workspace_bytes(N, T, H, K, V, in_dtype, packed));
    return KDA_ERR_WORKSPACE;
  }
  const int64_t e = elem_bytes(in_dtype);
  const int64_t w = sliced ? kSliceCols : V;
  char* p = static_cast<char*>(workspace);
  auto take = [&](int64_t bytes) {
    char* r = p;
    p += align256(bytes);
    return r;
  };
  char* split_ws = take(static_cast<int64_t>(chunk_split_workspace_bytes(N, T, H, K, w, in_dtype)));
  const int64_t rows = N * T;  // dense tokens
  const void *dq = q, *dk = k, *dg = g, *db = beta;
  const int32_t* valid = valid_lens;
  int st = KDA_OK;
  if (packed) {
    char* gq = take(rows * H * K * e);
    char* gk = take(rows * H * K * e);
    char* gg = take(rows * H * K * e);
    char* gb = take(rows * H * e);
    int32_t* len = reinterpret_cast<int32_t*>(take(N * 4));
    const int64_t kb = H * K * e;
    if ((st = move_rows(q, kb, gq, kb, kb, rows, T, 1, cu_seqlens, false, stream)) != KDA_OK) return st;
    if ((st = move_rows(k, kb, gk, kb, kb, rows, T, 1, cu_seqlens, false, stream)) != KDA_OK) return st;
    if ((st = move_rows(g, kb, gg, kb, kb, rows, T, 1, cu_seqlens, false, stream)) != KDA_OK) return st;
    if ((st = move_rows(beta, H * e, gb, H * e, H * e, rows, T, 1, cu_seqlens, false, stream)) != KDA_OK) return st;
    hipLaunchKernelGGL(bwd::doc_lengths_kernel, dim3(static_cast<unsigned>((N + 255) / 256)), dim3(256), 0, stream,
                       cu_seqlens, N, len);
    if ((st = check_launch("doc_lengths_kernel")) != KDA_OK) return st;
    dq = gq, dk = gk, dg = gg, db = gb, valid = len;
  }
  char* gv = take(rows * H * w * e);
  char* go = take(rows * H * w * e);
  char* gs_in = sliced ? take(N * H * K * w * 4) : nullptr;
  char* gs_out = sliced ? take(N * H * K * w * 4) : nullptr;
  const size_t split_bytes = chunk_split_workspace_bytes(N, T, H, K, w, in_dtype);
  for (int64_t c0 = 0; c0 < V; c0 += w) {
    const int64_t wc = V - c0 < w ? V - c0 : w;
    // value rows of this slice: one per (token, head), wc columns of V
    if ((st = move_rows(static_cast<const char*>(v) + c0 * e, V * e, gv, wc * e, wc * e, rows * H, T, H,
                        cu_seqlens, false, stream)) != KDA_OK)
      return st;
    const float* si = s_in;
    float* so = s_out;
    if (sliced) {
      // state rows of this slice: one per (sequence, head, key), wc columns of V
      if (s_in != nullptr &&
          (st = move_rows(s_in + c0, V * 4, gs_in, wc * 4, wc * 4, N * H * K, 1, 1, nullptr, false, stream)) != KDA_OK)
        return st;
      si = s_in != nullptr ? reinterpret_cast<const float*>(gs_in) : nullptr;
      so = s_out != nullptr ? reinterpret_cast<float*>(gs_out) : nullptr;
    }
    if ((st = launch_chunk_split(dq, dk, gv, dg, db, in_dtype, si, so, go, valid, N, T, H, K, wc, split_ws,
                                 split_bytes, stream)) != KDA_OK)
      return st;
    if ((st = move_rows(go, wc * e, static_cast<char*>(out) + c0 * e, V * e, wc * e, rows * H, T, H, cu_seqlens,
                        true, stream)) != KDA_OK)
      return st;
    if (sliced && s_out != nullptr &&
        (st = move_rows(gs_out, wc * 4, s_out + c0, V * 4, wc * 4, N * H * K, 1, 1, nullptr, true, stream)) != KDA_OK)
      return st;
  }
  return KDA_OK;
}

}  // namespace kda_host
