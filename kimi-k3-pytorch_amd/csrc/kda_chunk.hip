// Chunkwise KDA prefill on gfx950 bf16 MFMA (chunk C = 64, K = 128).
//
// Reference algorithm: src/kda/chunkwise.py:61-102 with the UT transform of
// src/kda/ut_transform.py:23-58.  For one chunk (rows i, j = 0..63, key
// channels c, lg = inclusive cumsum of g inside the chunk):
//   A_ij   = sum_c k_i k_j exp(lg_i - lg_j)            j <  i   (strict)
//   Aqk_ij = sum_c q_i k_j exp(lg_i - lg_j)            j <= i
//   L = I + diag(beta) A ;  [W | U] = L^{-1} diag(beta) [exp(lg) k | v]
//   V~ = U - W S ;  O = (exp(lg) q) S + Aqk V~ ;  S <- diag(exp lg_63) S + (exp(lg_63 - lg) k)^T V~
//
// Two kernels:
//  * kda_chunk_prepare: one workgroup per (chunk, head), fully parallel.
//    Computes the decay factors, A and Aqk on MFMA, the blocked
//    forward-substitution solve, and writes a per-chunk record whose
//    operands are already in MFMA fragment order (see "record layout").
//  * kda_chunk_scan: one wave per (sequence, head, 16-column V tile) walks
//    the chunks in order with its state slice S[:, 16 cols] in MFMA
//    accumulator registers (f32).  The accumulator layout of S converts to
//    the B-operand layout of the next product without any data movement: a
//    C tile lane holds rows 4g..4g+3 of one column, so two consecutive row
//    tiles give the 8 values a 16x16x32 B operand needs, with the reduction
//    index permuted; the A operands are stored pre-permuted to match.
//
// Numerical scheme for the decays (per-channel, any g <= 0):
//   alpha_j = exp(g_j); within each 16-row block J the running products
//   a_j = exp(lg_j - lg_{16J}) and E_j = exp(lg_{16J+15} - lg_j) are <= 1.
//   Off-diagonal blocks J < I use (k_i a_i) . (k_j E_j D_IJ) with
//   D_IJ = exp(lg_{16I} - lg_{16J+15}) <= 1; diagonal blocks use
//   (k_i a_i) . (k_j E_j / P_I) with P_I = exp(lg_{16I+15} - lg_{16I}).
//   No factor overflows unless a block decays by more than 2^-100; such
//   chunks take an exact pairwise-exponent path for the diagonal blocks (the
//   reference evaluates every tile with an explicit pairwise exponent,
//   src/kda/utils.py:128-136).
#include "kda_launch.h"

namespace kda {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;
constexpr int kKey = 128;
constexpr int kPrepThreads = 256;
constexpr float kExtremeDecay = 7.888609052210118e-31f;  // 2^-100

// ---- record layout (bytes, per chunk and head) ----------------------------
//  W   [I=4][s=4][lane=64][8] bf16 : A fragments of W (token tile I, channel step s)
//  Q   [I=4][s=4][lane=64][8] bf16 : A fragments of exp(lg) q
//  KT  [ct=8][s'=2][lane=64][8] bf16 : A fragments of (exp(lg_63 - lg) k)^T
//  A   [I=4][s'=2][lane=64][8] bf16 : A fragments of Aqk (token tile I, token step s')
//  U   [vt=V/16][I=4][lane=64][4] bf16 : C tiles of U (accumulator init of V~)
//  GAM [128] f32 : exp(lg_63) per key channel
// Fragment element e of lane (i, g) covers reduction index
//   32 s + (e < 4 ? 4 g + e : 16 + 4 g + e - 4),
// the order in which two stacked C tiles provide a B operand.
constexpr int64_t kRecW = 0;
constexpr int64_t kRecQ = 16384;
constexpr int64_t kRecKT = 32768;
constexpr int64_t kRecA = 49152;
constexpr int64_t kRecU = 57344;
__host__ __device__ constexpr int64_t rec_gam(int64_t V) { return kRecU + (V / 16) * 2048; }
__host__ __device__ constexpr int64_t rec_bytes(int64_t V) { return ((rec_gam(V) + 512 + 255) / 256) * 256; }

__device__ __forceinline__ f32x4_t mfma32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(bf16x4_t a, bf16x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c,
                                                     0, 0, 0);
}
template <class V>
__device__ __forceinline__ V negate_bf16(V x) {
  // flip the sign bit of every bf16 lane
  typedef unsigned short u16v __attribute__((ext_vector_type(sizeof(V) / 2)));
  u16v b = __builtin_bit_cast(u16v, x);
  b ^= (unsigned short)0x8000;
  return __builtin_bit_cast(V, b);
}

template <class IT>
__device__ __forceinline__ void load_pair(const IT* p, float& lo, float& hi) {
  typedef IT pair_t __attribute__((ext_vector_type(2)));
  const pair_t x = *reinterpret_cast<const pair_t*>(p);
  lo = to_float(x[0]);
  hi = to_float(x[1]);
}

// ---- chunk map ------------------------------------------------------------
// chunk_start[s] = sum_{s' < s} ceil(span_{s'} / 64);  chunk_start[N] = total chunks.
__global__ __launch_bounds__(1024) void chunk_map_kernel(SeqDesc seq, int64_t N, int32_t* chunk_start) {
  __shared__ int32_t part[1024];
  const int tid = threadIdx.x;
  const int64_t per = (N + 1023) / 1024;
  const int64_t b0 = tid * per;
  const int64_t b1 = (b0 + per < N) ? b0 + per : N;
  int32_t local = 0;
  for (int64_t s = b0; s < b1; ++s) local += static_cast<int32_t>((seq_range(seq, s).span + kChunk - 1) / kChunk);
  part[tid] = local;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int32_t run = part[tid] - local;
  for (int64_t s = b0; s < b1; ++s) {
    chunk_start[s] = run;
    run += static_cast<int32_t>((seq_range(seq, s).span + kChunk - 1) / kChunk);
  }
  if (tid == 1023) chunk_start[N] = part[1023];
}

__device__ __forceinline__ int64_t find_seq(const int32_t* chunk_start, int64_t N, int64_t c) {
  int64_t lo = 0, hi = N - 1;  // largest s with chunk_start[s] <= c
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (chunk_start[mid] <= c)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// ---- prepare kernel -------------------------------------------------------
struct PrepSmem {
  bf16 KA[kChunk][136];  // k_j * a_j          (natural: token rows, key channels)
  bf16 QA[kChunk][136];  // q_j * a_j
  bf16 KE[kChunk][136];  // k_j * E_j
  bf16 L[kChunk][72];    // beta_i * A_ij, strict lower (bf16, MFMA A operand)
  float Ld[4][16][16];   // diagonal blocks of L in f32 (for the block inverses)
  bf16 Tinv[4][16][16];  // inverses of the unit-lower diagonal blocks of L
  // Per-channel block factors.  G, A0 and P are only read while building Gs,
  // Ge and the pair scales; the pair scales then overlay them (each thread
  // owns one channel column of all of them, so the overlay needs no barrier).
  union {
    struct {
      float G[4][kKey];   // exp(lg_{16J+15} - lg_{16J-1})  (block decay incl. its first row)
      float A0[4][kKey];  // alpha at the first row of block J
      float P[4][kKey];   // exp(lg_{16J+15} - lg_{16J})
    };
    float Sc[10][kKey];   // per block pair (I, J <= I): D_IJ (J < I) or 1 / P_I (J = I)
  };
  float Gs[4][kKey];      // exp(lg_{16J})  (chunk start to block start, inclusive)
  float Ge[4][kKey];      // exp(lg_63 - lg_{16J+15})
  float beta[kChunk];
};

// two prepare workgroups must fit in the 160 KB of LDS of one CU
static_assert(2 * sizeof(PrepSmem) <= 160 * 1024, "prepare kernel LDS no longer allows two workgroups per CU");

template <class IT>
struct PrepArgs {
  const IT* __restrict__ q;
  const IT* __restrict__ k;
  const IT* __restrict__ v;
  const IT* __restrict__ g;
  const IT* __restrict__ beta;
  SeqDesc seq;
  const int32_t* __restrict__ chunk_start;
  unsigned char* __restrict__ records;
  int64_t N, H, V;
};

template <class IT>
__global__ __launch_bounds__(kPrepThreads, 2) void chunk_prepare_kernel(const PrepArgs<IT> a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  PrepSmem& sm = *reinterpret_cast<PrepSmem*>(smem_raw);
  const int64_t c = blockIdx.x;
  const int64_t h = blockIdx.y;
  if (c >= a.chunk_start[a.N]) return;  // uniform: grid is an upper bound
  const int64_t s = find_seq(a.chunk_start, a.N, c);
  const SeqRange sr = seq_range(a.seq, s);
  const int64_t lc = c - a.chunk_start[s];
  const int64_t tok0 = sr.start + kChunk * lc;
  const int n_span = static_cast<int>(sr.span - kChunk * lc < kChunk ? sr.span - kChunk * lc : kChunk);
  int64_t nv = sr.valid - kChunk * lc;
  const int n_valid = static_cast<int>(nv < 0 ? 0 : (nv > n_span ? n_span : nv));
  unsigned char* rec = a.records + (c * a.H + h) * rec_bytes(a.V);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n16 = lane & 15;
  const int g4 = lane >> 4;
  const int64_t krow = a.H * kKey;

  // ---- P1: per-channel decay factors (thread = channel pair cp, block J) ---
  int extreme_local = 0;
  {
    const int J = wave;
    const int cp = lane;
    float gv[2][16], kv[2][16], qv[2][16];
    {
      // all 48 paired loads are issued before any use (tokens past the valid
      // range read row tok0 instead and are zeroed afterwards)
      typedef IT pair_t __attribute__((ext_vector_type(2)));
      pair_t gp[16], kp[16], qp[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tl = 16 * J + r;
        const int64_t off = (tok0 + (tl < n_valid ? tl : 0)) * krow + h * kKey + 2 * cp;
        gp[r] = *reinterpret_cast<const pair_t*>(a.g + off);
        kp[r] = *reinterpret_cast<const pair_t*>(a.k + off);
        qp[r] = *reinterpret_cast<const pair_t*>(a.q + off);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool ok = 16 * J + r < n_valid;
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
          gv[ch][r] = ok ? to_float(gp[r][ch]) : 0.f;
          kv[ch][r] = ok ? to_float(kp[r][ch]) : 0.f;
          qv[ch][r] = ok ? to_float(qp[r][ch]) : 0.f;
        }
      }
    }
    float ka[2][16], qa[2][16], ke[2][16];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      float al[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) al[r] = fast_exp(gv[ch][r]);
      float run = 1.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (r > 0) run *= al[r];
        ka[ch][r] = kv[ch][r] * run;
        qa[ch][r] = qv[ch][r] * run;
      }
      const float p_blk = run;  // a at the last row = exp(lg_{16J+15} - lg_{16J})
      float suf = 1.f;
#pragma unroll
      for (int r = 15; r >= 0; --r) {
        ke[ch][r] = kv[ch][r] * suf;
        suf *= al[r];
      }
      const int cc = 2 * cp + ch;
      sm.P[J][cc] = p_blk;
      sm.A0[J][cc] = al[0];
      sm.G[J][cc] = al[0] * p_blk;
      if (!(p_blk >= kExtremeDecay)) extreme_local = 1;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tl = 16 * J + r;
      *reinterpret_cast<bf16x2_t*>(&sm.KA[tl][2 * cp]) = bf16x2_t{(bf16)ka[0][r], (bf16)ka[1][r]};
      *reinterpret_cast<bf16x2_t*>(&sm.QA[tl][2 * cp]) = bf16x2_t{(bf16)qa[0][r], (bf16)qa[1][r]};
      *reinterpret_cast<bf16x2_t*>(&sm.KE[tl][2 * cp]) = bf16x2_t{(bf16)ke[0][r], (bf16)ke[1][r]};
    }
  }
  if (tid < kChunk) sm.beta[tid] = tid < n_valid ? to_float(a.beta[(tok0 + tid) * a.H + h]) : 0.f;
  const int extreme = __syncthreads_or(extreme_local);

  // ---- P1b: block-level decay tables and gamma_C ---------------------------
  if (tid < kKey) {
    const int cc = tid;
    float G[4], A0[4], P[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      G[J] = sm.G[J][cc];
      A0[J] = sm.A0[J][cc];
      P[J] = sm.P[J][cc];
    }
    float pre = 1.f;
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      sm.Gs[J][cc] = pre * A0[J];
      pre *= G[J];
    }
    float post = 1.f;
#pragma unroll
    for (int J = 3; J >= 0; --J) {
      sm.Ge[J][cc] = post;
      post *= G[J];
    }
    reinterpret_cast<float*>(rec + rec_gam(a.V))[cc] = pre;  // exp(lg_63)
    // scale of the k_j E_j operand for block pair (I, J): D_IJ = alpha_{16I} prod_{J<J'<I} G_J'
    // for J < I, 1 / P_I on the diagonal (written over G/A0/P of this same channel)
    int pidx = 0;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int J = 0; J <= I; ++J, ++pidx) {
        float sc;
        if (J < I) {
          sc = A0[I];
#pragma unroll
          for (int jj = J + 1; jj < I; ++jj) sc *= G[jj];
        } else {
          sc = P[I] > 0.f ? 1.f / P[I] : 0.f;
        }
        sm.Sc[pidx][cc] = sc;
      }
    }
  }
  __syncthreads();

  // ---- export: Q~ and K~^T fragments (read-only on the tables) -------------
  for (int task = tid; task < 2048; task += kPrepThreads) {
    const int frag = (task >> 6) & 15;
    const int fl = task & 63;
    const int fi = fl & 15, fg = fl >> 4;
    bf16x8_t out;
    if (task < 1024) {  // Q~ = exp(lg) q : fragment (I, s), lane (i, g)
      const int I = frag >> 2, st = frag & 3;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int ch = 32 * st + (e < 4 ? 4 * fg + e : 16 + 4 * fg + e - 4);
        out[e] = (bf16)((float)sm.QA[16 * I + fi][ch] * sm.Gs[I][ch]);
      }
      *reinterpret_cast<bf16x8_t*>(rec + kRecQ + (static_cast<int64_t>(frag) * 64 + fl) * 16) = out;
    } else {  // K~^T : fragment (ct, s'), lane (c, g)
      const int ct = frag >> 1, st = frag & 1;
      const int ch = 16 * ct + fi;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tk = 32 * st + (e < 4 ? 4 * fg + e : 16 + 4 * fg + e - 4);
        out[e] = (bf16)((float)sm.KE[tk][ch] * sm.Ge[tk >> 4][ch]);
      }
      *reinterpret_cast<bf16x8_t*>(rec + kRecKT + (static_cast<int64_t>(frag) * 64 + fl) * 16) = out;
    }
  }

  // ---- P2: A (strict) and Aqk (causal) 16x16 blocks on MFMA ---------------
  {
    for (int p = wave; p < 10; p += 4) {
      // block pair p = I (I + 1) / 2 + J, J <= I
      const int I = p >= 6 ? 3 : (p >= 3 ? 2 : (p >= 1 ? 1 : 0));
      const int J = p - I * (I + 1) / 2;
      f32x4_t akk = {0.f, 0.f, 0.f, 0.f};
      f32x4_t aqk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int c0 = 32 * st + 8 * g4;
        const bf16x8_t ke = *reinterpret_cast<const bf16x8_t*>(&sm.KE[16 * J + n16][c0]);
        const f32x4_t sc0 = *reinterpret_cast<const f32x4_t*>(&sm.Sc[p][c0]);
        const f32x4_t sc1 = *reinterpret_cast<const f32x4_t*>(&sm.Sc[p][c0 + 4]);
        bf16x8_t af;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          af[e] = (bf16)((float)ke[e] * sc0[e]);
          af[4 + e] = (bf16)((float)ke[4 + e] * sc1[e]);
        }
        const bf16x8_t kb = *reinterpret_cast<const bf16x8_t*>(&sm.KA[16 * I + n16][c0]);
        const bf16x8_t qb = *reinterpret_cast<const bf16x8_t*>(&sm.QA[16 * I + n16][c0]);
        akk = mfma32(af, kb, akk);
        aqk = mfma32(af, qb, aqk);
      }
      // lane (n16, g4) holds Akk[16I + n16][16J + 4 g4 + r] (and likewise Aqk)
      const int i = 16 * I + n16;
      const float bi = sm.beta[i];
      bf16x4_t lrow;
      bf16x4_t qrow;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * J + 4 * g4 + r;
        const float vk = (j < i) ? akk[r] * bi : 0.f;
        lrow[r] = (bf16)vk;
        qrow[r] = (bf16)((j <= i) ? aqk[r] : 0.f);
        if (I == J) sm.Ld[I][n16][4 * g4 + r] = vk;
      }
      *reinterpret_cast<bf16x4_t*>(&sm.L[i][16 * J + 4 * g4]) = lrow;
      unsigned char* afrag = rec + kRecA + (static_cast<int64_t>(I * 2 + J / 2) * 64 + lane) * 16;
      *reinterpret_cast<bf16x4_t*>(afrag + (J & 1) * 8) = qrow;
      if (I == J && (I & 1) == 0) *reinterpret_cast<bf16x4_t*>(afrag + 8) = bf16x4_t{};  // tile J = I+1 is above
    }
  }
  __syncthreads();

  // ---- exact diagonal blocks for chunks with extreme decay ----------------
  if (extreme) {
    float* Lr = reinterpret_cast<float*>(&sm.QA[0][0]);  // [64][128] f32, overlays QA and KE (dead now)
    {
      const int J = wave, cp = lane;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        float run = 0.f;
        for (int r = 0; r < 16; ++r) {
          const int tl = 16 * J + r;
          const float gvv = tl < n_valid ? to_float(a.g[(tok0 + tl) * krow + h * kKey + 2 * cp + ch]) : 0.f;
          if (r > 0) run += gvv;
          Lr[tl * kKey + 2 * cp + ch] = run;
        }
      }
    }
    __syncthreads();
    for (int task = tid; task < 4 * 136; task += kPrepThreads) {
      const int I = task / 136;
      int p = task % 136;
      int il = 0;
      while ((il + 1) * (il + 2) / 2 <= p) ++il;
      const int jl = p - il * (il + 1) / 2;
      const int i = 16 * I + il, j = 16 * I + jl;
      float acc_k = 0.f, acc_q = 0.f;
      if (i < n_valid && j < n_valid) {
        const int64_t oi = (tok0 + i) * krow + h * kKey;
        const int64_t oj = (tok0 + j) * krow + h * kKey;
        for (int cc = 0; cc < kKey; ++cc) {
          const float e = fast_exp(Lr[i * kKey + cc] - Lr[j * kKey + cc]);
          const float kj = to_float(a.k[oj + cc]);
          acc_k += to_float(a.k[oi + cc]) * kj * e;
          acc_q += to_float(a.q[oi + cc]) * kj * e;
        }
      }
      if (jl < il) {
        const float vk = sm.beta[i] * acc_k;
        sm.L[i][j] = (bf16)vk;
        sm.Ld[I][il][jl] = vk;
      }
      const int fl = il + 16 * (jl >> 2);
      bf16* afrag = reinterpret_cast<bf16*>(rec + kRecA + (static_cast<int64_t>(I * 2 + I / 2) * 64 + fl) * 16);
      afrag[(I & 1) * 4 + (jl & 3)] = (bf16)acc_q;
    }
    __syncthreads();
  }

  // ---- P3: inverses of the four unit-lower diagonal blocks (f32) ----------
  if (lane < 16) {
    const int I = wave;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float acc = (r == lane) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < r; ++j) acc -= sm.Ld[I][r][j] * x[j];
      x[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sm.Tinv[I][r][lane] = (bf16)x[r];
  }
  __syncthreads();

  // ---- P4: blocked forward substitution  [W | U] = L^{-1} diag(beta) [Kgamma | v]
  // Wave w owns column tiles nt = w, w+4, ... of the 8 + V/16 tiles (8 key
  // tiles of W, V/16 value tiles of U) and walks the four row blocks once for
  // all of them, so the L and inverse fragments are read once per block and
  // the column tiles form independent MFMA chains.
  {
    constexpr int kMaxT = 6;  // up to (8 + 256/16) / 4 column tiles per wave
    const int n_tiles = 8 + static_cast<int>(a.V / 16);
    const int64_t vrow = a.H * a.V;
    int nts[kMaxT];
    int nown = 0;
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      nts[t] = wave + 4 * t;
      if (nts[t] < n_tiles) ++nown;
    }
    // right-hand sides diag(beta) [Kgamma | v], loaded up front
    float rhs[kMaxT][4][4];
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t >= nown) {
#pragma unroll
        for (int I = 0; I < 4; ++I)
#pragma unroll
          for (int r = 0; r < 4; ++r) rhs[t][I][r] = 0.f;
        continue;
      }
      const int nt = nts[t];
      const bool is_w = nt < 8;
      const int col = 16 * (is_w ? nt : nt - 8) + n16;
#pragma unroll
      for (int I = 0; I < 4; ++I) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tl = 16 * I + 4 * g4 + r;
          float val;
          if (is_w)
            val = (float)sm.KA[tl][col] * sm.Gs[I][col];
          else
            val = to_float(a.v[(tok0 + (tl < n_valid ? tl : 0)) * vrow + h * a.V + col]);
          rhs[t][I][r] = (tl < n_valid ? val : 0.f) * sm.beta[tl];
        }
      }
    }
    f32x4_t X[kMaxT][4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4_t acc[kMaxT];
#pragma unroll
      for (int t = 0; t < kMaxT; ++t) acc[t] = f32x4_t{rhs[t][I][0], rhs[t][I][1], rhs[t][I][2], rhs[t][I][3]};
#pragma unroll
      for (int J = 0; J < I; ++J) {
        const bf16x4_t la = negate_bf16(*reinterpret_cast<const bf16x4_t*>(&sm.L[16 * I + n16][16 * J + 4 * g4]));
#pragma unroll
        for (int t = 0; t < kMaxT; ++t) {
          if (t >= nown) continue;
          const bf16x4_t xb = {(bf16)X[t][J][0], (bf16)X[t][J][1], (bf16)X[t][J][2], (bf16)X[t][J][3]};
          acc[t] = mfma16(la, xb, acc[t]);
        }
      }
      const bf16x4_t ta = *reinterpret_cast<const bf16x4_t*>(&sm.Tinv[I][n16][4 * g4]);
#pragma unroll
      for (int t = 0; t < kMaxT; ++t) {
        if (t >= nown) continue;
        const bf16x4_t ab = {(bf16)acc[t][0], (bf16)acc[t][1], (bf16)acc[t][2], (bf16)acc[t][3]};
        X[t][I] = mfma16(ta, ab, f32x4_t{0.f, 0.f, 0.f, 0.f});
      }
    }
    // exports
#pragma unroll
    for (int t = 0; t < kMaxT; ++t) {
      if (t >= nown) continue;
      const int nt = nts[t];
      if (nt < 8) {
        // scatter into W fragments: channel 16 nt + n16 -> step st, lane group gq, element eq
        const int st = nt >> 1;
        const int gq = n16 >> 2;
        const int eq = 4 * (nt & 1) + (n16 & 3);
#pragma unroll
        for (int I = 0; I < 4; ++I) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int il = 4 * g4 + r;
            bf16* dst =
                reinterpret_cast<bf16*>(rec + kRecW + (static_cast<int64_t>(I * 4 + st) * 64 + il + 16 * gq) * 16);
            dst[eq] = (bf16)X[t][I][r];
          }
        }
      } else {
        const int vt = nt - 8;
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          *reinterpret_cast<bf16x4_t*>(rec + kRecU + (static_cast<int64_t>(vt * 4 + I) * 64 + lane) * 8) =
              bf16x4_t{(bf16)X[t][I][0], (bf16)X[t][I][1], (bf16)X[t][I][2], (bf16)X[t][I][3]};
        }
      }
    }
  }
}

// ---- scan kernel ----------------------------------------------------------
// One workgroup of three waves per (sequence, head, 32 value columns).
// Waves 0 and 1 ("compute") own the 16-column state slices
// S[:, 16 (2 wp + w) .. +16] in accumulator registers; they only read LDS,
// run MFMAs and issue output stores, and never wait on vector memory.
// Wave 2 ("copier") moves the next chunk's record (W, Q, KT, A fragments,
// the two U tiles and gamma: 60.5 KB) into the other of two LDS buffers with
// direct global->LDS loads and touches the record a few chunks ahead so that
// the copy hits L2.  The roles run separate loops with one barrier per chunk.
constexpr int kScanComputeWaves = 2;
constexpr int kScanThreads = 64 * (kScanComputeWaves + 1);
constexpr int kScanShared = 57344;                                       // W | Q | KT | A
constexpr int kScanBuf = kScanShared + kScanComputeWaves * 2048 + 512;   // + U tiles + gamma = 61952 B
constexpr int kScanUnits = kScanShared / 16;                             // 16-byte units of the shared part
constexpr int kScanPrefetch = 4;
constexpr int kWarmLoads = 8;                                            // 8 x 64 lanes x 128 B = 64 KB

template <class IT>
struct ScanArgs {
  IT* out;
  const float* s_in;
  float* s_out;
  SeqDesc seq;
  const int32_t* chunk_start;
  const unsigned char* records;
  int64_t N, H, V;
};

// copier wave: one chunk's record pieces into an LDS buffer
__device__ __forceinline__ void scan_copy(const unsigned char* rec, unsigned char* buf, int64_t vt0, int ntiles,
                                          int64_t gam_off, int lane) {
#pragma unroll 8
  for (int i = 0; i < kScanUnits / 64; ++i)  // 56 instructions of 64 x 16 B
    __builtin_amdgcn_global_load_lds(rec + (i * 64 + lane) * 16, buf + i * 1024, 16, 0, 0);
  for (int t = 0; t < 2 * ntiles; ++t)       // U tiles: 2 instructions each
    __builtin_amdgcn_global_load_lds(rec + kRecU + vt0 * 2048 + (t * 64 + lane) * 16, buf + kScanShared + t * 1024,
                                     16, 0, 0);
  if (lane < 32)  // gamma
    __builtin_amdgcn_global_load_lds(rec + gam_off + lane * 16, buf + kScanShared + kScanComputeWaves * 2048, 16, 0,
                                     0);
}

// copier wave: touch one dword of each 128-byte line of a future record's
// shared part (the words land in a scratch LDS area that is never read)
__device__ __forceinline__ void scan_warm_l2(const unsigned char* rec, unsigned char* scratch, int lane) {
#pragma unroll
  for (int k = 0; k < kWarmLoads; ++k) {
    int off = (k * 64 + lane) * 128;
    off = off < kScanShared - 4 ? off : kScanShared - 4;
    __builtin_amdgcn_global_load_lds(rec + off, scratch, 4, 0, 0);
  }
}

// barrier without a memory fence: the asm statements only stop the compiler
// from moving memory accesses across it; LDS ordering comes from the waits
// each role performs before arriving
__device__ __forceinline__ void scan_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <class IT>
__device__ __forceinline__ void scan_chunk(const unsigned char* buf, f32x4_t (&S)[8], int w, int lane,
                                           f32x4_t (&O)[4]) {
  // Two-stage software pipeline over the reduction steps: the fragments of
  // step st + 1 are read from LDS while the 8 products of step st run.
  auto load_wq = [&](int st, bf16x8_t (&wf)[4], bf16x8_t (&qf)[4]) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      wf[I] = *reinterpret_cast<const bf16x8_t*>(buf + kRecW + ((I * 4 + st) * 64 + lane) * 16);
      qf[I] = *reinterpret_cast<const bf16x8_t*>(buf + kRecQ + ((I * 4 + st) * 64 + lane) * 16);
    }
  };
  bf16x8_t wa[4], qa[4], wb[4], qb[4];
  bf16x4_t uf[4];
#pragma unroll
  for (int I = 0; I < 4; ++I)
    uf[I] = *reinterpret_cast<const bf16x4_t*>(buf + kScanShared + w * 2048 + (I * 64 + lane) * 8);
  load_wq(0, wa, qa);
  bf16x8_t Sb[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      Sb[st][r] = (bf16)S[2 * st][r];
      Sb[st][4 + r] = (bf16)S[2 * st + 1][r];
    }
  }
  f32x4_t Vt[4];
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    Vt[I] = f32x4_t{(float)uf[I][0], (float)uf[I][1], (float)uf[I][2], (float)uf[I][3]};
    O[I] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    bf16x8_t(&wc)[4] = (st & 1) ? wb : wa;
    bf16x8_t(&qc)[4] = (st & 1) ? qb : qa;
    if (st + 1 < 4) {
      if (st & 1)
        load_wq(st + 1, wa, qa);
      else
        load_wq(st + 1, wb, qb);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      Vt[I] = mfma32(negate_bf16(wc[I]), Sb[st], Vt[I]);
      O[I] = mfma32(qc[I], Sb[st], O[I]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // Aqk fragments used: (I, s') for s' <= I / 2 -> slots 0, 2, 4, 5, 6, 7;
  // gamma and the first half of the K~^T fragments
  bf16x8_t af[6];
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const int slot = j < 2 ? 2 * j : j + 2;
    af[j] = *reinterpret_cast<const bf16x8_t*>(buf + kRecA + (slot * 64 + lane) * 16);
  }
  const int g4 = lane >> 4;
  const float* gam = reinterpret_cast<const float*>(buf + kScanShared + kScanComputeWaves * 2048);
  f32x4_t gm[8];
  bf16x8_t kf[8][2];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    gm[ct] = *reinterpret_cast<const f32x4_t*>(gam + 16 * ct + 4 * g4);
#pragma unroll
    for (int st = 0; st < 2; ++st)
      kf[ct][st] = *reinterpret_cast<const bf16x8_t*>(buf + kRecKT + ((ct * 2 + st) * 64 + lane) * 16);
  }
  bf16x8_t Vb[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      Vb[st][r] = (bf16)Vt[2 * st][r];
      Vb[st][4 + r] = (bf16)Vt[2 * st + 1][r];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  O[0] = mfma32(af[0], Vb[0], O[0]);
  O[1] = mfma32(af[1], Vb[0], O[1]);
  O[2] = mfma32(af[2], Vb[0], O[2]);
  O[2] = mfma32(af[3], Vb[1], O[2]);
  O[3] = mfma32(af[4], Vb[0], O[3]);
  O[3] = mfma32(af[5], Vb[1], O[3]);
#pragma unroll
  for (int ct = 4; ct < 8; ++ct) {
    gm[ct] = *reinterpret_cast<const f32x4_t*>(gam + 16 * ct + 4 * g4);
#pragma unroll
    for (int st = 0; st < 2; ++st)
      kf[ct][st] = *reinterpret_cast<const bf16x8_t*>(buf + kRecKT + ((ct * 2 + st) * 64 + lane) * 16);
  }
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    S[ct] *= gm[ct];
#pragma unroll
    for (int st = 0; st < 2; ++st) S[ct] = mfma32(kf[ct][st], Vb[st], S[ct]);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ct = 4; ct < 8; ++ct) {
    S[ct] *= gm[ct];
#pragma unroll
    for (int st = 0; st < 2; ++st) S[ct] = mfma32(kf[ct][st], Vb[st], S[ct]);
  }
}

// Store a chunk's 64 x 16 output tile.  The accumulator layout (lane (n, g)
// holds rows 16 I + 4 g + r of column n) is transposed through a per-wave
// 2 KB LDS stage so that each lane writes 16 contiguous bytes of a row.
template <class IT>
__device__ __forceinline__ void scan_store_out(const f32x4_t (&O)[4], IT* out, int64_t tokbase, int64_t n_span,
                                               int64_t H, int64_t h, int64_t V, int64_t col0, int lane,
                                               IT* stage) {
  const int g4 = lane >> 4, n16 = lane & 15;
#pragma unroll
  for (int I = 0; I < 4; ++I) {
#pragma unroll
    for (int r = 0; r < 4; ++r) stage[(16 * I + 4 * g4 + r) * 16 + n16] = from_compute<IT>(O[I][r]);
  }
  // lanes now read what other lanes of the wave wrote: complete the writes and
  // keep the compiler from moving the reads above them
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = j * 32 + (lane >> 1);
    const int half = lane & 1;
    const uint4 val = *reinterpret_cast<const uint4*>(stage + row * 16 + 8 * half);
    if (row < n_span) *reinterpret_cast<uint4*>(out + ((tokbase + row) * H + h) * V + col0 + 8 * half) = val;
  }
}

template <class IT>
__global__ __launch_bounds__(kScanThreads) void chunk_scan_kernel(const ScanArgs<IT> a) {
  __shared__ __align__(16) unsigned char buf0[kScanBuf];
  __shared__ __align__(16) unsigned char buf1[kScanBuf];
  __shared__ __align__(16) unsigned char warm[256];
  __shared__ __align__(16) IT stage_all[kScanComputeWaves][64 * 16];  // output transpose, one tile per wave
  const int64_t nvt = a.V / 16;
  const int64_t nwp = (nvt + kScanComputeWaves - 1) / kScanComputeWaves;  // workgroups per (sequence, head)
  const int64_t bid = blockIdx.x;
  const int64_t wp = bid % nwp;
  const int64_t h = (bid / nwp) % a.H;
  const int64_t s = bid / (nwp * a.H);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int64_t vt0 = wp * kScanComputeWaves;
  const int ntiles = static_cast<int>(nvt - vt0 < kScanComputeWaves ? nvt - vt0 : kScanComputeWaves);
  const SeqRange sr = seq_range(a.seq, s);
  const int64_t c0 = a.chunk_start[s];
  const int64_t c1 = a.chunk_start[s + 1];
  const int64_t rb = rec_bytes(a.V);
  auto rec_of = [&](int64_t c) { return a.records + (c * a.H + h) * rb; };

  if (w == kScanComputeWaves) {
    // ---------------- copier wave ----------------
    const int64_t gam_off = rec_gam(a.V);
    for (int64_t p = c0 + 1; p < c1 && p <= c0 + kScanPrefetch; ++p) scan_warm_l2(rec_of(p), warm, lane);
    scan_copy(rec_of(c0), buf0, vt0, ntiles, gam_off, lane);
    __builtin_amdgcn_s_waitcnt(0);
    scan_barrier();
    // step c: the compute waves read buffer (c - c0) % 2; the copier fills the other
    // with chunk c + 1, waits for it (the warming loads issued after it may stay in
    // flight: a wave's vector memory loads retire in issue order), then arrives
    for (int64_t c = c0; c < c1; ++c) {
      const bool odd = ((c - c0) & 1) != 0;
      if (c + 1 < c1) {
        if (odd)
          scan_copy(rec_of(c + 1), buf0, vt0, ntiles, gam_off, lane);
        else
          scan_copy(rec_of(c + 1), buf1, vt0, ntiles, gam_off, lane);
      }
      // always exactly kWarmLoads warming loads (clamped to a valid record) so
      // that vmcnt(kWarmLoads) below means "the copy has landed"
      scan_warm_l2(rec_of(c + 1 + kScanPrefetch < c1 ? c + 1 + kScanPrefetch : c1 - 1), warm, lane);
      asm volatile("" ::: "memory");
      // s_waitcnt vmcnt(kWarmLoads) expcnt(7) lgkmcnt(15)
      __builtin_amdgcn_s_waitcnt((kWarmLoads & 15) | (7 << 4) | (15 << 8) | ((kWarmLoads >> 4) << 14));
      scan_barrier();
    }
    __builtin_amdgcn_s_waitcnt(0);  // no copy may land in LDS after the workgroup ends
    return;
  }

  // ---------------- compute waves ----------------
  const bool active = w < ntiles;
  const int n16 = lane & 15;
  const int g4 = lane >> 4;
  const int64_t col = 16 * (vt0 + w) + n16;
  const int64_t sbase = (s * a.H + h) * kKey * a.V;
  f32x4_t S[8];
#pragma unroll
  for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = 16 * ct + 4 * g4 + r;
      S[ct][r] = (a.s_in && active) ? a.s_in[sbase + row * a.V + col] : 0.f;
    }
  }
  scan_barrier();
  f32x4_t O[4];
  for (int64_t c = c0; c < c1; ++c) {
    const int64_t lc = c - c0;
    if (active) {
      if ((lc & 1) == 0)
        scan_chunk<IT>(buf0, S, w, lane, O);
      else
        scan_chunk<IT>(buf1, S, w, lane, O);
      const int64_t n_span = sr.span - kChunk * lc < kChunk ? sr.span - kChunk * lc : kChunk;
      scan_store_out<IT>(O, a.out, sr.start + kChunk * lc, n_span, a.H, h, a.V, col - n16, lane, stage_all[w]);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((63 & 15) | (7 << 4) | (0 << 8) | ((63 >> 4) << 14));  // lgkmcnt(0): LDS reads done
    scan_barrier();
  }
  if (a.s_out && active) {
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = 16 * ct + 4 * g4 + r;
        a.s_out[sbase + row * a.V + col] = S[ct][r];
      }
    }
  }
}

// ---- host side ------------------------------------------------------------
static int64_t chunk_bound(int64_t N, int64_t total_tokens) { return total_tokens / kChunk + N + 1; }

static bool mfma_path(int in_dtype, int state_dtype, int64_t K, int64_t V) {
  return (in_dtype == KDA_DTYPE_BF16 || in_dtype == KDA_DTYPE_F16) && state_dtype == KDA_DTYPE_F32 && K == kKey &&
         V % 16 == 0 && V >= 16 && V <= 256;
}

static size_t map_bytes(int64_t N) { return static_cast<size_t>(((N + 1) * 4 + 255) / 256 * 256); }

static void mark(kda_host::KernelEvents* ev, int i, hipStream_t stream) {
  if (ev != nullptr) {
    (void)hipEventRecord(ev->ev[i], stream);
    ev->n_launched = i;
  }
}

template <class IT>
static int run_chunk(const void* q, const void* k, const void* v, const void* g, const void* beta, const void* s_in,
                     void* s_out, void* out, const SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H,
                     int64_t V, void* workspace, hipStream_t stream, kda_host::KernelEvents* ev) {
  int32_t* chunk_start = static_cast<int32_t*>(workspace);
  unsigned char* records = static_cast<unsigned char*>(workspace) + map_bytes(N);
  mark(ev, 0, stream);
  hipLaunchKernelGGL(chunk_map_kernel, dim3(1), dim3(1024), 0, stream, seq, N, chunk_start);
  int st = kda_host::check_launch("chunk_map_kernel");
  if (st != KDA_OK) return st;
  mark(ev, 1, stream);

  static bool attr_done = false;
  const size_t smem = sizeof(PrepSmem);
  if (!attr_done) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_prepare_kernel<IT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)) != hipSuccess) {
      kda_host::set_detail("cannot reserve %zu bytes of LDS for chunk_prepare_kernel", smem);
      return KDA_ERR_LAUNCH;
    }
    attr_done = true;
  }
  PrepArgs<IT> pa;
  pa.q = static_cast<const IT*>(q);
  pa.k = static_cast<const IT*>(k);
  pa.v = static_cast<const IT*>(v);
  pa.g = static_cast<const IT*>(g);
  pa.beta = static_cast<const IT*>(beta);
  pa.seq = seq;
  pa.chunk_start = chunk_start;
  pa.records = records;
  pa.N = N;
  pa.H = H;
  pa.V = V;
  const int64_t nchunks = chunk_bound(N, total_tokens);
  hipLaunchKernelGGL(chunk_prepare_kernel<IT>, dim3(static_cast<unsigned>(nchunks), static_cast<unsigned>(H)),
                     dim3(kPrepThreads), smem, stream, pa);
  st = kda_host::check_launch("chunk_prepare_kernel");
  if (st != KDA_OK) return st;
  mark(ev, 2, stream);

  ScanArgs<IT> sa;
  sa.out = static_cast<IT*>(out);
  sa.s_in = static_cast<const float*>(s_in);
  sa.s_out = static_cast<float*>(s_out);
  sa.seq = seq;
  sa.chunk_start = chunk_start;
  sa.records = records;
  sa.N = N;
  sa.H = H;
  sa.V = V;
  const int64_t blocks = N * H * ((V / 16 + kScanComputeWaves - 1) / kScanComputeWaves);
  hipLaunchKernelGGL(chunk_scan_kernel<IT>, dim3(static_cast<unsigned>(blocks)), dim3(kScanThreads), 0, stream, sa);
  st = kda_host::check_launch("chunk_scan_kernel");
  mark(ev, 3, stream);
  return st;
}

}  // namespace kda

namespace kda_host {

size_t chunk_workspace_bytes(int64_t num_seqs, int64_t total_tokens, int64_t heads, int64_t key_dim,
                             int64_t value_dim, int in_dtype) {
  if (!kda::mfma_path(in_dtype, in_dtype == KDA_DTYPE_F64 ? KDA_DTYPE_F64 : KDA_DTYPE_F32, key_dim, value_dim))
    return 0;
  return kda::map_bytes(num_seqs) +
         static_cast<size_t>(kda::chunk_bound(num_seqs, total_tokens) * heads * kda::rec_bytes(value_dim));
}

int launch_chunk(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                 const void* s_in, void* s_out, int state_dtype, void* out, const kda::SeqDesc& seq, int64_t N,
                 int64_t total_tokens, int64_t H, int64_t K, int64_t V, void* workspace, size_t workspace_bytes,
                 hipStream_t stream, KernelEvents* ev) {
  using namespace kda;
  if (!mfma_path(in_dtype, state_dtype, K, V)) {
    mark(ev, 0, stream);
    const int st = launch_recurrent(q, k, v, g, beta, in_dtype, s_in, s_out, state_dtype, out, nullptr, seq, N, H,
                                    K, V, stream, false);
    mark(ev, 1, stream);
    return st;
  }
  if (workspace_bytes < chunk_workspace_bytes(N, total_tokens, H, K, V, in_dtype)) {
    set_detail("chunk_fwd: workspace too small");
    return KDA_ERR_WORKSPACE;
  }
  if (H > 65535 || chunk_bound(N, total_tokens) > 0x7fffffffLL || N * H * (V / 16) > 0x7fffffffLL) {
    set_detail("chunk_fwd: grid too large (H=%lld)", (long long)H);
    return KDA_ERR_UNSUPPORTED;
  }
  if (in_dtype == KDA_DTYPE_BF16)
    return run_chunk<bf16>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, V, workspace, stream, ev);
  return run_chunk<f16>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, V, workspace, stream, ev);
}

}  // namespace kda_host
