// Chunkwise KDA prefill on gfx950 bf16 MFMA (chunk C = 64, K <= 128 zero-padded
// to 128 channels, V <= 256).
//
// Reference algorithm: src/kda/chunkwise.py:61-102 with the UT transform of
// src/kda/ut_transform.py:23-58.  For one chunk (rows i, j = 0..63, key
// channels c, lg = inclusive cumsum of g inside the chunk):
//   A_ij   = sum_c k_i k_j exp(lg_i - lg_j)            j <  i   (strict)
//   Aqk_ij = sum_c q_i k_j exp(lg_i - lg_j)            j <= i
//   M = (I + diag(beta) A)^{-1} diag(beta)             (64 x 64, lower)
//   V~ = M (v - exp(lg) k S) ;  O = (exp(lg) q) S + Aqk V~ ;  S <- diag(exp lg_63) S + (exp(lg_63 - lg) k)^T V~
// The reference forms W = M exp(lg) k and U = M v (its UT transform,
// ut_transform.py:53-55) and then V~ = U - W S; multiplying M into
// (v - exp(lg) k S) instead is the same quantity and needs only the 64 x 64
// matrix M per chunk rather than the forward substitution of 8 + V/16
// column tiles.
//
// Every chunk is an affine map of the state, S_out = P_c S_in + R_c.  A
// sequence of chunks is cut into segments of L chunks so that the serial
// chain does not limit parallelism when batch * heads is small:
//  * phase A, chunk_segment_kernel<.., kSummary>: one workgroup per
//    (segment, head, 128-column group) prepares every chunk of its segment,
//    hands each chunk's M and Aqk fragments to phase C through the
//    workspace, and folds the segment into (P_g, Q_g) by running the chunk
//    recurrence on X = [Q | P] from X = [0 | I]: the V value columns give
//    Q_g, 128 more columns give P_g.  The first segment of a sequence starts
//    from the real initial state and directly yields the start state of the
//    second segment; the last segment only prepares its chunks.
//  * phase B, segment_combine_kernel: S_{g+1} = P_g S_g + Q_g along each
//    sequence, one workgroup per (sequence, head, 16-column tile).
//  * phase C, chunk_segment_kernel<.., kOutputMA>: one workgroup per
//    (segment, head, column group) re-runs its segment from the true start
//    state with M and Aqk from phase A and writes the outputs (and the final
//    state).
// When batch * heads alone fills the GPU, each sequence is one segment and
// only phase C runs, preparing every chunk itself (kOutput).
//
// Inside phases A and C a workgroup of 8 waves walks its chunks; per chunk
// it builds every chunk operand in LDS (decay factors, A and Aqk on MFMA,
// the diagonal-block inverses and M) and then the 4 scanner waves advance
// their 16-column state tiles, held in f32 MFMA accumulators.  The
// accumulator layout of a state tile converts to the B-operand layout of the
// next product without data movement: a C tile lane holds rows 4g..4g+3 of
// one column, so two consecutive row tiles give the 8 values a 16x16x32 B
// operand needs, with the reduction index permuted; the A operands are
// written pre-permuted to match.  The raw inputs of the next chunk are loaded
// into registers while the current chunk is scanned.
//
// Numerical scheme for the decays (per-channel g of either sign):
//   alpha_j = exp(g_j); within each 16-row block J the running products
//   a_j = exp(lg_j - lg_{16J}) and E_j = exp(lg_{16J+15} - lg_j) (<= 1 for
//   g <= 0).  Off-diagonal blocks J < I use (k_i a_i) . (k_j E_j D_IJ) with
//   D_IJ = exp(lg_{16I} - lg_{16J+15}); diagonal blocks use
//   (k_i a_i) . (k_j E_j / P_I) with P_I = exp(lg_{16I+15} - lg_{16I}).
//   Each factor is a product of at most one chunk's decays, and the product
//   of two factors is the pairwise exponent exp(lg_i - lg_j) itself, so the
//   bf16 operands carry the same relative rounding for any g; only a block
//   whose decay leaves [2^-100, 2^100] could overflow a factor, and such
//   chunks take an exact pairwise-exponent path for the diagonal blocks (the
//   reference evaluates every tile with an explicit pairwise exponent,
//   src/kda/utils.py:128-136).
#include <atomic>
#include <cstdlib>

#include "kda_launch.h"

namespace kda {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;
constexpr int kKey = 128;
constexpr int kColGroup = 128;  // value columns per workgroup
constexpr int kThreads = 512;   // 8 waves
constexpr float kExtremeDecay = 7.888609052210118e-31f;  // 2^-100
constexpr float kExtremeGrowth = 1.2676506002282294e30f;  // 2^100
constexpr int32_t kOneSegment = 0x3fffffff;              // L: every sequence is one segment

constexpr int kSummary = 0;   // phase A: segment summaries, and each chunk's M and Aqk
constexpr int kOutput = 1;    // phase C preparing every chunk itself (sequences of one segment)
constexpr int kOutputMA = 2;  // phase C reading each chunk's M and Aqk written by phase A
template <int MODE>
inline constexpr bool kWritesOut = MODE != kSummary;  // outputs, Q~, start states from phase B
template <int MODE>
inline constexpr bool kPrepares = MODE != kOutputMA;  // P2, the diagonal-block inverses and M in the loop
// M and Aqk of one (chunk, head) in the workspace: the six lower-triangular
// 64 x 64 A fragments of each, [M | Aqk][j = 0..5][lane][8] bf16 (j -> slot
// j < 2 ? 2 j : j + 2 of the [I][s'] fragment layout)
constexpr int64_t kMaBytes = 12 * 1024;
__host__ __device__ constexpr int lower_slot(int j) { return j < 2 ? 2 * j : j + 2; }

// ---- LDS map of chunk_segment_kernel (bytes) ------------------------------
// Natural bf16 tiles use a padded row of 136 elements; the k a, q a and k E
// tiles also shift each 16-row block by 64 bytes, so that the four rows a
// loader wave writes at once (one per block) fall in different LDS banks.
constexpr int kRow = 136;
constexpr int kNat = kChunk * kRow * 2 + 3 * 64;  // 17600
constexpr int kOffKA = 0;                   // bf16 [64][136] k_j a_j
constexpr int kOffQA = kOffKA + kNat;       // bf16 [64][136] q_j a_j    -> Kgamma fragments after P2
constexpr int kOffKE = kOffQA + kNat;       // bf16 [64][136] k_j E_j    -> M fragments after P2
constexpr int kOffL = kOffKE + kNat;        // bf16 [64][72] beta_i A_ij, strict lower
constexpr int kOffLd = kOffL + kChunk * 72 * 2;  // f32 [4][16][16] diagonal blocks of L
constexpr int kOffTinv = kOffLd + 4 * 256 * 4;   // bf16 [4][16][16] T_I = inverses of those blocks
constexpr int kOffTinvT = kOffTinv + 4 * 256 * 2;  // bf16 [4][16][16] T_I transposed
constexpr int kOffTab = kOffTinvT + 4 * 256 * 2;   // f32 pair scales [10][128]
constexpr int kOffGs = kOffTab + 10 * kKey * 4;     // f32 [4][128] exp(lg_{16J})
constexpr int kOffGe = kOffGs + 4 * kKey * 4;       // f32 [4][128] exp(lg_63 - lg_{16J+15})
constexpr int kOffBeta = kOffGe + 4 * kKey * 4;     // f32 [64]
constexpr int kOffVn = kOffBeta + 256;              // bf16 [64][136] v of the column group
constexpr int kOffQf = kOffVn + kNat;               // Q~ A fragments  [I=4][s=4][lane][8] bf16
constexpr int kOffKTf = kOffQf + 16384;             // K~^T A fragments [ct=8][s=2][lane][8]
constexpr int kOffAf = kOffKTf + 16384;             // Aqk A fragments [I=4][s=2][lane][8]
constexpr int kOffGam = kOffAf + 8192;              // f32 [128] exp(lg_63)
constexpr int kOffFlag = kOffGam + 512;             // int [4] extreme-decay flags of the loader waves
constexpr int kRowT = 72;                           // padded row of the channel-major tile
constexpr int kOffKEt = kOffFlag + 16;              // bf16 [128][72] k_j E_j, channel-major
constexpr int kSmemBytes = kOffKEt + kKey * kRowT * 2;
// -Kgamma = -exp(lg) k A fragments, 1 KB each (64 lanes x 8 bf16), fragment
// (I, s) at kgf_off<MODE>(I, s), [I][s]: in phase C with P2 over the q a
// tile, which is dead after P2; in phase C without P2 over the k E tile and
// in phase A over the channel-major k E tile, neither of which those modes
// use.
template <int MODE>
__host__ __device__ constexpr int kgf_off(int I, int s) {
  return MODE == kOutput     ? kOffQA + (I * 4 + s) * 1024
         : MODE == kOutputMA ? kOffKE + (I * 4 + s) * 1024
                             : kOffKEt + (I * 4 + s) * 1024;
}
// M = (I + diag(beta) A)^-1 diag(beta) A fragments [I=4][s=2][lane][8]: over
// the k E tile (dead after P2) when M is formed in the loop, over the L tile
// (unused) when it comes from phase A
template <int MODE>
__host__ __device__ constexpr int mf_off() {
  return MODE == kOutputMA ? kOffL : kOffKE;
}
// Lane slots of the Q~, -Kgamma and K~^T fragments.  Phase A and phase C
// without P2 write them straight from the loader registers (a loader thread
// holds 16 rows x 2 channels), and XOR-swizzle the slots so that a loader
// wave's 4- and 8-byte writes spread over the LDS banks; every swizzle
// permutes slots inside aligned groups of eight, which keeps the scanners'
// 16-byte fragment reads conflict-free.  Phase C with P2 exports whole
// 16-byte lanes from the natural tiles, unswizzled.
template <int MODE>
__device__ __forceinline__ int qk_slot(int I, int lane) {  // Q~ / -Kgamma fragment (I, s)
  return MODE != kOutput ? lane ^ ((4 * I + (lane >> 4)) & 7) : lane;
}
template <int MODE>
__device__ __forceinline__ int kt_slot(int ct, int lane) {  // K~^T fragment (ct, s')
  return MODE != kOutput ? lane ^ (ct & 1) : lane;
}
constexpr int kOffStage = kOffKA;  // output transpose [4 waves][64][32]
constexpr int kOffPnat = kOffKA;   // phase A: P_g natural bf16 [128][136]
static_assert(kSmemBytes <= 160 * 1024, "chunk_segment_kernel LDS exceeds one CU");
static_assert(kChunk * 72 * 2 >= 8192, "M fragments must fit in the L tile");
static_assert(mf_off<kSummary>() == kOffKE && mf_off<kOutput>() == kOffKE, "m_block_row writes M over the k E tile");
static_assert(kOffKEt % 16 == 0 && kOffGs % 16 == 0 && kOffGe % 16 == 0, "16-byte LDS accesses need aligned tiles");
static_assert(4 * 64 * 32 * 2 <= kNat, "output stage must fit in the k a tile");
static_assert(kOffStage + 4 * 64 * 32 * 2 <= kgf_off<kOutputMA>(0, 0) && kOffStage + 4 * 64 * 32 * 2 <= kOffVn,
              "phase C without P2 stores a chunk's outputs while the next chunk's operands are written");
static_assert(kKey * kRow * 2 <= 2 * kNat, "P transpose must fit in the k a and q a tiles");
static_assert(16384 <= kNat && 8192 <= kNat, "Kgamma and M fragments must fit in the q a and k E tiles");
static_assert(16384 <= kKey * kRowT * 2, "phase A Kgamma fragments must fit in the channel-major k E tile");
// Fragment element e of lane (i, g) covers reduction index
//   32 s + (e < 4 ? 4 g + e : 16 + 4 g + e - 4),
// the order in which two stacked C tiles provide a B operand.

__device__ __forceinline__ f32x4_t mfma32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(bf16x4_t a, bf16x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c,
                                                     0, 0, 0);
}
template <class V>
__device__ __forceinline__ V negate_bf16(V x) {
  // flip the sign bit of every bf16 lane, two lanes per 32-bit word
  typedef unsigned int u32v __attribute__((ext_vector_type(sizeof(V) / 4)));
  u32v b = __builtin_bit_cast(u32v, x);
  b ^= 0x80008000u;
  return __builtin_bit_cast(V, b);
}
__device__ __forceinline__ int perm_index(int e, int g) { return e < 4 ? 4 * g + e : 16 + 4 * g + e - 4; }

// The value of x, hidden from the optimiser (it cannot be hoisted or
// assumed loop-invariant).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Wave index of a thread, as a wave-uniform (scalar) value: conditions on it
// become scalar branches instead of exec-masked divergent regions.
__device__ __forceinline__ int wave_of(int tid) { return __builtin_amdgcn_readfirstlane(tid >> 6); }

template <class T>
__device__ __forceinline__ T* lds(unsigned char* base, int off) {
  return reinterpret_cast<T*>(base + off);
}
// Row `row` of a block-shifted natural tile at byte offset `off`.
__device__ __forceinline__ bf16* nat_row(unsigned char* sm, int off, int row) {
  return reinterpret_cast<bf16*>(sm + off + row * (kRow * 2) + (row >> 4) * 64);
}

// ---- chunk and segment maps -------------------------------------------------
// chunk_start[s] = sum_{s' < s} ceil(span_{s'} / 64), chunk_start[N] = total chunks;
// seg_start[s]   = sum_{s' < s} max(1, ceil(chunks_{s'} / L)).
__device__ __forceinline__ int32_t seq_chunks(const SeqDesc& seq, int64_t s) {
  return static_cast<int32_t>((seq_range(seq, s).span + kChunk - 1) / kChunk);
}
__device__ __forceinline__ int32_t seq_segments(int32_t chunks, int32_t L) {
  const int32_t n = (chunks + L - 1) / L;
  return n > 1 ? n : 1;
}

__global__ __launch_bounds__(1024) void chunk_map_kernel(SeqDesc seq, int64_t N, int32_t L, int32_t* chunk_start,
                                                         int32_t* seg_start) {
  __shared__ int32_t pc[1024];
  __shared__ int32_t ps[1024];
  const int tid = threadIdx.x;
  const int64_t per = (N + 1023) / 1024;
  const int64_t b0 = tid * per;
  const int64_t b1 = (b0 + per < N) ? b0 + per : N;
  int32_t lc = 0, ls = 0;
  for (int64_t s = b0; s < b1; ++s) {
    const int32_t c = seq_chunks(seq, s);
    lc += c;
    ls += seq_segments(c, L);
  }
  pc[tid] = lc;
  ps[tid] = ls;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t ac = tid >= off ? pc[tid - off] : 0;
    const int32_t as = tid >= off ? ps[tid - off] : 0;
    __syncthreads();
    pc[tid] += ac;
    ps[tid] += as;
    __syncthreads();
  }
  int32_t rc = pc[tid] - lc, rs = ps[tid] - ls;
  for (int64_t s = b0; s < b1; ++s) {
    chunk_start[s] = rc;
    seg_start[s] = rs;
    const int32_t c = seq_chunks(seq, s);
    rc += c;
    rs += seq_segments(c, L);
  }
  if (tid == 1023) {
    chunk_start[N] = pc[1023];
    seg_start[N] = ps[1023];
  }
}

__device__ __forceinline__ int64_t find_seq(const int32_t* start, int64_t N, int64_t x) {
  int64_t lo = 0, hi = N - 1;  // largest s with start[s] <= x
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (start[mid] <= x)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// ---- workspace layouts of the segment buffers --------------------------------
// seg_state / seg_q: f32 in accumulator order [seg][h][V/16 tiles][ct=8][lane][4]
//   (element r of lane (n, g) in row tile ct is row 16 ct + 4 g + r, column 16 t + n);
// seg_p: bf16 A fragments [seg][h][I=8][s=4][lane][8] of the 128x128 transition.
__host__ __device__ constexpr int64_t seg_state_floats(int64_t V) { return kKey * V; }
__host__ __device__ constexpr int64_t seg_p_elems() { return kKey * kKey; }

template <class IT>
struct SegArgs {
  const IT* __restrict__ q;
  const IT* __restrict__ k;
  const IT* __restrict__ v;
  const IT* __restrict__ g;
  const IT* __restrict__ beta;
  IT* __restrict__ out;
  const float* s_in;
  float* s_out;
  SeqDesc seq;
  const int32_t* __restrict__ chunk_start;  // [N+1], or nullptr for dense sequences (closed form)
  const int32_t* __restrict__ seg_start;    // [N+1], or nullptr for dense sequences (closed form)
  int64_t dense_chunks;                     // dense: chunks per sequence
  int64_t dense_segs;                       // dense: segments per sequence
  float* seg_state;
  float* seg_q;
  bf16* seg_p;
  bf16* chunk_ma;  // [chunk][h] M and Aqk fragments (kMaBytes), or nullptr
  int64_t N, H, K, V;  // K <= kKey, a multiple of 16: channels K..kKey-1 are zero padding inside the kernel
  int32_t L;
  // kernels that form g from decay logits (DECAY): `g` then points at the
  // logits z [tokens, H, K], and g = lower_bounded_decay(z + zbias[h],
  // exp(a_log[h]), g_min, clamp to [g_lo, g_hi]), rounded to the input type
  const IT* __restrict__ zbias;  // [H, K] or nullptr
  const float* __restrict__ a_log;  // [H]
  float g_min, g_lo, g_hi;
};

// Per-loader constants of the decay formed from logits: the bias of the
// thread's two channels, the head's scale exp(A_log[h]) and the clamp bounds.
struct DecayConsts {
  float b[2];
  bool ok[2];  // the channel is a real one (< K), not padding
  float scale, g_min, lo, hi;
};

template <class IT, bool DECAY>
__device__ __forceinline__ DecayConsts decay_consts(const SegArgs<IT>& a, int64_t h, int cp) {
  DecayConsts d{};
  if constexpr (DECAY) {
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      d.ok[ch] = 2 * cp + ch < a.K;
      d.b[ch] = (a.zbias && d.ok[ch]) ? to_float(a.zbias[h * a.K + 2 * cp + ch]) : 0.f;
    }
    d.scale = fexp(a.a_log[h]);
    d.g_min = a.g_min;
    d.lo = a.g_lo;
    d.hi = a.g_hi;
  }
  return d;
}

// g of one row and channel: the raw value, or (DECAY) the decay formed from
// its logit and rounded to the input type, as the gates kernel stores it;
// rows past the valid tokens decay by nothing (the operator mask,
// src/kda/utils.py:82-94), and neither do padding channels
template <class IT, bool DECAY>
__device__ __forceinline__ float g_value(float raw, const DecayConsts& d, int ch, bool valid) {
  if constexpr (DECAY) {
    const float gg = lower_bounded_decay(raw, d.b[ch], d.scale, d.g_min, d.lo, d.hi);
    return (valid && d.ok[ch]) ? to_float(from_compute<IT>(gg)) : 0.f;
  } else {
    return raw;
  }
}

// Chunk and segment maps: the arrays of chunk_map_kernel for packed
// documents, a closed form for dense sequences (every sequence has the same
// number of chunks and segments).
template <class A>
__device__ __forceinline__ int64_t chunk_start_of(const A& a, int64_t s) {
  return a.chunk_start ? a.chunk_start[s] : s * a.dense_chunks;
}
template <class A>
__device__ __forceinline__ int64_t seg_start_of(const A& a, int64_t s) {
  return a.seg_start ? a.seg_start[s] : s * a.dense_segs;
}
template <class A>
__device__ __forceinline__ int64_t seq_of_segment(const A& a, int64_t gsg) {
  return a.seg_start ? find_seq(a.seg_start, a.N, gsg) : gsg / a.dense_segs;
}

struct ChunkGeo {
  int64_t tok0;
  int n_span;
  int n_valid;
};

__device__ __forceinline__ ChunkGeo chunk_geo(const SeqRange& sr, int64_t lc) {
  ChunkGeo c;
  c.tok0 = sr.start + kChunk * lc;
  const int64_t rest = sr.span - kChunk * lc;
  c.n_span = static_cast<int>(rest < kChunk ? rest : kChunk);
  const int64_t nv = sr.valid - kChunk * lc;
  c.n_valid = static_cast<int>(nv < 0 ? 0 : (nv > c.n_span ? c.n_span : nv));
  return c;
}

// Raw inputs of one chunk, held in the registers of the four loader waves
// (4-7) between chunks: loader thread (block J = lane / 16, channel pair
// cp = 16 (wave - 4) + lane % 16) holds g, k (and q) of the 16 rows of block
// J, so the four blocks of a channel pair sit in lanes l, l + 16, l + 32,
// l + 48 of one wave; the 256 loader threads together hold the chunk's v
// slice of this column group and beta.
__device__ __forceinline__ int loader_block(int tid) { return (tid & 63) >> 4; }
__device__ __forceinline__ int loader_pair(int tid) { return 16 * (wave_of(tid) - 4) + (tid & 15); }
// Whether loader wave w holds channels the chunk reads.  With K <= 64 (four
// state row tiles) waves 6 and 7 hold channels 64..127, all padding, and no
// product reads them (P2, the state advance and the output reduce over the
// first 64 channels only): those waves skip the channel work of P1 and keep
// only their share of v, beta and the M/Aqk units.  With eight row tiles
// every channel's operands are read, the padding ones as zeros, so every
// wave forms them.
template <bool PAD, int KT>
__device__ __forceinline__ bool kChanWave(int w) { return !(PAD && KT == 4) || w < 6; }

template <class IT>
struct Raw {
  typedef IT pair_t __attribute__((ext_vector_type(2)));
  pair_t gp[16], kp[16], qp[16];
  uint4 vv[4];
  IT bt;
  uint4 ma[3];  // M and Aqk units t2, t2 + 256, t2 + 512 (phase C without P2)
};

// Raw buffer resource over `bytes` bytes from `base` (dword 3 is the gfx9
// family's untyped 32-bit data format).  The hardware checks each lane's
// offset against `bytes`: a load past it returns zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// One chunk's raw inputs as buffer resources over this head's rows of the
// chunk's valid tokens (rows past them read as zero), built once per chunk in
// scalar registers; every load then needs only a lane offset.
struct ChunkLoads {
  __amdgpu_buffer_rsrc_t g, k, q, v, beta, ma;
  int krow;  // bytes per token of q, k, g
};

// `active` false gives resources of zero size: every load returns zero and
// reads no memory, so the loads need no branch around them.
template <class IT>
__device__ __forceinline__ ChunkLoads chunk_loads(const SegArgs<IT>& a, const ChunkGeo& cg, int64_t c, int64_t h,
                                                  int64_t col0, bool active = true) {
  constexpr int64_t kEl = sizeof(IT);
  ChunkLoads cl;
  cl.krow = static_cast<int>(a.H * a.K * kEl);
  const int64_t nv = active ? cg.n_valid : 0;
  const int64_t kb = (cg.tok0 * a.H + h) * a.K * kEl;
  const int64_t kbytes = nv * cl.krow;
  cl.g = buffer_rsrc(reinterpret_cast<const char*>(a.g) + kb, kbytes);
  cl.k = buffer_rsrc(reinterpret_cast<const char*>(a.k) + kb, kbytes);
  cl.q = buffer_rsrc(reinterpret_cast<const char*>(a.q) + kb, kbytes);
  cl.v = buffer_rsrc(reinterpret_cast<const char*>(a.v) + ((cg.tok0 * a.H + h) * a.V + col0) * kEl,
                     nv * a.H * a.V * kEl);
  cl.beta = buffer_rsrc(reinterpret_cast<const char*>(a.beta) + (cg.tok0 * a.H + h) * kEl, nv * a.H * kEl);
  cl.ma = buffer_rsrc(a.chunk_ma ? reinterpret_cast<const char*>(a.chunk_ma) + (c * a.H + h) * kMaBytes : nullptr,
                      (a.chunk_ma && active) ? kMaBytes : 0);
  return cl;
}

// Lane offsets of a loader thread's v units in the chunk (-1: no unit) and
// in the LDS tile, and of beta, fixed for the whole segment.
struct LoaderLanes {
  int v[4];
  int vlds[4];
  int beta;
  int kcol;  // byte offset of the thread's channel pair in a q/k/g row, or past every chunk (padding channels)
};

template <class IT, bool PAD>
__device__ __forceinline__ LoaderLanes loader_lanes(const SegArgs<IT>& a, int vcg, int tid) {
  constexpr int kEl = sizeof(IT);
  const int t2 = tid - 256;
  const int upr = vcg / 8;  // 16-byte units per row
  LoaderLanes ll;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = t2 + 256 * i;
    const int row = u / upr;
    ll.v[i] = row < kChunk ? row * static_cast<int>(a.H * a.V * kEl) + 16 * (u % upr) : -1;
    ll.vlds[i] = row < kChunk ? (row * kRow + 8 * (u % upr)) * 2 : -1;
  }
  ll.beta = t2 < kChunk ? t2 * static_cast<int>(a.H * kEl) : -1;
  // a padding channel pair reads at 64 rows past the chunk's first row, beyond
  // every chunk's resource range, so its loads return zero
  const int cp = loader_pair(tid);
  ll.kcol = (!PAD || 2 * cp < a.K) ? 4 * cp : static_cast<int>(kChunk * a.H * a.K * kEl);
  return ll;
}

// Part PART (0..7) of the loads of one chunk's raw inputs: rows 2 PART and
// 2 PART + 1 of g, k and q of this thread's block, one 16-byte v unit on
// even parts, beta on the last and, in phase C without P2, one 16-byte unit
// of the chunk's M and Aqk fragments on parts 5-7.  Spreading the eight parts over a chunk's
// phases keeps any single moment's burst of requests small: issued at once,
// every CU's 64 KB would saturate HBM and stall the issuing waves.
template <class IT, int MODE, int PART>
__device__ __forceinline__ void load_raw_part(Raw<IT>& raw, const ChunkLoads& cl, const LoaderLanes& ll, int tid) {
  typedef typename Raw<IT>::pair_t pair_t;
  const int J = loader_block(tid);
#pragma unroll
  for (int r = 2 * PART; r < 2 * PART + 2; ++r) {
    const int off = (16 * J + r) * cl.krow + ll.kcol;
    raw.gp[r] = __builtin_bit_cast(pair_t, __builtin_amdgcn_raw_buffer_load_b32(cl.g, off, 0, 0));
    raw.kp[r] = __builtin_bit_cast(pair_t, __builtin_amdgcn_raw_buffer_load_b32(cl.k, off, 0, 0));
    raw.qp[r] = __builtin_bit_cast(pair_t, __builtin_amdgcn_raw_buffer_load_b32(cl.q, off, 0, 0));
  }
  if constexpr (MODE == kOutputMA && PART >= 5)
    raw.ma[PART - 5] = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(cl.ma, ((tid - 256) + 256 * (PART - 5)) * 16, 0, 0));
  if constexpr ((PART & 1) == 0) {
    const int i = PART / 2;
    if (ll.v[i] >= 0) raw.vv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(cl.v, ll.v[i], 0, 0));
  }
  if constexpr (PART == 7) {
    if (ll.beta >= 0) raw.bt = __builtin_bit_cast(IT, __builtin_amdgcn_raw_buffer_load_b16(cl.beta, ll.beta, 0, 0));
  }
}

template <class IT, int MODE>
__device__ __forceinline__ void load_raw(Raw<IT>& raw, const ChunkLoads& cl, const LoaderLanes& ll, int tid) {
  load_raw_part<IT, MODE, 0>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 1>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 2>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 3>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 4>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 5>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 6>(raw, cl, ll, tid);
  load_raw_part<IT, MODE, 7>(raw, cl, ll, tid);
}

// Where the loader waves are in a chunk's phases, for the spread loads of
// the next chunk: `load_part<P>()` issues part P (of zero-size resources past
// the segment's last chunk).  The loads carry no branch: a conditional load
// leaves its registers possibly pending on the other path, and the waits the
// compiler then places before reusing registers stall every later part.
template <class IT, int MODE>
struct NextLoads {
  Raw<IT>* raw;
  ChunkLoads cl;
  const LoaderLanes* ll;
  int tid;
  template <int P>
  __device__ __forceinline__ void load_part() const {
    load_raw_part<IT, MODE, P>(*raw, cl, *ll, tid);
  }
};

// Block row I of M = (I + B)^{-1} diag(beta) (B = diag(beta) A, strictly
// lower) as A fragments.  With N = (I + B)^{-1}, block row I of Z = N^T obeys
//   Z_II = T_I^T ;  Z_IJ = -T_J^T sum_{K=J+1..I} B_KJ^T Z_IK   (J < I),
// a chain in which Z_IK is the B operand of the next product.  In the
// accumulator layout lane (i, g) holds Z_IJ[4 g + r][i] = N[16 I + i][16 J + 4 g + r],
// which is half of an A fragment of M (rows i, reduction over j).
template <int I>
__device__ __forceinline__ void m_block_row(unsigned char* sm, int lane) {
  const int n16 = lane & 15;
  const int g4 = lane >> 4;
  bf16(*Lm)[72] = lds<bf16[72]>(sm, kOffL);
  bf16(*Tinv)[16][16] = lds<bf16[16][16]>(sm, kOffTinv);
  bf16(*TinvT)[16][16] = lds<bf16[16][16]>(sm, kOffTinvT);
  const float* betas = lds<float>(sm, kOffBeta);
  unsigned char* mf = sm + kOffKE;  // where the modes that form M keep it
  // every operand of the chain first (one LDS round trip):
  //   bt[J][K - J - 1] = B_KJ^T (lane (j, g) holds B[16K + 4g + r][16J + j]),
  //   ta[J] = -T_J^T (lane (j, g) holds T_J[4g + r][j]), b4[J] = beta of block J
  bf16x4_t tI = *reinterpret_cast<const bf16x4_t*>(&Tinv[I][n16][4 * g4]);  // T_I[i][4g + r]
  bf16x4_t bt[I > 0 ? I : 1][I > 0 ? I : 1];
  bf16x4_t ta[I > 0 ? I : 1];
  f32x4_t b4[I + 1];
#pragma unroll
  for (int J = 0; J <= I; ++J) b4[J] = *reinterpret_cast<const f32x4_t*>(&betas[16 * J + 4 * g4]);
#pragma unroll
  for (int J = 0; J < I; ++J) {
    ta[J] = negate_bf16(*reinterpret_cast<const bf16x4_t*>(&TinvT[J][n16][4 * g4]));
#pragma unroll
    for (int K = J + 1; K <= I; ++K)
#pragma unroll
      for (int r = 0; r < 4; ++r) bt[J][K - J - 1][r] = Lm[16 * K + 4 * g4 + r][16 * J + n16];
  }
  __builtin_amdgcn_sched_barrier(0);
  auto put = [&](int J, const f32x4_t& z) {  // M_IJ = N_IJ diag(beta_J)
    *reinterpret_cast<bf16x4_t*>(mf + ((I * 2 + J / 2) * 64 + lane) * 16 + (J & 1) * 8) =
        bf16x4_t{(bf16)(z[0] * b4[J][0]), (bf16)(z[1] * b4[J][1]), (bf16)(z[2] * b4[J][2]), (bf16)(z[3] * b4[J][3])};
  };
  f32x4_t Z[I + 1];
  Z[I] = f32x4_t{(float)tI[0], (float)tI[1], (float)tI[2], (float)tI[3]};
  put(I, Z[I]);
  if constexpr ((I & 1) == 0)  // block (I, I + 1) is above the diagonal
    *reinterpret_cast<bf16x4_t*>(mf + ((I * 2 + I / 2) * 64 + lane) * 16 + 8) = bf16x4_t{};
#pragma unroll
  for (int J = I - 1; J >= 0; --J) {
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int K = J + 1; K <= I; ++K) {
      const bf16x4_t zb = {(bf16)Z[K][0], (bf16)Z[K][1], (bf16)Z[K][2], (bf16)Z[K][3]};
      acc = mfma16(bt[J][K - J - 1], zb, acc);
    }
    const bf16x4_t ab = {(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
    Z[J] = mfma16(ta[J], ab, f32x4_t{0.f, 0.f, 0.f, 0.f});
    put(J, Z[J]);
  }
}

// ---- per-chunk preparation: every chunk operand, in LDS ---------------------
// P1 of one chunk, computed by a loader thread (block J, channel pair cp)
// from the raw inputs into registers: the decayed rows k a, q a, k E as bf16
// pairs, the per-channel decay tables of block J (from the four blocks'
// products, exchanged between the lanes that hold them), the v slice (bf16)
// and beta.  The loaders compute it for chunk c + 1 while the scanners
// advance the state through chunk c, and write it to LDS at the top of the
// next chunk (p1_write).
struct P1Out {
  uint32_t ka[16], qa[16], ke[16];  // bf16 pairs (channels 2cp, 2cp + 1) of rows 16 J + r
  uint32_t kg[16], kt[16];          // phase A: -Kgamma and K~ rows, written straight into fragments
  float gs[2];                      // exp(lg_{16J})
  float ge[2];                      // exp(lg_63 - lg_{16J+15})
  float gam[2];                     // exp(lg_63)
  float sc[4][2];                   // scales of block pairs (J, J'), J' <= J
  int ext;                          // some block of the wave's channels decays past 2^-100
  uint4 vv[4];                      // bf16 v units of this thread (zero past the valid rows)
  float bt;                         // beta of row t2 (< 64), zero past the valid rows
  uint4 ma[3];                      // M and Aqk units (phase C without P2)
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(bf16)lo, (bf16)hi});
}

template <class IT, int MODE, bool DECAY>
__device__ __forceinline__ void p1_math(P1Out& po, const Raw<IT>& raw, const ChunkGeo& cg, int vcg, int tid,
                                        const DecayConsts& dc, bool chan = true) {
  // rows past the chunk's valid tokens were read as zero (g = 0, k = q = 0),
  // so they give a unit decay and zero operands without a test (a decay
  // formed from logits is zeroed there explicitly).  `chan` false (a loader
  // wave whose channels are all padding and never read): only v and beta.
  const int J = loader_block(tid);
  const int lane = tid & 63;
  po.ext = 0;
  if (chan) {
  float al[2][16];
  float pj[2] = {1.f, 1.f};  // P_J = exp(lg_{16J+15} - lg_{16J})
#pragma unroll
  for (int r = 0; r < 16; ++r) {
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      al[ch][r] = fast_exp(g_value<IT, DECAY>(to_float(raw.gp[r][ch]), dc, ch, 16 * J + r < cg.n_valid));
      if (r > 0) pj[ch] *= al[ch][r];
    }
  }
  // Block J's products P_J and alpha at its first row A0_J give G_J = A0_J P_J,
  // the decay across the block; the other blocks' G come from lanes l ^ 16,
  // l ^ 32, l ^ 48.
  //   Gs_J = A0_J prod_{J' < J} G_J',  Ge_J = prod_{J' > J} G_J',  gamma = prod G_J',
  //   pair (J, J') scale: A0_J prod_{J' < j < J} G_j (J' < J), 1 / P_J (J' = J).
  bool ext = false;
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    const float a0 = al[ch][0];
    ext = ext || !(pj[ch] >= kExtremeDecay && pj[ch] <= kExtremeGrowth);
    float G[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) G[jb] = __shfl(a0 * pj[ch], (lane & 15) + 16 * jb);
    float pre = 1.f, post = 1.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      pre *= jb < J ? G[jb] : 1.f;
      post *= jb > J ? G[jb] : 1.f;
    }
    po.gs[ch] = pre * a0;
    po.ge[ch] = post;
    po.gam[ch] = G[0] * G[1] * G[2] * G[3];
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      float sc = a0;
#pragma unroll
      for (int jj = 1; jj < 3; ++jj) sc *= (jj > jp && jj < J) ? G[jj] : 1.f;
      po.sc[jp][ch] = jp < J ? sc : (pj[ch] > 0.f ? 1.f / pj[ch] : 0.f);
    }
  }
  po.ext = __any(ext) ? 1 : 0;
  // k a, q a (and in phase A -Kgamma = -k a Gs) forward; k E (and K~ = k E Ge) backward
  float run[2] = {1.f, 1.f};
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float kv[2], qv[2];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      if (r > 0) run[ch] *= al[ch][r];
      kv[ch] = to_float(raw.kp[r][ch]) * run[ch];
      qv[ch] = to_float(raw.qp[r][ch]) * run[ch];
    }
    po.ka[r] = pack_bf16x2(kv[0], kv[1]);
    po.qa[r] = pack_bf16x2(qv[0], qv[1]);
    if constexpr (MODE == kSummary) po.kg[r] = pack_bf16x2(-kv[0] * po.gs[0], -kv[1] * po.gs[1]);
  }
  float suf[2] = {1.f, 1.f};
#pragma unroll
  for (int r = 15; r >= 0; --r) {
    float kv[2];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) kv[ch] = to_float(raw.kp[r][ch]) * suf[ch];
    po.ke[r] = pack_bf16x2(kv[0], kv[1]);
    if constexpr (MODE == kSummary) po.kt[r] = pack_bf16x2(kv[0] * po.ge[0], kv[1] * po.ge[1]);
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) suf[ch] *= al[ch][r];
  }
  }  // chan
  const int t2 = tid - 256;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 val = raw.vv[i];  // rows past the valid ones were read as zero
    if constexpr (sizeof(IT) == 2 && !__is_same(IT, bf16)) {
      // f16 inputs: convert the 8 values to bf16 operands
      typedef IT h8_t __attribute__((ext_vector_type(8)));
      const h8_t x = __builtin_bit_cast(h8_t, val);
      bf16x8_t y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (bf16)to_float(x[e]);
      val = __builtin_bit_cast(uint4, y);
    }
    po.vv[i] = val;
  }
  po.bt = (t2 < kChunk && t2 < cg.n_valid) ? to_float(raw.bt) : 0.f;
}

// Operand rows of a loader thread (block J, channel pair cp) written straight
// into A fragments.  A wave owns channels 32 s .. 32 s + 31 (s = wave - 4):
// for an operand that reduces over channels (Q~, -Kgamma) they are reduction
// step s, and channel pair (2 cp, 2 cp + 1) of row 16 J + r is one 4-byte
// piece of lane (r, g) of fragment (J, s) at `frag`.
template <int MODE>
__device__ __forceinline__ void write_channel_frags(unsigned char* frag, const uint32_t (&x)[16], int J, int lane) {
  const int m = lane & 15;
  const int g = (m & 7) >> 1;                  // channel 32 s + 2 m: lane group g,
  const int eb = 4 * (m & 1) + 8 * (m >> 3);  // byte 2 e of the lane's 16 bytes
#pragma unroll
  for (int r = 0; r < 16; ++r) *reinterpret_cast<uint32_t*>(frag + qk_slot<MODE>(J, r + 16 * g) * 16 + eb) = x[r];
}
// K~ rows into the K~^T fragments, which reduce over rows: channel ch is row
// ch % 16 of row tile ct = ch / 16, and rows 16 J + 4 g .. 16 J + 4 g + 3 are
// one 8-byte half of lane (ch % 16, g) of reduction step J / 2.
template <int MODE>
__device__ __forceinline__ void write_kt_frags(unsigned char* sm, const uint32_t (&kt)[16], int J, int cp) {
#pragma unroll
  for (int chp = 0; chp < 2; ++chp) {
    const int ch = 2 * cp + chp;
    const int ct = ch >> 4;
    unsigned char* frag = sm + kOffKTf + (ct * 2 + (J >> 1)) * 1024 + (J & 1) * 8;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      uint32_t w[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const uint32_t a = kt[4 * gg + 2 * h2], b = kt[4 * gg + 2 * h2 + 1];
        w[h2] = chp == 0 ? (a & 0xffffu) | (b << 16) : (a >> 16) | (b & 0xffff0000u);
      }
      *reinterpret_cast<uint2*>(frag + kt_slot<MODE>(ct, (ch & 15) + 16 * gg) * 16) = uint2{w[0], w[1]};
    }
  }
}

// The part of P1 that only P2 and M read: the k a and q a tiles, the pair
// scales, the extreme-decay flags and beta.  Phase A, whose state advance
// reads none of them, writes it while the scanners advance the previous
// chunk (p1_write_early); the other modes write it with the rest.
template <int MODE>
inline constexpr bool kEarlyP1 = MODE == kSummary;
template <int MODE>
__device__ __forceinline__ void p1_write_early(unsigned char* sm, const P1Out& po, int tid, bool chan = true) {
  const int J = loader_block(tid);
  const int cp = loader_pair(tid);
  float(*Sc)[kKey] = lds<float[kKey]>(sm, kOffTab);
  float* betas = lds<float>(sm, kOffBeta);
  if (chan) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tl = 16 * J + r;
      *reinterpret_cast<uint32_t*>(nat_row(sm, kOffKA, tl) + 2 * cp) = po.ka[r];
      *reinterpret_cast<uint32_t*>(nat_row(sm, kOffQA, tl) + 2 * cp) = po.qa[r];
    }
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const int cc = 2 * cp + ch;
#pragma unroll
      for (int jp = 0; jp < 4; ++jp)
        if (jp <= J) Sc[J * (J + 1) / 2 + jp][cc] = po.sc[jp][ch];
    }
  }
  if ((tid & 63) == 0) lds<int>(sm, kOffFlag)[wave_of(tid) - 4] = po.ext;
  const int t2 = tid - 256;
  if (t2 < kChunk) betas[t2] = po.bt;
}

// Writes P1 (loader waves) and joins every wave at the first barrier of the
// chunk.
template <int MODE, bool LOADER>
__device__ __forceinline__ void p1_write(unsigned char* sm, const P1Out& po, const LoaderLanes* ll, int tid,
                                         bool chan = true) {
  if constexpr (LOADER) {
    const int J = loader_block(tid);
    const int cp = loader_pair(tid);
    bf16(*KEt)[kRowT] = lds<bf16[kRowT]>(sm, kOffKEt);
    float(*Gs)[kKey] = lds<float[kKey]>(sm, kOffGs);
    float(*Ge)[kKey] = lds<float[kKey]>(sm, kOffGe);
    float* gam = lds<float>(sm, kOffGam);
    if constexpr (!kEarlyP1<MODE>) p1_write_early<MODE>(sm, po, tid, chan);
    if (chan) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tl = 16 * J + r;
      if constexpr (kPrepares<MODE>) *reinterpret_cast<uint32_t*>(nat_row(sm, kOffKE, tl) + 2 * cp) = po.ke[r];
    }
    // phase A writes the state advance's operands later (p1_write_late)
    if constexpr (MODE != kSummary) {
      // channel-major k E: rows 16 J .. 16 J + 15 of channels 2 cp, 2 cp + 1
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        uint32_t w[8];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          w[m] = ch == 0 ? (po.ke[2 * m] & 0xffffu) | (po.ke[2 * m + 1] << 16)
                         : (po.ke[2 * m] >> 16) | (po.ke[2 * m + 1] & 0xffff0000u);
        *reinterpret_cast<uint4*>(&KEt[2 * cp + ch][16 * J]) = uint4{w[0], w[1], w[2], w[3]};
        *reinterpret_cast<uint4*>(&KEt[2 * cp + ch][16 * J + 8]) = uint4{w[4], w[5], w[6], w[7]};
      }
    }
    if constexpr (MODE != kSummary) {
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        const int cc = 2 * cp + ch;
        if constexpr (MODE == kOutput) {
          Gs[J][cc] = po.gs[ch];
          Ge[J][cc] = po.ge[ch];
        }
        if (J == 0) gam[cc] = po.gam[ch];
      }
    }
    }  // chan
    if constexpr (MODE != kSummary) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (ll->vlds[i] >= 0) *reinterpret_cast<uint4*>(sm + kOffVn + ll->vlds[i]) = po.vv[i];
    }
  }
  __syncthreads();
}

// Phase A: the operands that only the state advance reads (-Kgamma and K~^T
// fragments straight from the registers, gamma, the v tile), written by the
// loader waves while waves 0-3 form the diagonal-block inverses, so that the
// first barrier of the chunk waits for the k E tile alone.  None of these
// tiles is touched between the previous chunk's state advance and this one's.
template <int MODE>
__device__ __forceinline__ void p1_write_late(unsigned char* sm, const P1Out& po, const LoaderLanes& ll, int tid,
                                              bool chan = true) {
  const int J = loader_block(tid);
  const int cp = loader_pair(tid);
  if (chan) {
    write_channel_frags<MODE>(sm + kgf_off<MODE>(J, wave_of(tid) - 4), po.kg, J, tid & 63);
    write_kt_frags<MODE>(sm, po.kt, J, cp);
    float* gam = lds<float>(sm, kOffGam);
    if (J == 0) {
      gam[2 * cp] = po.gam[0];
      gam[2 * cp + 1] = po.gam[1];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (ll.vlds[i] >= 0) *reinterpret_cast<uint4*>(sm + kOffVn + ll.vlds[i]) = po.vv[i];
}

// P1 of phase C without P2, which needs no natural tiles: the loader thread
// turns its rows straight into operand values,
//   Q~ = exp(lg) q,  -Kgamma = -exp(lg) k  (running products from exp(lg_{16J})),
//   K~ = exp(lg_63 - lg) k                 (running products back from exp(lg_63 - lg_{16J+15})),
// with the block products of the other three blocks of its channels taken
// from the lanes that hold them.  Rows past the chunk's valid tokens were read
// as zero (g = 0, k = q = 0), so they give zero operands and a unit decay.
template <class IT, bool DECAY>
__device__ __forceinline__ void p1_math_ma(P1Out& po, const Raw<IT>& raw, int tid, int n_valid,
                                           const DecayConsts& dc, bool chan = true) {
  const int J = loader_block(tid);
  const int lane = tid & 63;
  if (chan) {  // false: a loader wave whose channels are all padding and never read (v and M, Aqk only)
  float al[2][16];
  float pj[2] = {1.f, 1.f};
#pragma unroll
  for (int r = 0; r < 16; ++r) {
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      al[ch][r] = fast_exp(g_value<IT, DECAY>(to_float(raw.gp[r][ch]), dc, ch, 16 * J + r < n_valid));
      if (r > 0) pj[ch] *= al[ch][r];
    }
  }
  float x[2], y[2];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    const float a0 = al[ch][0];
    float G[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) G[jb] = __shfl(a0 * pj[ch], (lane & 15) + 16 * jb);
    float pre = 1.f, post = 1.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      pre *= jb < J ? G[jb] : 1.f;
      post *= jb > J ? G[jb] : 1.f;
    }
    x[ch] = pre * a0;  // exp(lg_{16J})
    y[ch] = post;      // exp(lg_63 - lg_{16J+15})
    po.gam[ch] = G[0] * G[1] * G[2] * G[3];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float kv[2], qv[2];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      if (r > 0) x[ch] *= al[ch][r];
      kv[ch] = to_float(raw.kp[r][ch]) * x[ch];
      qv[ch] = to_float(raw.qp[r][ch]) * x[ch];
    }
    po.qa[r] = pack_bf16x2(qv[0], qv[1]);
    po.ka[r] = pack_bf16x2(-kv[0], -kv[1]);
  }
#pragma unroll
  for (int r = 15; r >= 0; --r) {
    po.ke[r] = pack_bf16x2(to_float(raw.kp[r][0]) * y[0], to_float(raw.kp[r][1]) * y[1]);
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) y[ch] *= al[ch][r];
  }
  }  // chan
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 val = raw.vv[i];
    if constexpr (sizeof(IT) == 2 && !__is_same(IT, bf16)) {
      typedef IT h8_t __attribute__((ext_vector_type(8)));
      const h8_t xv = __builtin_bit_cast(h8_t, val);
      bf16x8_t yv;
#pragma unroll
      for (int e = 0; e < 8; ++e) yv[e] = (bf16)to_float(xv[e]);
      val = __builtin_bit_cast(uint4, yv);
    }
    po.vv[i] = val;
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) po.ma[k] = raw.ma[k];
}

// Writes P1 of phase C without P2 into the fragment tiles the scanners read,
// issuing parts 0-5 of the next chunk's loads between the writes.  A loader
// wave owns channels 32 s .. 32 s + 31 (s = wave - 4), which are reduction
// step s of the Q~ and -Kgamma fragments: channel pair (2 cp, 2 cp + 1) of
// row 16 J + r is one 4-byte piece of lane (r, g) of fragment (J, s).  Of
// the K~^T fragments, channel ch is row ch % 16 of row tile ch / 16, and
// rows 16 J + 4 g .. 16 J + 4 g + 3 are one 8-byte half of lane (ch % 16, g)
// of reduction step J / 2.
template <class IT, int MODE>
__device__ __forceinline__ void p1_write_ma(unsigned char* sm, const P1Out& po, const LoaderLanes& ll, int tid,
                                            const NextLoads<IT, MODE>& nl, bool chan = true) {
  const int lane = tid & 63;
  const int J = loader_block(tid);
  const int cp = loader_pair(tid);
  const int s = wave_of(tid) - 4;
  nl.template load_part<0>();
  nl.template load_part<1>();
  if (chan) {
    write_channel_frags<MODE>(sm + kOffQf + (J * 4 + s) * 1024, po.qa, J, lane);
    write_channel_frags<MODE>(sm + kgf_off<MODE>(J, s), po.ka, J, lane);
  }
  nl.template load_part<2>();
  nl.template load_part<3>();
  if (chan) write_kt_frags<MODE>(sm, po.ke, J, cp);
  nl.template load_part<4>();
  nl.template load_part<5>();
  if (chan && J == 0) {
    float* gam = lds<float>(sm, kOffGam);
    gam[2 * cp] = po.gam[0];
    gam[2 * cp + 1] = po.gam[1];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (ll.vlds[i] >= 0) *reinterpret_cast<uint4*>(sm + kOffVn + ll.vlds[i]) = po.vv[i];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int u = (tid - 256) + 256 * k;  // [M | Aqk][j][lane]
    const int slot = lower_slot((u >> 6) % 6);
    *reinterpret_cast<uint4*>(sm + (u < 384 ? mf_off<MODE>() : kOffAf) + (slot * 64 + (u & 63)) * 16) = po.ma[k];
  }
}

// Everything after P1 (reads only LDS, plus global q/k/g on the rare
// extreme-decay path).
template <class IT, int MODE, bool LOADER, bool DECAY, int KT>
__device__ __forceinline__ void prepare_mid(unsigned char* sm, const SegArgs<IT>& a, const ChunkGeo& cg, int64_t h,
                                            int vcg, int tid, const NextLoads<IT, MODE>& nl,
                                            const P1Out* po = nullptr, const LoaderLanes* ll = nullptr,
                                            bool chan = true) {
  const int lane = tid & 63;
  const int wave = wave_of(tid);
  const int n16 = lane & 15;
  const int g4 = lane >> 4;
  const int n_valid = cg.n_valid;
  bf16(*Lm)[72] = lds<bf16[72]>(sm, kOffL);
  float(*Ld)[16][16] = lds<float[16][16]>(sm, kOffLd);
  bf16(*Tinv)[16][16] = lds<bf16[16][16]>(sm, kOffTinv);
  bf16(*TinvT)[16][16] = lds<bf16[16][16]>(sm, kOffTinvT);
  bf16(*KEt)[kRowT] = lds<bf16[kRowT]>(sm, kOffKEt);
  float(*Sc)[kKey] = lds<float[kKey]>(sm, kOffTab);  // pair scales [10][128]
  float(*Gs)[kKey] = lds<float[kKey]>(sm, kOffGs);
  float(*Ge)[kKey] = lds<float[kKey]>(sm, kOffGe);
  float* betas = lds<float>(sm, kOffBeta);
  const int* flags = lds<int>(sm, kOffFlag);

  static_assert(MODE != kOutputMA, "phase C without P2 builds its operands in p1_write_ma");

  if constexpr (LOADER) {
    nl.template load_part<0>();
    nl.template load_part<1>();
  }
  if constexpr (MODE == kOutput) {
    // phase C: every wave exports Q~ and K~^T and takes block pairs of P2;
    // the loaders export -Kgamma during P3
  // ---- export: Q~ (phase C) and K~^T fragments ------------------------------
    // element e of lane (i, g) of fragment s covers index 32 s + 4 g + e (e < 4)
    // and 32 s + 16 + 4 g + e - 4: two runs of four, one 8-byte read each.  Task
    // tid + 512 k is a Q~ fragment lane for k < 2 (phase C) and a K~^T one
    // otherwise; every task's reads go out before any is used.
    {
      constexpr int k0 = MODE == kOutput ? 0 : 2;
      bf16x4_t lo[4], hi[4];
      f32x4_t slo[4], shi[4];
  #pragma unroll
      for (int k = k0; k < 4; ++k) {
        const int task = tid + kThreads * k;
        const int frag = (task >> 6) & 15;
        const int fi = task & 15, fg = (task >> 4) & 3;
        if (k < 2) {  // Q~ = exp(lg) q : fragment (I, s), lane (i, g)
          const int I = frag >> 2, c0 = 32 * (frag & 3) + 4 * fg;
          const bf16* row = nat_row(sm, kOffQA, 16 * I + fi);
          lo[k] = *reinterpret_cast<const bf16x4_t*>(row + c0);
          hi[k] = *reinterpret_cast<const bf16x4_t*>(row + c0 + 16);
          slo[k] = *reinterpret_cast<const f32x4_t*>(&Gs[I][c0]);
          shi[k] = *reinterpret_cast<const f32x4_t*>(&Gs[I][c0 + 16]);
        } else {  // K~^T : fragment (ct, s'), lane (c, g); rows r0.. and r0 + 16.. each sit in one block
          const int ch = 16 * (frag >> 1) + fi, r0 = 32 * (frag & 1) + 4 * fg;
          lo[k] = *reinterpret_cast<const bf16x4_t*>(&KEt[ch][r0]);
          hi[k] = *reinterpret_cast<const bf16x4_t*>(&KEt[ch][r0 + 16]);
          slo[k][0] = Ge[r0 >> 4][ch];
          shi[k][0] = Ge[(r0 + 16) >> 4][ch];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
      for (int k = k0; k < 4; ++k) {
        const int task = tid + kThreads * k;
        bf16x8_t o;
  #pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = (bf16)((float)lo[k][e] * (k < 2 ? slo[k][e] : slo[k][0]));
          o[4 + e] = (bf16)((float)hi[k][e] * (k < 2 ? shi[k][e] : shi[k][0]));
        }
        *lds<bf16x8_t>(sm, (k < 2 ? kOffQf : kOffKTf) + (task & 1023) * 16) = o;
      }
    }
  
    if constexpr (LOADER) nl.template load_part<2>();
    // ---- P2: A (strict) and Aqk (causal) 16x16 blocks on MFMA ---------------
    for (int p = wave; p < 10; p += 8) {
      // block pair p = I (I + 1) / 2 + J, J <= I
      const int I = p >= 6 ? 3 : (p >= 3 ? 2 : (p >= 1 ? 1 : 0));
      const int J = p - I * (I + 1) / 2;
      // the operands of two reduction steps at a time (two LDS round trips per pair)
      const bf16* ke_row = nat_row(sm, kOffKE, 16 * J + n16);
      const bf16* ka_row = nat_row(sm, kOffKA, 16 * I + n16);
      const bf16* qa_row = nat_row(sm, kOffQA, 16 * I + n16);
      const int i = 16 * I + n16;
      const float bi = betas[i];
      f32x4_t akk = {0.f, 0.f, 0.f, 0.f};
      f32x4_t aqk = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
      for (int half = 0; half < KT / 4; ++half) {
        bf16x8_t ke[2], kb[2], qb[2];
        f32x4_t sc0[2], sc1[2];
  #pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int c0 = 32 * (2 * half + u) + 8 * g4;
          ke[u] = *reinterpret_cast<const bf16x8_t*>(ke_row + c0);
          sc0[u] = *reinterpret_cast<const f32x4_t*>(&Sc[p][c0]);
          sc1[u] = *reinterpret_cast<const f32x4_t*>(&Sc[p][c0 + 4]);
          kb[u] = *reinterpret_cast<const bf16x8_t*>(ka_row + c0);
          qb[u] = *reinterpret_cast<const bf16x8_t*>(qa_row + c0);
        }
        __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
        for (int u = 0; u < 2; ++u) {
          bf16x8_t af;
  #pragma unroll
          for (int e = 0; e < 4; ++e) {
            af[e] = (bf16)((float)ke[u][e] * sc0[u][e]);
            af[4 + e] = (bf16)((float)ke[u][4 + e] * sc1[u][e]);
          }
          akk = mfma32(af, kb[u], akk);
          aqk = mfma32(af, qb[u], aqk);
        }
      }
      // lane (n16, g4) holds A[16I + n16][16J + 4 g4 + r] (and likewise Aqk)
      bf16x4_t lrow;
      bf16x4_t qrow;
  #pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * J + 4 * g4 + r;
        const float vk = (j < i) ? akk[r] * bi : 0.f;
        lrow[r] = (bf16)vk;
        qrow[r] = (bf16)((j <= i) ? aqk[r] : 0.f);
        if (I == J) Ld[I][n16][4 * g4 + r] = vk;
      }
      *reinterpret_cast<bf16x4_t*>(&Lm[i][16 * J + 4 * g4]) = lrow;
      {
        unsigned char* afrag = sm + kOffAf + ((I * 2 + J / 2) * 64 + lane) * 16;
        *reinterpret_cast<bf16x4_t*>(afrag + (J & 1) * 8) = qrow;
        if (I == J && (I & 1) == 0) *reinterpret_cast<bf16x4_t*>(afrag + 8) = bf16x4_t{};  // tile J = I+1 is above
      }
    }
  } else {
    // phase A: block pair p of P2 (A and Aqk) goes to wave p, and pairs 8
    // and 9 to waves 0 and 1 (the K~^T and -Kgamma fragments came with P1)
    // ---- A (strict) and Aqk (causal) 16x16 block pair p on MFMA -------------
    auto p2_pair = [&](int p) {
      // block pair p = I (I + 1) / 2 + J, J <= I
      const int I = p >= 6 ? 3 : (p >= 3 ? 2 : (p >= 1 ? 1 : 0));
      const int J = p - I * (I + 1) / 2;
      // the operands of two reduction steps at a time (two LDS round trips per pair)
      const bf16* ke_row = nat_row(sm, kOffKE, 16 * J + n16);
      const bf16* ka_row = nat_row(sm, kOffKA, 16 * I + n16);
      const bf16* qa_row = nat_row(sm, kOffQA, 16 * I + n16);
      const int i = 16 * I + n16;
      const float bi = betas[i];
      f32x4_t akk = {0.f, 0.f, 0.f, 0.f};
      f32x4_t aqk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int half = 0; half < KT / 4; ++half) {
        bf16x8_t ke[2], kb[2], qb[2];
        f32x4_t sc0[2], sc1[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int c0 = 32 * (2 * half + u) + 8 * g4;
          ke[u] = *reinterpret_cast<const bf16x8_t*>(ke_row + c0);
          sc0[u] = *reinterpret_cast<const f32x4_t*>(&Sc[p][c0]);
          sc1[u] = *reinterpret_cast<const f32x4_t*>(&Sc[p][c0 + 4]);
          kb[u] = *reinterpret_cast<const bf16x8_t*>(ka_row + c0);
          qb[u] = *reinterpret_cast<const bf16x8_t*>(qa_row + c0);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          bf16x8_t af;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            af[e] = (bf16)((float)ke[u][e] * sc0[u][e]);
            af[4 + e] = (bf16)((float)ke[u][4 + e] * sc1[u][e]);
          }
          akk = mfma32(af, kb[u], akk);
          aqk = mfma32(af, qb[u], aqk);
        }
      }
      // lane (n16, g4) holds A[16I + n16][16J + 4 g4 + r] (and likewise Aqk)
      bf16x4_t lrow;
      bf16x4_t qrow;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * J + 4 * g4 + r;
        const float vk = (j < i) ? akk[r] * bi : 0.f;
        lrow[r] = (bf16)vk;
        qrow[r] = (bf16)((j <= i) ? aqk[r] : 0.f);
        if (I == J) Ld[I][n16][4 * g4 + r] = vk;
      }
      *reinterpret_cast<bf16x4_t*>(&Lm[i][16 * J + 4 * g4]) = lrow;
      {
        unsigned char* afrag = sm + kOffAf + ((I * 2 + J / 2) * 64 + lane) * 16;
        *reinterpret_cast<bf16x4_t*>(afrag + (J & 1) * 8) = qrow;
        if (I == J && (I & 1) == 0) *reinterpret_cast<bf16x4_t*>(afrag + 8) = bf16x4_t{};  // tile J = I+1 is above
      }
    };
    if (wave < 4) {
      p2_pair(wave);
      if (wave < 2) p2_pair(wave + 8);
    } else {
      if constexpr (LOADER) nl.template load_part<2>();
      p2_pair(wave);
    }
  }
  if constexpr (LOADER) nl.template load_part<3>();
  __syncthreads();

  if constexpr (LOADER) nl.template load_part<4>();
  // ---- exact diagonal blocks for chunks with extreme decay ----------------
  if (flags[0] | flags[1] | flags[2] | flags[3]) {
    float* Lr = lds<float>(sm, kOffQA);  // [64][128] f32 over the dead q a and k E tiles
    const int64_t krow = a.H * a.K;
    if (wave < 4) {
      const int J = wave, cp = lane;
      const DecayConsts dc = decay_consts<IT, DECAY>(a, h, cp);
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        float run = 0.f;
        for (int r = 0; r < 16; ++r) {
          const int tl = 16 * J + r;
          const float gvv =
              (tl < n_valid && 2 * cp + ch < a.K)
                  ? g_value<IT, DECAY>(to_float(a.g[(cg.tok0 + tl) * krow + h * a.K + 2 * cp + ch]), dc, ch, true)
                  : 0.f;
          if (r > 0) run += gvv;
          Lr[tl * kKey + 2 * cp + ch] = run;
        }
      }
    }
    __syncthreads();
    for (int task = tid; task < 4 * 136; task += kThreads) {
      const int I = task / 136;
      const int p = task % 136;
      int il = 0;
      while ((il + 1) * (il + 2) / 2 <= p) ++il;
      const int jl = p - il * (il + 1) / 2;
      const int i = 16 * I + il, j = 16 * I + jl;
      float acc_k = 0.f, acc_q = 0.f;
      if (i < n_valid && j < n_valid) {
        const int64_t oi = (cg.tok0 + i) * krow + h * a.K;
        const int64_t oj = (cg.tok0 + j) * krow + h * a.K;
        for (int cc = 0; cc < a.K; ++cc) {
          const float e = fast_exp(Lr[i * kKey + cc] - Lr[j * kKey + cc]);
          const float kj = to_float(a.k[oj + cc]);
          acc_k += to_float(a.k[oi + cc]) * kj * e;
          acc_q += to_float(a.q[oi + cc]) * kj * e;
        }
      }
      if (jl < il) {
        const float vk = betas[i] * acc_k;
        Lm[i][j] = (bf16)vk;
        Ld[I][il][jl] = vk;
      }
      {
        const int fl = il + 16 * (jl >> 2);
        bf16* afrag = reinterpret_cast<bf16*>(sm + kOffAf + ((I * 2 + I / 2) * 64 + fl) * 16);
        afrag[(I & 1) * 4 + (jl & 3)] = (bf16)acc_q;
      }
    }
    __syncthreads();
  }

  if constexpr (LOADER) nl.template load_part<5>();
  // ---- P3: inverses T_I of the four unit-lower diagonal blocks (f32), waves
  // 0-3; meanwhile (phase C) waves 4-7 export Kgamma = exp(lg) k over the dead
  // q a tile
  if (wave < 4) {
    if (lane < 16) {
      // column `lane` of T_I, row by row.  Row r + 1 of L is read while row r
      // is formed (its entries j < r + 1 only), and each row's sum runs in two
      // independent halves, so neither the LDS latency nor one long chain of
      // dependent FMAs sets the pace.
      const int I = wave;
      float x[16];
      f32x4_t cur[4] = {}, nxt[4] = {};
      x[0] = lane == 0 ? 1.f : 0.f;
      Tinv[I][0][lane] = (bf16)x[0];
      cur[0] = *reinterpret_cast<const f32x4_t*>(&Ld[I][1][0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) {
        if (r + 1 < 16) {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            if (4 * q4 < r + 1) nxt[q4] = *reinterpret_cast<const f32x4_t*>(&Ld[I][r + 1][4 * q4]);
        }
        float acc0 = (r == lane) ? 1.f : 0.f;
        float acc1 = 0.f;
#pragma unroll
        for (int j = 0; j < r; ++j) {
          if (j & 1)
            acc1 -= cur[j >> 2][j & 3] * x[j];
          else
            acc0 -= cur[j >> 2][j & 3] * x[j];
        }
        x[r] = acc0 + acc1;
        Tinv[I][r][lane] = (bf16)x[r];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) cur[q4] = nxt[q4];
        __builtin_amdgcn_sched_barrier(0);
      }
      bf16x8_t t0, t1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        t0[e] = (bf16)x[e];
        t1[e] = (bf16)x[8 + e];
      }
      *reinterpret_cast<bf16x8_t*>(&TinvT[I][lane][0]) = t0;
      *reinterpret_cast<bf16x8_t*>(&TinvT[I][lane][8]) = t1;
    }
  } else {
    // phase C: -Kgamma : fragment (I, s), lane (i, g); tasks tid - 256 + 256 k, reads first
    if constexpr (MODE == kOutput) {
      bf16x4_t lo[4], hi[4];
      f32x4_t glo[4], ghi[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int task = tid - 256 + 256 * k;
        const int frag = task >> 6;
        const int fi = task & 15, fg = (task >> 4) & 3;
        const int I = frag >> 2, c0 = 32 * (frag & 3) + 4 * fg;
        const bf16* row = nat_row(sm, kOffKA, 16 * I + fi);
        lo[k] = *reinterpret_cast<const bf16x4_t*>(row + c0);
        hi[k] = *reinterpret_cast<const bf16x4_t*>(row + c0 + 16);
        glo[k] = *reinterpret_cast<const f32x4_t*>(&Gs[I][c0]);
        ghi[k] = *reinterpret_cast<const f32x4_t*>(&Gs[I][c0 + 16]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        bf16x8_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = (bf16)(-(float)lo[k][e] * glo[k][e]);
          o[4 + e] = (bf16)(-(float)hi[k][e] * ghi[k][e]);
        }
        *lds<bf16x8_t>(sm, kgf_off<MODE>(0, 0) + (tid - 256 + 256 * k) * 16) = o;
      }
    }
    if constexpr (LOADER && MODE == kSummary) p1_write_late<MODE>(sm, *po, *ll, tid, chan);
    if constexpr (LOADER) nl.template load_part<6>();
  }
  __syncthreads();

  // ---- P4: M = (I + B)^{-1} diag(beta), B = diag(beta) A strictly lower.
  // With N = (I + B)^{-1}, block row I of Z = N^T satisfies
  //   Z_II = T_I^T ;  Z_IJ = -T_J^T sum_{K=J+1..I} B_KJ^T Z_IK   (J < I),
  // a chain in which Z_IK is the B operand of the next product.  In the
  // accumulator layout lane (i, g) holds Z_IJ[4 g + r][i] = N[16 I + i][16 J + 4 g + r],
  // which is half of an A fragment of M (rows i, reduction over j); the
  // fragments go over the dead k E tile.  Wave I < 4 owns block row I.
}

// ---- P4: M, block row I by wave I < 4 (the loader waves are free here) ------
struct NoWork {
  __device__ __forceinline__ void operator()() const {}
};
// `loader_work` runs on the loader waves, which M does not need, before the
// barrier.
template <class IT, int MODE, bool LOADER, class F = NoWork>
__device__ __forceinline__ void prepare_m(unsigned char* sm, int tid, const NextLoads<IT, MODE>& nl,
                                          const F& loader_work = F{}) {
  if constexpr (!kPrepares<MODE>) return;  // M comes with the chunk's loads
  const int lane = tid & 63;
  const int wave = wave_of(tid);
  if constexpr (LOADER) {
    nl.template load_part<7>();
    loader_work();
  }
  switch (wave) {
    case 0: m_block_row<0>(sm, lane); break;
    case 1: m_block_row<1>(sm, lane); break;
    case 2: m_block_row<2>(sm, lane); break;
    case 3: m_block_row<3>(sm, lane); break;
    default: break;
  }
  __syncthreads();
}

// ---- per-chunk state advance of one wave's pair of 16-column tiles ----------
// ut[t] >= 0: U tile index of tile t (value columns); -1: a transition column
// (U = 0).  Phase C also forms O = Q~ S + Aqk V~ for both tiles.  KT: the row
// tiles of the state that carry channels (8, or 4 when K <= 64: the rows past
// them stay zero, so the products over them are skipped).
template <int MODE, int KT>
__device__ __forceinline__ void scan_pair(const unsigned char* sm, f32x4_t (&S)[2][8], const int (&ut)[2], int lane,
                                          f32x4_t (&O)[2][4]) {
  const int g4 = lane >> 4;
  const int n16 = lane & 15;
  const bf16(*Vn)[kRow] = reinterpret_cast<const bf16(*)[kRow]>(sm + kOffVn);
  // Y = v - Kgamma S (value columns) or -Kgamma S (transition columns): the
  // products start from zero and v is added after them, so that its LDS reads
  // overlap the MFMA chain instead of delaying its first step
  f32x4_t Y[2][4];
  bf16 vin[2][4][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      Y[t][I] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (ut[t] >= 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) vin[t][I][r] = Vn[16 * I + 4 * g4 + r][16 * ut[t] + n16];
      }
      if constexpr (kWritesOut<MODE>) O[t][I] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  }
  // one reduction step at a time: the B operands of the step come from row
  // tiles 2 st and 2 st + 1 of the state, and the -Kgamma and Q~ fragments of
  // the step serve both tiles (Q~ S is the first part of the output); the
  // fragments of step st + 1 are read while the products of step st run
  auto load_step = [&](int st, bf16x8_t (&kf)[4], bf16x8_t (&qf)[4]) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      kf[I] = *reinterpret_cast<const bf16x8_t*>(sm + kgf_off<MODE>(I, st) + qk_slot<MODE>(I, lane) * 16);
      if constexpr (kWritesOut<MODE>)
        qf[I] = *reinterpret_cast<const bf16x8_t*>(sm + kOffQf + ((I * 4 + st) * 64 + qk_slot<MODE>(I, lane)) * 16);
    }
  };
  bf16x8_t kfa[4], qfa[4], kfb[4], qfb[4];
  load_step(0, kfa, qfa);
#pragma unroll
  for (int st = 0; st < KT / 2; ++st) {
    bf16x8_t(&kf)[4] = (st & 1) ? kfb : kfa;
    bf16x8_t(&qf)[4] = (st & 1) ? qfb : qfa;
    if (st + 1 < KT / 2) {
      if (st & 1)
        load_step(st + 1, kfa, qfa);
      else
        load_step(st + 1, kfb, qfb);
    }
    bf16x8_t sb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sb[t][r] = (bf16)S[t][2 * st][r];
        sb[t][4 + r] = (bf16)S[t][2 * st + 1][r];
      }
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int t = 0; t < 2; ++t) Y[t][I] = mfma32(kf[I], sb[t], Y[t][I]);
      if constexpr (kWritesOut<MODE>) {
#pragma unroll
        for (int t = 0; t < 2; ++t) O[t][I] = mfma32(qf[I], sb[t], O[t][I]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (ut[t] >= 0) {
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int r = 0; r < 4; ++r) Y[t][I][r] += (float)vin[t][I][r];
    }
  }
  // lower-triangular 64 x 64 fragments (I, s') with s' <= I / 2 sit in slots 0, 2, 4, 5, 6, 7
  auto lower_product = [&](int off, const bf16x8_t (&xb)[2][2], f32x4_t (&acc)[2][4]) {
    bf16x8_t af[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const int slot = j < 2 ? 2 * j : j + 2;
      af[j] = *reinterpret_cast<const bf16x8_t*>(sm + off + (slot * 64 + lane) * 16);
    }
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const int I = j < 2 ? j : (j < 4 ? 2 : 3);
      const int sp = (j == 3 || j == 5) ? 1 : 0;
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[t][I] = mfma32(af[j], xb[t][sp], acc[t][I]);
    }
  };
  auto pack = [&](const f32x4_t (&x)[2][4], bf16x8_t (&xb)[2][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          xb[t][st][r] = (bf16)x[t][2 * st][r];
          xb[t][st][4 + r] = (bf16)x[t][2 * st + 1][r];
        }
      }
    }
  };
  // V~ = M Y
  bf16x8_t Yb[2][2];
  pack(Y, Yb);
  f32x4_t Vt[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int I = 0; I < 4; ++I) Vt[t][I] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  lower_product(mf_off<MODE>(), Yb, Vt);
  bf16x8_t Vb[2][2];
  pack(Vt, Vb);
  // the output product takes V~ as hi + lo (x = bf16(x) + bf16(x - bf16(x)),
  // about 16 bits): V~'s rounding is the largest operand error of the output
  // (measured at B=1, T=8192, H=16, K=V=128: 5.7e-3 -> 4.5e-3 against the
  // f32 oracle, for 12 more MFMAs per tile pair; at K <= 64 it left the
  // error unchanged, so those shapes skip it).  The state update keeps the
  // bf16 V~: splitting it too cut the state's error from 1.9e-3 to 4e-4 but
  // cost 2.5% of the prefill.
  constexpr bool kSplitV = kWritesOut<MODE> && KT == 8;
  bf16x8_t Vl[2][2];
  if constexpr (kSplitV) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          Vl[t][st][r] = (bf16)(Vt[t][2 * st][r] - (float)Vb[t][st][r]);
          Vl[t][st][4 + r] = (bf16)(Vt[t][2 * st + 1][r] - (float)Vb[t][st][4 + r]);
        }
  }
  // O += Aqk V~
  if constexpr (kWritesOut<MODE>) {
    lower_product(kOffAf, Vb, O);
    if constexpr (kSplitV) lower_product(kOffAf, Vl, O);
  }
  // S <- diag(gamma) S + K~^T V~
  const float* gam = reinterpret_cast<const float*>(sm + kOffGam);
#pragma unroll
  for (int h4 = 0; h4 < KT / 4; ++h4) {
    bf16x8_t kt[4][2];
    f32x4_t gm[4];
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int ct = 4 * h4 + c4;
      gm[c4] = *reinterpret_cast<const f32x4_t*>(gam + 16 * ct + 4 * g4);
#pragma unroll
      for (int sp = 0; sp < 2; ++sp)
        kt[c4][sp] = *reinterpret_cast<const bf16x8_t*>(sm + kOffKTf + ((ct * 2 + sp) * 64 + kt_slot<MODE>(ct, lane)) * 16);
    }
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int ct = 4 * h4 + c4;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        S[t][ct] *= gm[c4];
        S[t][ct] = mfma32(kt[c4][0], Vb[t][0], S[t][ct]);
        S[t][ct] = mfma32(kt[c4][1], Vb[t][1], S[t][ct]);
      }
    }
  }
}

// Store a chunk's 64 x (16 ntile) output slice of one wave.  The accumulator
// layout (lane (n, g) holds rows 16 I + 4 g + r of column n) is transposed
// through a per-wave 4 KB LDS stage so that each lane writes 16 contiguous
// bytes of a row.
template <class IT>
__device__ __forceinline__ void store_out(const f32x4_t (&O)[2][4], int ntile, IT* out, const ChunkGeo& cg,
                                          int64_t H, int64_t h, int64_t V, int64_t col, int lane, IT* stage) {
  const int g4 = lane >> 4, n16 = lane & 15;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
#pragma unroll
      for (int r = 0; r < 4; ++r) stage[(16 * I + 4 * g4 + r) * 32 + 16 * t + n16] = from_compute<IT>(O[t][I][r]);
    }
  }
  // lanes now read what other lanes of the wave wrote: complete the writes and
  // keep the compiler from moving the reads above them
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int unit = lane + 64 * u;
    const int row = unit >> 2;
    const int c8 = unit & 3;
    const uint4 val = *reinterpret_cast<const uint4*>(stage + row * 32 + 8 * c8);
    if (row < cg.n_span && c8 < 2 * ntile)
      *reinterpret_cast<uint4*>(out + ((cg.tok0 + row) * H + h) * V + col + 8 * c8) = val;
  }
}

// ---- phases A and C -----------------------------------------------------------
// Waves 0-3 (scanners) hold the state tiles: in phase C wave w owns tiles
// 2w, 2w+1 of the column group; in phase A with the transition tracked it
// also owns tiles 2w+8, 2w+9 (the 16 tiles are [value tiles | transition
// tiles]).  Waves 4-7 (loaders) hold the raw inputs of the next chunk.  The
// two roles run separate loops with the same barriers, so neither role's
// registers are live in the other's code.
// DECAY: g formed from decay logits; PAD: K < 128, channels K..127 are zero
// padding (K == 128 compiles without any of the padding checks)
template <class IT, int MODE, bool DECAY, bool PAD, int KT>
__global__ __launch_bounds__(kThreads) void chunk_segment_kernel(const SegArgs<IT> a) {
  extern __shared__ __align__(16) unsigned char sm[];
  // one-dimensional grid, segment slowest: the workgroups past the real
  // segment count (the grid is an upper bound) are all at the end, so the
  // active ones spread evenly over the XCDs
  const int64_t ncg = (a.V + kColGroup - 1) / kColGroup;
  const int64_t gsg = blockIdx.x / (a.H * ncg);
  const int64_t h = (blockIdx.x / ncg) % a.H;
  const int64_t cgi = blockIdx.x % ncg;
  if (gsg >= seg_start_of(a, a.N)) return;  // uniform
  const int64_t s = seq_of_segment(a, gsg);
  const int64_t lg = gsg - seg_start_of(a, s);
  const int64_t nseg = seg_start_of(a, s + 1) - seg_start_of(a, s);
  // the last segment needs no summary; phase A still prepares its chunks' M and Aqk
  const bool scan_state = !(MODE == kSummary && lg == nseg - 1);
  const SeqRange sr = seq_range(a.seq, s);
  const int64_t cs = chunk_start_of(a, s);
  const int64_t c_begin = cs + lg * a.L;
  const int64_t c_end_seq = chunk_start_of(a, s + 1);
  const int64_t c_end = (c_begin + a.L < c_end_seq) ? c_begin + a.L : c_end_seq;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = wave_of(tid);
  // scanner slot: with K <= 64 the output phases put their value tiles on
  // scanners 2 and 3, which share SIMDs with loader waves 6 and 7 (their
  // channels all padding, kChanWave), so that no SIMD runs a busy scanner
  // and a busy loader
  const int sw = (KT == 4 && kWritesOut<MODE>) ? (w ^ 2) : w;
  const int n16 = lane & 15;
  const int g4 = lane >> 4;
  const int64_t col0 = cgi * kColGroup;
  const int vcg = static_cast<int>(a.V - col0 < kColGroup ? a.V - col0 : kColGroup);
  const int nvt = vcg / 16;
  const bool track_p = MODE == kSummary && lg > 0 && cgi == 0;
  const int ntiles = nvt + (track_p ? KT : 0);  // value tiles, then one transition tile per channel row tile
  const int64_t sbase = (s * a.H + h) * a.K * a.V;
  constexpr int kPairs = MODE == kSummary ? 2 : 1;  // tile pairs per scanner wave

  f32x4_t S[kPairs][2][8];
  if (w < 4) {
    // ---------------- scanners ----------------
#pragma unroll
    for (int pp = 0; pp < kPairs; ++pp) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int tile = 2 * sw + 8 * pp + t;
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
          if (tile < nvt) {
            if (lg == 0) {
              // K is a multiple of 16: a row tile is all real or all padding
              const bool real = a.s_in != nullptr && (!PAD || 16 * ct < a.K);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int64_t row = 16 * ct + 4 * g4 + r;
                S[pp][t][ct][r] = real ? a.s_in[sbase + row * a.V + col0 + 16 * tile + n16] : 0.f;
              }
            } else if (kWritesOut<MODE>) {
              const float* p = a.seg_state + (gsg * a.H + h) * seg_state_floats(a.V) +
                               ((col0 / 16 + tile) * 8 + ct) * 256 + lane * 4;
              S[pp][t][ct] = *reinterpret_cast<const f32x4_t*>(p);
            } else {
              S[pp][t][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
          } else if (tile < ntiles) {  // transition columns start at the identity
#pragma unroll
            for (int r = 0; r < 4; ++r)
              S[pp][t][ct][r] = (16 * ct + 4 * g4 + r == 16 * (tile - nvt) + n16) ? 1.f : 0.f;
          } else {
            S[pp][t][ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
    if constexpr (MODE == kOutputMA) {
      // two barriers per chunk: the loaders' operand writes end at the first,
      // the scanners' reads of them at the second; the outputs of a chunk are
      // stored (through a stage that the operand writes do not touch) while
      // the loaders write the next chunk's operands
      for (int64_t c = c_begin; c < c_end; ++c) {
        const ChunkGeo geo = chunk_geo(sr, c - cs);
        const int tid_c = opaque(tid);
        __syncthreads();
        const int tile0 = 2 * sw;
        f32x4_t O[2][4];
        const int ut[2] = {tile0 < nvt ? tile0 : -1, tile0 + 1 < nvt ? tile0 + 1 : -1};
        if (tile0 < ntiles) scan_pair<MODE, KT>(sm, S[0], ut, tid_c & 63, O);
        __syncthreads();
        if (tile0 < ntiles) {
          const int nt = ntiles - tile0 < 2 ? ntiles - tile0 : 2;
          store_out<IT>(O, nt, a.out, geo, a.H, h, a.V, col0 + 16 * tile0, tid_c & 63,
                        lds<IT>(sm, kOffStage + w * 4096));
        }
      }
    } else {
    P1Out none;
    const NextLoads<IT, MODE> nl{};
    for (int64_t c = c_begin; c < c_end; ++c) {
      const ChunkGeo geo = chunk_geo(sr, c - cs);
      // an opaque copy of the thread index keeps the compiler from hoisting
      // the many lane-dependent LDS addresses of a chunk out of the loop,
      // where they would stay live (and spill) next to the state tiles
      const int tid_c = opaque(tid);
      p1_write<MODE, false>(sm, none, nullptr, tid_c);
      prepare_mid<IT, MODE, false, DECAY, KT>(sm, a, geo, h, vcg, tid_c, nl);
      prepare_m<IT, MODE, false>(sm, tid_c, nl);
#pragma unroll
      for (int pp = 0; pp < kPairs; ++pp) {
        const int tile0 = 2 * sw + 8 * pp;
        if (tile0 < ntiles && scan_state) {
          const int ut[2] = {tile0 < nvt ? tile0 : -1, tile0 + 1 < nvt ? tile0 + 1 : -1};
          f32x4_t O[2][4];
          scan_pair<MODE, KT>(sm, S[pp], ut, tid_c & 63, O);
          if constexpr (kWritesOut<MODE>) {
            const int nt = ntiles - tile0 < 2 ? ntiles - tile0 : 2;
            store_out<IT>(O, nt, a.out, geo, a.H, h, a.V, col0 + 16 * tile0, tid_c & 63,
                          lds<IT>(sm, kOffStage + w * 4096));
          }
        }
      }
      __syncthreads();
    }
    }
  } else if constexpr (MODE == kOutputMA) {
    // ---------------- loaders, phase C without P2 ----------------
    Raw<IT> raw;
    P1Out po;
    const LoaderLanes ll = loader_lanes<IT, PAD>(a, vcg, tid);
    const DecayConsts dc = decay_consts<IT, DECAY>(a, h, loader_pair(tid));
    const bool chan = kChanWave<PAD, KT>(w);
    if (c_begin < c_end) {
      const ChunkGeo g0 = chunk_geo(sr, c_begin - cs);
      load_raw<IT, MODE>(raw, chunk_loads<IT>(a, g0, c_begin, h, col0), ll, tid);
      p1_math_ma<IT, DECAY>(po, raw, tid, g0.n_valid, dc, chan);
    }
    for (int64_t c = c_begin; c < c_end; ++c) {
      const int tid_c = opaque(tid);
      const NextLoads<IT, MODE> nl{&raw, chunk_loads<IT>(a, chunk_geo(sr, c + 1 - cs), c + 1, h, col0, c + 1 < c_end),
                                   &ll, tid_c};
      p1_write_ma<IT, MODE>(sm, po, ll, tid_c, nl, chan);
      __syncthreads();
      nl.template load_part<6>();
      nl.template load_part<7>();
      if (c + 1 < c_end) p1_math_ma<IT, DECAY>(po, raw, tid_c, chunk_geo(sr, c + 1 - cs).n_valid, dc, chan);
      __syncthreads();
    }
  } else {
    // ---------------- loaders ----------------
    // The raw inputs of chunk c + 1 are loaded in eight parts spread over
    // the phases of chunk c (one burst of every CU's 64 KB would saturate the
    // memory system and stall the issuing waves); while the scanners advance
    // the state through chunk c the loaders turn them into P1 registers.  All
    // eight parts are loaded and consumed within one iteration: raw inputs
    // carried across the loop edge end up copied between registers, which
    // waits for the loads.
    Raw<IT> raw;
    P1Out po;
    const LoaderLanes ll = loader_lanes<IT, PAD>(a, vcg, tid);
    const DecayConsts dc = decay_consts<IT, DECAY>(a, h, loader_pair(tid));
    const bool chan = kChanWave<PAD, KT>(w);
    if (c_begin < c_end) {
      const ChunkGeo g0 = chunk_geo(sr, c_begin - cs);
      load_raw<IT, MODE>(raw, chunk_loads<IT>(a, g0, c_begin, h, col0), ll, tid);
      p1_math<IT, MODE, DECAY>(po, raw, g0, vcg, tid, dc, chan);
      if constexpr (kEarlyP1<MODE>) p1_write_early<MODE>(sm, po, tid, chan);
    }
    for (int64_t c = c_begin; c < c_end; ++c) {
      const ChunkGeo geo = chunk_geo(sr, c - cs);
      const int tid_c = opaque(tid);
      p1_write<MODE, true>(sm, po, &ll, tid_c, chan);
      const NextLoads<IT, MODE> nl{&raw, chunk_loads<IT>(a, chunk_geo(sr, c + 1 - cs), c + 1, h, col0, c + 1 < c_end),
                                   &ll, tid_c};
      prepare_mid<IT, MODE, true, DECAY, KT>(sm, a, geo, h, vcg, tid_c, nl, &po, &ll, chan);
      // hand the chunk's M and Aqk fragments to phase C (one column group
      // writes them, 16-byte units [M | Aqk][j][lane]): Aqk, final since P2,
      // while waves 0-3 form M; M after it, while the scanners only read it
      const bool hand_off = MODE == kSummary && a.chunk_ma != nullptr && cgi == 0;
      unsigned char* ma_dst = hand_off ? reinterpret_cast<unsigned char*>(a.chunk_ma) + (c * a.H + h) * kMaBytes
                                       : nullptr;
      auto hand_units = [&](bool aqk) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const int u = (tid_c - 256) + 256 * k;
          if ((u >= 384) == aqk) {
            const int slot = lower_slot((u >> 6) % 6);
            *reinterpret_cast<uint4*>(ma_dst + u * 16) =
                *reinterpret_cast<const uint4*>(sm + (aqk ? kOffAf : mf_off<MODE>()) + (slot * 64 + (u & 63)) * 16);
          }
        }
      };
      prepare_m<IT, MODE, true>(sm, tid_c, nl, [&] {
        if (hand_off) hand_units(true);
      });
      if (hand_off) hand_units(false);
      if (c + 1 < c_end) {
        p1_math<IT, MODE, DECAY>(po, raw, chunk_geo(sr, c + 1 - cs), vcg, tid_c, dc, chan);
        // the k a and q a tiles, pair scales, flags and beta of chunk c + 1:
        // P2 and M of chunk c are done, and the state advance reads none of them
        if constexpr (kEarlyP1<MODE>) p1_write_early<MODE>(sm, po, tid_c, chan);
      }
      __syncthreads();
    }
  }

  // ---- end of the segment ----------------------------------------------------
  if constexpr (kWritesOut<MODE>) {
    if (w < 4 && lg == nseg - 1 && a.s_out != nullptr) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int tile = 2 * sw + t;
        if (tile >= nvt) continue;
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
          if (PAD && 16 * ct >= a.K) break;  // padding rows (K is a multiple of 16)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t row = 16 * ct + 4 * g4 + r;
            a.s_out[sbase + row * a.V + col0 + 16 * tile + n16] = S[0][t][ct][r];
          }
        }
      }
    }
  } else {
    if (!scan_state) return;  // uniform: the last segment has no summary
    // value tiles: the start state of the next segment (first segment) or Q_g
    float* dst = (lg == 0) ? a.seg_state + ((gsg + 1) * a.H + h) * seg_state_floats(a.V)
                           : a.seg_q + (gsg * a.H + h) * seg_state_floats(a.V);
    bf16(*Pn)[kRow] = lds<bf16[kRow]>(sm, kOffPnat);
    if (w < 4) {
#pragma unroll
      for (int pp = 0; pp < kPairs; ++pp) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int tile = 2 * sw + 8 * pp + t;
          if (tile < nvt) {
#pragma unroll
            for (int ct = 0; ct < 8; ++ct)
              *reinterpret_cast<f32x4_t*>(dst + ((col0 / 16 + tile) * 8 + ct) * 256 + lane * 4) = S[pp][t][ct];
          } else if (tile < ntiles) {
            // transition tile -> natural bf16 [i][j] in LDS
            const int j = 16 * (tile - nvt) + n16;
#pragma unroll
            for (int ct = 0; ct < 8; ++ct)
#pragma unroll
              for (int r = 0; r < 4; ++r) Pn[16 * ct + 4 * g4 + r][j] = (bf16)S[pp][t][ct][r];
          }
        }
      }
    }
    if (track_p) {
      // natural P_g in LDS -> A fragments in the workspace
      __syncthreads();
      bf16* pdst = a.seg_p + (gsg * a.H + h) * seg_p_elems();
      for (int f = tid; f < 8 * 4 * 64; f += kThreads) {
        const int I = f >> 8, st = (f >> 6) & 3, fl = f & 63;
        const int i = 16 * I + (fl & 15), gq = fl >> 4;
        // columns past the KT row tiles have no transition tile (their channels
        // are padding, and the state rows they would multiply are zero): zeros
        bf16x4_t lo = bf16x4_t{}, hi = bf16x4_t{};
        if (st < KT / 2) {
          lo = *reinterpret_cast<const bf16x4_t*>(&Pn[i][32 * st + 4 * gq]);
          hi = *reinterpret_cast<const bf16x4_t*>(&Pn[i][32 * st + 16 + 4 * gq]);
        }
        *reinterpret_cast<bf16x8_t*>(pdst + static_cast<int64_t>(f) * 8) =
            bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  }
}

// ---- phase B: S_{g+1} = P_g S_g + Q_g along each sequence ---------------------
// One workgroup of 8 waves per (sequence, head, 16-column tile); wave ct owns
// output row tile ct.  The state moves between waves as bf16 B-operand
// halves through LDS (double-buffered, one barrier per segment); P_g and
// Q_g of the next kCombineDepth segments are in flight in registers.  The
// step loop is unrolled by kCombineDepth with every load unconditional (the
// segment index clamped) and the last group padded with steps whose results
// are dropped, so each register set is reloaded at one fixed place and the
// waits for a step's operands cover only that step's loads (an early exit
// from the unrolled group would join the loop's back edge, where the compiler
// then waits for every load in flight).  The start state is loaded before the
// prefetches, so the first step waits for its own operands only.  Each step
// moves 40 KB through the CU's vector memory path (the 32 KB of P_g this
// column tile needs whole, Q_g's slice and the stored state), which sets its
// pace more than load latency does: two steps ahead measured fastest (13.1 us
// for 14 steps at T=8192, H=16 against 14.8 us four ahead, whose prologue
// burst and padded steps cost more than the shorter lead).
constexpr int kCombineDepth = 2;

struct CombineArgs {
  const int32_t* seg_start;  // [N+1], or nullptr for dense sequences
  int64_t dense_segs;
  float* seg_state;
  const float* seg_q;
  const bf16* seg_p;
  int64_t N, H, V;
};

__global__ __launch_bounds__(512) void segment_combine_kernel(const CombineArgs a) {
  __shared__ __align__(16) bf16x4_t Sh[2][8][64];
  const int64_t s = blockIdx.x;
  const int64_t h = blockIdx.y;
  const int64_t tile = blockIdx.z;
  const int64_t g0 = seg_start_of(a, s);
  const int64_t nseg = seg_start_of(a, s + 1) - g0;
  if (nseg <= 2) return;  // phase A already produced every start state
  const int last = static_cast<int>(nseg - 2);  // steps lg = 1..last produce the start state of segment lg + 1
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int ct = wave_of(tid);
  // this lane's element of segment g0 + g: base + g * stride
  const int64_t st_stride = a.H * seg_state_floats(a.V);
  const int64_t p_stride = a.H * seg_p_elems();
  const float* q_base = a.seg_q + (g0 * a.H + h) * seg_state_floats(a.V) + (tile * 8 + ct) * 256 + lane * 4;
  float* s_base = a.seg_state + (g0 * a.H + h) * seg_state_floats(a.V) + (tile * 8 + ct) * 256 + lane * 4;
  const bf16* p_base = a.seg_p + (g0 * a.H + h) * seg_p_elems() + (ct * 4 * 64 + lane) * 8;

  bf16x8_t Pf[kCombineDepth][4];
  f32x4_t Qv[kCombineDepth];
  auto load_step = [&](int d, int lg) {
    const int g = lg < last ? lg : last;
#pragma unroll
    for (int st = 0; st < 4; ++st) Pf[d][st] = *reinterpret_cast<const bf16x8_t*>(p_base + g * p_stride + st * 64 * 8);
    Qv[d] = *reinterpret_cast<const f32x4_t*>(q_base + g * st_stride);
  };
  const f32x4_t x = *reinterpret_cast<const f32x4_t*>(s_base + st_stride);
#pragma unroll
  for (int d = 0; d < kCombineDepth; ++d) load_step(d, 1 + d);
  Sh[0][ct][lane] = bf16x4_t{(bf16)x[0], (bf16)x[1], (bf16)x[2], (bf16)x[3]};
  __syncthreads();
  for (int lg0 = 1; lg0 <= last; lg0 += kCombineDepth) {
#pragma unroll
    for (int d = 0; d < kCombineDepth; ++d) {
      const int lg = lg0 + d;
      const int buf = (lg - 1) & 1;
      f32x4_t acc = Qv[d];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x4_t lo = Sh[buf][2 * st][lane];
        const bf16x4_t hi = Sh[buf][2 * st + 1][lane];
        const bf16x8_t sb = bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc = mfma32(Pf[d][st], sb, acc);
      }
      load_step(d, lg + kCombineDepth);
      if (lg <= last) *reinterpret_cast<f32x4_t*>(s_base + (lg + 1) * st_stride) = acc;
      Sh[buf ^ 1][ct][lane] = bf16x4_t{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
      __syncthreads();
    }
  }
}

// ---- host side ------------------------------------------------------------
static bool mfma_path(int in_dtype, int state_dtype, int64_t K, int64_t V) {
  return (in_dtype == KDA_DTYPE_BF16 || in_dtype == KDA_DTYPE_F16) && state_dtype == KDA_DTYPE_F32 && K <= kKey &&
         K % 16 == 0 &&
         V % 16 == 0 && V >= 16 && V <= 256;
}

static int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

// How a prefill is cut into segments: L chunks per segment, or one segment
// per sequence when (sequences x heads x column groups) alone fill the GPU.
struct Plan {
  int32_t L;
  bool segmented;
  int64_t ncg;
  int64_t segs_bound;    // upper bound on the total number of segments
  int64_t chunks_bound;  // upper bound on the total number of chunks
};

// The schedule override of kda_set_segment_chunks: L >= 1 forces L chunks
// per segment, 0 one segment per sequence, -1 (the default) the plan below.
// The result does not depend on it (tests use it to cover both schedules at
// small sizes); the environment plays no part in the schedule.
static std::atomic<int64_t> g_segment_override{-1};
static int64_t segment_override() { return g_segment_override.load(std::memory_order_relaxed); }

// `longest` (packed documents only, 0 when unknown): the longest document in
// tokens.  Documents of uneven length that alone fill the GPU would leave it
// idle while the longest runs on (one workgroup per document and head): when
// the longest document is well past the chunk-steps per CU of a balanced
// pass, every document is cut into segments of that many chunks (short ones
// stay one segment), which spreads the long chains over the CUs the short
// documents free.
static Plan make_plan(int64_t N, int64_t total_tokens, int64_t H, int64_t V, int64_t longest) {
  Plan p;
  p.ncg = (V + kColGroup - 1) / kColGroup;
  const int64_t cus = device_cus();
  const int64_t chunks_bound = total_tokens / kChunk + N;
  p.chunks_bound = chunks_bound;
  const int64_t work = (total_tokens / kChunk) * H * p.ncg;  // chunk-workgroups of one pass
  const int64_t forced = segment_override();
  if (forced > 0) {
    p.L = static_cast<int32_t>(forced < kOneSegment ? forced : kOneSegment - 1);
    p.segmented = true;
    p.segs_bound = chunks_bound / p.L + N + 1;
    return p;
  }
  const int64_t per_cu = (work + cus - 1) / cus;  // chunk-steps per CU of a balanced pass
  const int64_t longest_chunks = (longest + kChunk - 1) / kChunk;
  const bool uneven = forced != 0 && N > 1 && per_cu >= 2 && 4 * longest_chunks > 5 * per_cu;
  if (uneven && work >= 2 * cus) {
    p.L = static_cast<int32_t>(per_cu < kOneSegment ? per_cu : kOneSegment - 1);
    p.segmented = true;
    p.segs_bound = chunks_bound / p.L + N + 1;
  } else if (forced == 0 || N * H * p.ncg * 4 >= cus * 3 || work < 2 * cus) {
    p.L = kOneSegment;
    p.segmented = false;
    p.segs_bound = N;
  } else {
    int64_t L = (work + cus - 1) / cus;
    if (L < 2) L = 2;
    p.L = static_cast<int32_t>(L);
    p.segmented = true;
    p.segs_bound = chunks_bound / L + N + 1;
  }
  return p;
}

// The scheduling hint of a call: packed documents carry the longest
// document's length in `dense_span` (0 when the caller does not know it).
inline int64_t plan_longest(const SeqDesc& seq) { return seq.cu_seqlens != nullptr ? seq.dense_span : 0; }

static size_t map_bytes(int64_t N) { return static_cast<size_t>(((2 * (N + 1)) * 4 + 255) / 256 * 256); }

static size_t segment_bytes(const Plan& p, int64_t H, int64_t V) {
  if (!p.segmented) return 0;
  const size_t st = static_cast<size_t>(p.segs_bound * H * seg_state_floats(V)) * 4;
  const size_t pp = static_cast<size_t>(p.segs_bound * H * seg_p_elems()) * 2;
  const size_t ma = static_cast<size_t>(p.chunks_bound * H * kMaBytes);
  return 2 * st + pp + ma;
}

static void mark(kda_host::KernelEvents* ev, int i, hipStream_t stream) {
  if (ev != nullptr) {
    (void)hipEventRecord(ev->ev[i], stream);
    ev->n_launched = i;
  }
}

template <class IT, int MODE, bool DECAY, bool PAD, int KT>
static int launch_segments(const SegArgs<IT>& sa, const Plan& p, int64_t H, hipStream_t stream) {
  if (!kda_host::reserve_lds(reinterpret_cast<const void*>(&chunk_segment_kernel<IT, MODE, DECAY, PAD, KT>),
                             kSmemBytes)) {
    kda_host::set_detail("cannot reserve %d bytes of LDS for chunk_segment_kernel", kSmemBytes);
    return KDA_ERR_LAUNCH;
  }
  hipLaunchKernelGGL((chunk_segment_kernel<IT, MODE, DECAY, PAD, KT>), dim3(static_cast<unsigned>(p.segs_bound * H * p.ncg)),
                     dim3(kThreads), kSmemBytes, stream, sa);
  return kda_host::check_launch(MODE == kSummary ? "chunk_segment_kernel<summary>" : "chunk_segment_kernel<output>");
}

// Decay formed in the kernel from logits (kda_chunk_fwd_decay); null for a g input.
struct DecayInput {
  const void* zbias;
  const float* a_log;
  float g_min;
};

template <class IT, bool DECAY, bool PAD, int KT>
static int run_chunk_k(const void* q, const void* k, const void* v, const void* g, const void* beta, const void* s_in,
                     void* s_out, void* out, const SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H,
                     int64_t K, int64_t V, void* workspace, hipStream_t stream, kda_host::KernelEvents* ev,
                     const DecayInput* decay) {
  const Plan p = make_plan(N, total_tokens, H, V, plan_longest(seq));
  int32_t* chunk_start = static_cast<int32_t*>(workspace);
  int32_t* seg_start = chunk_start + (N + 1);
  unsigned char* segbuf = static_cast<unsigned char*>(workspace) + map_bytes(N);
  const size_t st_bytes = p.segmented ? static_cast<size_t>(p.segs_bound * H * seg_state_floats(V)) * 4 : 0;

  SegArgs<IT> sa;
  sa.q = static_cast<const IT*>(q);
  sa.k = static_cast<const IT*>(k);
  sa.v = static_cast<const IT*>(v);
  sa.g = static_cast<const IT*>(g);
  sa.beta = static_cast<const IT*>(beta);
  sa.out = static_cast<IT*>(out);
  sa.s_in = static_cast<const float*>(s_in);
  sa.s_out = static_cast<float*>(s_out);
  sa.seq = seq;
  const bool dense = seq.cu_seqlens == nullptr;
  sa.chunk_start = dense ? nullptr : chunk_start;
  sa.seg_start = dense ? nullptr : seg_start;
  sa.dense_chunks = dense ? (seq.dense_span + kChunk - 1) / kChunk : 0;
  {
    const int64_t nseg = dense ? (sa.dense_chunks + p.L - 1) / p.L : 0;
    sa.dense_segs = nseg > 1 ? nseg : 1;
  }
  sa.seg_state = p.segmented ? reinterpret_cast<float*>(segbuf) : nullptr;
  sa.seg_q = p.segmented ? reinterpret_cast<float*>(segbuf + st_bytes) : nullptr;
  sa.seg_p = p.segmented ? reinterpret_cast<bf16*>(segbuf + 2 * st_bytes) : nullptr;
  sa.chunk_ma = p.segmented ? reinterpret_cast<bf16*>(segbuf + 2 * st_bytes +
                                                      static_cast<size_t>(p.segs_bound * H * seg_p_elems()) * 2)
                            : nullptr;
  sa.N = N;
  sa.H = H;
  sa.K = K;
  sa.V = V;
  sa.L = p.L;
  sa.zbias = nullptr;
  sa.a_log = nullptr;
  sa.g_min = 0.f;
  sa.g_lo = sa.g_hi = 0.f;
  if (DECAY) {
    // eps of the input type, as torch.finfo gives it (src/kda/decay.py:40)
    const float eps = __is_same(IT, bf16) ? 0.0078125f : 0.0009765625f;
    sa.zbias = static_cast<const IT*>(decay->zbias);
    sa.a_log = decay->a_log;
    sa.g_min = decay->g_min;
    sa.g_lo = eps;
    sa.g_hi = 1.f - eps;
  }

  mark(ev, 0, stream);
  int st = KDA_OK;
  if (ev != nullptr && dense) ev->empty |= 1u;  // dense batches need no chunk map
  if (!dense) {
    hipLaunchKernelGGL(chunk_map_kernel, dim3(1), dim3(1024), 0, stream, seq, N, p.L, chunk_start, seg_start);
    st = kda_host::check_launch("chunk_map_kernel");
    if (st != KDA_OK) return st;
  }
  mark(ev, 1, stream);
  if (p.segmented) {
    st = launch_segments<IT, kSummary, DECAY, PAD, KT>(sa, p, H, stream);
    if (st != KDA_OK) return st;
    mark(ev, 2, stream);
    CombineArgs ca{sa.seg_start, sa.dense_segs, sa.seg_state, sa.seg_q, sa.seg_p, N, H, V};
    hipLaunchKernelGGL(segment_combine_kernel, dim3(static_cast<unsigned>(N), static_cast<unsigned>(H),
                                                    static_cast<unsigned>(V / 16)),
                       dim3(512), 0, stream, ca);
    st = kda_host::check_launch("segment_combine_kernel");
    if (st != KDA_OK) return st;
    mark(ev, 3, stream);
  } else {
    mark(ev, 2, stream);
    mark(ev, 3, stream);
    if (ev != nullptr) ev->empty |= 6u;  // one segment per sequence: no summaries, no combine
  }
  st = p.segmented ? launch_segments<IT, kOutputMA, DECAY, PAD, KT>(sa, p, H, stream)
                   : launch_segments<IT, kOutput, DECAY, PAD, KT>(sa, p, H, stream);
  mark(ev, 4, stream);
  return st;
}

template <class IT, bool DECAY>
static int run_chunk(const void* q, const void* k, const void* v, const void* g, const void* beta, const void* s_in,
                     void* s_out, void* out, const SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H,
                     int64_t K, int64_t V, void* workspace, hipStream_t stream, kda_host::KernelEvents* ev,
                     const DecayInput* decay) {
  // K == 128 runs without padding checks; K <= 64 (the reference's shipped
  // model profiles use 64) carries its channels in four row tiles of the state
  if (K == kKey)
    return run_chunk_k<IT, DECAY, false, 8>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V,
                                            workspace, stream, ev, decay);
  if (K <= kKey / 2)
    return run_chunk_k<IT, DECAY, true, 4>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V,
                                           workspace, stream, ev, decay);
  return run_chunk_k<IT, DECAY, true, 8>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V,
                                         workspace, stream, ev, decay);
}

}  // namespace kda

namespace kda_host {

void chunk_plan(int64_t num_seqs, int64_t total_tokens, int64_t longest, int64_t heads, int64_t key_dim,
                int64_t value_dim, int in_dtype, int64_t* chunks_per_segment, int64_t* segments) {
  if (!kda::mfma_path(in_dtype, in_dtype == KDA_DTYPE_F64 ? KDA_DTYPE_F64 : KDA_DTYPE_F32, key_dim, value_dim)) {
    // the split-bf16 chunk path where it applies (-2): dense sequences, and
    // packed documents whose longest length the caller passes; everything
    // else (f64 inputs, K past 128) the exact recurrence kernel (-1)
    *chunks_per_segment = chunk_split_general(in_dtype, KDA_DTYPE_F32, key_dim, value_dim) ? -2 : -1;
    *segments = num_seqs;
    return;
  }
  const kda::Plan p = kda::make_plan(num_seqs, total_tokens, heads, value_dim, longest);
  *chunks_per_segment = p.segmented ? p.L : 0;
  *segments = p.segs_bound;
}

size_t chunk_workspace_bytes(int64_t num_seqs, int64_t total_tokens, int64_t longest, int64_t heads,
                             int64_t key_dim, int64_t value_dim, int in_dtype) {
  if (!kda::mfma_path(in_dtype, in_dtype == KDA_DTYPE_F64 ? KDA_DTYPE_F64 : KDA_DTYPE_F32, key_dim, value_dim)) {
    // the split-bf16 chunk path: packed documents (longest > 0) as a padded
    // batch of the longest document's tokens, dense sequences as they are;
    // the recurrence kernel needs none
    if (!chunk_split_general(in_dtype, KDA_DTYPE_F32, key_dim, value_dim) || num_seqs <= 0) return 0;
    if (longest > 0)
      return chunk_split_general_workspace_bytes(num_seqs, longest, heads, key_dim, value_dim, in_dtype, true);
    return chunk_split_general_workspace_bytes(num_seqs, (total_tokens + num_seqs - 1) / num_seqs, heads, key_dim,
                                               value_dim, in_dtype, false);
  }
  const kda::Plan p = kda::make_plan(num_seqs, total_tokens, heads, value_dim, longest);
  return kda::map_bytes(num_seqs) + kda::segment_bytes(p, heads, value_dim);
}

// Whether a call off the MFMA path takes the split-bf16 chunk path: a shape
// that path covers, as dense sequences or as packed documents whose longest
// length (dense_span) the caller passes (without it the padded batch cannot
// be sized, and the exact recurrence runs).
static bool split_call(const kda::SeqDesc& seq, int64_t N, int64_t total_tokens, int in_dtype, int state_dtype,
                       int64_t K, int64_t V) {
  if (!chunk_split_general(in_dtype, state_dtype, K, V) || N <= 0 || seq.dense_span <= 0) return false;
  return seq.cu_seqlens != nullptr ? seq.valid_lens == nullptr : N * seq.dense_span == total_tokens;
}

size_t chunk_call_workspace_bytes(const kda::SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H, int64_t K,
                                  int64_t V, int in_dtype, int state_dtype) {
  if (kda::mfma_path(in_dtype, state_dtype, K, V))
    return chunk_workspace_bytes(N, total_tokens, kda::plan_longest(seq), H, K, V, in_dtype);
  if (split_call(seq, N, total_tokens, in_dtype, state_dtype, K, V))
    return chunk_split_general_workspace_bytes(N, seq.dense_span, H, K, V, in_dtype, seq.cu_seqlens != nullptr);
  return 0;
}

int launch_chunk(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                 const void* s_in, void* s_out, int state_dtype, void* out, const kda::SeqDesc& seq, int64_t N,
                 int64_t total_tokens, int64_t H, int64_t K, int64_t V, void* workspace, size_t workspace_bytes,
                 hipStream_t stream, KernelEvents* ev) {
  using namespace kda;
  if (!mfma_path(in_dtype, state_dtype, K, V)) {
    if (split_call(seq, N, total_tokens, in_dtype, state_dtype, K, V)) {
      // the chunk path of split-bf16 products (packed documents as a padded
      // batch, value widths past 128 in column slices)
      mark(ev, 0, stream);
      const int st = launch_chunk_split_general(q, k, v, g, beta, in_dtype, static_cast<const float*>(s_in),
                                                static_cast<float*>(s_out), out, seq.cu_seqlens, seq.valid_lens, N,
                                                seq.dense_span, total_tokens, H, K, V, workspace, workspace_bytes,
                                                stream);
      mark(ev, 1, stream);
      return st;
    }
    mark(ev, 0, stream);
    const int st = launch_recurrent(q, k, v, g, beta, in_dtype, s_in, s_out, state_dtype, out, nullptr, seq, N, H,
                                    K, V, stream, false);
    mark(ev, 1, stream);
    return st;
  }
  if (workspace_bytes < chunk_workspace_bytes(N, total_tokens, plan_longest(seq), H, K, V, in_dtype)) {
    set_detail("chunk_fwd: workspace too small");
    return KDA_ERR_WORKSPACE;
  }
  const Plan p = make_plan(N, total_tokens, H, V, plan_longest(seq));
  if (H > 65535 || p.segs_bound * H * p.ncg > 0x7fffffffLL || N > 0x7fffffffLL) {
    set_detail("chunk_fwd: grid too large (N=%lld, H=%lld)", (long long)N, (long long)H);
    return KDA_ERR_UNSUPPORTED;
  }
  if (in_dtype == KDA_DTYPE_BF16)
    return run_chunk<bf16, false>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V, workspace, stream,
                                  ev, nullptr);
  return run_chunk<f16, false>(q, k, v, g, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V, workspace, stream, ev,
                               nullptr);
}

int launch_chunk_decay(const void* q, const void* k, const void* v, const void* z, const void* zbias,
                       const float* a_log, float g_min, const void* beta, int in_dtype, const void* s_in, void* s_out,
                       int state_dtype, void* out, const kda::SeqDesc& seq, int64_t N, int64_t total_tokens, int64_t H,
                       int64_t K, int64_t V, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace kda;
  if (!mfma_path(in_dtype, state_dtype, K, V)) {
    set_detail("chunk_fwd_decay: the fused decay needs the MFMA path (bf16/f16 inputs, f32 state, K <= 128 a multiple of 16, "
               "V a multiple of 16 in 16..256); form g with kda_gates_fwd and call kda_chunk_fwd");
    return KDA_ERR_UNSUPPORTED;
  }
  if (workspace_bytes < chunk_workspace_bytes(N, total_tokens, plan_longest(seq), H, K, V, in_dtype)) {
    set_detail("chunk_fwd_decay: workspace too small");
    return KDA_ERR_WORKSPACE;
  }
  const Plan p = make_plan(N, total_tokens, H, V, plan_longest(seq));
  if (H > 65535 || p.segs_bound * H * p.ncg > 0x7fffffffLL || N > 0x7fffffffLL) {
    set_detail("chunk_fwd_decay: grid too large (N=%lld, H=%lld)", (long long)N, (long long)H);
    return KDA_ERR_UNSUPPORTED;
  }
  const DecayInput d{zbias, a_log, g_min};
  if (in_dtype == KDA_DTYPE_BF16)
    return run_chunk<bf16, true>(q, k, v, z, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V, workspace, stream,
                                 nullptr, &d);
  return run_chunk<f16, true>(q, k, v, z, beta, s_in, s_out, out, seq, N, total_tokens, H, K, V, workspace, stream,
                              nullptr, &d);
}

void set_segment_override(int64_t chunks) { kda::g_segment_override.store(chunks, std::memory_order_relaxed); }

}  // namespace kda_host
