// Cache plumbing for serving: the batch reorder (beam search) and the clone of
// a decode cache, every tensor of every layer in one launch.  A decode cache
// holds, per KDA layer, the f32 recurrent state [B,H,K,V], three ShortConv
// histories [B,K_conv-1,width] and the int64 sequence offsets [B]; all of them
// are batch-major, so a reorder is a gather of batch rows of each tensor
// (out[i] = src[index[i]]) and a clone is the same gather with the identity
// index.  One HBM stream: each selected row is read once and written once.
#include "kda_launch.h"

namespace kda {

constexpr int kCacheMaxTensors = 64;                      // tensors per launch
constexpr int kGatherThreads = 256;
constexpr int kGatherPer = 2;                               // units per thread per tile
constexpr int kGatherTile = kGatherThreads * kGatherPer;    // units per tile

struct GatherDesc {
  const unsigned char* src;
  unsigned char* dst;
  int64_t row_units;      // units per row (unit = 1 << shift bytes)
  int64_t tile0;          // first tile of this tensor within the launch
  int32_t tiles_per_row;  // > 1 only when a row is longer than a tile
  int32_t rows_per_tile;  // > 1 only when several rows fit in a tile
  int32_t shift;          // log2 of the unit: 4 (16 bytes) when sizes and addresses allow
  int32_t pad;
};

struct GatherArgs {
  GatherDesc d[kCacheMaxTensors];
  const int64_t* index;  // [n_out] source row of each output row; null = identity
  int64_t n_out, n_src;
  int* status;           // set to 1 when an index is out of range (null: not reported)
  int32_t n;             // descriptors in use
};
static_assert(sizeof(GatherArgs) <= 4096, "the descriptors travel in the kernel argument block");

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

template <int S>
struct UnitOf;
template <>
struct UnitOf<4> {
  typedef u32x4 type;
};
template <>
struct UnitOf<3> {
  typedef u32x2 type;
};
template <>
struct UnitOf<2> {
  typedef unsigned type;
};
template <>
struct UnitOf<1> {
  typedef unsigned short type;
};
template <>
struct UnitOf<0> {
  typedef unsigned char type;
};

__device__ __forceinline__ int64_t gather_block(unsigned b, unsigned nb) {
  const unsigned per = nb / 8, rem = nb % 8, x = b % 8;
  return static_cast<int64_t>(x) * per + (x < rem ? x : rem) + b / 8;
}

__device__ __forceinline__ bool source_row(const GatherArgs& a, int64_t row, int64_t& srow) {
  srow = a.index ? a.index[row] : row;
  if (srow >= 0 && srow < a.n_src) return true;
  if (a.status) *a.status = 1;
  return false;
}

template <int S>
__device__ __forceinline__ void gather_tile(const GatherArgs& a, const GatherDesc& d, int64_t local) {
  typedef typename UnitOf<S>::type U;
  const U* src = reinterpret_cast<const U*>(d.src);
  U* dst = reinterpret_cast<U*>(d.dst);
  const int tid = threadIdx.x;
  if (d.rows_per_tile == 1) {
    // a slice of kGatherTile units of one row: all loads in flight, then all
    // stores, non-temporal (the output is not read back by this pass).  Two
    // 16-byte units per thread in 256-thread tiles measured fastest (6.1 TB/s
    // on an 8.9 GB reorder, against 5.7 at four units and 3.7 at eight; 5.4
    // at four units with plain stores).
    const int64_t row = local / d.tiles_per_row;
    const int64_t c0 = (local - row * d.tiles_per_row) * kGatherTile;
    int64_t srow;
    if (!source_row(a, row, srow)) return;
    const U* s = src + srow * d.row_units;
    U* o = dst + row * d.row_units;
    U v[kGatherPer];
#pragma unroll
    for (int j = 0; j < kGatherPer; ++j) {
      const int64_t c = c0 + j * kGatherThreads + tid;
      if (c < d.row_units) v[j] = s[c];
    }
#pragma unroll
    for (int j = 0; j < kGatherPer; ++j) {
      const int64_t c = c0 + j * kGatherThreads + tid;
      if (c < d.row_units) __builtin_nontemporal_store(v[j], o + c);
    }
  } else {
    // several short rows: unit e of the tile is column e % row_units of row e / row_units
    const int64_t r0 = local * d.rows_per_tile;
    const int64_t left = a.n_out - r0;
    const int nrow = left < d.rows_per_tile ? static_cast<int>(left) : d.rows_per_tile;
    const int ru = static_cast<int>(d.row_units), n = nrow * ru;
#pragma unroll
    for (int j = 0; j < kGatherPer; ++j) {
      const int e = j * kGatherThreads + tid;
      if (e < n) {
        const int r = e / ru, c = e - r * ru;
        int64_t srow;
        if (source_row(a, r0 + r, srow)) dst[(r0 + r) * ru + c] = src[srow * ru + c];
      }
    }
  }
}

__global__ __launch_bounds__(kGatherThreads) void cache_gather_kernel(const GatherArgs a) {
  const int64_t tile = gather_block(blockIdx.x, gridDim.x);
  // the descriptor whose tile range holds this tile (tile0 ascends)
  int lo = 0, hi = a.n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.d[mid].tile0 <= tile)
      lo = mid;
    else
      hi = mid - 1;
  }
  const GatherDesc& d = a.d[lo];
  const int64_t local = tile - d.tile0;
  switch (d.shift) {
    case 4:
      gather_tile<4>(a, d, local);
      break;
    case 3:
      gather_tile<3>(a, d, local);
      break;
    case 2:
      gather_tile<2>(a, d, local);
      break;
    case 1:
      gather_tile<1>(a, d, local);
      break;
    default:
      gather_tile<0>(a, d, local);
      break;
  }
}

}  // namespace kda

namespace kda_host {

static int low_zero_bits(uint64_t x) {
  int s = 0;
  while (s < 4 && !(x & (uint64_t{1} << s))) ++s;
  return s;
}

static bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return na > 0 && nb > 0 && pa < pb + static_cast<uintptr_t>(nb) && pb < pa + static_cast<uintptr_t>(na);
}

int launch_cache_gather(const void* const* src, void* const* dst, const int64_t* row_bytes, int n_tensors,
                        const int64_t* index, int64_t n_src, int64_t n_out, int* status, hipStream_t stream) {
  if (n_tensors < 0 || n_src < 0 || n_out < 0 || (n_tensors > 0 && (!src || !dst || !row_bytes))) {
    set_detail("cache_gather: bad tensor count, row count or null descriptor arrays");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  if (!index && n_out != n_src) {
    set_detail("cache_gather: without an index the output has the source's %lld rows, not %lld",
               (long long)n_src, (long long)n_out);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  for (int t = 0; t < n_tensors; ++t) {
    const int64_t rb = row_bytes[t];
    if (rb < 0) {
      set_detail("cache_gather: tensor %d has negative row bytes", t);
      return KDA_ERR_INVALID_ARGUMENT;
    }
    if (rb == 0 || n_out == 0) continue;
    if (!dst[t] || (!src[t] && n_src > 0)) {
      set_detail("cache_gather: tensor %d has a null pointer", t);
      return KDA_ERR_INVALID_ARGUMENT;
    }
    if (rb > INT64_MAX / (n_src > n_out ? n_src : n_out)) {
      set_detail("cache_gather: tensor %d is too large", t);
      return KDA_ERR_INVALID_ARGUMENT;
    }
    for (int u = 0; u < n_tensors; ++u)  // an output may not overlap any source or another output
      if (row_bytes[u] > 0 && (overlaps(dst[t], rb * n_out, src[u], row_bytes[u] * n_src) ||
                               (u != t && overlaps(dst[t], rb * n_out, dst[u], row_bytes[u] * n_out)))) {
        set_detail("cache_gather: output %d overlaps tensor %d", t, u);
        return KDA_ERR_INVALID_ARGUMENT;
      }
  }
  if (n_out == 0) return KDA_OK;
  if (n_src == 0) {
    set_detail("cache_gather: gathering %lld rows from an empty batch", (long long)n_out);
    return KDA_ERR_INVALID_ARGUMENT;
  }
  kda::GatherArgs args{};
  args.index = index;
  args.n_out = n_out;
  args.n_src = n_src;
  args.status = status;
  int64_t tiles = 0;
  auto flush = [&]() -> int {
    if (args.n == 0) return KDA_OK;
    if (tiles > 0x7fffffffLL) {
      set_detail("cache_gather: grid too large");
      return KDA_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL(kda::cache_gather_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kda::kGatherThreads), 0,
                       stream, args);
    const int rc = check_launch("cache_gather_kernel");
    args.n = 0;
    tiles = 0;
    return rc;
  };
  for (int t = 0; t < n_tensors; ++t) {
    const int64_t rb = row_bytes[t];
    if (rb == 0) continue;
    kda::GatherDesc d{};
    d.src = static_cast<const unsigned char*>(src[t]);
    d.dst = static_cast<unsigned char*>(dst[t]);
    d.shift = low_zero_bits(static_cast<uint64_t>(rb) | reinterpret_cast<uintptr_t>(src[t]) |
                            reinterpret_cast<uintptr_t>(dst[t]) | (uint64_t{1} << 4));
    d.row_units = rb >> d.shift;
    int64_t ntile;
    if (d.row_units * 2 > kda::kGatherTile) {
      const int64_t tpr = (d.row_units + kda::kGatherTile - 1) / kda::kGatherTile;
      if (tpr > 0x7fffffffLL) {
        set_detail("cache_gather: tensor %d rows are too long", t);
        return KDA_ERR_UNSUPPORTED;
      }
      d.tiles_per_row = static_cast<int32_t>(tpr);
      d.rows_per_tile = 1;
      ntile = n_out * tpr;
    } else {
      d.tiles_per_row = 1;
      d.rows_per_tile = static_cast<int32_t>(kda::kGatherTile / d.row_units);
      ntile = (n_out + d.rows_per_tile - 1) / d.rows_per_tile;
    }
    if (args.n == kda::kCacheMaxTensors || tiles + ntile > 0x7fffffffLL) {
      const int rc = flush();
      if (rc != KDA_OK) return rc;
    }
    d.tile0 = tiles;
    tiles += ntile;
    args.d[args.n++] = d;
  }
  return flush();
}

}  // namespace kda_host
