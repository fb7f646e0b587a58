// The chunkwise prefill for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): kda_chunk_fwd with its workspace taken from a file-scope device
// array instead of a caller buffer.
//
// `scratch` is a host-side stand-in in host code, not a device address: its
// device address is looked up once per device with hipGetSymbolAddress (each
// GPU holds its own copy at its own address, for as long as the process
// runs) and only that pointer is handed to the kernels.  Every call on one
// GPU shares that GPU's array: calls that overlap on one GPU (two streams, or
// two host threads) race on it.  Nothing in the array needs to start at zero:
// every workspace word a prefill reads (chunk and segment maps, segment
// summaries and start states, each chunk's M and Aqk) is written earlier in
// the same call.
#include <mutex>

#include "kda_launch.h"

static constexpr size_t kScratchBytes = static_cast<size_t>(KDA_NOALLOC_SCRATCH_BYTES);
static_assert(kScratchBytes % 256 == 0, "scratch size must keep 256-byte alignment");

// the workspace of kda_chunk_fwd_noalloc, one copy per device
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace kda_host {

// Device address of this device's scratch array (looked up on the first call
// on each device, with that device current).
int noalloc_scratch(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_detail("chunk_fwd_noalloc: no current HIP device (or device index >= %d)", kMaxDevices);
    return KDA_ERR_LAUNCH;
  }
  if (stream != nullptr) {
    int sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev) {
      set_detail("chunk_fwd_noalloc: the stream belongs to device %d, the current device is %d", sdev, dev);
      return KDA_ERR_INVALID_ARGUMENT;
    }
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_detail("chunk_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                 hipGetErrorString(e));
      return KDA_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return KDA_OK;
}

}  // namespace kda_host

extern "C" int kda_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                     int in_dtype, const void* initial_state, void* final_state, int state_dtype,
                                     void* out, const int32_t* cu_seqlens, int64_t dense_span,
                                     const int32_t* valid_lens, int64_t num_seqs, int64_t total_tokens,
                                     int64_t heads, int64_t key_dim, int64_t value_dim, void* stream) {
  using namespace kda_host;
  if (num_seqs <= 0 || total_tokens <= 0 || heads <= 0 || key_dim <= 0 || value_dim <= 0) {
    set_detail("chunk_fwd_noalloc: sizes must be positive");
    return KDA_ERR_INVALID_ARGUMENT;
  }
  // the size check comes before any device call: an oversize request launches nothing
  const kda::SeqDesc seq{cu_seqlens, dense_span, valid_lens};
  const size_t need = chunk_call_workspace_bytes(seq, num_seqs, total_tokens, heads, key_dim, value_dim, in_dtype,
                                                 state_dtype);
  if (need > kScratchBytes) {
    set_detail("chunk_fwd_noalloc: this prefill needs %zu workspace bytes; the static scratch holds %zu "
               "(use kda_chunk_fwd with a caller workspace)",
               need, kScratchBytes);
    return KDA_ERR_WORKSPACE;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int st = noalloc_scratch(s, &ws);
  if (st != KDA_OK) return st;
  // the same argument checks and kernels as kda_chunk_fwd, on the scratch array
  return kda_chunk_fwd(q, k, v, g, beta, in_dtype, initial_state, final_state, state_dtype, out, cu_seqlens,
                       dense_span, valid_lens, num_seqs, total_tokens, heads, key_dim, value_dim, ws, kScratchBytes,
                       stream);
}
