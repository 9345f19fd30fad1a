// Decode kernels for bf16 K/V caches (instantiated per KV type so the
// translation units build in parallel).
#include "pa_decode_mfma.hpp"

namespace pa {
hipError_t launch_decode_bf16(const DecodeParams& p, int gc, hipStream_t stream) {
  if (decode_mfma_eligible<KvBF16>(p, gc)) return launch_decode_mfma<KvBF16>(p, gc, stream);
  return launch_decode_kv<KvBF16>(p, gc, stream);
}
}  // namespace pa
