// Decode kernels for f16 K/V caches (instantiated per KV type so the
// translation units build in parallel).
#include "pa_decode_mfma.hpp"

namespace pa {
hipError_t launch_decode_f16(const DecodeParams& p, int gc, hipStream_t stream) {
  if (decode_mfma_eligible<KvF16>(p, gc)) return launch_decode_mfma<KvF16>(p, gc, stream);
  return launch_decode_kv<KvF16>(p, gc, stream);
}
}  // namespace pa
