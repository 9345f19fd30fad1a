// Decode kernels for f64 K/V caches (instantiated per KV type so the
// translation units build in parallel).
#include "pa_decode.hpp"

namespace pa {
hipError_t launch_decode_f64(const DecodeParams& p, int gc, hipStream_t stream) {
  return launch_decode_kv<KvF64>(p, gc, stream);
}
}  // namespace pa
