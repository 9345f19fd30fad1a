// Decode kernels for FP8 (E4M3) K/V caches (instantiated per KV type so the
// translation units build in parallel).
#include "pa_decode.hpp"

namespace pa {
hipError_t launch_decode_fp8(const DecodeParams& p, int gc, hipStream_t stream) {
  return launch_decode_kv<KvFP8>(p, gc, stream);
}
}  // namespace pa
