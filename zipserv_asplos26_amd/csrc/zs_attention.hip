// zs_attention.hip -- decode attention over compressed / dense KV (gfx950).
#include <hip/hip_runtime.h>

#include "../../include/zipserv.h"

extern "C" size_t zs_decode_attention_workspace_bytes(int, int, int, int, int) { return 0; }

extern "C" int zs_decode_attention(void*, const uint16_t*, const zs_kv_compressed_t*,
                                   const zs_kv_compressed_t*, const int32_t*, int, int, int, int,
                                   int, float, uint16_t*, float*, void*, size_t, int) {
  return ZS_E_UNSUPPORTED;
}

extern "C" int zs_decode_attention_dense(void*, const uint16_t*, const uint16_t*, const uint16_t*,
                                         const int32_t*, int, int, int, int, int, int, float,
                                         uint16_t*, float*, void*, size_t, int) {
  return ZS_E_UNSUPPORTED;
}
