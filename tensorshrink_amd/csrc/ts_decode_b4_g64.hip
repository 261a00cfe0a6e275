// Decode kernels for 4-bit layers (uniform or NF4 / Lloyd-Max codebook); group size 64.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_decode.h"

namespace ts {

int decode_b4_g64(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st) {
  (void)L;
  return bf16 ? launch_decode<4, 64, true, false, false, 32>(g, st) : launch_decode<4, 64, false, false, false, 32>(g, st);
}

}  // namespace ts
