// Decode kernels for 2-bit layers (uniform or companded 4-level codebook); group size 64.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_decode.h"

namespace ts {

int decode_b2_g64(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st) {
  (void)L;
  return bf16 ? launch_decode<2, 64, true, false, false, 4>(g, st) : launch_decode<2, 64, false, false, false, 4>(g, st);
}

}  // namespace ts
