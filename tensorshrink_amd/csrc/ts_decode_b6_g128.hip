// Decode kernels for 6-bit layers: residual VQ, a 4-bit uniform stage plus a 2-bit uniform
// residual stage, both applied in the same pass; group size 128.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_decode.h"

namespace ts {

int decode_b6_g128(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st) {
  (void)L;
  return bf16 ? launch_decode<4, 128, true, false, true, 4>(g, st) : launch_decode<4, 128, false, false, true, 4>(g, st);
}

}  // namespace ts
