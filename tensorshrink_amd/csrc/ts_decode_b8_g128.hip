// Decode kernels for 8-bit layers: uniform codes (exact in bf16/f16 as integers) or a
// 256-entry codebook (NF8) as a (hi, lo) pair of bf16/f16 values, so the
// codebook value keeps ~16 mantissa bits; group size 128.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_decode.h"

namespace ts {

int decode_b8_g128(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st) {
  (void)L;
  if (L->codebook)
    return bf16 ? launch_decode<8, 128, true, true, false, 16>(g, st) : launch_decode<8, 128, false, true, false, 16>(g, st);
  return bf16 ? launch_decode<8, 128, true, false, false, 1>(g, st) : launch_decode<8, 128, false, false, false, 1>(g, st);
}

}  // namespace ts
