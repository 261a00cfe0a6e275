// Prefill kernels for 8-bit layers (uniform or NF8 codebook); group size 128.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_prefill.h"

namespace ts {

int prefill_b8_g128(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st) {
  if (L->codebook)
    return bf16 ? launch_prefill_tiles<8, 128, true, true, false>(a, st)
                : launch_prefill_tiles<8, 128, false, true, false>(a, st);
  return bf16 ? launch_prefill_tiles<8, 128, true, false, false>(a, st)
              : launch_prefill_tiles<8, 128, false, false, false>(a, st);
}

}  // namespace ts
