// Prefill kernels for 4-bit layers (uniform or NF4 / Lloyd-Max codebook); group size 256.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_prefill.h"

namespace ts {

int prefill_b4_g256(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st) {
  if (L->codebook)
    return bf16 ? launch_prefill_tiles<4, 256, true, true, false>(a, st)
                : launch_prefill_tiles<4, 256, false, true, false>(a, st);
  return bf16 ? launch_prefill_tiles<4, 256, true, false, false>(a, st)
              : launch_prefill_tiles<4, 256, false, false, false>(a, st);
}

}  // namespace ts
