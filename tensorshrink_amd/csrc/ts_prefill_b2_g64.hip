// Prefill kernels for 2-bit layers (uniform or companded codebook); group size 64.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_prefill.h"

namespace ts {

int prefill_b2_g64(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st) {
  if (L->codebook)
    return bf16 ? launch_prefill_tiles<2, 64, true, true, false>(a, st)
                : launch_prefill_tiles<2, 64, false, true, false>(a, st);
  return bf16 ? launch_prefill_tiles<2, 64, true, false, false>(a, st)
              : launch_prefill_tiles<2, 64, false, false, false>(a, st);
}

}  // namespace ts
