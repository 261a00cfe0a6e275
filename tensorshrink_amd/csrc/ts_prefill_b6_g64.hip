// Prefill kernels for 6-bit RVQ layers (4-bit uniform stage + 2-bit uniform residual); group size 64.
// (One translation unit per bit width and group size keeps builds parallel.)
#include "ts_prefill.h"

namespace ts {

int prefill_b6_g64(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st) {
  (void)L;
  return bf16 ? launch_prefill_tiles<4, 64, true, false, true>(a, st)
              : launch_prefill_tiles<4, 64, false, false, true>(a, st);
}

}  // namespace ts
