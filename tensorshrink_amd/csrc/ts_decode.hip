// Decode entry point: fills the kernel arguments from a ts_qlayer and hands
// them to the per-bit-width dispatcher. The kernel itself is in ts_decode.h.
#include "ts_decode.h"

namespace ts {

int decode_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                   int64_t ldy, int y_dtype, const uint16_t* bias, hipStream_t st) {
  DecodeArgs a{};
  a.packed = L->packed;
  a.pstride = L->packed_stride;
  a.scale = L->scale;
  a.gmin = L->gmin;
  a.dqsc = L->dq_scale_codes;
  a.dqsm = L->dq_scale_meta;
  a.dqgc = L->dq_gmin_codes;
  a.dqgm = L->dq_gmin_meta;
  a.dq_gs = (uint32_t)(L->dq_group_size > 0 ? L->dq_group_size : 1);
  a.s2packed = L->stage2_packed;
  a.s2stride = L->stage2_stride;
  a.s2scale = L->stage2_scale;
  a.s2gmin = L->stage2_gmin;
  // The kernel's table loads are unconditional. With no outliers (or no
  // codebook, or no bias) they read entry 0 of the packed buffer (at least 16
  // bytes), and the values are never used.
  if (L->n_outliers > 0 && !L->tile_outliers) return TS_NOT_COVERED;  // needs the per-tile slots
  const void* dummy = L->packed;
  const bool has_out = L->n_outliers > 0;
  a.slots = has_out ? L->tile_outliers : static_cast<const uint64_t*>(dummy);
  a.cap = has_out ? (int32_t)L->tile_outlier_cap : 0;
  a.cbsrc = L->codebook ? L->codebook : static_cast<const float*>(dummy);
  a.cb_is_table = L->codebook ? 1 : 0;
  a.x = x;
  a.ldx = ldx;
  a.y = y;
  a.ldy = ldy;
  a.y_dtype = y_dtype;
  a.bias = bias;
  a.bias_src = bias ? bias : static_cast<const uint16_t*>(dummy);
  a.bias_mul = bias ? 1 : 0;
  a.N = L->rows;
  a.cols = L->cols;
  a.K = L->padded_cols;
  a.n_groups = L->n_groups;
  a.n_tiles = ts_cdiv(L->rows, 16);
  a.M = (int)M;
  const bool bf16 = x_dtype == TS_BF16;
  switch (L->bits * 1000 + L->group_size) {
    case 2064: return decode_b2_g64(L, a, bf16, st);
    case 2128: return decode_b2_g128(L, a, bf16, st);
    case 2256: return decode_b2_g256(L, a, bf16, st);
    case 4032: return decode_b4_g32(L, a, bf16, st);
    case 4064: return decode_b4_g64(L, a, bf16, st);
    case 4128: return decode_b4_g128(L, a, bf16, st);
    case 4256: return decode_b4_g256(L, a, bf16, st);
    case 6064: return decode_b6_g64(L, a, bf16, st);
    case 6128: return decode_b6_g128(L, a, bf16, st);
    case 8032: return decode_b8_g32(L, a, bf16, st);
    case 8064: return decode_b8_g64(L, a, bf16, st);
    case 8128: return decode_b8_g128(L, a, bf16, st);
    default: return TS_NOT_COVERED;
  }
}

}  // namespace ts
