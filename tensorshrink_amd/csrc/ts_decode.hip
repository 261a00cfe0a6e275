// Decode entry point: fills the kernel arguments from a ts_qlayer and hands
// them to the per-bit-width dispatcher. The kernel itself is in ts_decode.h.
#include "ts_decode.h"

#include <cstring>

namespace ts {

// float -> bf16 / f16 bits, rounding to nearest even: the kernel's own
// conversions (ts_f2bf, and the f16 cast), here on the host.
static uint16_t host_f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static uint16_t host_f2h(float f) {
  const _Float16 h = (_Float16)f;
  uint16_t u;
  std::memcpy(&u, &h, 2);
  return u;
}

// Kernel arguments of one layer; NOT_COVERED when it has outliers but
// neither per-tile outlier slots nor the CSR row offsets.
static int fill_args(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                     int64_t ldy, int y_dtype, const uint16_t* bias, DecodeArgs& a, DecodeCsr& c) {
  a = DecodeArgs{};
  a.packed = L->packed;
  a.pstride = L->packed_stride;
  a.scale = L->scale;
  a.gmin = L->gmin;
  a.dqsc = L->dq_scale_codes;
  a.dqsm = L->dq_scale_meta;
  a.dqgc = L->dq_gmin_codes;
  a.dqgm = L->dq_gmin_meta;
  a.dq_gs = (uint32_t)(L->dq_group_size > 0 ? L->dq_group_size : 1);
  a.dqm_bytes = L->dq_scale_codes ? (uint32_t)(ts_cdiv(L->rows * L->n_groups, (int64_t)a.dq_gs) * 4) : 0u;
  a.s2packed = L->stage2_packed;
  a.s2stride = L->stage2_stride;
  a.s2scale = L->stage2_scale;
  a.s2gmin = L->stage2_gmin;
  // The kernel's table loads are unconditional. With no outliers (or no
  // codebook, or no bias) they read entry 0 of the packed buffer (at least 16
  // bytes), and the values are never used.
  const void* dummy = L->packed;
  const bool has_out = L->n_outliers > 0;
  const bool slots = has_out && L->tile_outliers && L->tile_outlier_cap > 0;
  const bool csr = has_out && !slots && L->outlier_row_ptr && L->outlier_row && L->outlier_col && L->outlier_delta;
  if (has_out && !slots && !csr) return TS_NOT_COVERED;
  a.slots = slots ? L->tile_outliers : static_cast<const uint64_t*>(dummy);
  a.cap = slots ? (int32_t)L->tile_outlier_cap : (csr ? -1 : 0);
  c.row_ptr = csr ? L->outlier_row_ptr : static_cast<const int32_t*>(dummy);
  c.row = csr ? L->outlier_row : static_cast<const int32_t*>(dummy);
  c.col = csr ? L->outlier_col : static_cast<const int32_t*>(dummy);
  c.delta = csr ? L->outlier_delta : static_cast<const uint16_t*>(dummy);
  a.cbsrc = L->codebook ? L->codebook : static_cast<const float*>(dummy);
  const int ncb = 1 << (L->bits == 6 ? 4 : L->bits);
  a.cb_mode = !L->codebook ? CB_UNIFORM : (L->codebook_host && ncb <= 16) ? CB_INLINE : CB_DEVICE;
  if (a.cb_mode != CB_DEVICE) {
    // The table entries, as the kernel uses them: centred on the middle of
    // the codebook's range, cb0 = (cb[0] + cb[last]) / 2, for 2- and 4-bit
    // codebooks (NF, Lloyd-Max; uniform grids and RVQ stage 1 keep cb0 = 0),
    // then rounded to the activation type.
    float v[16];
    for (int j = 0; j < 16; ++j) v[j] = a.cb_mode == CB_INLINE ? L->codebook_host[j < ncb ? j : 0] : (float)j;
    const bool centre = a.cb_mode == CB_INLINE && (L->bits == 4 || L->bits == 2);
    a.cb0 = centre ? 0.5f * (v[0] + v[ncb - 1]) : 0.f;
    for (int j = 0; j < 16; ++j) a.cbq[j] = x_dtype == TS_BF16 ? host_f2bf(v[j] - a.cb0) : host_f2h(v[j] - a.cb0);
  }
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
  return TS_OK;
}

static int dispatch(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st) {
  switch (L->bits * 1000 + L->group_size) {
    case 2064: return decode_b2_g64(L, g, bf16, st);
    case 2128: return decode_b2_g128(L, g, bf16, st);
    case 2256: return decode_b2_g256(L, g, bf16, st);
    case 4032: return decode_b4_g32(L, g, bf16, st);
    case 4064: return decode_b4_g64(L, g, bf16, st);
    case 4128: return decode_b4_g128(L, g, bf16, st);
    case 4256: return decode_b4_g256(L, g, bf16, st);
    case 6064: return decode_b6_g64(L, g, bf16, st);
    case 6128: return decode_b6_g128(L, g, bf16, st);
    case 8032: return decode_b8_g32(L, g, bf16, st);
    case 8064: return decode_b8_g64(L, g, bf16, st);
    case 8128: return decode_b8_g128(L, g, bf16, st);
    default: return TS_NOT_COVERED;
  }
}

int decode_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                   int64_t ldy, int y_dtype, const uint16_t* bias, hipStream_t st) {
  DecodeGroup g{};
  const int rc = fill_args(L, x, M, ldx, x_dtype, y, ldy, y_dtype, bias, g.a[0], g.csr[0]);
  if (rc != TS_OK) return rc;
  g.tile_end[0] = g.a[0].n_tiles;
  g.n = 1;
  return dispatch(L, g, x_dtype == TS_BF16, st);
}

// Layers that can share one launch: the same bit width, group size, column
// count, padding, codebook kind, double-quant kind and stage-2 kind.
static bool same_format(const ts_qlayer* a, const ts_qlayer* b) {
  return a->bits == b->bits && a->group_size == b->group_size && a->cols == b->cols &&
         a->padded_cols == b->padded_cols && a->n_groups == b->n_groups &&
         (a->codebook != nullptr) == (b->codebook != nullptr) &&
         (a->dq_scale_codes != nullptr) == (b->dq_scale_codes != nullptr) &&
         (a->stage2_packed != nullptr) == (b->stage2_packed != nullptr);
}

int decode_forward_group(const ts_qlayer* const* layers, int n, const uint16_t* x, int64_t M, int64_t ldx,
                         int x_dtype, void* const* y, const int64_t* ldy, int y_dtype,
                         const uint16_t* const* bias, hipStream_t st) {
  if (n < 1 || n > DEC_GMAX) return TS_NOT_COVERED;
  DecodeGroup g{};
  int64_t tiles = 0;
  for (int l = 0; l < n; ++l) {
    if (!same_format(layers[0], layers[l])) return TS_NOT_COVERED;
    const int rc =
        fill_args(layers[l], x, M, ldx, x_dtype, y[l], ldy[l], y_dtype, bias ? bias[l] : nullptr, g.a[l], g.csr[l]);
    if (rc != TS_OK) return rc;
    tiles += g.a[l].n_tiles;
    g.tile_end[l] = tiles;
  }
  g.n = n;
  return dispatch(layers[0], g, x_dtype == TS_BF16, st);
}

}  // namespace ts
