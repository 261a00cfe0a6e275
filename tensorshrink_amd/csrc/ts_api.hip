// extern "C" entry points of libtensorshrink_hip.so (declared in
// include/tensorshrink_hip.h). Argument checking and dispatch only; the
// kernels live in ts_decode.hip, ts_prefill.hip, ts_gemm.hip, ts_aux.hip,
// ts_quantize.hip.
#include <algorithm>

#include "ts_common.h"

namespace ts {
int decode_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                   int64_t ldy, int y_dtype, const uint16_t* bias, hipStream_t st);
int decode_forward_group(const ts_qlayer* const* layers, int n, const uint16_t* x, int64_t M, int64_t ldx,
                         int x_dtype, void* const* y, const int64_t* ldy, int y_dtype,
                         const uint16_t* const* bias, hipStream_t st);
int prefill_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                    int64_t ldy, int y_dtype, const uint16_t* bias, void* ws, size_t ws_bytes, hipStream_t st);
size_t prefill_partials_bytes(const ts_qlayer* L, int64_t M);
int generic_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                    int64_t ldy, int y_dtype, const uint16_t* bias, hipStream_t st);
int dequantize(const ts_qlayer* L, int mode, const int32_t* oidx, const uint16_t* oval, int64_t n_oidx,
               void* w_out, int64_t ldw, int dt, hipStream_t st);
size_t gemm_ws_bytes(const ts_qlayer* L);
int gemm_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y, int64_t ldy,
                 int y_dtype, const uint16_t* bias, void* ws, size_t ws_bytes, hipStream_t st);
// Above the decode sizes the forward dequantizes the layer into the
// workspace and runs one library GEMM, when the caller provides it (the
// reference switches to dequantize + F.linear above 64 rows; measured here the
// GEMM path is faster than the fused MFMA kernel from 17 rows on).
constexpr int64_t GEMM_MIN_M = 17;
// Up to DEC_M_MAX rows of x per launch the decode kernel runs them as blocks
// of 16 tokens that share each code-table read (the reference's fused kernel
// covers M <= 64, modules.py:881-894). Above 16 rows it competes with the
// fused MFMA prefill kernel, which splits K where its tiles would leave CUs
// idle. Measured on MI355X (NF4 / NF8 / 2-bit / 6-bit RVQ layers of 1024-28672
// rows, K = 4096-28672): decode wins up to 32 rows (24 when K > 8192) on
// layers of at most 256 16-row tiles with codes of at most 6 bits; 8-bit
// layers (by at most 3 us at 17-24 rows on the smallest ones) and taller
// layers run the prefill kernel from 17 rows.
constexpr int64_t DEC_M_MAX = 64;
inline bool decode_mid_m(const ts_qlayer* L, int64_t M) {
  if (M <= 16) return true;
  return L->bits != 8 && ts_cdiv(L->rows, 16) <= 256 && M <= (L->cols > 8192 ? 24 : 32);
}
// Grouped decode launches (q/k/v, gate/up) above 16 rows: up to 32 rows while
// the group has at most this many 16-row tiles in all. Measured: q/k/v of a
// 4096-wide model (384 tiles) in one decode launch takes 26-52 us at 17-32
// rows against 60-73 us for three prefill launches (2-bit to NF8); gate/up
// (1792 tiles) loses to two prefill launches from 24 rows (17 at 8 and 2 bits).
constexpr int64_t DEC_GROUP_TILES_MAX = 768;
int outlier_row_ptr(const int32_t* row, int64_t n, int64_t rows, int32_t* row_ptr, hipStream_t st);
int tile_outlier_max(const int32_t* rp, int64_t rows, int32_t* out, hipStream_t st);
int build_tile_outliers(const int32_t* rp, const int32_t* orow, const int32_t* ocol, const uint16_t* odelta,
                        int64_t rows, int64_t cap, uint64_t* slots, hipStream_t st);
int build_colsorted_outliers(const int32_t* rp, const int32_t* ocol, const uint16_t* odelta, int64_t rows,
                             uint32_t* out, hipStream_t st);
size_t outlier_tables_ws(int64_t n);
int build_outlier_tables(const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n, int32_t* orow,
                         int32_t* ocol, uint16_t* odelta, int32_t* row_ptr, void* ws, size_t ws_bytes,
                         hipStream_t st);
int apply_outlier_correction(float* out, int64_t M, int64_t ldo, const void* x, int64_t ldx, int xdt,
                             const int32_t* row_ptr, const int32_t* col, const uint16_t* delta, int64_t rows,
                             hipStream_t st);
int build_outlier_tables_noalloc(const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n,
                                 int32_t* orow, int32_t* ocol, uint16_t* odelta, int32_t* row_ptr, hipStream_t st);
size_t topk_ws_bytes(int64_t n, int64_t k);
int topk_count(const ts_qinput* in, int64_t k, void* ws, size_t ws_bytes, int64_t* n_cand, hipStream_t st);
int topk_write(const ts_qinput* in, int64_t k, void* ws, int64_t* cidx, float* cval, hipStream_t st);
int topk_select(const int64_t* cidx, const float* cval, int64_t nc, int64_t n, int64_t k, int64_t* out_idx,
                float* out_val);
int quantize_groups(const ts_qinput* in, const ts_group_opts* o, uint8_t* packed, int64_t pstride, uint16_t* s16,
                    uint16_t* g16, float* s32, float* g32, hipStream_t st);
int lm_sample(const ts_qinput* in, const ts_group_opts* o, const float* s32, const float* g32, const int64_t* idx,
              int64_t n, float* out, hipStream_t st);
int lloyd_max_fit_host(const float* x, int64_t m, const float* init, int32_t n_levels, int32_t iters, float* out);
int double_quantize(const uint16_t* v, int64_t n, int64_t dqgs, uint8_t* codes, uint16_t* meta, uint16_t* recon,
                    hipStream_t st);
int rvq_residual(const ts_qinput* in, const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n,
                 float* res, hipStream_t st);
int sq_error_sums(const ts_qinput* in, const void* d, int ddt, double* sums, hipStream_t st);
int gather_f16(const void* w, int dt, const int64_t* idx, int64_t n, uint16_t* out, hipStream_t st);
}  // namespace ts

static inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

static bool layer_ok(const ts_qlayer* L) {
  if (!L || !L->packed || L->rows <= 0 || L->cols <= 0 || L->group_size <= 0) return false;
  if (L->bits != 2 && L->bits != 4 && L->bits != 8 && L->bits != 6) return false;
  if (L->padded_cols < L->cols || L->padded_cols % L->group_size != 0) return false;
  if (L->n_groups != L->padded_cols / L->group_size) return false;
  const bool dq = L->dq_scale_codes != nullptr;
  if (dq && (!L->dq_scale_meta || !L->dq_gmin_codes || !L->dq_gmin_meta || L->dq_group_size <= 0)) return false;
  if (!dq && (!L->scale || !L->gmin)) return false;
  if (L->n_outliers > 0 && (!L->outlier_row || !L->outlier_col || !L->outlier_delta || !L->outlier_row_ptr))
    return false;
  if (L->bits == 6 && (!L->stage2_packed || !L->stage2_scale || !L->stage2_gmin)) return false;
  if (L->tile_outliers && L->tile_outlier_cap <= 0) return false;
  return true;
}

extern "C" {

const char* ts_status_str(int s) {
  switch (s) {
    case TS_OK: return "ok";
    case TS_NOT_COVERED: return "shape or format not covered by the kernels";
    case TS_BAD_ARG: return "bad argument";
    case TS_HIP_ERROR: return "HIP runtime error";
    case TS_WORKSPACE: return "workspace too small";
    default: return "unknown status";
  }
}

const char* ts_version(void) { return "tensorshrink_hip 0.1.0 (gfx950)"; }

size_t ts_forward_workspace_bytes(const ts_qlayer* layer, int64_t M) {
  if (!layer_ok(layer) || M < ts::GEMM_MIN_M) return 0;
  return ts::gemm_ws_bytes(layer);
}

size_t ts_forward_partials_bytes(const ts_qlayer* layer, int64_t M) {
  if (!layer_ok(layer) || ts::decode_mid_m(layer, M)) return 0;
  const size_t b = ts::prefill_partials_bytes(layer, M);
  // always below the library path's workspace, which takes precedence
  return b < ts::gemm_ws_bytes(layer) ? b : 0;
}

int ts_qlinear_forward(const ts_qlayer* L, const void* x, int64_t M, int64_t ldx, int x_dtype, void* y, int64_t ldy,
                       int y_dtype, const void* bias, void* workspace, size_t workspace_bytes, void* stream) {
  if (!layer_ok(L) || !x || !y || M < 0) return TS_BAD_ARG;
  if (x_dtype != TS_BF16 && x_dtype != TS_F16) return TS_BAD_ARG;
  if (y_dtype != TS_BF16 && y_dtype != TS_F16 && y_dtype != TS_F32) return TS_BAD_ARG;
  if (y_dtype != TS_F32 && y_dtype != x_dtype) return TS_BAD_ARG;
  if (ldx < L->cols || ldy < L->rows) return TS_BAD_ARG;
  if (M == 0) return TS_OK;
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* bp = static_cast<const uint16_t*>(bias);
  // The tiled kernels read x in aligned 16-byte chunks.
  const bool aligned = (L->cols % 8 == 0) && (ldx % 8 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  int rc = TS_NOT_COVERED;
  if (M >= ts::GEMM_MIN_M && workspace)
    rc = ts::gemm_forward(L, xp, M, ldx, x_dtype, y, ldy, y_dtype, bp, workspace, workspace_bytes, S(stream));
  if (rc == TS_NOT_COVERED && aligned) {
    // the decode kernel in passes of at most DEC_M_MAX rows; the first pass
    // decides coverage (the format checks run before any launch)
    auto decode_passes = [&]() {
      const size_t ybytes = y_dtype == TS_F32 ? 4 : 2;
      int r = TS_NOT_COVERED;
      for (int64_t m0 = 0; m0 < M; m0 += ts::DEC_M_MAX) {
        r = ts::decode_forward(L, xp + m0 * ldx, std::min(ts::DEC_M_MAX, M - m0), ldx, x_dtype,
                               static_cast<char*>(y) + m0 * ldy * ybytes, ldy, y_dtype, bp, S(stream));
        if (r != TS_OK) break;
      }
      return r;
    };
    const bool dec = ts::decode_mid_m(L, M);
    if (dec) rc = decode_passes();
    if (rc == TS_NOT_COVERED && M > 16)
      rc = ts::prefill_forward(L, xp, M, ldx, x_dtype, y, ldy, y_dtype, bp, workspace, workspace_bytes, S(stream));
    // layers the prefill kernel does not take (group sizes below 64 with
    // columns not a multiple of 64, columns past its 16-bit outlier walk):
    // the decode kernel's token blocks before the one-thread-per-output kernel
    if (rc == TS_NOT_COVERED && !dec) rc = decode_passes();
  }
  if (rc == TS_NOT_COVERED) rc = ts::generic_forward(L, xp, M, ldx, x_dtype, y, ldy, y_dtype, bp, S(stream));
  return rc;
}

int ts_qlinear_forward_group(const ts_qlayer* const* layers, int n_layers, const void* x, int64_t M, int64_t ldx,
                             int x_dtype, void* const* y, const int64_t* ldy, int y_dtype,
                             const void* const* bias, void* stream) {
  if (!layers || !y || !ldy || !x || M < 0 || n_layers < 1) return TS_BAD_ARG;
  if (x_dtype != TS_BF16 && x_dtype != TS_F16) return TS_BAD_ARG;
  if (y_dtype != TS_BF16 && y_dtype != TS_F16 && y_dtype != TS_F32) return TS_BAD_ARG;
  if (y_dtype != TS_F32 && y_dtype != x_dtype) return TS_BAD_ARG;
  for (int l = 0; l < n_layers; ++l) {
    const ts_qlayer* L = layers[l];
    if (!layer_ok(L) || !y[l] || ldx < L->cols || ldy[l] < L->rows) return TS_BAD_ARG;
  }
  if (M == 0) return TS_OK;
  const ts_qlayer* L0 = layers[0];
  const bool aligned = (L0->cols % 8 == 0) && (ldx % 8 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  if (!aligned || M > 32) return TS_NOT_COVERED;
  if (M > 16) {
    int64_t tiles = 0;
    for (int l = 0; l < n_layers; ++l) tiles += ts_cdiv(layers[l]->rows, 16);
    if (tiles > ts::DEC_GROUP_TILES_MAX) return TS_NOT_COVERED;
  }
  return ts::decode_forward_group(layers, n_layers, static_cast<const uint16_t*>(x), M, ldx, x_dtype, y, ldy, y_dtype,
                                  reinterpret_cast<const uint16_t* const*>(bias), S(stream));
}

int ts_apply_outlier_correction(float* out, int64_t M, int64_t ldo, const void* x, int64_t ldx, int x_dtype,
                                const int32_t* row_ptr, const int32_t* col, const uint16_t* delta, int64_t rows,
                                void* stream) {
  if (!out || !x || !row_ptr || !col || !delta || M < 0 || rows < 0) return TS_BAD_ARG;
  if (x_dtype != TS_BF16 && x_dtype != TS_F16) return TS_BAD_ARG;
  return ts::apply_outlier_correction(out, M, ldo, x, ldx, x_dtype, row_ptr, col, delta, rows, S(stream));
}

int ts_dequantize(const ts_qlayer* L, int mode, const int32_t* outlier_idx, const uint16_t* outlier_val,
                  int64_t n_outlier_idx, void* w_out, int64_t ldw, int out_dtype, void* stream) {
  if (!layer_ok(L) || !w_out || ldw < L->cols) return TS_BAD_ARG;
  if (mode != TS_DEQ_CODEC && mode != TS_DEQ_QLINEAR) return TS_BAD_ARG;
  if (mode == TS_DEQ_CODEC && n_outlier_idx > 0 && (!outlier_idx || !outlier_val)) return TS_BAD_ARG;
  if (out_dtype != TS_F16 && out_dtype != TS_BF16 && out_dtype != TS_F32) return TS_BAD_ARG;
  return ts::dequantize(L, mode, outlier_idx, outlier_val, n_outlier_idx, w_out, ldw, out_dtype, S(stream));
}

int ts_outlier_row_ptr(const int32_t* outlier_row, int64_t n, int64_t rows, int32_t* row_ptr, void* stream) {
  if ((n > 0 && !outlier_row) || !row_ptr || rows < 0) return TS_BAD_ARG;
  return ts::outlier_row_ptr(outlier_row, n, rows, row_ptr, S(stream));
}

size_t ts_outlier_tables_workspace_bytes(int64_t n, int64_t rows) {
  (void)rows;
  return n > 0 ? ts::outlier_tables_ws(n) : 0;
}

int ts_tile_outlier_max(const int32_t* row_ptr, int64_t rows, int32_t* max_count, void* stream) {
  if (!row_ptr || !max_count || rows <= 0) return TS_BAD_ARG;
  return ts::tile_outlier_max(row_ptr, rows, max_count, S(stream));
}

int ts_build_tile_outliers(const int32_t* row_ptr, const int32_t* orow, const int32_t* ocol, const uint16_t* odelta,
                           int64_t rows, int64_t cap, uint64_t* slots, void* stream) {
  if (!row_ptr || !orow || !ocol || !odelta || !slots || rows <= 0 || cap <= 0) return TS_BAD_ARG;
  return ts::build_tile_outliers(row_ptr, orow, ocol, odelta, rows, cap, slots, S(stream));
}

int ts_build_colsorted_outliers(const int32_t* row_ptr, const int32_t* ocol, const uint16_t* odelta, int64_t rows,
                                uint32_t* out, void* stream) {
  if (!row_ptr || !ocol || !odelta || !out || rows < 0) return TS_BAD_ARG;
  return ts::build_colsorted_outliers(row_ptr, ocol, odelta, rows, out, S(stream));
}

int ts_build_outlier_tables(const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n, int32_t* orow,
                            int32_t* ocol, uint16_t* odelta, int32_t* row_ptr, void* ws, size_t ws_bytes,
                            void* stream) {
  if (!L || !L->packed || n < 0 || (n > 0 && (!idx || !val || !orow || !ocol || !odelta))) return TS_BAD_ARG;
  if (n > 0 && (L->rows * L->cols) > ((int64_t)1 << 31)) return TS_NOT_COVERED;  // int32 flat indices
  return ts::build_outlier_tables(L, idx, val, n, orow, ocol, odelta, row_ptr, ws, ws_bytes, S(stream));
}

int ts_build_outlier_tables_noalloc(const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n,
                                    int32_t* orow, int32_t* ocol, uint16_t* odelta, int32_t* row_ptr, void* stream) {
  if (!L || !L->packed || n < 0 || (n > 0 && (!idx || !val || !orow || !ocol || !odelta))) return TS_BAD_ARG;
  if (n > 0 && (L->rows * L->cols) > ((int64_t)1 << 31)) return TS_NOT_COVERED;  // int32 flat indices
  return ts::build_outlier_tables_noalloc(L, idx, val, n, orow, ocol, odelta, row_ptr, S(stream));
}

size_t ts_topk_workspace_bytes(int64_t n, int64_t k) { return (k > 0 && k < n) ? ts::topk_ws_bytes(n, k) : 0; }

int ts_topk_candidates_count(const ts_qinput* in, int64_t k, void* ws, size_t ws_bytes, int64_t* n_candidates,
                             void* stream) {
  if (!in || !in->w || in->rows <= 0 || in->cols <= 0 || !n_candidates) return TS_BAD_ARG;
  return ts::topk_count(in, k, ws, ws_bytes, n_candidates, S(stream));
}

int ts_topk_candidates_write(const ts_qinput* in, int64_t k, void* ws, int64_t* cand_idx, float* cand_val,
                             void* stream) {
  if (!in || !in->w || !ws || !cand_idx || !cand_val) return TS_BAD_ARG;
  return ts::topk_write(in, k, ws, cand_idx, cand_val, S(stream));
}

int ts_topk_select(const int64_t* cand_idx, const float* cand_val, int64_t n_candidates, int64_t n, int64_t k,
                   int64_t* out_idx, float* out_val) {
  if (!cand_idx || !cand_val || !out_idx || !out_val) return TS_BAD_ARG;
  return ts::topk_select(cand_idx, cand_val, n_candidates, n, k, out_idx, out_val);
}

int ts_quantize_groups(const ts_qinput* in, const ts_group_opts* opts, uint8_t* packed, int64_t packed_stride,
                       uint16_t* scale16, uint16_t* gmin16, float* scale32, float* gmin32, void* stream) {
  if (!in || !in->w || !opts || !packed || !scale16 || !gmin16) return TS_BAD_ARG;
  if (opts->bits != 2 && opts->bits != 4 && opts->bits != 8) return TS_BAD_ARG;
  if (opts->group_size <= 0 || (scale32 == nullptr) != (gmin32 == nullptr)) return TS_BAD_ARG;
  return ts::quantize_groups(in, opts, packed, packed_stride, scale16, gmin16, scale32, gmin32, S(stream));
}

int ts_lm_sample(const ts_qinput* in, const ts_group_opts* opts, const float* scale32, const float* gmin32,
                 const int64_t* idx, int64_t n, float* out, void* stream) {
  if (!in || !opts || !scale32 || !gmin32 || (n > 0 && (!idx || !out))) return TS_BAD_ARG;
  return ts::lm_sample(in, opts, scale32, gmin32, idx, n, out, S(stream));
}

int ts_lloyd_max_fit_host(const float* samples, int64_t m, const float* linspace_init, int32_t n_levels,
                          int32_t iters, float* out_centroids) {
  if (!samples || !linspace_init || !out_centroids) return TS_BAD_ARG;
  return ts::lloyd_max_fit_host(samples, m, linspace_init, n_levels, iters, out_centroids);
}

int ts_double_quantize(const uint16_t* values16, int64_t n, int64_t dq_group_size, uint8_t* codes, uint16_t* meta,
                       uint16_t* recon16, void* stream) {
  if (!values16 || !codes || !meta) return TS_BAD_ARG;
  return ts::double_quantize(values16, n, dq_group_size, codes, meta, recon16, S(stream));
}

int ts_rvq_residual(const ts_qinput* in, const ts_qlayer* stage1, const int32_t* outlier_idx,
                    const uint16_t* outlier_val, int64_t n_outliers, float* residual, void* stream) {
  if (!in || !stage1 || !residual || stage1->bits != 4) return TS_BAD_ARG;
  return ts::rvq_residual(in, stage1, outlier_idx, outlier_val, n_outliers, residual, S(stream));
}

int ts_sq_error_sums(const ts_qinput* in, const void* deq, int deq_dtype, double* sums2, void* stream) {
  if (!in || !deq || !sums2) return TS_BAD_ARG;
  return ts::sq_error_sums(in, deq, deq_dtype, sums2, S(stream));
}

int ts_gather_f16(const void* w, int w_dtype, const int64_t* idx, int64_t n, uint16_t* out, void* stream) {
  if (n > 0 && (!w || !idx || !out)) return TS_BAD_ARG;
  return ts::gather_f16(w, w_dtype, idx, n, out, S(stream));
}

}  // extern "C"
