/*
 * tensorshrink_hip.h - C ABI of libtensorshrink_hip.so, the MI355X (gfx950)
 * implementation of tensorshrink's GOAP quantized-linear path.
 *
 * All entry points are extern "C", take plain device pointers and sizes, run
 * on the caller's HIP stream, never synchronize the device, never allocate in
 * steady state and keep no hidden per-thread state. A status code is returned;
 * TS_NOT_COVERED mirrors the reference's "return None = not covered" contract
 * (triton_kernels.py:740-745), every other non-zero code is an error.
 *
 * Buffer formats are the reference's QuantLinear buffers (modules.py:337-464)
 * and QuantizedTensor fields (codec.py:102-151), byte for byte:
 *   packed          u8  [rows, padded_cols*bits/8]  2-bit: cols 4j..4j+3 at bits
 *                                                    0-1,2-3,4-5,6-7; 4-bit: col 2j
 *                                                    low nibble, 2j+1 high nibble
 *   scale, gmin     f16 [rows, n_groups]            (absent under double quant)
 *   dq_*_codes      u8  [n_super * dq_group_size]   flat row-major over [rows, n_groups]
 *   dq_*_meta       f16 [n_super, 2]                (meta_scale, meta_min)
 *   codebook        f32 [1 << bits]                 NF or Lloyd-Max grid, or NULL
 *   outlier_row/col i32 [n_outliers]                stable-sorted by row
 *   outlier_delta   f16 [n_outliers]                val - base dequant value
 *   stage2_*        RVQ (bits = 6) residual stage: 2-bit packed + f16 scale/gmin
 */
#ifndef TENSORSHRINK_HIP_H
#define TENSORSHRINK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  TS_OK = 0,
  TS_NOT_COVERED = 1, /* shape/format outside what the kernels cover */
  TS_BAD_ARG = 2,     /* inconsistent sizes or NULL where a buffer is required */
  TS_HIP_ERROR = 3,   /* a HIP runtime call or launch failed */
  TS_WORKSPACE = 4    /* workspace smaller than ts_*_workspace_bytes() asked for */
} ts_status;

typedef enum { TS_F16 = 0, TS_BF16 = 1, TS_F32 = 2 } ts_dtype;

/* Non-owning view of one quantized linear layer (QuantLinear's buffers). */
typedef struct {
  int32_t bits;        /* 2, 4, 8, or 6 (RVQ: 4-bit stage 1 + 2-bit stage 2) */
  int32_t group_size;
  int64_t rows;        /* out_features */
  int64_t cols;        /* in_features */
  int64_t padded_cols; /* cols rounded up to a multiple of group_size */
  int64_t n_groups;
  const uint8_t* packed;
  int64_t packed_stride; /* bytes per packed row */
  const uint16_t* scale; /* f16 [rows, n_groups]; NULL under double quant */
  const uint16_t* gmin;
  const uint8_t* dq_scale_codes; /* NULL unless double quant */
  const uint16_t* dq_scale_meta;
  const uint8_t* dq_gmin_codes;
  const uint16_t* dq_gmin_meta;
  int64_t dq_group_size; /* 0 unless double quant */
  const float* codebook; /* f32 [1 << bits] or NULL (uniform grid) */
  const int32_t* outlier_row;
  const int32_t* outlier_col;
  const uint16_t* outlier_delta; /* f16 */
  int64_t n_outliers;
  const int32_t* outlier_row_ptr; /* i32 [rows + 1] CSR offsets into the row-sorted
                                     outlier tables (ts_outlier_row_ptr builds it) */
  const uint8_t* stage2_packed;   /* RVQ only: u8 [rows, padded_cols/4] */
  int64_t stage2_stride;
  const uint16_t* stage2_scale;   /* RVQ only: f16 [rows, n_groups] */
  const uint16_t* stage2_gmin;
  /* Outliers regrouped per 16-row tile for the decode kernel (derived from the
   * CSR tables by ts_build_tile_outliers; no counterpart in the reference):
   * tile t owns slots [t * tile_outlier_cap, (t + 1) * tile_outlier_cap), each
   * u64 = col | (row - 16 t) << 32 | f16 delta bits << 48; unused slots are 0.
   * NULL / 0 when the layer has no outliers, or to make the decode kernel read
   * the outliers through outlier_row_ptr instead (outliers crowded into a few
   * tiles, where every tile padded to the fullest one would be too large). */
  const uint64_t* tile_outliers;
  int64_t tile_outlier_cap;
  /* Optional host copy of `codebook` (no counterpart in the reference). With
   * at most 16 entries the decode kernel then takes the values as launch
   * arguments instead of reading them from device memory, where that read
   * would queue behind the layer's weight stream. NULL: read `codebook`. */
  const float* codebook_host;
  /* Outliers of each row in column order (derived from the row-sorted tables
   * by ts_build_colsorted_outliers; no counterpart in the reference): entry k
   * of row r's CSR range [outlier_row_ptr[r], outlier_row_ptr[r + 1]) is
   * col | f16 delta bits << 16, ascending in col. The prefill kernel walks a
   * row's outliers with it while it dequantizes the row; without it (and
   * with outliers) the forward above 16 rows runs the generic kernel. */
  const uint32_t* outlier_colsorted;
} ts_qlayer;

const char* ts_status_str(int status);

/* Library version string. */
const char* ts_version(void);

/* Bytes of device workspace ts_qlinear_forward uses for M activation rows:
 * 0 up to 16 rows (the decode kernel), else room for the dequantized layer
 * (rows x cols in the activation dtype) plus the GEMM library's workspace. */
size_t ts_forward_workspace_bytes(const ts_qlayer* layer, int64_t M);

/* Bytes of device workspace (16-byte aligned) with which ts_qlinear_forward's
 * fused prefill kernel splits K across workgroups for M activation rows: the
 * splits' fp32 partial sums, k_split x M x rows x 4 bytes, k_split <= 8. Not 0
 * only where the launch plan estimates a split faster: tiles that would leave
 * compute units idle (few rows or small M, e.g. 4096 x 14336 at M = 256), or
 * 256 x 256 tiles that fill them only when split (the same layer at M =
 * 2048). 0 where the decode kernel runs. Always below
 * ts_forward_workspace_bytes(layer, M), so a workspace of this size never
 * selects the GEMM library path. No counterpart in the reference (its Triton
 * kernels do not split K). */
size_t ts_forward_partials_bytes(const ts_qlayer* layer, int64_t M);

/*
 * y[M, rows] = x[M, cols] @ W^T + outliers (+ bias), fp32 accumulation, stored
 * in y_dtype. Replaces fused_quantized_linear (triton_kernels.py:714-945) and,
 * for large M, the dequantize_weight + outlier scatter + F.linear path
 * (modules.py:896-922): M <= 16 runs the HBM-bound decode kernel; M > 16
 * with a workspace of ts_forward_workspace_bytes(layer, M) bytes dequantizes
 * the layer into it and runs one hipBLASLt GEMM (bias in its epilogue);
 * otherwise the decode kernel on blocks of 16 tokens where that is the faster
 * kernel for the shape (M <= 32, or <= 24 when cols > 8192, on layers of at
 * most 4096 rows with codes of at most 6 bits), else the fused MFMA prefill
 * kernel, which splits K across workgroups when the workspace holds
 * ts_forward_partials_bytes(layer, M) bytes and that size is not 0 (layers
 * the prefill kernel does not take: the decode kernel in passes of 64 rows,
 * else a one-thread-per-output kernel). x_dtype is TS_BF16 or TS_F16; bias
 * (may be NULL) has x_dtype. ldx/ldy are row strides in elements. Calls that
 * share a workspace must be ordered on one stream.
 */
int ts_qlinear_forward(const ts_qlayer* layer, const void* x, int64_t M, int64_t ldx, int x_dtype,
                       void* y, int64_t ldy, int y_dtype, const void* bias,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * The forward above for n (1..4) layers that read the same x (q/k/v, gate/up)
 * in one launch: y[l][M, rows_l] = x @ W_l^T (+ bias[l]). Covers M <= 16, and
 * M <= 32 when the layers have at most 12288 rows in all (q/k/v; not the
 * taller gate/up, where per-layer prefill launches win), with layers of one
 * format (bits, group size, cols, codebook / double-quant / stage-2 kind);
 * returns TS_NOT_COVERED otherwise, and the caller runs
 * ts_qlinear_forward per layer. No counterpart in the reference, which calls
 * fused_quantized_linear once per QuantLinear (modules.py:896-905); this
 * replaces that sequence of calls for layers sharing an input. bias may be
 * NULL, as may any bias[l].
 */
int ts_qlinear_forward_group(const ts_qlayer* const* layers, int n_layers, const void* x, int64_t M, int64_t ldx,
                             int x_dtype, void* const* y, const int64_t* ldy, int y_dtype,
                             const void* const* bias, void* stream);

/*
 * out[m, row[k]] += x[m, col[k]] * delta[k] on an fp32 [M, ldo] buffer.
 * Replaces apply_outlier_correction (triton_kernels.py:948-991). Row-sorted
 * tables are reduced per row without atomics.
 */
int ts_apply_outlier_correction(float* out, int64_t M, int64_t ldo, const void* x, int64_t ldx, int x_dtype,
                                const int32_t* outlier_row_ptr, const int32_t* outlier_col,
                                const uint16_t* outlier_delta, int64_t rows, void* stream);

/*
 * Dense dequantization of a layer into w_out [rows, cols] (row stride ldw).
 * mode TS_DEQ_CODEC: the codec's dequantize_tensor (codec.py:761-807):
 *   float32 reconstruction, outliers overwritten with outlier_val, cast to
 *   out_dtype (round to nearest even). Needs outlier_idx/outlier_val (codec
 *   order, flat indices) passed separately.
 * mode TS_DEQ_QLINEAR: the QuantLinear view: outliers become base + delta.
 * Replaces dequantize_weight (triton_kernels.py:1114-1186).
 */
enum { TS_DEQ_CODEC = 0, TS_DEQ_QLINEAR = 1 };
int ts_dequantize(const ts_qlayer* layer, int mode, const int32_t* outlier_idx, const uint16_t* outlier_val,
                  int64_t n_outlier_idx, void* w_out, int64_t ldw, int out_dtype, void* stream);

/* CSR row offsets for row-sorted outlier tables: row_ptr[r] = first k with
 * outlier_row[k] >= r, for r in [0, rows]. */
int ts_outlier_row_ptr(const int32_t* outlier_row, int64_t n_outliers, int64_t rows, int32_t* row_ptr,
                       void* stream);

/*
 * Per-tile outlier slots (ts_qlayer.tile_outliers) from the row-sorted CSR
 * tables. ts_tile_outlier_max writes the largest outlier count of any 16-row
 * tile to *max_count (device int32); the caller picks cap >= that count and
 * allocates ceil(rows / 16) * cap slots for ts_build_tile_outliers. Lets the
 * decode kernel load a tile's outliers at a fixed address instead of through
 * the row offsets (a dependent load on its critical path).
 */
int ts_tile_outlier_max(const int32_t* outlier_row_ptr, int64_t rows, int32_t* max_count, void* stream);
int ts_build_tile_outliers(const int32_t* outlier_row_ptr, const int32_t* outlier_row, const int32_t* outlier_col,
                           const uint16_t* outlier_delta, int64_t rows, int64_t cap, uint64_t* slots, void* stream);

/*
 * ts_build_outlier_tables with no workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc). No counterpart in the reference. The sort scratch is a
 * fixed 8 MiB device array inside the library (one per GPU, held until the
 * process ends): the call allocates nothing, and n_outliers is limited to
 * 262144 (TS_BAD_ARG above; the config-scale layers hold at most 234,881).
 * All calls on one GPU share that array, so calls that overlap on one GPU
 * (concurrent streams or host threads) race; order them on one stream.
 */
int ts_build_outlier_tables_noalloc(const ts_qlayer* layer, const int32_t* outlier_idx, const uint16_t* outlier_val,
                                    int64_t n_outliers, int32_t* outlier_row, int32_t* outlier_col,
                                    uint16_t* outlier_delta, int32_t* outlier_row_ptr, void* stream);

/* ts_qlayer.outlier_colsorted from the row-sorted CSR tables: each row's
 * entries (col | f16 delta << 16) sorted by column. out: u32 [n_outliers].
 * Needs every column below 65535. */
int ts_build_colsorted_outliers(const int32_t* outlier_row_ptr, const int32_t* outlier_col,
                                const uint16_t* outlier_delta, int64_t rows, uint32_t* out, void* stream);

/*
 * QuantLinear construction (modules.py:414-448, 649-715): from codec-order
 * outlier_idx/outlier_val, write outlier_row/col stable-sorted by row and
 * outlier_delta = f16(f32(val) - base), base = codeval * scale + gmin with the
 * float32 scale/gmin QuantLinear reconstructs. workspace: see
 * ts_outlier_tables_workspace_bytes.
 */
size_t ts_outlier_tables_workspace_bytes(int64_t n_outliers, int64_t rows);
int ts_build_outlier_tables(const ts_qlayer* layer, const int32_t* outlier_idx, const uint16_t* outlier_val,
                            int64_t n_outliers, int32_t* outlier_row, int32_t* outlier_col,
                            uint16_t* outlier_delta, int32_t* outlier_row_ptr, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * GOAP quantize (codec.py:453-675, gpu_quantize.py:52-166), split in phases so
 * the host can run the one sequential step (the exact top-k order) in between.
 *
 * Phase 1 ts_topk_candidates_count + _write: |w| as float32, a per-segment
 * histogram lower bound of the running k-th largest value, and compaction of
 * every position that can enter the top-k heap, in index order.
 * Phase 2 ts_topk_select (host, C++): replays libstdc++'s heap selection over
 * the candidates, giving torch.topk's CPU order (ties included).
 * Phase 3 ts_quantize_groups: clamp to [-t, t], per-(row, group) min/max,
 * scale, code assignment (uniform round / codebook midpoint search), packing.
 * Phase 4 ts_double_quantize: uint8 double quantization of f16 scale/gmin.
 */
typedef struct {
  const void* w;     /* [rows, cols] row-major, dtype w_dtype */
  int w_dtype;       /* TS_F16, TS_BF16 or TS_F32 */
  int64_t rows, cols;
} ts_qinput;

size_t ts_topk_workspace_bytes(int64_t n, int64_t k);
/* Histograms, segment bounds and per-chunk candidate counts into `workspace`;
 * synchronizes the stream and returns the candidate count in *n_candidates. */
int ts_topk_candidates_count(const ts_qinput* in, int64_t k, void* workspace, size_t workspace_bytes,
                             int64_t* n_candidates, void* stream);
/* Writes the candidates (flat index, |w| as float32) in index order into
 * device arrays of at least *n_candidates entries, reusing `workspace` from
 * the count call. */
int ts_topk_candidates_write(const ts_qinput* in, int64_t k, void* workspace, int64_t* cand_idx,
                             float* cand_val, void* stream);
/* Host: exact torch.topk (CPU, largest, sorted) order over a candidate stream
 * that starts with positions [0, k) and contains every position the heap
 * would admit; n = total element count. For k * 64 > n the stream must be the
 * whole array (nth_element regime). Host arrays. */
int ts_topk_select(const int64_t* cand_idx, const float* cand_val, int64_t n_candidates, int64_t n, int64_t k,
                   int64_t* out_idx, float* out_val);

typedef struct {
  int32_t bits;          /* 2, 4, 8 */
  int32_t group_size;
  float threshold;       /* clamp bound t (ignored when clamp == 0) */
  int32_t clamp;
  const float* codebook; /* sorted f32 code grid (device) or NULL (uniform round) */
  int32_t codebook_len;
} ts_group_opts;

/* Clamp to [-t, t], pad columns with the last one, per-(row, group) min/max,
 * scale = max((max - min) / (2^b - 1), 1e-8), codes (round half-even, or the
 * codebook midpoint search with ties to the lower code) and packing.
 * packed: u8 [rows, packed_stride]; scale16/gmin16: f16 [rows, n_groups];
 * scale32/gmin32 (optional, both or neither): the float32 values. */
int ts_quantize_groups(const ts_qinput* in, const ts_group_opts* opts, uint8_t* packed, int64_t packed_stride,
                       uint16_t* scale16, uint16_t* gmin16, float* scale32, float* gmin32, void* stream);

/* Normalized value (x - gmin) / scale at n flat positions of the padded
 * [rows, padded_cols] tensor: the Lloyd-Max fit sample (codec.py:327-331). */
int ts_lm_sample(const ts_qinput* in, const ts_group_opts* opts, const float* scale32, const float* gmin32,
                 const int64_t* idx, int64_t n, float* out, void* stream);

/* Host: Lloyd-Max fit (codec.py:320-361) over float32 samples with the
 * reference's arithmetic: init = linspace_init (n_levels values), `iters`
 * rounds of midpoint assignment and sequential float32 sums. Writes the
 * sorted centroids. Host arrays. */
int ts_lloyd_max_fit_host(const float* samples, int64_t m, const float* linspace_init, int32_t n_levels,
                          int32_t iters, float* out_centroids);

/* out[i] = f16(w[idx[i]]) (outlier values, codec.py:537). */
int ts_gather_f16(const void* w, int w_dtype, const int64_t* idx, int64_t n, uint16_t* out, void* stream);

/* Double quantization (codec.py:380-417) of an f16 array of n values:
 * codes u8 [n_super*dq_gs], meta f16 [n_super, 2], recon f16 [n] (the
 * f16-rounded reconstruction QuantizedTensor.scale/gmin carry). */
int ts_double_quantize(const uint16_t* values16, int64_t n, int64_t dq_group_size, uint8_t* codes,
                       uint16_t* meta, uint16_t* recon16, void* stream);

/* float32 residual w - dequant(stage 1) for RVQ (codec.py:703-707). */
int ts_rvq_residual(const ts_qinput* in, const ts_qlayer* stage1, const int32_t* outlier_idx,
                    const uint16_t* outlier_val, int64_t n_outliers, float* residual, void* stream);

/* sum((w - dequant)^2) and sum(w^2) in float64 for relative_error (codec.py:850-857). */
int ts_sq_error_sums(const ts_qinput* in, const void* deq, int deq_dtype, double* sums2, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TENSORSHRINK_HIP_H */
