// Prefill entry point (the kernel is in ts_prefill.h) and the generic
// fallback kernel for shapes and formats the tiled kernels do not cover.
#include "ts_prefill.h"

namespace ts {

// y[m][n] = cast(sum_s part[s][m][n] + bias[n]); four outputs of a row per
// thread when N % 4 == 0 (16-byte partial reads), else one.
template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int P, int64_t M,
                                                            int64_t N, const uint16_t* __restrict__ bias, void* y,
                                                            int64_t ldy, int y_dtype) {
  constexpr int V = VEC ? 4 : 1;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (i >= M * N) return;
  const int64_t m = i / N, n = i - m * N;
  float v[V];
  if constexpr (VEC) {
    float4 t = *reinterpret_cast<const float4*>(part + i);
    for (int s = 1; s < P; ++s) {
      const float4 u = *reinterpret_cast<const float4*>(part + (int64_t)s * M * N + i);
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    float t = part[i];
    for (int s = 1; s < P; ++s) t += part[(int64_t)s * M * N + i];
    v[0] = t;
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (bias) v[j] += XT<BF16>::to_f(bias[n + j]);
    const int64_t off = m * ldy + n + j;
    if (y_dtype == TS_F32) reinterpret_cast<float*>(y)[off] = v[j];
    else reinterpret_cast<uint16_t*>(y)[off] = XT<BF16>::from_f(v[j]);
  }
}

int launch_splitk_reduce(const PrefillArgs& a, bool bf16, hipStream_t st) {
  const bool vec = a.N % 4 == 0;
  const int64_t threads = vec ? a.M * a.N / 4 : a.M * a.N;
  const dim3 grid((unsigned)ts_cdiv(threads, 256)), block(256);
  const uint16_t* b = a.bias;
  if (bf16) {
    if (vec) hipLaunchKernelGGL((splitk_reduce_kernel<true, true>), grid, block, 0, st, a.part, a.k_split, a.M, a.N, b, a.y, a.ldy, a.y_dtype);
    else hipLaunchKernelGGL((splitk_reduce_kernel<true, false>), grid, block, 0, st, a.part, a.k_split, a.M, a.N, b, a.y, a.ldy, a.y_dtype);
  } else {
    if (vec) hipLaunchKernelGGL((splitk_reduce_kernel<false, true>), grid, block, 0, st, a.part, a.k_split, a.M, a.N, b, a.y, a.ldy, a.y_dtype);
    else hipLaunchKernelGGL((splitk_reduce_kernel<false, false>), grid, block, 0, st, a.part, a.k_split, a.M, a.N, b, a.y, a.ldy, a.y_dtype);
  }
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// The launchers' (bits, codebook) template arguments for a layer: 6-bit
// (RVQ) layers run the 4-bit kernel without a codebook.
static int prefill_bits(const ts_qlayer* L) { return L->bits == 6 ? 4 : L->bits; }
static bool prefill_codebook(const ts_qlayer* L) { return L->bits != 6 && L->codebook != nullptr; }

size_t prefill_partials_bytes(const ts_qlayer* L, int64_t M) {
  if (M <= 16 || L->padded_cols % PF_BK != 0) return 0;
  return prefill_part_bytes(prefill_plan(M, L->rows, L->padded_cols, prefill_bits(L), prefill_codebook(L)), M, L->rows);
}

int prefill_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                    int64_t ldy, int y_dtype, const uint16_t* bias, void* ws, size_t ws_bytes, hipStream_t st) {
  if (L->padded_cols % PF_BK != 0) return TS_NOT_COVERED;
  const bool has_out = L->n_outliers > 0;
  // Outliers are walked per row in column order with 16-bit columns; the walk
  // stops at column 0xffff, which must lie past the last k-step's end.
  if (has_out && (L->outlier_colsorted == nullptr || L->outlier_row_ptr == nullptr ||
                  L->padded_cols + 2 * PF_BK > (int64_t)PF_NO_COL))
    return TS_NOT_COVERED;
  PrefillArgs a{};
  a.packed = L->packed;
  a.pstride = L->packed_stride;
  a.scale = L->scale;
  a.gmin = L->gmin;
  a.dqsc = L->dq_scale_codes;
  a.dqsm = L->dq_scale_meta;
  a.dqgc = L->dq_gmin_codes;
  a.dqgm = L->dq_gmin_meta;
  if (L->dq_scale_codes) {  // super-group index by shift
    const int64_t g = L->dq_group_size;
    if (g <= 0 || (g & (g - 1)) != 0) return TS_NOT_COVERED;
    while ((int64_t(1) << a.dq_shift) < g) ++a.dq_shift;
  }
  // table pointers the kernel reads unconditionally get a valid dummy
  const void* dummy = L->packed;
  a.codebook = L->codebook ? L->codebook : static_cast<const float*>(dummy);
  a.s2packed = L->stage2_packed;
  a.s2stride = L->stage2_stride;
  a.s2scale = L->stage2_scale;
  a.s2gmin = L->stage2_gmin;
  a.has_out = has_out ? 1 : 0;
  a.orow_ptr = has_out ? L->outlier_row_ptr : static_cast<const int32_t*>(dummy);
  a.ocs = has_out ? L->outlier_colsorted : static_cast<const uint32_t*>(dummy);
  a.ocs_bytes = has_out ? (uint32_t)(L->n_outliers * 4) : 4u;
  a.x = x;
  a.ldx = ldx;
  a.y = y;
  a.ldy = ldy;
  a.y_dtype = y_dtype;
  a.bias = bias;
  a.M = M;
  a.N = L->rows;
  a.K = L->padded_cols;
  a.cols = L->cols;
  a.n_groups = L->n_groups;
  // Extents of the buffers the kernel reads through 32-bit byte offsets.
  const int64_t stage1_bits = L->bits == 6 ? 4 : L->bits;
  const int64_t x_bytes = ((M - 1) * ldx + L->cols) * 2;
  const int64_t p_bytes = (L->rows - 1) * L->packed_stride + L->padded_cols * stage1_bits / 8;
  const int64_t meta = L->rows * L->n_groups;
  const int64_t dqm = L->dq_scale_codes ? ts_cdiv(meta, L->dq_group_size) * 4 : 0;
  const int64_t s2 = L->stage2_packed ? (L->rows - 1) * L->stage2_stride + L->padded_cols / 4 : 0;
  constexpr int64_t lim = int64_t(1) << 31;
  if (x_bytes >= lim || p_bytes >= lim || 2 * meta >= lim || dqm >= lim || s2 >= lim || 4 * L->n_outliers >= lim)
    return TS_NOT_COVERED;
  a.x_bytes = (uint32_t)x_bytes;
  a.p_bytes = (uint32_t)p_bytes;
  a.meta_elems = (uint32_t)meta;
  a.dqm_bytes = (uint32_t)dqm;
  a.s2_bytes = (uint32_t)s2;
  // K split when the plan asks for one and the workspace holds the partials;
  // else the best unsplit tile
  PrefillPlan plan = prefill_plan(M, L->rows, L->padded_cols, prefill_bits(L), prefill_codebook(L));
  const size_t pb = prefill_part_bytes(plan, M, L->rows);
  a.k_split = 1;
  a.part = nullptr;
  if (pb > 0 && ws && ws_bytes >= pb && (reinterpret_cast<uintptr_t>(ws) & 15) == 0) {
    a.k_split = plan.splits;
    a.part = static_cast<float*>(ws);
  } else if (plan.splits > 1) {
    plan = prefill_plan(M, L->rows, L->padded_cols, prefill_bits(L), prefill_codebook(L), false);
  }
  a.bm = plan.bm;
  a.bn = plan.bn;
  const bool bf16 = x_dtype == TS_BF16;
  switch (L->bits * 1000 + L->group_size) {
    case 2064: return prefill_b2_g64(L, a, bf16, st);
    case 2128: return prefill_b2_g128(L, a, bf16, st);
    case 2256: return prefill_b2_g256(L, a, bf16, st);
    case 4032: return prefill_b4_g32(L, a, bf16, st);
    case 4064: return prefill_b4_g64(L, a, bf16, st);
    case 4128: return prefill_b4_g128(L, a, bf16, st);
    case 4256: return prefill_b4_g256(L, a, bf16, st);
    case 6064: return prefill_b6_g64(L, a, bf16, st);
    case 6128: return prefill_b6_g128(L, a, bf16, st);
    case 8032: return prefill_b8_g32(L, a, bf16, st);
    case 8064: return prefill_b8_g64(L, a, bf16, st);
    case 8128: return prefill_b8_g128(L, a, bf16, st);
    default: return TS_NOT_COVERED;
  }
}

// ---------------------------------------------------------------------------
// Generic fallback for shapes the tiled kernels do not cover (odd group sizes,
// ragged columns): one thread per output, on-the-fly float32 dequant.
// ---------------------------------------------------------------------------
TS_DEV float g_value(const ts_qlayer& L, int64_t row, int64_t col) {
  const uint8_t* p = L.packed + row * L.packed_stride;
  uint32_t c;
  if (L.bits == 2) c = (p[col >> 2] >> (2 * (col & 3))) & 3u;
  else if (L.bits == 4 || L.bits == 6) c = (p[col >> 1] >> (4 * (col & 1))) & 15u;
  else c = p[col];
  const float cv = (L.codebook && L.bits != 6) ? L.codebook[c] : (float)c;
  const int64_t g = col / L.group_size;
  const int64_t flat = row * L.n_groups + g;
  float s, gm;
  if (L.dq_scale_codes) {
    const int64_t sup = flat / L.dq_group_size;
    s = (float)L.dq_scale_codes[flat] * ts_h2f(L.dq_scale_meta[2 * sup]) + ts_h2f(L.dq_scale_meta[2 * sup + 1]);
    gm = (float)L.dq_gmin_codes[flat] * ts_h2f(L.dq_gmin_meta[2 * sup]) + ts_h2f(L.dq_gmin_meta[2 * sup + 1]);
  } else {
    s = ts_h2f(L.scale[flat]);
    gm = ts_h2f(L.gmin[flat]);
  }
  float w = cv * s + gm;
  if (L.bits == 6) {
    const uint8_t* p2 = L.stage2_packed + row * L.stage2_stride;
    const float c2 = (float)((p2[col >> 2] >> (2 * (col & 3))) & 3u);
    w += c2 * ts_h2f(L.stage2_scale[flat]) + ts_h2f(L.stage2_gmin[flat]);
  }
  return w;
}

template <bool BF16>
__global__ void generic_kernel(const ts_qlayer L, const uint16_t* x, int64_t M, int64_t ldx, void* y, int64_t ldy,
                               int ydt, const uint16_t* bias) {
  const int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t m = blockIdx.y;
  if (n >= L.rows || m >= M) return;
  float acc = 0.f;
  for (int64_t k = 0; k < L.cols; ++k) acc += XT<BF16>::to_f(x[m * ldx + k]) * g_value(L, n, k);
  if (L.n_outliers > 0 && L.outlier_row_ptr) {
    for (int32_t o = L.outlier_row_ptr[n]; o < L.outlier_row_ptr[n + 1]; ++o)
      acc += XT<BF16>::to_f(x[m * ldx + L.outlier_col[o]]) * ts_h2f(L.outlier_delta[o]);
  }
  if (bias) acc += XT<BF16>::to_f(bias[n]);
  if (ydt == TS_F32) reinterpret_cast<float*>(y)[m * ldy + n] = acc;
  else reinterpret_cast<uint16_t*>(y)[m * ldy + n] = XT<BF16>::from_f(acc);
}

int generic_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                    int64_t ldy, int y_dtype, const uint16_t* bias, hipStream_t st) {
  dim3 grid((unsigned)ts_cdiv(L->rows, 256), (unsigned)M);
  if (x_dtype == TS_BF16)
    hipLaunchKernelGGL(generic_kernel<true>, grid, dim3(256), 0, st, *L, x, M, ldx, y, ldy, y_dtype, bias);
  else
    hipLaunchKernelGGL(generic_kernel<false>, grid, dim3(256), 0, st, *L, x, M, ldx, y, ldy, y_dtype, bias);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

}  // namespace ts
