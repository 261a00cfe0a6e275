// Dense dequantization, QuantLinear outlier tables and the standalone outlier
// correction. Everything here that the reference defines bit-for-bit
// (dequantize_tensor, _outlier_base_val, _compute_outlier_delta) keeps the
// reference's float32 operation order: separate multiply and add, no FMA
// contraction, round-to-nearest-even narrowing.
#include <cstring>

#include <rocprim/rocprim.hpp>

#include <mutex>

#include "ts_common.h"

namespace ts {

// Code value at (row, col) of a packed layer: the raw code or codebook[code]
// as float32 (modules.py:664-694, codec.py:775-788).
TS_DEV float code_value(const ts_qlayer& L, int64_t row, int64_t col) {
  const uint8_t* p = L.packed + row * L.packed_stride;
  uint32_t c;
  if (L.bits == 2) c = (p[col >> 2] >> (2 * (col & 3))) & 3u;
  else if (L.bits == 4 || L.bits == 6) c = (p[col >> 1] >> (4 * (col & 1))) & 15u;
  else c = p[col];
  if (L.codebook && L.bits != 6) return L.codebook[c];
  return (float)c;
}

// float32 scale/gmin of (row, group): DQ reconstruction codes*ms + mm
// (codec.py:420-435 / modules.py:573-579) or the f16 values.
TS_DEV void scale_gmin_f32(const ts_qlayer& L, int64_t row, int64_t g, float& s, float& gm) {
#pragma clang fp contract(off)
  const int64_t flat = row * L.n_groups + g;
  if (L.dq_scale_codes) {
    const int64_t sup = flat / L.dq_group_size;
    s = (float)L.dq_scale_codes[flat] * ts_h2f(L.dq_scale_meta[2 * sup]) + ts_h2f(L.dq_scale_meta[2 * sup + 1]);
    gm = (float)L.dq_gmin_codes[flat] * ts_h2f(L.dq_gmin_meta[2 * sup]) + ts_h2f(L.dq_gmin_meta[2 * sup + 1]);
  } else {
    s = ts_h2f(L.scale[flat]);
    gm = ts_h2f(L.gmin[flat]);
  }
}

TS_DEV float base_value(const ts_qlayer& L, int64_t row, int64_t col) {
#pragma clang fp contract(off)
  const int64_t g = col / L.group_size;
  float s, gm;
  scale_gmin_f32(L, row, g, s, gm);
  const float cv = code_value(L, row, col);
  return cv * s + gm;
}

// RVQ stage 2 value (codec.py:836-844): uniform 2-bit, f16 scale/gmin.
TS_DEV float stage2_value(const ts_qlayer& L, int64_t row, int64_t col) {
#pragma clang fp contract(off)
  const uint8_t* p = L.stage2_packed + row * L.stage2_stride;
  const float c = (float)((p[col >> 2] >> (2 * (col & 3))) & 3u);
  const int64_t flat = row * L.n_groups + col / L.group_size;
  return c * ts_h2f(L.stage2_scale[flat]) + ts_h2f(L.stage2_gmin[flat]);
}

TS_DEV void store_out(void* out, int64_t off, int dt, float v) {
  if (dt == TS_F32) reinterpret_cast<float*>(out)[off] = v;
  else if (dt == TS_BF16) reinterpret_cast<uint16_t*>(out)[off] = ts_f2bf(v);
  else reinterpret_cast<uint16_t*>(out)[off] = ts_f2h(v);
}

// Pass 1: every position gets cast(base (+ RVQ stage 2)).
__global__ void dequant_base_kernel(const ts_qlayer L, void* out, int64_t ldw, int dt) {
#pragma clang fp contract(off)
  const int64_t row = blockIdx.y;
  for (int64_t col = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; col < L.cols;
       col += (int64_t)gridDim.x * blockDim.x) {
    float v = base_value(L, row, col);
    if (L.bits == 6) v = v + stage2_value(L, row, col);
    store_out(out, row * ldw + col, dt, v);
  }
}

// Pass 1, vectorised: 8-column chunks (inside one group), the codes in one
// 2/4/8-byte load, scale/gmin once per chunk, one 16-byte store (two for
// f32). Same float32 operations as base_value / stage2_value, in the same
// order, so the output is bit-identical.
// Two floats -> packed (lo, hi) bf16 / f16, round to nearest even, the same
// bits as ts_f2bf / ts_f2h: bf16 through one v_cvt_pk_bf16_f32, with a NaN
// replaced by ts_f2bf's canonical 0x7fc0.
template <int DT>
TS_DEV uint32_t pack_pair(float a, float b) {
  if constexpr (DT == TS_BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {a, b};
    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    if (__builtin_isnan(a) || __builtin_isnan(b))
      r = (__builtin_isnan(a) ? 0x7fc0u : (r & 0xffffu)) | ((__builtin_isnan(b) ? 0x7fc0u : (r >> 16)) << 16);
    return r;
  } else {
    return (uint32_t)ts_f2h(a) | ((uint32_t)ts_f2h(b) << 16);
  }
}

// Index math of the vectorised pass in 32 bits (the host checks the sizes);
// group sizes are powers of two, the double-quant group size usually.
struct DqvGeom {
  uint32_t cpr;       // 8-column chunks per row
  uint32_t nchunks;   // rows x cpr
  uint32_t gshift;    // log2(group_size)
  uint32_t dqshift;   // log2(dq_group_size), or 0xff: divide
};

// Raw inputs of one 8-column chunk (inside one group: group sizes are
// multiples of 8). A lane loads all of its chunks before it stores any: the
// stores may alias the loads as far as the compiler knows, so loads written
// after a store stay after it, and a wave would then hold one chunk's loads
// in flight at a time.
struct DqChunk {
  uint32_t row, col0, flat;
  ts_u32x2 code;   // 8 codes: 8 bytes (8-bit), .x (4-bit), .x low half (2-bit)
  uint32_t sc, gc;  // DQ: u8 scale/gmin codes; otherwise f16 scale/gmin bits
  uint32_t ms, mg;  // DQ: (mult, offset) f16 pairs of the super-group
  uint32_t w2, s2, g2;  // RVQ stage 2: 8 2-bit codes, f16 scale/gmin bits
};

template <int BITS, bool DQ>
TS_DEV void dequant_chunk_load(const ts_qlayer& L, const DqvGeom& g, uint32_t ci, DqChunk& c) {
  c.row = ci / g.cpr;
  c.col0 = (ci - c.row * g.cpr) * 8u;
  c.flat = c.row * (uint32_t)L.n_groups + (c.col0 >> g.gshift);
  if constexpr (DQ) {  // scale_gmin_f32
    const uint32_t sup = g.dqshift != 0xffu ? c.flat >> g.dqshift : c.flat / (uint32_t)L.dq_group_size;
    c.ms = *reinterpret_cast<const uint32_t*>(L.dq_scale_meta + 2 * sup);
    c.mg = *reinterpret_cast<const uint32_t*>(L.dq_gmin_meta + 2 * sup);
    c.sc = L.dq_scale_codes[c.flat];
    c.gc = L.dq_gmin_codes[c.flat];
  } else {
    c.sc = L.scale[c.flat];
    c.gc = L.gmin[c.flat];
  }
  const uint8_t* p = L.packed + (int64_t)c.row * L.packed_stride;
  if constexpr (BITS == 8) c.code = ts_ld8(p + c.col0);
  else if constexpr (BITS == 2) c.code.x = *reinterpret_cast<const uint16_t*>(p + c.col0 / 4);
  else c.code.x = ts_ld4(p + c.col0 / 2);  // 4-bit codes (and the 4-bit stage 1 of 6-bit RVQ)
  if constexpr (BITS == 6) {
    c.w2 = *reinterpret_cast<const uint16_t*>(L.stage2_packed + (int64_t)c.row * L.stage2_stride + c.col0 / 4);
    c.s2 = L.stage2_scale[c.flat];
    c.g2 = L.stage2_gmin[c.flat];
  }
}

template <int BITS, int DT, bool DQ>
TS_DEV void dequant_chunk_store(const ts_qlayer& L, const float* cbs, bool use_cb, const DqChunk& c, void* out,
                                int64_t ldw) {
#pragma clang fp contract(off)
  float s, gm;
  if constexpr (DQ) {
    s = (float)c.sc * ts_h2f((uint16_t)c.ms) + ts_h2f((uint16_t)(c.ms >> 16));
    gm = (float)c.gc * ts_h2f((uint16_t)c.mg) + ts_h2f((uint16_t)(c.mg >> 16));
  } else {
    s = ts_h2f((uint16_t)c.sc);
    gm = ts_h2f((uint16_t)c.gc);
  }
  uint32_t k[8];
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = ((i < 4 ? c.code.x : c.code.y) >> (8 * (i & 3))) & 0xffu;
  } else if constexpr (BITS == 2) {
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = (c.code.x >> (2 * i)) & 3u;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = (c.code.x >> (4 * i)) & 15u;
  }
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float cv = use_cb ? cbs[k[i]] : (float)k[i];
    v[i] = cv * s + gm;
  }
  if constexpr (BITS == 6) {
    const float s2 = ts_h2f((uint16_t)c.s2), g2 = ts_h2f((uint16_t)c.g2);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] + ((float)((c.w2 >> (2 * i)) & 3u) * s2 + g2);
  }
  const int64_t off = (int64_t)c.row * ldw + c.col0;
  if (c.col0 + 8u <= (uint32_t)L.cols) {
    if constexpr (DT == TS_F32) {
      float* o = reinterpret_cast<float*>(out) + off;
      *reinterpret_cast<ts_f32x4*>(o) = ts_f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<ts_f32x4*>(o + 4) = ts_f32x4{v[4], v[5], v[6], v[7]};
    } else {
      *reinterpret_cast<ts_u32x4*>(reinterpret_cast<uint16_t*>(out) + off) =
          ts_u32x4{pack_pair<DT>(v[0], v[1]), pack_pair<DT>(v[2], v[3]), pack_pair<DT>(v[4], v[5]),
                   pack_pair<DT>(v[6], v[7])};
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (c.col0 + i < (uint32_t)L.cols) store_out(out, off + i, DT, v[i]);
  }
}

// BITS: 2, 4, 8, or 6 (4-bit stage 1 + 2-bit stage 2). Each wave covers 256
// consecutive 8-column chunks, lane l taking chunks l, l + 64, l + 128,
// l + 192: every load and store instruction of a wave then covers one
// contiguous span (1 KB of bf16 output per store). Chunks past the end load
// the last chunk's inputs (in bounds) and store nothing.
template <int BITS, int DT, bool DQ>
__global__ __launch_bounds__(256) void dequant_vec_kernel(const ts_qlayer L, void* out, int64_t ldw, DqvGeom g) {
  __shared__ float cbs[256];
  const uint32_t base = (blockIdx.x * 4u + (threadIdx.x >> 6)) * 256u + (threadIdx.x & 63u);
  DqChunk c[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) dequant_chunk_load<BITS, DQ>(L, g, min(base + 64u * j, g.nchunks - 1u), c[j]);
  // the codebook after the chunk loads, so that they are in flight while it
  // arrives; the barrier waits for LDS only, not for the chunk loads
  const float* cb = L.codebook;
  const bool use_cb = cb != nullptr && BITS != 6;
  if (use_cb) {
    for (int i = threadIdx.x; i < (1 << (BITS == 6 ? 4 : BITS)); i += blockDim.x) cbs[i] = cb[i];
  }
  ts_lds_barrier();
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j)
    if (base + 64u * j < g.nchunks) dequant_chunk_store<BITS, DT, DQ>(L, cbs, use_cb, c[j], out, ldw);
}

template <int BITS, bool DQ>
void launch_dequant_vec_dt(const ts_qlayer& L, void* out, int64_t ldw, int dt, const DqvGeom& g, dim3 grid,
                           hipStream_t st) {
  if (dt == TS_F32) hipLaunchKernelGGL((dequant_vec_kernel<BITS, TS_F32, DQ>), grid, dim3(256), 0, st, L, out, ldw, g);
  else if (dt == TS_BF16) hipLaunchKernelGGL((dequant_vec_kernel<BITS, TS_BF16, DQ>), grid, dim3(256), 0, st, L, out, ldw, g);
  else hipLaunchKernelGGL((dequant_vec_kernel<BITS, TS_F16, DQ>), grid, dim3(256), 0, st, L, out, ldw, g);
}

template <int BITS>
void launch_dequant_vec(const ts_qlayer& L, void* out, int64_t ldw, int dt, hipStream_t st) {
  DqvGeom g;
  g.cpr = (uint32_t)ts_cdiv(L.cols, 8);
  g.nchunks = (uint32_t)(L.rows * g.cpr);
  g.gshift = (uint32_t)__builtin_ctzll((unsigned long long)L.group_size);
  const int64_t dqgs = L.dq_group_size;
  g.dqshift = (dqgs > 0 && (dqgs & (dqgs - 1)) == 0) ? (uint32_t)__builtin_ctzll((unsigned long long)dqgs) : 0xffu;
  const dim3 grid((unsigned)ts_cdiv(g.nchunks, 1024));
  if (L.dq_scale_codes) launch_dequant_vec_dt<BITS, true>(L, out, ldw, dt, g, grid, st);
  else launch_dequant_vec_dt<BITS, false>(L, out, ldw, dt, g, grid, st);
}

// Pass 2, codec view (codec.py:793-796, 823-846): the outlier position takes
// f32(outlier_val) (+ RVQ stage 2), then the cast.
__global__ void dequant_outlier_codec_kernel(const ts_qlayer L, void* out, int64_t ldw, int dt, const int32_t* idx,
                                             const uint16_t* val, int64_t n) {
#pragma clang fp contract(off)
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  const int64_t f = idx[o];
  const int64_t r = f / L.cols, c = f % L.cols;
  float v = ts_h2f(val[o]);
  if (L.bits == 6) v = v + stage2_value(L, r, c);
  store_out(out, r * ldw + c, dt, v);
}

// Pass 2, QuantLinear view (modules.py:786-802 in float32): base + delta.
__global__ void dequant_outlier_qlinear_kernel(const ts_qlayer L, void* out, int64_t ldw, int dt) {
#pragma clang fp contract(off)
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= L.n_outliers) return;
  const int64_t r = L.outlier_row[o], c = L.outlier_col[o];
  float v = base_value(L, r, c) + ts_h2f(L.outlier_delta[o]);
  if (L.bits == 6) v = v + stage2_value(L, r, c);
  store_out(out, r * ldw + c, dt, v);
}

// row_ptr[r] = first k with row[k] >= r (lower bound), r in [0, rows].
__global__ void row_ptr_kernel(const int32_t* row, int64_t n, int64_t rows, int32_t* row_ptr) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r > rows) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (row[mid] < r) lo = mid + 1;
    else hi = mid;
  }
  row_ptr[r] = (int32_t)lo;
}

__global__ void split_idx_kernel(const int32_t* idx, int64_t n, int64_t cols, uint32_t* key, uint32_t* pos) {
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  key[o] = (uint32_t)((int64_t)idx[o] / cols);
  pos[o] = (uint32_t)o;
}

// Sorted position o <- codec position perm[o]; delta per modules.py:700-715.
__global__ void outlier_delta_kernel(const ts_qlayer L, const int32_t* idx, const uint16_t* val,
                                     const uint32_t* perm, int64_t n, int32_t* orow, int32_t* ocol,
                                     uint16_t* odelta) {
#pragma clang fp contract(off)
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  const int64_t src = perm[o];
  const int64_t f = idx[src];
  const int64_t r = f / L.cols;
  const int64_t c = f % L.cols;
  orow[o] = (int32_t)r;
  ocol[o] = (int32_t)c;
  const float base = base_value(L, r, c);
  odelta[o] = ts_f2h(ts_h2f(val[src]) - base);
}

// out[m, r] += sum over the row's outliers of x[m, col] * delta (row-sorted
// CSR; one thread per (m, row), no atomics).
template <bool BF16>
__global__ void outlier_correction_kernel(float* out, int64_t M, int64_t ldo, const uint16_t* x, int64_t ldx,
                                          const int32_t* row_ptr, const int32_t* col, const uint16_t* delta,
                                          int64_t rows) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t m = blockIdx.y;
  if (r >= rows || m >= M) return;
  const int32_t o0 = row_ptr[r], o1 = row_ptr[r + 1];
  if (o0 == o1) return;
  float acc = 0.f;
  for (int32_t o = o0; o < o1; ++o) acc += XT<BF16>::to_f(x[m * ldx + col[o]]) * ts_h2f(delta[o]);
  out[m * ldo + r] += acc;
}

int dequantize(const ts_qlayer* Lp, int mode, const int32_t* oidx, const uint16_t* oval, int64_t n_oidx,
               void* w_out, int64_t ldw, int dt, hipStream_t st) {
  const ts_qlayer& L = *Lp;
  // 16-byte stores need 16-byte aligned rows; the 8-column chunks need group
  // sizes that are multiples of 8 and code rows whose loads stay aligned
  const int esz = dt == TS_F32 ? 4 : 2;
  // code loads of 8 columns: 2 (2-bit), 4 (4-bit) or 8 (8-bit) bytes, so rows
  // and bases aligned to 8 (2 for the 2-bit stage-2 plane); 32-bit index
  // math; power-of-two group size; (scale, min) meta pairs read as one
  // 4-byte word
  const bool vec = (ldw * esz) % 16 == 0 && (reinterpret_cast<uintptr_t>(w_out) & 15) == 0 &&
                   L.rows * L.n_groups < ((int64_t)1 << 31) && L.rows * ts_cdiv(L.cols, 8) < ((int64_t)1 << 31) &&
                   (L.group_size & (L.group_size - 1)) == 0 &&
                   (!L.dq_scale_codes || ((reinterpret_cast<uintptr_t>(L.dq_scale_meta) & 3) == 0 &&
                                          (reinterpret_cast<uintptr_t>(L.dq_gmin_meta) & 3) == 0)) &&
                   L.group_size % 8 == 0 && (L.packed_stride % 8) == 0 &&
                   (reinterpret_cast<uintptr_t>(L.packed) & 7) == 0 &&
                   (L.bits != 6 || ((L.stage2_stride % 2) == 0 && (reinterpret_cast<uintptr_t>(L.stage2_packed) & 1) == 0));
  if (vec) {
    if (L.bits == 2) launch_dequant_vec<2>(L, w_out, ldw, dt, st);
    else if (L.bits == 4) launch_dequant_vec<4>(L, w_out, ldw, dt, st);
    else if (L.bits == 6) launch_dequant_vec<6>(L, w_out, ldw, dt, st);
    else launch_dequant_vec<8>(L, w_out, ldw, dt, st);
  } else {
    dim3 grid((unsigned)std::min<int64_t>(ts_cdiv(L.cols, 256), 64), (unsigned)L.rows);
    hipLaunchKernelGGL(dequant_base_kernel, grid, dim3(256), 0, st, L, w_out, ldw, dt);
  }
  TS_CHECK_LAUNCH();
  if (mode == TS_DEQ_CODEC && n_oidx > 0) {
    hipLaunchKernelGGL(dequant_outlier_codec_kernel, dim3((unsigned)ts_cdiv(n_oidx, 256)), dim3(256), 0, st, L,
                       w_out, ldw, dt, oidx, oval, n_oidx);
    TS_CHECK_LAUNCH();
  } else if (mode == TS_DEQ_QLINEAR && L.n_outliers > 0) {
    hipLaunchKernelGGL(dequant_outlier_qlinear_kernel, dim3((unsigned)ts_cdiv(L.n_outliers, 256)), dim3(256), 0,
                       st, L, w_out, ldw, dt);
    TS_CHECK_LAUNCH();
  }
  return TS_OK;
}

int outlier_row_ptr(const int32_t* row, int64_t n, int64_t rows, int32_t* row_ptr, hipStream_t st) {
  hipLaunchKernelGGL(row_ptr_kernel, dim3((unsigned)ts_cdiv(rows + 1, 256)), dim3(256), 0, st, row, n, rows,
                     row_ptr);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

size_t outlier_tables_ws(int64_t n) {
  size_t sort_bytes = 0;
  (void)rocprim::radix_sort_pairs(nullptr, sort_bytes, (uint32_t*)nullptr, (uint32_t*)nullptr,
                                                (uint32_t*)nullptr, (uint32_t*)nullptr, (size_t)n, 0, 32);
  const size_t arr = ((size_t)n * 4 + 255) / 256 * 256;
  return 4 * arr + (sort_bytes + 255) / 256 * 256 + 256;
}

int build_outlier_tables(const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n, int32_t* orow,
                         int32_t* ocol, uint16_t* odelta, int32_t* row_ptr, void* ws, size_t ws_bytes,
                         hipStream_t st) {
  if (n == 0) {
    if (row_ptr) return outlier_row_ptr(orow, 0, L->rows, row_ptr, st);
    return TS_OK;
  }
  if (ws_bytes < outlier_tables_ws(n)) return TS_WORKSPACE;
  const size_t arr = ((size_t)n * 4 + 255) / 256 * 256;
  char* p = static_cast<char*>(ws);
  uint32_t* key_in = reinterpret_cast<uint32_t*>(p);
  uint32_t* key_out = reinterpret_cast<uint32_t*>(p + arr);
  uint32_t* pos_in = reinterpret_cast<uint32_t*>(p + 2 * arr);
  uint32_t* pos_out = reinterpret_cast<uint32_t*>(p + 3 * arr);
  void* tmp = p + 4 * arr;
  size_t tmp_bytes = ws_bytes - 4 * arr;
  hipLaunchKernelGGL(split_idx_kernel, dim3((unsigned)ts_cdiv(n, 256)), dim3(256), 0, st, idx, n, L->cols, key_in,
                     pos_in);
  TS_CHECK_LAUNCH();
  int end_bit = 1;
  while (end_bit < 32 && ((int64_t)1 << end_bit) <= L->rows) ++end_bit;
  // LSD radix sort is stable: equal rows keep codec (top-k) order, as
  // np.argsort(kind="stable") does in modules.py:422.
  if (rocprim::radix_sort_pairs(tmp, tmp_bytes, key_in, key_out, pos_in, pos_out, (size_t)n, 0, end_bit, st) !=
      hipSuccess)
    return TS_HIP_ERROR;
  hipLaunchKernelGGL(outlier_delta_kernel, dim3((unsigned)ts_cdiv(n, 256)), dim3(256), 0, st, *L, idx, val,
                     pos_out, n, orow, ocol, odelta);
  TS_CHECK_LAUNCH();
  if (row_ptr) return outlier_row_ptr(orow, n, L->rows, row_ptr, st);
  return TS_OK;
}

// ---------------------------------------------------------------------------
// ts_build_outlier_tables without a caller workspace: the sort scratch is a
// fixed device array, so the call allocates nothing (for callers that cannot
// call hipMalloc: graph capture, serving loops). Host code reaches the array
// only through the address hipGetSymbolAddress returns for the current
// device (each device holds its own copy); the array's name is a host-side
// stand-in that is never passed to a kernel or copy. Every call on one device
// shares the array, so calls that overlap on one device race; the sort writes
// every scratch byte it reads, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(8) << 20;
constexpr int64_t NOALLOC_MAX_OUTLIERS = 262144;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
void* g_scratch[MAX_DEVICES];
int g_scratch_rc[MAX_DEVICES];
std::once_flag g_scratch_once[MAX_DEVICES];

// Device address of `scratch` on the current device, looked up once per device.
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return TS_HIP_ERROR;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess && p ? TS_OK : TS_HIP_ERROR;
    g_scratch[dev] = p;
  });
  *out = g_scratch[dev];
  return g_scratch_rc[dev];
}
}  // namespace

int build_outlier_tables_noalloc(const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n,
                                 int32_t* orow, int32_t* ocol, uint16_t* odelta, int32_t* row_ptr, hipStream_t st) {
  if (n > NOALLOC_MAX_OUTLIERS) return TS_BAD_ARG;
  const size_t need = n > 0 ? outlier_tables_ws(n) : 0;
  if (need > NOALLOC_SCRATCH_BYTES) return TS_WORKSPACE;
  void* p = nullptr;
  const int rc = scratch_address(&p);
  if (rc != TS_OK) return rc;
  return build_outlier_tables(L, idx, val, n, orow, ocol, odelta, row_ptr, p, NOALLOC_SCRATCH_BYTES, st);
}

// Largest outlier count over 16-row tiles: one workgroup, strided over tiles.
__global__ __launch_bounds__(1024) void tile_max_kernel(const int32_t* __restrict__ rp, int64_t rows,
                                                        int32_t* __restrict__ out) {
  __shared__ int32_t part[1024];
  const int64_t n_tiles = ts_cdiv(rows, 16);
  int32_t best = 0;
  for (int64_t t = threadIdx.x; t < n_tiles; t += 1024) {
    const int32_t c = rp[std::min<int64_t>(16 * t + 16, rows)] - rp[16 * t];
    best = c > best ? c : best;
  }
  part[threadIdx.x] = best;
  __syncthreads();
  for (int s = 512; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s && part[threadIdx.x + s] > part[threadIdx.x]) part[threadIdx.x] = part[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = part[0];
}

// Slot i of tile t: outlier rp[16t] + i of the row-sorted tables, or 0.
__global__ __launch_bounds__(256) void tile_slots_kernel(const int32_t* __restrict__ rp, const int32_t* __restrict__ orow,
                                                         const int32_t* __restrict__ ocol,
                                                         const uint16_t* __restrict__ odelta, int64_t rows,
                                                         int64_t cap, uint64_t* __restrict__ slots) {
  const int64_t t = blockIdx.x;
  const int32_t k0 = rp[16 * t], k1 = rp[std::min<int64_t>(16 * t + 16, rows)];
  for (int64_t i = threadIdx.x; i < cap; i += 256) {
    const int64_t k = k0 + i;
    uint64_t v = 0;
    if (k < k1)
      v = (uint64_t)(uint32_t)ocol[k] | ((uint64_t)(uint32_t)(orow[k] - 16 * t) << 32) |
          ((uint64_t)odelta[k] << 48);
    slots[t * cap + i] = v;
  }
}

// One thread per row: the row's entries as col | delta << 16, insertion-sorted
// by column (rows hold a handful of outliers at the configured fractions).
__global__ __launch_bounds__(256) void colsorted_kernel(const int32_t* __restrict__ rp,
                                                        const int32_t* __restrict__ ocol,
                                                        const uint16_t* __restrict__ odelta, int64_t rows,
                                                        uint32_t* __restrict__ out) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int32_t k0 = rp[r], k1 = rp[r + 1];
  for (int32_t k = k0; k < k1; ++k) {
    const uint32_t e = ((uint32_t)ocol[k] & 0xffffu) | ((uint32_t)odelta[k] << 16);
    int32_t j = k;
    while (j > k0 && (out[j - 1] & 0xffffu) > (e & 0xffffu)) {
      out[j] = out[j - 1];
      --j;
    }
    out[j] = e;
  }
}

int build_colsorted_outliers(const int32_t* rp, const int32_t* ocol, const uint16_t* odelta, int64_t rows,
                             uint32_t* out, hipStream_t st) {
  if (rows <= 0) return TS_OK;
  hipLaunchKernelGGL(colsorted_kernel, dim3((unsigned)ts_cdiv(rows, 256)), dim3(256), 0, st, rp, ocol, odelta, rows,
                     out);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

int tile_outlier_max(const int32_t* rp, int64_t rows, int32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(tile_max_kernel, dim3(1), dim3(1024), 0, st, rp, rows, out);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

int build_tile_outliers(const int32_t* rp, const int32_t* orow, const int32_t* ocol, const uint16_t* odelta,
                        int64_t rows, int64_t cap, uint64_t* slots, hipStream_t st) {
  hipLaunchKernelGGL(tile_slots_kernel, dim3((unsigned)ts_cdiv(rows, 16)), dim3(256), 0, st, rp, orow, ocol, odelta,
                     rows, cap, slots);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

int apply_outlier_correction(float* out, int64_t M, int64_t ldo, const void* x, int64_t ldx, int xdt,
                             const int32_t* row_ptr, const int32_t* col, const uint16_t* delta, int64_t rows,
                             hipStream_t st) {
  if (M <= 0 || rows <= 0) return TS_OK;
  dim3 grid((unsigned)ts_cdiv(rows, 256), (unsigned)M);
  if (xdt == TS_BF16)
    hipLaunchKernelGGL(outlier_correction_kernel<true>, grid, dim3(256), 0, st, out, M, ldo,
                       static_cast<const uint16_t*>(x), ldx, row_ptr, col, delta, rows);
  else
    hipLaunchKernelGGL(outlier_correction_kernel<false>, grid, dim3(256), 0, st, out, M, ldo,
                       static_cast<const uint16_t*>(x), ldx, row_ptr, col, delta, rows);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

}  // namespace ts
