// Prefill (M > 16) quantized linear on the matrix cores.
//
// Replaces the reference's large-M path: dequantize_weight into a dense
// compute-dtype W (triton_kernels.py:1114-1186), the outlier scatter onto W
// (modules.py:912-919) and F.linear (modules.py:920). Here W never exists in
// HBM: each workgroup dequantizes its BN x 64 weight tile straight into LDS
// as bf16/f16, folds that tile's outliers into it (w = cast(f32(w) + delta),
// as modules.py:918 does on the dense W), and feeds MFMA f32_32x32x16 with
// fp32 accumulation.
//
// Tile: BM x BN x 64 per workgroup of 4 waves (2 x 2), each wave
// (BM/2) x (BN/2) as (BM/64) x (BN/64) MFMA 32x32 blocks. x and W tiles are
// double-buffered in LDS with a 16-byte-chunk XOR swizzle (chunk c of row r
// stored at c ^ (r & 7)) so the MFMA operand reads and the tile writes are
// both bank-conflict free. One barrier per k-step.
#include "ts_common.h"

namespace ts {

struct PrefillArgs {
  const uint8_t* packed;
  int64_t pstride;
  const uint16_t* scale;
  const uint16_t* gmin;
  const uint8_t* dqsc;
  const uint16_t* dqsm;
  const uint8_t* dqgc;
  const uint16_t* dqgm;
  uint32_t dq_gs;
  const float* codebook;
  const uint8_t* s2packed;
  int64_t s2stride;
  const uint16_t* s2scale;
  const uint16_t* s2gmin;
  const int32_t* orow_ptr;
  const int32_t* ocol;
  const uint16_t* odelta;
  const uint16_t* x;
  int64_t ldx;
  void* y;
  int64_t ldy;
  int y_dtype;
  const uint16_t* bias;
  int64_t M, N, K;  // K = padded_cols (multiple of 64)
  int64_t cols;
  int64_t n_groups;
  int64_t m_tiles, n_tiles;
};

constexpr int BK = 64;

typedef __bf16 ts_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 ts_f16x2 __attribute__((ext_vector_type(2)));
typedef float ts_f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed (lo, hi) bf16/f16 pair, round to nearest even
// (v_cvt_pk_bf16_f32 on gfx950).
template <bool BF16>
TS_DEV uint32_t to_pair(float lo, float hi) {
  const ts_f32x2 v = {lo, hi};
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ts_bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ts_f16x2));
}

TS_DEV void pf_scale_gmin(const PrefillArgs& a, int64_t row, int64_t g, float& s, float& gm) {
  const int64_t flat = row * a.n_groups + g;
  if (a.dqsc) {
    const uint32_t sup = (uint32_t)flat / a.dq_gs;
    s = __fadd_rn(__fmul_rn((float)a.dqsc[flat], ts_h2f(a.dqsm[2 * sup])), ts_h2f(a.dqsm[2 * sup + 1]));
    gm = __fadd_rn(__fmul_rn((float)a.dqgc[flat], ts_h2f(a.dqgm[2 * sup])), ts_h2f(a.dqgm[2 * sup + 1]));
  } else {
    s = ts_h2f(a.scale[flat]);
    gm = ts_h2f(a.gmin[flat]);
  }
}

// LDS offset (in uint16 elements) of 16-byte chunk c of row r in a [rows][64] tile.
TS_DEV int swz(int r, int c) { return r * BK + ((c ^ (r & 7)) << 3); }

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, int BM, int BN>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int A_CHUNKS = BM * 8 / 256;          // 16-byte x chunks per thread per k-step
  constexpr int CPT = BN * BK / 256;              // weight codes per thread per k-step
  constexpr int TPR = BK / CPT;                   // threads per weight row
  constexpr int WB = CPT * BITS / 8;              // packed bytes per thread per k-step
  constexpr int WB2 = CPT / 4;                    // RVQ stage-2 bytes
  constexpr int CBN = (CB && BITS == 8) ? 256 : 16;
  constexpr int OMAX = 8;                         // outliers per row staged in LDS
  static_assert(CPT % 32 == 0 || CPT == 16, "weight chunk");
  static_assert(WB % 4 == 0, "packed chunk");
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* As = reinterpret_cast<uint16_t*>(smem);             // [2][BM][64]
  uint16_t* Bs = As + 2 * BM * BK;                              // [2][BN][64]
  float* cbs = reinterpret_cast<float*>(Bs + 2 * BN * BK);      // codebook
  int32_t* ocs = reinterpret_cast<int32_t*>(cbs + CBN);         // [BN][OMAX] outlier columns of each tile row
  float* ods = reinterpret_cast<float*>(ocs + BN * OMAX);       // [BN][OMAX] outlier deltas

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-aware tile order: consecutive workgroups go to different XCDs, so map
  // blockIdx so that the 8 workgroups sharing an XCD walk down one column of
  // M tiles of the same weight tile (W bytes then hit that XCD's L2).
  const int64_t nblk = a.m_tiles * a.n_tiles;
  int64_t bid = blockIdx.x;
  {
    const int64_t per_xcd = nblk / 8;
    if (per_xcd * 8 == nblk) bid = (bid % 8) * per_xcd + bid / 8;
  }
  const int64_t mt = bid % a.m_tiles, nt = bid / a.m_tiles;
  const int64_t m0 = mt * BM, n0 = nt * BN;

  if (CB) {
    for (int i = tid; i < CBN; i += 256) cbs[i] = a.codebook[i];
  }

  // weight-row ownership for the dequant
  const int wr = tid / TPR;                 // row within the tile
  const int wpart = tid % TPR;              // which CPT-code slice of the k-step
  const int64_t wrow = min(n0 + wr, a.N - 1);
  const uint8_t* wp = a.packed + wrow * a.pstride + (wpart * CPT * BITS) / 8;
  const uint8_t* wp2 = RVQ ? a.s2packed + wrow * a.s2stride + (wpart * CPT) / 4 : nullptr;
  const int32_t o_begin = a.orow_ptr ? a.orow_ptr[wrow] : 0;
  const int32_t o_end = (a.orow_ptr && n0 + wr < a.N) ? a.orow_ptr[wrow + 1] : o_begin;
  const int o_cnt = (int)(o_end - o_begin);
  if (wpart == 0) {
    for (int i = 0; i < OMAX && i < o_cnt; ++i) {
      ocs[wr * OMAX + i] = a.ocol[o_begin + i];
      ods[wr * OMAX + i] = ts_h2f(a.odelta[o_begin + i]);
    }
  }

  ts_u32x4 areg[A_CHUNKS];
  uint32_t wreg[WB / 4];
  uint32_t wreg2[RVQ ? (WB2 + 3) / 4 : 1];
  float sreg[CPT / 32 > 0 ? CPT / 32 : 1][4];

  auto gload = [&](int64_t kt) {
    const int64_t k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int ch = tid + i * 256;
      const int r = ch >> 3, c = ch & 7;
      const int64_t m = m0 + r;
      const int64_t col = k0 + c * 8;
      areg[i] = (m < a.M && col < a.cols) ? ts_ld16(a.x + m * a.ldx + col) : ts_u32x4{0u, 0u, 0u, 0u};
    }
    const uint8_t* p = wp + (k0 * BITS) / 8;
    if constexpr (WB % 16 == 0) {
#pragma unroll
      for (int i = 0; i < WB / 16; ++i) {
        const ts_u32x4 v = ts_ld16(p + 16 * i);
        wreg[4 * i] = v.x; wreg[4 * i + 1] = v.y; wreg[4 * i + 2] = v.z; wreg[4 * i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < WB / 4; ++i) wreg[i] = ts_ld4(p + 4 * i);
    }
    if constexpr (RVQ) {
      const uint8_t* p2 = wp2 + k0 / 4;
#pragma unroll
      for (int i = 0; i < (WB2 + 3) / 4; ++i) wreg2[i] = (WB2 >= 4) ? ts_ld4(p2 + 4 * i) : *(const uint16_t*)(p2);
    }
    // one (scale, gmin) per 32-code sub-chunk (GS is a multiple of 32)
#pragma unroll
    for (int sc = 0; sc < (CPT >= 32 ? CPT / 32 : 1); ++sc) {
      const int64_t g = (k0 + wpart * CPT + sc * 32) / GS;
      pf_scale_gmin(a, wrow, g, sreg[sc][0], sreg[sc][1]);
      if constexpr (RVQ) {
        sreg[sc][2] = ts_h2f(a.s2scale[wrow * a.n_groups + g]);
        sreg[sc][3] = ts_h2f(a.s2gmin[wrow * a.n_groups + g]);
      }
    }
  };

  auto lstore = [&](int buf, int64_t kt) {
    uint16_t* Ab = As + buf * BM * BK;
    uint16_t* Bb = Bs + buf * BN * BK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int ch = tid + i * 256;
      const int r = ch >> 3, c = ch & 7;
      *reinterpret_cast<ts_u32x4*>(Ab + swz(r, c)) = areg[i];
    }
    // dequantize CPT codes of row wr, 8 at a time (one 16-byte chunk)
#pragma unroll
    for (int c8 = 0; c8 < CPT / 8; ++c8) {
      const int sc = CPT >= 32 ? (c8 * 8) / 32 : 0;
      const float s = sreg[sc][0], gm = sreg[sc][1];
      float cv[8];
      if constexpr (BITS == 4) {
        // one dword = 8 codes; spread even/odd nibbles into bytes
        const uint32_t d = wreg[c8];
        if constexpr (CB) {
          const uint32_t lo = (d << 2) & 0x3c3c3c3cu, hi = (d >> 2) & 0x3c3c3c3cu;  // 4*code per byte
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            cv[2 * e] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(cbs) + ((lo >> (8 * e)) & 0xffu));
            cv[2 * e + 1] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(cbs) + ((hi >> (8 * e)) & 0xffu));
          }
        } else {
          const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            cv[2 * e] = (float)((lo >> (8 * e)) & 0xffu);
            cv[2 * e + 1] = (float)((hi >> (8 * e)) & 0xffu);
          }
        }
      } else if constexpr (BITS == 2) {
        const uint32_t d = wreg[c8 >> 1] >> (16 * (c8 & 1));  // 8 codes in 16 bits
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t c = (d >> (2 * e)) & 3u;
          cv[e] = CB ? cbs[c] : (float)c;
        }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t d = wreg[2 * c8 + h];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t c = (d >> (8 * e)) & 0xffu;
            cv[4 * h + e] = CB ? cbs[c] : (float)c;
          }
        }
      }
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(cv[e], s, gm);
      if constexpr (RVQ) {
        const float s2 = sreg[sc][2], g2 = sreg[sc][3];
        const uint32_t d2 = wreg2[c8 >> 1] >> (16 * (c8 & 1));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += __builtin_fmaf((float)((d2 >> (2 * e)) & 3u), s2, g2);
      }
      ts_u32x4 pk;
      pk.x = to_pair<BF16>(v[0], v[1]);
      pk.y = to_pair<BF16>(v[2], v[3]);
      pk.z = to_pair<BF16>(v[4], v[5]);
      pk.w = to_pair<BF16>(v[6], v[7]);
      const int chunk = (wpart * CPT) / 8 + c8;
      *reinterpret_cast<ts_u32x4*>(Bb + swz(wr, chunk)) = pk;
    }
    // fold this row's outliers that land in the k-step into the tile
    if (o_cnt > 0) {
      const int64_t kc0 = kt * BK + wpart * CPT;
      const int nl = o_cnt < OMAX ? o_cnt : OMAX;
      for (int i = 0; i < o_cnt; ++i) {
        const int64_t col = i < nl ? ocs[wr * OMAX + i] : a.ocol[o_begin + i];
        if (col >= kc0 && col < kc0 + CPT) {
          const float dl = i < nl ? ods[wr * OMAX + i] : ts_h2f(a.odelta[o_begin + i]);
          const int kk = (int)(col - kt * BK);
          uint16_t* p = Bb + swz(wr, kk >> 3) + (kk & 7);
          *p = XT<BF16>::from_f(XT<BF16>::to_f(*p) + dl);
        }
      }
    }
  };

  ts_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = ts_f32x16{};

  const int64_t KT = a.K / BK;
  __syncthreads();  // codebook
  gload(0);
  lstore(0, 0);
  __syncthreads();
  for (int64_t kt = 0; kt < KT; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < KT) gload(kt + 1);
    const uint16_t* Ab = As + buf * BM * BK;
    const uint16_t* Bb = Bs + buf * BN * BK;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int c = 2 * s + (lane >> 5);
      ts_u32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * (BM / 2) + 32 * i + (lane & 31);
        af[i] = *reinterpret_cast<const ts_u32x4*>(Ab + swz(r, c));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * (BN / 2) + 32 * j + (lane & 31);
        bf[j] = *reinterpret_cast<const ts_u32x4*>(Bb + swz(r, c));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = ts_mfma32x32x16<BF16>(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < KT) lstore(buf ^ 1, kt + 1);
    __syncthreads();
  }

  // epilogue: bias, cast, store
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + wn * (BN / 2) + 32 * j + (lane & 31);
    if (n >= a.N) continue;
    const float b = a.bias ? XT<BF16>::to_f(a.bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= a.M) continue;
        const float v = acc[i][j][r] + b;
        const int64_t off = m * a.ldy + n;
        if (a.y_dtype == TS_F32) reinterpret_cast<float*>(a.y)[off] = v;
        else reinterpret_cast<uint16_t*>(a.y)[off] = XT<BF16>::from_f(v);
      }
    }
  }
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, int BM, int BN>
static int launch_prefill(PrefillArgs a, hipStream_t st) {
  constexpr int CBN = (CB && BITS == 8) ? 256 : 16;
  const size_t smem = (size_t)2 * (BM + BN) * BK * 2 + CBN * 4 + (size_t)BN * 8 * 8;
  auto kern = prefill_kernel<BITS, GS, BF16, CB, RVQ, BM, BN>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess)
      return TS_HIP_ERROR;
    attr_set = true;
  }
  a.m_tiles = ts_cdiv(a.M, BM);
  a.n_tiles = ts_cdiv(a.N, BN);
  hipLaunchKernelGGL(kern, dim3((unsigned)(a.m_tiles * a.n_tiles)), dim3(256), smem, st, a);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ>
static int pick_tile(PrefillArgs& a, hipStream_t st) {
  // 256 x 256 tiles when they fill the chip, 256 x 128 otherwise.
  const int64_t t256 = ts_cdiv(a.M, 256) * ts_cdiv(a.N, 256);
  if (t256 >= 256) return launch_prefill<BITS, GS, BF16, CB, RVQ, 256, 256>(a, st);
  return launch_prefill<BITS, GS, BF16, CB, RVQ, 256, 128>(a, st);
}

template <bool BF16>
static int dispatch_prefill(const ts_qlayer* L, PrefillArgs& a, hipStream_t st) {
  const bool cb = L->codebook != nullptr;
  const int gs = L->group_size;
#define TS_PF_GS(BITS, CBV, RVQV)                                              \
  do {                                                                         \
    if (gs == 128) return pick_tile<BITS, 128, BF16, CBV, RVQV>(a, st);        \
    if (gs == 64) return pick_tile<BITS, 64, BF16, CBV, RVQV>(a, st);          \
    if (gs == 256) return pick_tile<BITS, 256, BF16, CBV, RVQV>(a, st);        \
    if (gs == 32) return pick_tile<BITS, 32, BF16, CBV, RVQV>(a, st);          \
    return TS_NOT_COVERED;                                                     \
  } while (0)
  if (L->bits == 6) TS_PF_GS(4, false, true);
  if (L->bits == 4) { if (cb) TS_PF_GS(4, true, false); TS_PF_GS(4, false, false); }
  if (L->bits == 2) { if (cb) TS_PF_GS(2, true, false); TS_PF_GS(2, false, false); }
  if (L->bits == 8) { if (cb) TS_PF_GS(8, true, false); TS_PF_GS(8, false, false); }
#undef TS_PF_GS
  return TS_NOT_COVERED;
}

int prefill_forward(const ts_qlayer* L, const uint16_t* x, int64_t M, int64_t ldx, int x_dtype, void* y,
                    int64_t ldy, int y_dtype, const uint16_t* bias, hipStream_t st) {
  if (L->padded_cols % BK != 0) return TS_NOT_COVERED;
  PrefillArgs a{};
  a.packed = L->packed;
  a.pstride = L->packed_stride;
  a.scale = L->scale;
  a.gmin = L->gmin;
  a.dqsc = L->dq_scale_codes;
  a.dqsm = L->dq_scale_meta;
  a.dqgc = L->dq_gmin_codes;
  a.dqgm = L->dq_gmin_meta;
  a.dq_gs = (uint32_t)(L->dq_group_size > 0 ? L->dq_group_size : 1);
  a.codebook = L->codebook;
  a.s2packed = L->stage2_packed;
  a.s2stride = L->stage2_stride;
  a.s2scale = L->stage2_scale;
  a.s2gmin = L->stage2_gmin;
  a.orow_ptr = L->n_outliers > 0 ? L->outlier_row_ptr : nullptr;
  a.ocol = L->outlier_col;
  a.odelta = L->outlier_delta;
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
  return x_dtype == TS_BF16 ? dispatch_prefill<true>(L, a, st) : dispatch_prefill<false>(L, a, st);
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
