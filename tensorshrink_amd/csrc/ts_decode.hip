// Decode (M <= 16) quantized linear: y[M, N] = x[M, K] W^T + outliers + bias.
//
// Replaces the reference's fused Triton GEMV/skinny-GEMM
// (triton_kernels.py:278-541, dispatched at modules.py:881-894) and its
// standalone outlier pass (triton_kernels.py:543-576, 940-941).
//
// Mapping (one 16-row tile of W per workgroup, K split across its waves):
//   * MFMA f32_16x16x32 (bf16 or f16). Lane l owns W row r0 + l%16 (B column)
//     and x row l%16 (A row); lane group q = l/16 owns a quarter of every
//     quantization group, so one group is GS/32 MFMAs over that lane set.
//   * Each lane streams its quarter-group of packed codes with one or two
//     coalesced 16-byte loads per group (8/4 bytes for narrow groups).
//   * Codes become bf16/f16 pairs through an LDS table indexed by the packed
//     byte (4-bit: one u32 = two codes; 2-bit: one u64 = four codes), kept in
//     REP bank-private copies so random bytes never collide on a bank.
//   * The per-group affine is factorised out of the MFMA:
//         y += s[n,g] * (x . cb[c]) + gmin[n,g] * (x . 1)
//     with both dot products on the matrix core and s/gmin in float32
//     (rebuilt from double-quant codes in-register, modules.py:573-579).
//   * Partial sums of the K-split waves are reduced in LDS; the row-sorted
//     outliers of the tile (CSR slice, no search, no global atomics) are added
//     with LDS float atomics, then bias, then the compute-dtype store.
#include "ts_common.h"

namespace ts {

struct DecodeArgs {
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
  const int32_t* orow;
  const int32_t* ocol;
  const uint16_t* odelta;
  const uint16_t* x;
  int64_t ldx;
  void* y;
  int64_t ldy;
  int y_dtype;
  const uint16_t* bias;
  int64_t N;
  int64_t cols;
  int64_t n_groups;
  int M;
  int gpw;  // groups per wave
};

template <bool BF16>
TS_DEV uint32_t pack2(float lo, float hi) {
  return (uint32_t)XT<BF16>::from_f(lo) | ((uint32_t)XT<BF16>::from_f(hi) << 16);
}

// Per-(row, group) scale and gmin in float32 (codec.py:740-758 semantics).
TS_DEV void load_scale_gmin(const DecodeArgs& a, int64_t row, int64_t g, float& s, float& gm) {
  const int64_t flat = row * a.n_groups + g;
  if (a.dqsc) {
    const uint32_t sup = (uint32_t)flat / a.dq_gs;
    const float sc = (float)a.dqsc[flat];
    const float gc = (float)a.dqgc[flat];
    s = __fadd_rn(__fmul_rn(sc, ts_h2f(a.dqsm[2 * sup])), ts_h2f(a.dqsm[2 * sup + 1]));
    gm = __fadd_rn(__fmul_rn(gc, ts_h2f(a.dqgm[2 * sup])), ts_h2f(a.dqgm[2 * sup + 1]));
  } else {
    s = ts_h2f(a.scale[flat]);
    gm = ts_h2f(a.gmin[flat]);
  }
}

template <int NB>
struct Bytes {
  uint32_t d[(NB + 3) / 4];
};

template <int NB>
TS_DEV Bytes<NB> load_bytes(const uint8_t* p) {
  Bytes<NB> b;
  if constexpr (NB == 32) {
    ts_u32x4 v0 = ts_ld16(p), v1 = ts_ld16(p + 16);
    b.d[0] = v0.x; b.d[1] = v0.y; b.d[2] = v0.z; b.d[3] = v0.w;
    b.d[4] = v1.x; b.d[5] = v1.y; b.d[6] = v1.z; b.d[7] = v1.w;
  } else if constexpr (NB == 16) {
    ts_u32x4 v = ts_ld16(p);
    b.d[0] = v.x; b.d[1] = v.y; b.d[2] = v.z; b.d[3] = v.w;
  } else if constexpr (NB == 8) {
    ts_u32x2 v = ts_ld8(p);
    b.d[0] = v.x; b.d[1] = v.y;
  } else if constexpr (NB == 4) {
    b.d[0] = ts_ld4(p);
  } else if constexpr (NB == 2) {
    b.d[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
    static_assert(NB == 1, "unsupported chunk");
    b.d[0] = *p;
  }
  return b;
}

TS_DEV uint32_t byte_of(const uint32_t* d, int i) { return (d[i >> 2] >> (8 * (i & 3))) & 0xffu; }

// LDS table layouts (REP copies interleaved so lane%REP picks its own bank).
template <int REP>
struct Tables {
  uint32_t* t4;  // [256][REP]        two codes of a nibble-packed byte
  uint2* t2;     // [256][REP]        four codes of a crumb-packed byte
  uint32_t* t8;  // [256][REP]        (hi, lo) split of one 8-bit codebook entry
};

template <int BITS, int GS, bool BF16, bool CB8, bool RVQ, int REP>
__global__ __launch_bounds__(512) void decode_kernel(const DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int GB = GS * BITS / 8;        // packed bytes per row per group
  constexpr int LB = GB / 4;               // bytes per lane per group
  constexpr int NMF = (BITS == 8 && CB8) ? GS / 16 : GS / 32;  // MFMAs per group
  constexpr int CPM = (BITS == 8 && CB8) ? 4 : 8;              // codes per lane per MFMA
  constexpr int GB2 = GS / 4;              // RVQ stage-2 bytes per row per group
  constexpr int LB2 = GB2 / 4;
  constexpr bool USE_T4 = (BITS == 4);
  constexpr bool USE_T2 = (BITS == 2) || RVQ;
  constexpr bool USE_T8 = (BITS == 8) && CB8;
  constexpr int U = 4;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int n = lane & 15;
  const int q = lane >> 4;
  const int rsl = lane & (REP - 1);
  const int64_t r0 = (int64_t)blockIdx.x * 16;

  // ---- LDS carve-up ------------------------------------------------------
  unsigned char* sp = smem;
  uint32_t* t4 = nullptr;
  uint2* t2 = nullptr;
  uint32_t* t8 = nullptr;
  if constexpr (USE_T4) { t4 = reinterpret_cast<uint32_t*>(sp); sp += 256 * REP * 4; }
  if constexpr (USE_T2) { t2 = reinterpret_cast<uint2*>(sp); sp += 256 * REP * 8; }
  if constexpr (USE_T8) { t8 = reinterpret_cast<uint32_t*>(sp); sp += 256 * REP * 4; }
  float* red = reinterpret_cast<float*>(sp);       // [nwaves][64][4]
  sp += nwaves * 64 * 4 * 4;
  float* ys = reinterpret_cast<float*>(sp);        // [16][17]

  // ---- codebook tables ---------------------------------------------------
  const float* cb = a.codebook;
  for (int e = tid; e < 256 * REP; e += blockDim.x) {
    const int b = e / REP;
    if constexpr (USE_T4) {
      const float lo = cb ? cb[b & 15] : (float)(b & 15);
      const float hi = cb ? cb[b >> 4] : (float)(b >> 4);
      t4[e] = pack2<BF16>(lo, hi);
    }
    if constexpr (USE_T2) {
      // RVQ stage 2 is always a uniform grid; a 2-bit layer uses its codebook.
      const float* c2 = RVQ ? nullptr : cb;
      float v[4];
      for (int j = 0; j < 4; ++j) {
        const int c = (b >> (2 * j)) & 3;
        v[j] = c2 ? c2[c] : (float)c;
      }
      t2[e] = make_uint2(pack2<BF16>(v[0], v[1]), pack2<BF16>(v[2], v[3]));
    }
    if constexpr (USE_T8) {
      const float v = cb[b];
      const uint16_t hb = XT<BF16>::from_f(v);
      const float hv = XT<BF16>::to_f(hb);
      const uint16_t lb = XT<BF16>::from_f(v - hv);
      t8[e] = (uint32_t)hb | ((uint32_t)lb << 16);
    }
  }
  for (int e = tid; e < 16 * 17; e += blockDim.x) ys[e] = 0.f;
  __syncthreads();

  const int64_t row = (r0 + n < a.N) ? (r0 + n) : (a.N - 1);
  const uint8_t* wp = a.packed + row * a.pstride + q * LB;
  const uint8_t* wp2 = RVQ ? (a.s2packed + row * a.s2stride + q * LB2) : nullptr;
  const bool xrow = n < a.M;
  const uint16_t* xp = a.x + (int64_t)n * a.ldx + q * (GS / 4);

  const int64_t g_begin = (int64_t)wave * a.gpw;
  const int64_t g_end = min(g_begin + (int64_t)a.gpw, a.n_groups);

  ts_f32x4 yacc = {0.f, 0.f, 0.f, 0.f};
  constexpr uint32_t ONE = XT<BF16>::ONE;
  const ts_u32x4 ones = CB8 ? ts_u32x4{ONE, ONE, ONE, ONE}
                            : ts_u32x4{ONE | (ONE << 16), ONE | (ONE << 16), ONE | (ONE << 16), ONE | (ONE << 16)};

  for (int64_t g0 = g_begin; g0 < g_end; g0 += U) {
    Bytes<LB> wb[U];
    Bytes<(LB2 > 0 ? LB2 : 1)> wb2[U];
    float s[U], gm[U], s2[U], gm2[U];
    ts_u32x4 xa[U][NMF];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t g = g0 + u;
      const bool live = g < g_end;
      const int64_t gg = live ? g : g_begin;
      wb[u] = load_bytes<LB>(wp + gg * GB);
      if constexpr (RVQ) wb2[u] = load_bytes<LB2>(wp2 + gg * GB2);
      load_scale_gmin(a, row, gg, s[u], gm[u]);
      if constexpr (RVQ) {
        s2[u] = ts_h2f(a.s2scale[row * a.n_groups + gg]);
        gm2[u] = ts_h2f(a.s2gmin[row * a.n_groups + gg]);
      }
      const int64_t c0 = gg * GS + q * (GS / 4);
#pragma unroll
      for (int j = 0; j < NMF; ++j) {
        const int64_t col = c0 + j * CPM;
        const bool ok = live && xrow && (col < a.cols);
        if constexpr (CPM == 8) {
          xa[u][j] = ok ? ts_ld16(xp + gg * GS + j * CPM) : ts_u32x4{0u, 0u, 0u, 0u};
        } else {
          ts_u32x2 v = ok ? ts_ld8(xp + gg * GS + j * CPM) : ts_u32x2{0u, 0u};
          // (x_k, x_k) pairs so one (hi, lo) table word multiplies x_k twice.
          xa[u][j] = ts_u32x4{__builtin_amdgcn_perm(v.x, v.x, 0x05040100u),
                              __builtin_amdgcn_perm(v.x, v.x, 0x07060302u),
                              __builtin_amdgcn_perm(v.y, v.y, 0x05040100u),
                              __builtin_amdgcn_perm(v.y, v.y, 0x07060302u)};
        }
      }
      if (!live) { s[u] = 0.f; gm[u] = 0.f; if constexpr (RVQ) { s2[u] = 0.f; gm2[u] = 0.f; } }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ts_f32x4 aw = {0.f, 0.f, 0.f, 0.f};
      ts_f32x4 ax = {0.f, 0.f, 0.f, 0.f};
      ts_f32x4 aw2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NMF; ++j) {
        ts_u32x4 b;
        if constexpr (BITS == 4) {
          const int b0 = 4 * j;
          b = ts_u32x4{t4[byte_of(wb[u].d, b0 + 0) * REP + rsl], t4[byte_of(wb[u].d, b0 + 1) * REP + rsl],
                       t4[byte_of(wb[u].d, b0 + 2) * REP + rsl], t4[byte_of(wb[u].d, b0 + 3) * REP + rsl]};
        } else if constexpr (BITS == 2) {
          const uint2 e0 = t2[byte_of(wb[u].d, 2 * j + 0) * REP + rsl];
          const uint2 e1 = t2[byte_of(wb[u].d, 2 * j + 1) * REP + rsl];
          b = ts_u32x4{e0.x, e0.y, e1.x, e1.y};
        } else if constexpr (CB8) {
          b = ts_u32x4{t8[byte_of(wb[u].d, 4 * j + 0) * REP + rsl], t8[byte_of(wb[u].d, 4 * j + 1) * REP + rsl],
                       t8[byte_of(wb[u].d, 4 * j + 2) * REP + rsl], t8[byte_of(wb[u].d, 4 * j + 3) * REP + rsl]};
        } else {
          uint32_t pr[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float f0 = (float)byte_of(wb[u].d, 8 * j + 2 * t);
            const float f1 = (float)byte_of(wb[u].d, 8 * j + 2 * t + 1);
            if constexpr (BF16)
              pr[t] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0),
                                            0x07060302u);
            else
              pr[t] = pack2<false>(f0, f1);
          }
          b = ts_u32x4{pr[0], pr[1], pr[2], pr[3]};
        }
        aw = ts_mfma16x16x32<BF16>(xa[u][j], b, aw);
        ax = ts_mfma16x16x32<BF16>(xa[u][j], ones, ax);
        if constexpr (RVQ) {
          const uint2 e0 = t2[byte_of(wb2[u].d, 2 * j + 0) * REP + rsl];
          const uint2 e1 = t2[byte_of(wb2[u].d, 2 * j + 1) * REP + rsl];
          aw2 = ts_mfma16x16x32<BF16>(xa[u][j], ts_u32x4{e0.x, e0.y, e1.x, e1.y}, aw2);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = yacc[i];
        v = __builtin_fmaf(s[u], aw[i], v);
        v = __builtin_fmaf(gm[u], ax[i], v);
        if constexpr (RVQ) {
          v = __builtin_fmaf(s2[u], aw2[i], v);
          v = __builtin_fmaf(gm2[u], ax[i], v);
        }
        yacc[i] = v;
      }
    }
  }

  // ---- K-split reduction ---------------------------------------------------
  *reinterpret_cast<ts_f32x4*>(red + (wave * 64 + lane) * 4) = yacc;
  __syncthreads();
  for (int t = tid; t < 256; t += blockDim.x) {
    const int l = t >> 2, i = t & 3;
    float acc = 0.f;
    for (int w = 0; w < nwaves; ++w) acc += red[(w * 64 + l) * 4 + i];
    const int m = 4 * (l >> 4) + i;
    ys[m * 17 + (l & 15)] += acc;
  }
  // ---- fused outlier correction (row-sorted CSR slice of this tile) --------
  if (a.orow_ptr) {
    const int64_t r1 = min(r0 + 16, a.N);
    const int32_t o0 = a.orow_ptr[r0];
    const int32_t o1 = a.orow_ptr[r1];
    __syncthreads();
    for (int32_t o = o0 + tid; o < o1; o += blockDim.x) {
      const int rr = a.orow[o] - (int)r0;
      const int64_t col = a.ocol[o];
      const float d = ts_h2f(a.odelta[o]);
      for (int m = 0; m < a.M; ++m) {
        const float xv = XT<BF16>::to_f(a.x[(int64_t)m * a.ldx + col]);
        atomicAdd(&ys[m * 17 + rr], xv * d);
      }
    }
  }
  __syncthreads();
  // ---- bias + store ----------------------------------------------------------
  for (int t = tid; t < 16 * a.M; t += blockDim.x) {
    const int m = t >> 4, nn = t & 15;
    const int64_t r = r0 + nn;
    if (r >= a.N) continue;
    float v = ys[m * 17 + nn];
    if (a.bias) v += XT<BF16>::to_f(a.bias[r]);
    const int64_t off = (int64_t)m * a.ldy + r;
    if (a.y_dtype == TS_F32)
      reinterpret_cast<float*>(a.y)[off] = v;
    else if (a.y_dtype == TS_BF16)
      reinterpret_cast<uint16_t*>(a.y)[off] = ts_f2bf(v);
    else
      reinterpret_cast<uint16_t*>(a.y)[off] = ts_f2h(v);
  }
}

template <int BITS, bool CB8, bool RVQ, int REP>
static size_t decode_smem(int nwaves) {
  size_t s = 0;
  if (BITS == 4) s += 256 * REP * 4;
  if (BITS == 2 || RVQ) s += 256 * REP * 8;
  if (BITS == 8 && CB8) s += 256 * REP * 4;
  s += (size_t)nwaves * 64 * 16;
  s += 16 * 17 * 4;
  return s;
}

template <int BITS, int GS, bool BF16, bool CB8, bool RVQ, int REP>
static int launch_decode(const DecodeArgs& a, int nwaves, hipStream_t st) {
  const size_t smem = decode_smem<BITS, CB8, RVQ, REP>(nwaves);
  auto kern = decode_kernel<BITS, GS, BF16, CB8, RVQ, REP>;
  static bool attr_set = false;  // raising the dynamic-LDS cap is idempotent
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess)
      return TS_HIP_ERROR;
    attr_set = true;
  }
  const dim3 grid((unsigned)ts_cdiv(a.N, 16));
  hipLaunchKernelGGL(kern, grid, dim3(64 * nwaves), smem, st, a);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// Choose the K split: enough waves to keep ~8 per CU busy, at least 4 groups
// per wave so the per-wave prologue/epilogue stays small.
static int pick_waves(int64_t N, int64_t n_groups) {
  int w = 8;
  while (w > 1 && n_groups < (int64_t)w * 2) w >>= 1;
  (void)N;
  return w;
}

template <bool BF16>
static int dispatch_decode_dtype(const ts_qlayer* L, DecodeArgs& a, hipStream_t st) {
  const int nw = pick_waves(a.N, a.n_groups);
  a.gpw = (int)ts_cdiv(a.n_groups, nw);
  const int gs = L->group_size;
  const bool cb = L->codebook != nullptr;
  constexpr int R = 32;
  if (L->bits == 6) {
    if (gs == 128) return launch_decode<4, 128, BF16, false, true, 16>(a, nw, st);
    if (gs == 64) return launch_decode<4, 64, BF16, false, true, 16>(a, nw, st);
    if (gs == 256) return launch_decode<4, 256, BF16, false, true, 16>(a, nw, st);
    return TS_NOT_COVERED;
  }
  if (L->bits == 4) {
    if (gs == 128) return launch_decode<4, 128, BF16, false, false, R>(a, nw, st);
    if (gs == 64) return launch_decode<4, 64, BF16, false, false, R>(a, nw, st);
    if (gs == 32) return launch_decode<4, 32, BF16, false, false, R>(a, nw, st);
    if (gs == 256) return launch_decode<4, 256, BF16, false, false, R>(a, nw, st);
    return TS_NOT_COVERED;
  }
  if (L->bits == 2) {
    if (gs == 128) return launch_decode<2, 128, BF16, false, false, 16>(a, nw, st);
    if (gs == 64) return launch_decode<2, 64, BF16, false, false, 16>(a, nw, st);
    if (gs == 32) return launch_decode<2, 32, BF16, false, false, 16>(a, nw, st);
    if (gs == 256) return launch_decode<2, 256, BF16, false, false, 16>(a, nw, st);
    return TS_NOT_COVERED;
  }
  if (L->bits == 8) {
    if (cb) {
      if (gs == 128) return launch_decode<8, 128, BF16, true, false, R>(a, nw, st);
      if (gs == 64) return launch_decode<8, 64, BF16, true, false, R>(a, nw, st);
      if (gs == 32) return launch_decode<8, 32, BF16, true, false, R>(a, nw, st);
      return TS_NOT_COVERED;
    }
    if (gs == 128) return launch_decode<8, 128, BF16, false, false, 1>(a, nw, st);
    if (gs == 64) return launch_decode<8, 64, BF16, false, false, 1>(a, nw, st);
    if (gs == 32) return launch_decode<8, 32, BF16, false, false, 1>(a, nw, st);
    return TS_NOT_COVERED;
  }
  return TS_NOT_COVERED;
}

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
  a.codebook = L->codebook;
  a.s2packed = L->stage2_packed;
  a.s2stride = L->stage2_stride;
  a.s2scale = L->stage2_scale;
  a.s2gmin = L->stage2_gmin;
  a.orow_ptr = L->n_outliers > 0 ? L->outlier_row_ptr : nullptr;
  a.orow = L->outlier_row;
  a.ocol = L->outlier_col;
  a.odelta = L->outlier_delta;
  a.x = x;
  a.ldx = ldx;
  a.y = y;
  a.ldy = ldy;
  a.y_dtype = y_dtype;
  a.bias = bias;
  a.N = L->rows;
  a.cols = L->cols;
  a.n_groups = L->n_groups;
  a.M = (int)M;
  return x_dtype == TS_BF16 ? dispatch_decode_dtype<true>(L, a, st) : dispatch_decode_dtype<false>(L, a, st);
}

}  // namespace ts
