// Prefill (M > 16) quantized linear on the matrix cores.
//
// Replaces the reference's large-M path: dequantize_weight into a dense
// compute-dtype W (triton_kernels.py:1114-1186), the outlier scatter onto W
// (modules.py:912-919) and F.linear (modules.py:920). W never exists in HBM:
// each workgroup dequantizes its BN x 64 weight tile straight into LDS as
// bf16/f16 (codebook / double-quant affine in float32, one rounding), folds
// the tile's outliers into it and feeds MFMA f32_32x32x16 with fp32
// accumulation.
//
// Tile 256 x BN x 64 per workgroup of 4 waves, one wave per SIMD (2 x 2
// waves, each 128 x BN/2 as 4 x BN/64 MFMA blocks of 32 x 32; the
// accumulators live in AGPRs). Sized for gfx950's budget per CU and clock:
// one 32x32x16 MFMA takes 32 cycles of a SIMD, and the LDS moves about 190 B
// per cycle. A 128 x 128 wave tile reads 8 KB of operands per 16 MFMAs
// (64 B per MFMA-cycle over the CU); with the tile stores and the codebook
// lookups the LDS stays near 60 % of its rate, so the k-loop can run at the
// MFMA rate. Each weight element is dequantized once per workgroup.
//   * All global reads are raw buffer loads (64-bit bases in SGPRs, 32-bit
//     offsets) into register stages: weights two k-steps ahead, x (two
//     register sets) two k-steps ahead. No load is conditional, so the
//     compiler's wait counts stay exact and a wait never drains younger
//     loads.
//   * One k-step = 4 MFMA sub-steps over LDS buffer `cur`. The operand
//     fragments of sub-step s + 1 are read before sub-step s's MFMAs; the next
//     stage's dequant (codebook lookup, scale, convert, write to buffer
//     `cur ^ 1`) and x store are spread over sub-steps 0-2. The one LDS
//     barrier per k-step sits before sub-step 3, whose fragments are already
//     in registers, so the next k-step's first fragment reads overlap its
//     MFMAs.
//   * LDS tiles use a 16-byte-chunk XOR swizzle (chunk c of row r at
//     c ^ (r & 7)): tile writes and MFMA operand reads are conflict free.
//   * Codebooks sit in LDS in bank-interleaved copies, so random code
//     lookups spread over the banks.
//   * Outliers: each weight row is dequantized by one thread (two for
//     BN = 128) that walks the row's outliers in column order (a derived
//     column-sorted table) and adds each delta into the element it has just
//     written with an LDS packed add (ds_pk_add_bf16 / _f16), i.e.
//     w = cast(cast(w) + cast(delta)), as modules.py:918 folds them into the
//     dense W. The next entry is loaded a k-step ahead; a second outlier of the
//     same row in one k-step waits for its load.
#pragma once
#include <algorithm>
#include <mutex>

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
  uint32_t dq_shift;      // log2 of the double-quant super-group size
  const float* codebook;  // or any valid float array when there is none
  const uint8_t* s2packed;
  int64_t s2stride;
  const uint16_t* s2scale;
  const uint16_t* s2gmin;
  const int32_t* orow_ptr;  // CSR row offsets (any valid int array without outliers)
  const uint32_t* ocs;      // column-sorted entries: col | f16 delta << 16
  int32_t has_out;
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
  // byte extents of the buffers read through buffer resources (all < 2^31)
  uint32_t x_bytes, p_bytes, meta_elems, dqm_bytes, s2_bytes, ocs_bytes;
};

constexpr int PF_BM = 256;
constexpr int PF_BK = 64;
constexpr uint32_t PF_NO_COL = 0xffffu;  // column of the "no more outliers" entry

typedef __bf16 ts_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 ts_f16x2 __attribute__((ext_vector_type(2)));
typedef float ts_f32x2 __attribute__((ext_vector_type(2)));
typedef short ts_s16x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed (lo, hi) bf16/f16 pair, round to nearest even
// (v_cvt_pk_bf16_f32 on gfx950).
template <bool BF16>
TS_DEV uint32_t to_pair(float lo, float hi) {
  const ts_f32x2 v = {lo, hi};
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ts_bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ts_f16x2));
}

// LDS offset (in uint16 elements) of 16-byte chunk c of row r in a [rows][64] tile.
TS_DEV int swz(int r, int c) { return r * PF_BK + ((c ^ (r & 7)) << 3); }

// Workgroup index -> tile index, so that the workgroups one XCD runs (the
// hardware deals workgroups out to the 8 XCDs round robin) take consecutive
// tiles: the 256-row M tiles of one weight tile then share that XCD's L2.
TS_DEV int64_t xcd_tile(int64_t b, int64_t n) {
  const int64_t x = b & 7, i = b >> 3;
  const int64_t q = n >> 3, r = n & 7;  // XCD x runs q + (x < r) workgroups
  return x * q + min(x, r) + i;
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN>
__global__ __launch_bounds__(256, 1) void prefill_kernel(const PrefillArgs a_in) {
  constexpr int BM = PF_BM, BK = PF_BK, NT = 256;
  constexpr int TM = 4;                         // 32-row blocks per wave along M (128 rows)
  constexpr int TN = BN / 64;                   // 32-column blocks per wave along N (BN / 2)
  constexpr int TPR = NT / BN;                  // threads per weight row (1 or 2)
  constexpr int CPT = BK / TPR;                 // weight codes per thread per k-step (64 or 32)
  constexpr int C8 = CPT / 8;                   // 8-code chunks per thread per k-step
  constexpr int SB = RVQ ? 4 : BITS;            // stage-1 bits
  constexpr int WB = CPT * SB / 8;              // stage-1 packed bytes per thread per k-step
  constexpr int WW = WB / 4;                    // ... in dwords
  constexpr int WW2 = RVQ ? CPT / 16 : 1;       // stage-2 dwords (16 two-bit codes each)
  constexpr int NGT = CPT > GS ? CPT / GS : 1;  // groups a thread's codes span in a k-step
  constexpr int CBN = CB ? (1 << BITS) : 1;
  constexpr int CBC = (CB && BITS == 8) ? 16 : 32;  // codebook copies (bank spread)
  constexpr int XCH = BM * 8 / NT;              // 16-byte x chunks per thread per k-step
  static_assert(WB >= 8 && WB % 8 == 0, "packed chunk");
  static_assert(GS % BK == 0 || BK % GS == 0, "group size");
  extern __shared__ __align__(16) unsigned char smem[];

  // Kernel arguments fetched once, kept in SGPRs (see the decode kernel).
  PrefillArgs a = a_in;
#define TS_PG(f) ts_pin_global(a.f)
#define TS_PS(f) ts_pin_scalar(a.f)
  TS_PG(packed); TS_PG(scale); TS_PG(gmin); TS_PG(dqsc); TS_PG(dqsm); TS_PG(dqgc); TS_PG(dqgm); TS_PG(codebook);
  TS_PG(orow_ptr); TS_PG(ocs); TS_PG(x); TS_PG(y);
  TS_PS(pstride); TS_PS(dq_shift); TS_PS(has_out); TS_PS(ldx); TS_PS(ldy); TS_PS(y_dtype); TS_PS(M); TS_PS(N);
  TS_PS(K); TS_PS(cols); TS_PS(n_groups); TS_PS(m_tiles); TS_PS(n_tiles);
  TS_PS(x_bytes); TS_PS(p_bytes); TS_PS(meta_elems); TS_PS(dqm_bytes); TS_PS(s2_bytes); TS_PS(ocs_bytes);
  if constexpr (RVQ) { TS_PG(s2packed); TS_PS(s2stride); TS_PG(s2scale); TS_PG(s2gmin); }
#undef TS_PG
#undef TS_PS

  uint16_t* As = reinterpret_cast<uint16_t*>(smem);          // [2][BM][64]
  uint16_t* Bs = As + 2 * BM * BK;                           // [2][BN][64]
  float* cbs = reinterpret_cast<float*>(Bs + 2 * BN * BK);   // [CBN][CBC]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const uint32_t cb_lane = lane % CBC;

  const int64_t tile = xcd_tile(blockIdx.x, a.m_tiles * a.n_tiles);
  const int64_t mt = tile % a.m_tiles, nt = tile / a.m_tiles;
  const int64_t m0 = mt * BM, n0 = nt * BN;

  const __amdgpu_buffer_rsrc_t rx = ts_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rw = ts_rsrc(a.packed, a.p_bytes);
  const __amdgpu_buffer_rsrc_t rsc = DQ ? ts_rsrc(a.dqsc, a.meta_elems) : ts_rsrc(a.scale, 2 * a.meta_elems);
  const __amdgpu_buffer_rsrc_t rgc = DQ ? ts_rsrc(a.dqgc, a.meta_elems) : ts_rsrc(a.gmin, 2 * a.meta_elems);
  const __amdgpu_buffer_rsrc_t rsm = ts_rsrc(DQ ? a.dqsm : a.scale, DQ ? a.dqm_bytes : 4);
  const __amdgpu_buffer_rsrc_t rgm = ts_rsrc(DQ ? a.dqgm : a.gmin, DQ ? a.dqm_bytes : 4);
  const __amdgpu_buffer_rsrc_t rw2 = ts_rsrc(RVQ ? a.s2packed : a.packed, RVQ ? a.s2_bytes : 4);
  const __amdgpu_buffer_rsrc_t rs2s = ts_rsrc(RVQ ? a.s2scale : a.scale, RVQ ? 2 * a.meta_elems : 4);
  const __amdgpu_buffer_rsrc_t rs2g = ts_rsrc(RVQ ? a.s2gmin : a.gmin, RVQ ? 2 * a.meta_elems : 4);
  const __amdgpu_buffer_rsrc_t roc = ts_rsrc(a.ocs, a.ocs_bytes);

  // weight-row ownership for the dequant
  const int wr = tid / TPR;     // row within the tile
  const int wpart = tid % TPR;  // which CPT-code slice of the k-step
  const int64_t wrow = min(n0 + wr, a.N - 1);
  const uint32_t woff = (uint32_t)(wrow * a.pstride) + (wpart * CPT * SB) / 8;
  const uint32_t woff2 = RVQ ? (uint32_t)(wrow * a.s2stride) + (wpart * CPT) / 4 : 0u;
  const uint32_t gbase = (uint32_t)(wrow * a.n_groups) + (wpart * CPT) / GS;
  const int KT = (int)(a.K / BK);

  // ---- raw load stage (registers only; nothing computes on the data here) --
  struct Stage {
    uint32_t w[WW];
    uint32_t w2[WW2];
    uint32_t sc[NGT], gc[NGT];  // DQ codes, or f16 scale / gmin bits
    uint32_t sm[NGT], gm[NGT];  // DQ (meta_scale, meta_min) f16 pairs
    uint32_t s2[NGT];           // RVQ stage-2 (scale, gmin) f16 bits
  };
  // x: thread tid owns chunk column tid & 7 of rows tid / 8 + 32 i. Rows
  // past M and chunks whose columns lie past `cols` are read at offsets past
  // the buffer's extent (bit 31 set for the latter), which the buffer load
  // returns as zeros; those rows are never stored.
  ts_u32x4 X[XCH];
  const uint32_t xbase = (uint32_t)((m0 + (tid >> 3)) * a.ldx) * 2u + (tid & 7) * 16u;
  const uint32_t xstep = (uint32_t)(32 * a.ldx * 2);
  const int xcol = (tid & 7) * 8;
  auto load_x = [&](int kt, ts_u32x4* xr) {
    kt = min(kt, KT - 1);
    const uint32_t kb = (uint32_t)kt * (BK * 2);
    const uint32_t oob = (kt * BK + xcol < a.cols) ? 0u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int64_t m = m0 + (tid >> 3) + 32 * i;
      xr[i] = ts_bld16s(rx, (m < a.M ? xbase + i * xstep : 0x7fffffffu) | oob, kb);
    }
  };
  auto store_x = [&](int buf, const ts_u32x4* xr) {
    uint16_t* Ab = As + buf * BM * BK;
#pragma unroll
    for (int i = 0; i < XCH; ++i)
      *reinterpret_cast<ts_u32x4*>(Ab + swz((tid >> 3) + 32 * i, tid & 7)) = xr[i];
  };
  auto load_stage = [&](int kt, Stage& S) {
    kt = min(kt, KT - 1);  // a stage past the end re-reads the last k-step (never used)
    const uint32_t off = woff + (uint32_t)kt * (BK * SB / 8);
    if constexpr (WB % 16 == 0) {
#pragma unroll
      for (int i = 0; i < WB / 16; ++i) {
        const ts_u32x4 v = ts_bld16(rw, off + 16 * i);
        S.w[4 * i] = v.x; S.w[4 * i + 1] = v.y; S.w[4 * i + 2] = v.z; S.w[4 * i + 3] = v.w;
      }
    } else {
      const ts_u32x2 v = ts_bld8(rw, off);
      S.w[0] = v.x; S.w[1] = v.y;
    }
    if constexpr (RVQ) {
      const uint32_t off2 = woff2 + (uint32_t)kt * (BK / 4);
      if constexpr (WW2 == 4) {
        const ts_u32x4 v = ts_bld16(rw2, off2);
        S.w2[0] = v.x; S.w2[1] = v.y; S.w2[2] = v.z; S.w2[3] = v.w;
      } else {
        const ts_u32x2 v = ts_bld8(rw2, off2);
        S.w2[0] = v.x; S.w2[1] = v.y;
      }
    }
    const uint32_t g0 = gbase + (uint32_t)(kt * BK) / GS;
#pragma unroll
    for (int t = 0; t < NGT; ++t) {
      const uint32_t flat = g0 + t;
      if constexpr (DQ) {
        const uint32_t sup = flat >> a.dq_shift;
        S.sc[t] = ts_bld1(rsc, flat);
        S.gc[t] = ts_bld1(rgc, flat);
        S.sm[t] = ts_bld4(rsm, 4 * sup);
        S.gm[t] = ts_bld4(rgm, 4 * sup);
      } else {
        S.sc[t] = ts_bld2(rsc, 2 * flat);
        S.gc[t] = ts_bld2(rgc, 2 * flat);
      }
      if constexpr (RVQ) S.s2[t] = ts_bld2(rs2s, 2 * flat) | (ts_bld2(rs2g, 2 * flat) << 16);
    }
  };

  // ---- dequant of one stage into LDS, in 3 parts --------------------------
  // Per-group scale and offset of a stage (float32; modules.py:573-579 for
  // the double-quant codes: code * meta_scale + meta_min).
  struct Scales {
    float s[NGT], g[NGT], s2[NGT], g2[NGT];
  };
  auto scales = [&](const Stage& S, Scales& Q) {
#pragma unroll
    for (int t = 0; t < NGT; ++t) {
      if constexpr (DQ) {
        Q.s[t] = __fadd_rn(__fmul_rn((float)S.sc[t], ts_h2f(S.sm[t] & 0xffffu)), ts_h2f(S.sm[t] >> 16));
        Q.g[t] = __fadd_rn(__fmul_rn((float)S.gc[t], ts_h2f(S.gm[t] & 0xffffu)), ts_h2f(S.gm[t] >> 16));
      } else {
        Q.s[t] = ts_h2f((uint16_t)S.sc[t]);
        Q.g[t] = ts_h2f((uint16_t)S.gc[t]);
      }
      if constexpr (RVQ) {
        Q.s2[t] = ts_h2f((uint16_t)(S.s2[t] & 0xffffu));
        Q.g2[t] = ts_h2f((uint16_t)(S.s2[t] >> 16));
      }
    }
  };
  // Chunk c8 (8 codes) of the thread's slice -> 8 bf16/f16 values in LDS.
  auto dq_chunk = [&](const Stage& S, const Scales& Q, int c8, uint16_t* Bb) {
    constexpr int GC = GS / 8;  // chunks per group
    const int t = NGT > 1 ? c8 / GC : 0;
    const float s = Q.s[t], gm = Q.g[t];
    float cv[8];
    if constexpr (SB == 8) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t d = S.w[2 * c8 + h];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t c = (d >> (8 * e)) & 0xffu;
          cv[4 * h + e] = CB ? cbs[c * CBC + cb_lane] : (float)c;
        }
      }
    } else if constexpr (SB == 4) {
      const uint32_t d = S.w[c8];
      if constexpr (CB) {
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[e] = cbs[((d >> (4 * e)) & 15u) * CBC + cb_lane];
      } else {
        uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
        asm volatile("" : "+v"(lo), "+v"(hi));  // keeps the byte-select conversions (v_cvt_f32_ubyteN)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cv[2 * e] = (float)((lo >> (8 * e)) & 0xffu);
          cv[2 * e + 1] = (float)((hi >> (8 * e)) & 0xffu);
        }
      }
    } else {  // 2-bit: 8 codes in 16 bits
      const uint32_t d = S.w[c8 >> 1] >> (16 * (c8 & 1));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t c = (d >> (2 * e)) & 3u;
        cv[e] = CB ? cbs[c * CBC + cb_lane] : (float)c;
      }
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(cv[e], s, gm);
    if constexpr (RVQ) {
      const uint32_t d2 = S.w2[c8 >> 1] >> (16 * (c8 & 1));
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += __builtin_fmaf((float)((d2 >> (2 * e)) & 3u), Q.s2[t], Q.g2[t]);
    }
    ts_u32x4 pk;
    pk.x = to_pair<BF16>(v[0], v[1]);
    pk.y = to_pair<BF16>(v[2], v[3]);
    pk.z = to_pair<BF16>(v[4], v[5]);
    pk.w = to_pair<BF16>(v[6], v[7]);
    *reinterpret_cast<ts_u32x4*>(Bb + swz(wr, wpart * C8 + c8)) = pk;
  };
  // part p of 3 covers chunks [p * C8 / 3, (p + 1) * C8 / 3)
  auto dq_part = [&](const Stage& S, const Scales& Q, int p, int buf) {
    uint16_t* Bb = Bs + buf * BN * BK;
#pragma unroll
    for (int c8 = 0; c8 < C8; ++c8)
      if (c8 >= p * C8 / 3 && c8 < (p + 1) * C8 / 3) dq_chunk(S, Q, c8, Bb);
  };

  // ---- outliers: this row's entries in column order, folded into the tile --
  // e: the next entry (column >= the current k-step's start), en: the one
  // after it when !en_stale; ptr: the table index of en; tld: the entry at
  // ptr loaded during the previous k-step.
  uint32_t e = PF_NO_COL, en = PF_NO_COL, tld = PF_NO_COL;
  uint32_t ptr = 0, oend = 0;
  bool en_stale = true;
  auto oload = [&](uint32_t i) { return ts_bld4(roc, 4u * i); };
  auto fold_outliers = [&](int kt, int buf) {
    if (!a.has_out) return;
    if (en_stale) {
      en = ptr < oend ? tld : PF_NO_COL;
      en_stale = false;
    }
    const uint32_t k0 = (uint32_t)kt * BK;
    uint32_t* Bw = reinterpret_cast<uint32_t*>(Bs + buf * BN * BK);
    while ((e & 0xffffu) < k0 + BK) {  // rare: at most one row in 16 k-steps at 0.1 % outliers
      const int cc = (int)((e & 0xffffu) - k0);
      if (TPR == 1 || (cc >> 5) == wpart) {
        const int h = swz(wr, cc >> 3) + (cc & 7);  // element offset in the tile
        const float d = ts_h2f((uint16_t)(e >> 16));
        const uint32_t dv = (uint32_t)(BF16 ? ts_f2bf(d) : (uint16_t)(e >> 16)) << (16 * (h & 1));
        if constexpr (BF16) {
          __builtin_amdgcn_ds_atomic_fadd_v2bf16((__attribute__((address_space(3))) ts_s16x2*)(Bw + (h >> 1)),
                                                 __builtin_bit_cast(ts_s16x2, dv));
        } else {
          __builtin_amdgcn_ds_atomic_fadd_v2f16((__attribute__((address_space(3))) ts_f16x2*)(Bw + (h >> 1)),
                                                __builtin_bit_cast(ts_f16x2, dv));
        }
      }
      if (en_stale) en = ptr < oend ? oload(ptr) : PF_NO_COL;  // second entry in one k-step
      e = en;
      ++ptr;
      en_stale = true;
    }
  };
  auto fetch_outlier = [&]() {
    if (!a.has_out) return;
    tld = oload(min(ptr, oend > 0 ? oend - 1 : 0u));
  };

  // ---- prologue --------------------------------------------------------------
  Stage S0, S1;
  load_x(0, X);
  load_stage(0, S0);
  load_stage(1, S1);
  if constexpr (CB) {
    for (int i = tid; i < CBN * CBC; i += NT) cbs[i] = a.codebook[i / CBC];
  }
  if (a.has_out) {
    const int64_t r = min(n0 + wr, a.N);  // a row past N has an empty range
    const uint32_t rb = (uint32_t)a.orow_ptr[r];
    oend = (uint32_t)a.orow_ptr[min(r + 1, a.N)];
    e = rb < oend ? a.ocs[rb] : PF_NO_COL;
    ptr = rb + 1;
    tld = oload(min(ptr, oend > 0 ? oend - 1 : 0u));
  }
  ts_lds_barrier();  // codebook copies
  {
    Scales Q;
    scales(S0, Q);
#pragma unroll
    for (int p = 0; p < 3; ++p) dq_part(S0, Q, p, 0);
  }
  fold_outliers(0, 0);
  fetch_outlier();
  store_x(0, X);
  load_stage(2, S0);
  ts_lds_barrier();

  ts_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = ts_f32x16{};

  // MFMA operand fragments of one 16-wide k slice (sub-step s of a k-step).
  struct Frag {
    ts_u32x4 a[TM], b[TN];
  };
  auto read_frag = [&](int buf, int s, Frag& F) {
    const uint16_t* Ab = As + buf * BM * BK;
    const uint16_t* Bb = Bs + buf * BN * BK;
    const int c = 2 * s + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i)
      F.a[i] = *reinterpret_cast<const ts_u32x4*>(Ab + swz(wm * (BM / 2) + 32 * i + (lane & 31), c));
#pragma unroll
    for (int j = 0; j < TN; ++j)
      F.b[j] = *reinterpret_cast<const ts_u32x4*>(Bb + swz(wn * (BN / 2) + 32 * j + (lane & 31), c));
  };
  auto mfma = [&](const Frag& F) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = ts_mfma32x32x16<BF16>(F.a[i], F.b[j], acc[i][j]);
  };

  Frag F0, F1;
  read_frag(0, 0, F0);
  // One k-step: x for k-step kt + 1 is loaded into X; stage S (k-step kt + 1)
  // is dequantized into buffer nxt over sub-steps 0-2 and refilled with
  // k-step kt + 3; X is stored to nxt; barrier; sub-step 3 runs on fragments
  // already in registers while the next k-step's first fragments are read.
  auto kstep = [&](int kt, Stage& S) {
    const int cur = kt & 1, nxt = cur ^ 1;
    Scales Q;
    load_x(kt + 1, X);
    scales(S, Q);
    read_frag(cur, 1, F1);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F0);
    dq_part(S, Q, 0, nxt);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 2, F0);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F1);
    dq_part(S, Q, 1, nxt);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 3, F1);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F0);
    dq_part(S, Q, 2, nxt);
    fold_outliers(kt + 1, nxt);
    fetch_outlier();
    load_stage(kt + 3, S);
    store_x(nxt, X);
    ts_lds_barrier();
    read_frag(nxt, 0, F0);
    mfma(F1);
  };
  // two k-steps per iteration (the stages alternate), one exit
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    kstep(kt, S1);
    kstep(kt + 1, S0);
  }
  if (kt < KT) kstep(kt, S1);

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

template <int BITS, bool CB, int BN>
constexpr size_t prefill_smem() {
  constexpr int CBN = CB ? (1 << BITS) : 0;
  constexpr int CBC = (CB && BITS == 8) ? 16 : 32;
  return (size_t)2 * (PF_BM + BN) * PF_BK * 2 + (size_t)CBN * CBC * 4;
}

// Raises a kernel's dynamic LDS limit once per device (thread safe).
inline bool ts_set_smem_once(const void* kern, size_t smem, std::once_flag* flags, bool* ok) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::call_once(flags[dev], [&] {
    ok[dev] = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) == hipSuccess;
  });
  return ok[dev];
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN>
inline int launch_prefill(PrefillArgs a, hipStream_t st) {
  constexpr size_t smem = prefill_smem<BITS, CB, BN>();
  static_assert(smem <= 160 * 1024, "LDS budget");
  auto kern = prefill_kernel<BITS, GS, BF16, CB, RVQ, DQ, BN>;
  static std::once_flag flags[64];
  static bool ok[64];
  if (!ts_set_smem_once(reinterpret_cast<const void*>(kern), smem, flags, ok)) return TS_HIP_ERROR;
  a.m_tiles = ts_cdiv(a.M, PF_BM);
  a.n_tiles = ts_cdiv(a.N, BN);
  hipLaunchKernelGGL(kern, dim3((unsigned)(a.m_tiles * a.n_tiles)), dim3(256), smem, st, a);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// 256 x 256 tiles when they fill the CUs, else 256 x 128.
template <int BITS, int GS, bool BF16, bool CB, bool RVQ>
inline int launch_prefill_tiles(PrefillArgs& a, hipStream_t st) {
  const bool wide = ts_cdiv(a.M, PF_BM) * ts_cdiv(a.N, 256) >= 256;
  const bool dq = a.dqsc != nullptr;
  if (wide) {
    return dq ? launch_prefill<BITS, GS, BF16, CB, RVQ, true, 256>(a, st)
              : launch_prefill<BITS, GS, BF16, CB, RVQ, false, 256>(a, st);
  }
  return dq ? launch_prefill<BITS, GS, BF16, CB, RVQ, true, 128>(a, st)
            : launch_prefill<BITS, GS, BF16, CB, RVQ, false, 128>(a, st);
}

// Per-(bit width, group size) launchers, one translation unit each
// (ts_prefill_b<bits>_g<gs>.hip).
int prefill_b2_g64(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b2_g128(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b2_g256(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b4_g32(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b4_g64(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b4_g128(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b4_g256(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b6_g64(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b6_g128(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b8_g32(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b8_g64(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);
int prefill_b8_g128(const ts_qlayer* L, PrefillArgs& a, bool bf16, hipStream_t st);

}  // namespace ts
