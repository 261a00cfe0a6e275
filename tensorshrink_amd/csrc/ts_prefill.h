// Prefill (M > 16) quantized linear on the matrix cores.
//
// Replaces the reference's large-M path: dequantize_weight into a dense
// compute-dtype W (triton_kernels.py:1114-1186), the outlier scatter onto W
// (modules.py:912-919) and F.linear (modules.py:920). W never exists in HBM:
// each workgroup dequantizes its BN x 64 weight tile straight into LDS as
// bf16/f16 (codebook / double-quant affine in float32, one rounding), folds
// that tile's outliers in (w = cast(f32(w) + delta), as modules.py:918 does on
// the dense W) and feeds MFMA f32_32x32x16 with fp32 accumulation.
//
// Tile: 256 x BN x 64 per workgroup of NW waves (NW/2 along M, 2 along N),
// each wave (512/NW) x BN/2 as MFMA 32x32 blocks. NW = 8 (two waves per
// SIMD, so one wave's LDS and barrier waits overlap the other's MFMAs) is
// the default; NW = 4 gives one wave per SIMD with 128 x BN/2 wave tiles.
//   * All global reads are raw buffer loads (64-bit bases in SGPRs, 32-bit
//     offsets) into register stages: weights two k-steps ahead, x (two
//     register sets) two k-steps ahead. Nothing computes on loaded data in the
//     load phase and no load is conditional, so the compiler's wait counts
//     stay exact and a wait never drains younger loads.
//   * Each k-step runs 4 MFMA sub-steps on LDS buffer `cur`. The operand
//     fragments and codebook values of sub-step s + 1 are read from LDS before
//     sub-step s's MFMAs; the next k-step's dequant (scale, convert, write to
//     buffer `cur ^ 1`) is spread over the sub-steps. One LDS-only barrier
//     per k-step (a __syncthreads would drain the prefetch).
//   * LDS tiles use a 16-byte-chunk XOR swizzle (chunk c of row r at
//     c ^ (r & 7)): both the tile writes and the MFMA operand reads are
//     bank-conflict free.
//   * Codebooks sit in LDS as 32 bank-interleaved copies, one per lane of a
//     half-wave, so random code lookups are conflict free.
//   * Outliers: each tile row's outliers (up to OMAX) are staged in LDS
//     sorted by column at the start; the threads owning the row walk them
//     with a moving pointer. Outliers of a row beyond OMAX (none at the
//     configured outlier fractions) are added to the output in the epilogue.
#pragma once
#include <algorithm>

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
  const int32_t* orow_ptr;  // CSR row offsets, or any valid int array when rp_mul == 0
  int64_t rp_mul;
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
  // byte extents of the buffers read through buffer resources (all < 2^31)
  uint32_t x_bytes, p_bytes, meta_elems, dqm_bytes, s2_bytes;
};

constexpr int PF_BM = 256;
constexpr int PF_BK = 64;
constexpr int PF_OMAX = 32;  // outliers per tile row staged in LDS
#ifndef PF_NW
#define PF_NW 8  // waves per workgroup
#endif

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

// LDS offset (in uint16 elements) of 16-byte chunk c of row r in a [rows][64] tile.
TS_DEV int swz(int r, int c) { return r * PF_BK + ((c ^ (r & 7)) << 3); }

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN, int NW>
__global__ __launch_bounds__(64 * NW, NW / 4) void prefill_kernel(const PrefillArgs a_in) {
  constexpr int BM = PF_BM, BK = PF_BK;
  constexpr int NT = 64 * NW;                  // threads
  constexpr int WGM = NW / 2;                  // waves along M (two along N)
  constexpr int TM = BM / WGM / 32, TN = BN / 64;
  constexpr int A_CHUNKS = BM * 8 / NT;       // 16-byte x chunks per thread per k-step
  constexpr int CPT = BN * BK / NT;           // weight codes per thread per k-step
  constexpr int TPR = BK / CPT;               // threads per weight row
  constexpr int WB = CPT * BITS / 8;          // packed bytes per thread per k-step
  constexpr int WB2 = RVQ ? CPT / 4 : 0;      // RVQ stage-2 bytes
  constexpr int C8 = CPT / 8;                 // 8-code chunks per thread per k-step
  constexpr int NGT = CPT >= GS ? CPT / GS : 1;  // groups a thread's codes span in a k-step
  constexpr int CBN = (CB && BITS == 8) ? 256 : 16;
  static_assert(C8 % 4 == 0 || C8 == 2, "dequant chunks per sub-step");
  static_assert(WB % 4 == 0, "packed chunk");
  extern __shared__ __align__(16) unsigned char smem[];
  // The codebook is static LDS (its address folds into the ds_read offset),
  // in 32 copies interleaved entry-major: copy l of entry e at [e * 32 + l],
  // i.e. in bank l. Lane l reads copy l % 32, so a wave's 64 random lookups
  // are bank-conflict free (two passes) whatever the codes.
  __shared__ float cbs[CB ? CBN * 32 : 1];

  // Kernel arguments fetched once, kept in SGPRs (see the decode kernel).
  PrefillArgs a = a_in;
#define TS_PG(f) ts_pin_global(a.f)
#define TS_PS(f) ts_pin_scalar(a.f)
  TS_PG(packed); TS_PG(scale); TS_PG(gmin); TS_PG(dqsc); TS_PG(dqsm); TS_PG(dqgc); TS_PG(dqgm); TS_PG(codebook);
  TS_PG(orow_ptr); TS_PG(ocol); TS_PG(odelta); TS_PG(x); TS_PG(y);
  TS_PS(pstride); TS_PS(dq_shift); TS_PS(rp_mul); TS_PS(ldx); TS_PS(ldy); TS_PS(y_dtype); TS_PS(M); TS_PS(N); TS_PS(K);
  TS_PS(cols); TS_PS(n_groups); TS_PS(m_tiles); TS_PS(n_tiles);
  TS_PS(x_bytes); TS_PS(p_bytes); TS_PS(meta_elems); TS_PS(dqm_bytes); TS_PS(s2_bytes);
  if constexpr (RVQ) { TS_PG(s2packed); TS_PS(s2stride); TS_PG(s2scale); TS_PG(s2gmin); }
#undef TS_PG
#undef TS_PS

  uint16_t* As = reinterpret_cast<uint16_t*>(smem);             // [2][BM][64]
  uint16_t* Bs = As + 2 * BM * BK;                              // [2][BN][64]
  uint32_t* ol = reinterpret_cast<uint32_t*>(Bs + 2 * BN * BK);  // [BN][OMAX] col | f16 delta << 16
  int32_t* ocnt = reinterpret_cast<int32_t*>(ol + BN * PF_OMAX);  // [BN] outliers per tile row

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t cb_lane = lane & 31;  // codebook copy of this lane
  const int wm = wave % WGM, wn = wave / WGM;

  // XCD-aware tile order: consecutive workgroups go to different XCDs, so map
  // blockIdx so that the workgroups sharing an XCD walk down one column of M
  // tiles of the same weight tile (W bytes then hit that XCD's L2).
  const int64_t nblk = a.m_tiles * a.n_tiles;
  int64_t bid = blockIdx.x;
  {
    const int64_t per_xcd = nblk / 8;
    if (per_xcd * 8 == nblk) bid = (bid % 8) * per_xcd + bid / 8;
  }
  const int64_t mt = bid % a.m_tiles, nt = bid / a.m_tiles;
  const int64_t m0 = mt * BM, n0 = nt * BN;

  // Buffer resources: 64-bit bases in SGPRs, 32-bit byte offsets per lane.
  const __amdgpu_buffer_rsrc_t rx = ts_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rw = ts_rsrc(a.packed, a.p_bytes);
  const __amdgpu_buffer_rsrc_t rsc = DQ ? ts_rsrc(a.dqsc, a.meta_elems) : ts_rsrc(a.scale, 2 * a.meta_elems);
  const __amdgpu_buffer_rsrc_t rgc = DQ ? ts_rsrc(a.dqgc, a.meta_elems) : ts_rsrc(a.gmin, 2 * a.meta_elems);
  const __amdgpu_buffer_rsrc_t rsm = ts_rsrc(DQ ? a.dqsm : a.scale, DQ ? a.dqm_bytes : 4);
  const __amdgpu_buffer_rsrc_t rgm = ts_rsrc(DQ ? a.dqgm : a.gmin, DQ ? a.dqm_bytes : 4);
  const __amdgpu_buffer_rsrc_t rw2 = ts_rsrc(RVQ ? a.s2packed : a.packed, RVQ ? a.s2_bytes : 4);
  const __amdgpu_buffer_rsrc_t rs2s = ts_rsrc(RVQ ? a.s2scale : a.scale, RVQ ? 2 * a.meta_elems : 4);
  const __amdgpu_buffer_rsrc_t rs2g = ts_rsrc(RVQ ? a.s2gmin : a.gmin, RVQ ? 2 * a.meta_elems : 4);

  // weight-row ownership for the dequant
  const int wr = tid / TPR;     // row within the tile
  const int wpart = tid % TPR;  // which CPT-code slice of the k-step
  const int64_t wrow = min(n0 + wr, a.N - 1);
  const uint32_t woff = (uint32_t)(wrow * a.pstride) + (wpart * CPT * BITS) / 8;
  const uint32_t woff2 = RVQ ? (uint32_t)(wrow * a.s2stride) + (wpart * CPT) / 4 : 0u;
  // flat group index of the thread's first group at k-step 0; k-step kt adds
  // kt * 64 / GS (GS divides 64 or 64 divides GS, so groups never straddle)
  static_assert(GS % BK == 0 || BK % GS == 0, "group size");
  const uint32_t gbase = (uint32_t)(wrow * a.n_groups) + (wpart * CPT) / GS;
  const int KT = (int)(a.K / BK);

  // ---- raw load stage (registers only; nothing computes on the data here) --
  struct Stage {
    uint32_t w[WB / 4];
    uint32_t w2[RVQ ? (WB2 + 3) / 4 : 1];
    uint32_t sc[NGT], gc[NGT];   // DQ codes, or f16 scale / gmin bits
    uint32_t sm[NGT], gm[NGT];   // DQ (meta_scale, meta_min) f16 pairs
    uint32_t s2[NGT];            // RVQ stage-2 (scale, gmin) f16 bits
  };
  // x chunks of one k-step, in two register sets: the loads for k-step
  // kt + 2 are issued at the start of k-step kt and stored to LDS at the end
  // of k-step kt + 1, so every wait is for loads a full k-step old and never
  // drains younger ones. Row offsets are clamped to the last row; columns
  // past `cols` are zeroed in store_x.
  ts_u32x4 X0[A_CHUNKS], X1[A_CHUNKS];
  uint32_t xoff[A_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int ch = tid + i * NT;
    xoff[i] = (uint32_t)(min(m0 + (ch >> 3), a.M - 1) * a.ldx) * 2u + (ch & 7) * 16u;
  }
  // A chunk whose columns lie past `cols` (all eight: cols % 8 == 0) is read
  // at an offset with bit 31 set, past the buffer's extent, which the buffer
  // load returns as zeros.
  const int xcol = (tid & 7) * 8;  // the same column slot for all of a thread's chunks
  // The k-step's byte offset goes in the scalar offset; a lane whose columns
  // are out of range ORs bit 31 into its vector offset, which is range checked.
  auto load_x = [&](int kt, ts_u32x4* xr) {
    kt = min(kt, KT - 1);
    const uint32_t kb = (uint32_t)kt * (BK * 2);
    const uint32_t oob = (kt * BK + xcol < a.cols) ? 0u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) xr[i] = ts_bld16s(rx, xoff[i] | oob, kb);
  };
  auto store_x = [&](int buf, const ts_u32x4* xr) {
    uint16_t* Ab = As + buf * BM * BK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int ch = tid + i * NT;
      *reinterpret_cast<ts_u32x4*>(Ab + swz(ch >> 3, ch & 7)) = xr[i];
    }
  };
  auto load_stage = [&](int kt, Stage& S) {
    kt = min(kt, KT - 1);  // a stage past the end re-reads the last k-step (never used)
    const uint32_t off = woff + (uint32_t)kt * (BK * BITS / 8);
    if constexpr (WB % 16 == 0) {
#pragma unroll
      for (int i = 0; i < WB / 16; ++i) {
        const ts_u32x4 v = ts_bld16(rw, off + 16 * i);
        S.w[4 * i] = v.x; S.w[4 * i + 1] = v.y; S.w[4 * i + 2] = v.z; S.w[4 * i + 3] = v.w;
      }
    } else if constexpr (WB == 8) {
      const ts_u32x2 v = ts_bld8(rw, off);
      S.w[0] = v.x; S.w[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < WB / 4; ++i) S.w[i] = ts_bld4(rw, off + 4 * i);
    }
    if constexpr (RVQ) {
      const uint32_t off2 = woff2 + (uint32_t)kt * (BK / 4);
      if constexpr (WB2 >= 4) {
#pragma unroll
        for (int i = 0; i < WB2 / 4; ++i) S.w2[i] = ts_bld4(rw2, off2 + 4 * i);
      } else {
        S.w2[0] = ts_bld2(rw2, off2);
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

  // ---- dequant of one stage into LDS, in 4 parts (one per MFMA sub-step) ---
  // Split in two so the code-value fetch (codebook reads from LDS) of part
  // p + 1 is in flight while part p's MFMAs run: lookup() gives the float code
  // values of the part's chunks, finish() scales, converts and writes them.
  constexpr int CP = C8 >= 4 ? C8 / 4 : 1;  // 8-code chunks per part
  struct Codes {
    float v[CP][8];
  };
  auto chunk_of = [&](int part, int cc) { return (C8 >= 4 ? part * CP : part) + cc; };
  auto lookup = [&](const Stage& S, int part, Codes& C) {
    if (C8 < 4 && part >= C8) return;
#pragma unroll
    for (int cc = 0; cc < CP; ++cc) {
      const int c8 = chunk_of(part, cc);
      float* cv = C.v[cc];
      if constexpr (BITS == 4) {
        const uint32_t d = S.w[c8];
        if constexpr (CB) {
#pragma unroll
          for (int e = 0; e < 8; ++e) cv[e] = cbs[(((d >> (4 * e)) & 15u) << 5) | cb_lane];
        } else {
          uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
          asm volatile("" : "+v"(lo), "+v"(hi));  // keeps the byte-select conversions (v_cvt_f32_ubyteN)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            cv[2 * e] = (float)((lo >> (8 * e)) & 0xffu);
            cv[2 * e + 1] = (float)((hi >> (8 * e)) & 0xffu);
          }
        }
      } else if constexpr (BITS == 2) {
        const uint32_t d = S.w[c8 >> 1] >> (16 * (c8 & 1));  // 8 codes in 16 bits
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t c = (d >> (2 * e)) & 3u;
          cv[e] = CB ? cbs[(c << 5) | cb_lane] : (float)c;
        }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t d = S.w[2 * c8 + h];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t c = (d >> (8 * e)) & 0xffu;
            cv[4 * h + e] = CB ? cbs[(c << 5) | cb_lane] : (float)c;
          }
        }
      }
    }
  };
  // Per-group scale and offset of a stage (float32, modules.py:573-579 for
  // the double-quant codes), computed once per k-step.
  struct Scales {
    float s[NGT], g[NGT];
  };
  auto scales = [&](const Stage& S, Scales& Q) {
#pragma unroll
    for (int t = 0; t < NGT; ++t) {
      if constexpr (DQ) {  // code * meta_scale + meta_min
        Q.s[t] = __fadd_rn(__fmul_rn((float)S.sc[t], ts_h2f(S.sm[t] & 0xffffu)), ts_h2f(S.sm[t] >> 16));
        Q.g[t] = __fadd_rn(__fmul_rn((float)S.gc[t], ts_h2f(S.gm[t] & 0xffffu)), ts_h2f(S.gm[t] >> 16));
      } else {
        Q.s[t] = ts_h2f((uint16_t)S.sc[t]);
        Q.g[t] = ts_h2f((uint16_t)S.gc[t]);
      }
    }
  };
  auto finish = [&](const Stage& S, const Scales& Q, int part, int buf, const Codes& C) {
    if (C8 < 4 && part >= C8) return;
    uint16_t* Bb = Bs + buf * BN * BK;
#pragma unroll
    for (int cc = 0; cc < CP; ++cc) {
      const int c8 = chunk_of(part, cc);
      const int t = (c8 * 8) / (CPT >= GS ? GS : CPT);  // group of this chunk within the thread's codes
      const int tg = NGT > 1 ? t : 0;
      const float s = Q.s[tg], gm = Q.g[tg];
      const float* cv = C.v[cc];
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(cv[e], s, gm);
      if constexpr (RVQ) {
        const float s2 = ts_h2f((uint16_t)(S.s2[tg] & 0xffffu)), g2 = ts_h2f((uint16_t)(S.s2[tg] >> 16));
        const uint32_t d2 = S.w2[c8 >> 1] >> (16 * (c8 & 1));
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
  };
  // Moving pointer over this row's sorted outliers.
  int opos = 0;
  int oncnt = 0;  // staged outliers of this row (set after staging)
  int64_t o_begin = 0, o_count = 0;
  // Fold this row's outliers that land in the thread's slice of k-step kt
  // into the dequantized tile (w = cast(f32(w) + delta), modules.py:918).
  auto fold_outliers = [&](int buf, int kt) {
    uint16_t* Bb = Bs + buf * BN * BK;
    const int k0 = kt * BK;
    if (o_count > 0) {
      const int kc0 = k0 + wpart * CPT, kc1 = kc0 + CPT;
      while (opos < oncnt) {
        const uint32_t e = ol[wr * PF_OMAX + opos];
        const int col = (int)(e & 0xffffu);
        if (col >= kc1) break;
        if (col >= kc0) {
          const int kk = col - k0;
          uint16_t* p = Bb + swz(wr, kk >> 3) + (kk & 7);
          *p = XT<BF16>::from_f(XT<BF16>::to_f(*p) + ts_h2f((uint16_t)(e >> 16)));
        }
        ++opos;
      }
    }
  };

  // ---- prologue --------------------------------------------------------------
  Stage S0, S1;
  load_x(0, X0);
  load_stage(0, S0);
  load_x(1, X1);
  load_stage(1, S1);
  if constexpr (CB) {
    for (int i = tid; i < CBN * 32; i += NT) cbs[i] = a.codebook[i >> 5];
  }
  // stage each tile row's first OMAX outliers, sorted by column (K < 65536)
  {
    const int64_t rb = a.orow_ptr[min(wrow, a.N) * a.rp_mul];
    const int64_t re = a.orow_ptr[min(wrow + 1, a.N) * a.rp_mul];
    o_begin = rb;
    o_count = (n0 + wr < a.N) ? re - rb : 0;
    if (wpart == 0) {
      const int n = (int)min<int64_t>(o_count, PF_OMAX);
      uint32_t* lst = ol + wr * PF_OMAX;
      for (int i = 0; i < n; ++i) {
        const uint32_t e = (uint32_t)a.ocol[rb + i] | ((uint32_t)a.odelta[rb + i] << 16);
        int j = i;
        while (j > 0 && (lst[j - 1] & 0xffffu) > (e & 0xffffu)) {
          lst[j] = lst[j - 1];
          --j;
        }
        lst[j] = e;
      }
      ocnt[wr] = n;
    }
  }
  ts_lds_barrier();
  oncnt = ocnt[wr];
#pragma unroll
  for (int part = 0; part < 4; ++part) {
    Codes C;
    Scales Q;
    scales(S0, Q);
    lookup(S0, part, C);
    finish(S0, Q, part, 0, C);
  }
  fold_outliers(0, 0);
  store_x(0, X0);
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
  auto read_frag = [&](int cur, int s, Frag& F) {
    const uint16_t* Ab = As + cur * BM * BK;
    const uint16_t* Bb = Bs + cur * BN * BK;
    const int c = 2 * s + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) F.a[i] = *reinterpret_cast<const ts_u32x4*>(Ab + swz(wm * (BM / WGM) + 32 * i + (lane & 31), c));
#pragma unroll
    for (int j = 0; j < TN; ++j) F.b[j] = *reinterpret_cast<const ts_u32x4*>(Bb + swz(wn * (BN / 2) + 32 * j + (lane & 31), c));
  };
  auto mfma = [&](const Frag& F) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = ts_mfma32x32x16<BF16>(F.a[i], F.b[j], acc[i][j]);
  };

  // One k-step. The LDS reads (operand fragments, code values) of sub-step
  // s + 1 are issued before sub-step s's MFMAs, whose shadow then covers
  // their latency and the VALU work of finish(). x for k-step kt + 2 is
  // issued into XL at the start; the dequant of stage S (k-step kt + 1) goes
  // to the other LDS buffer; S is refilled with k-step kt + 3; then x for
  // k-step kt + 1 (issued a k-step ago, in XS) is stored to the other buffer.
  auto kstep = [&](int kt, Stage& S, ts_u32x4* XL, const ts_u32x4* XS) {
    const int cur = kt & 1, nxt = cur ^ 1;
    Frag F0, F1;
    Codes C0, C1;
    Scales Q;
    read_frag(cur, 0, F0);
    lookup(S, 0, C0);
    scales(S, Q);
    load_x(kt + 2, XL);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 1, F1);
    lookup(S, 1, C1);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F0);
    finish(S, Q, 0, nxt, C0);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 2, F0);
    lookup(S, 2, C0);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F1);
    finish(S, Q, 1, nxt, C1);
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 3, F1);
    lookup(S, 3, C1);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F0);
    finish(S, Q, 2, nxt, C0);
    __builtin_amdgcn_sched_barrier(0);
    mfma(F1);
    finish(S, Q, 3, nxt, C1);
    fold_outliers(nxt, kt + 1);
    load_stage(kt + 3, S);
    store_x(nxt, XS);
    ts_lds_barrier();
  };
  // two k-steps per iteration (stages and x sets alternate), one exit
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    kstep(kt, S1, X0, X1);
    kstep(kt + 1, S0, X1, X0);
  }
  if (kt < KT) kstep(kt, S1, X0, X1);

  // epilogue: outliers of rows beyond OMAX (x * delta in fp32), bias, cast, store
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + wn * (BN / 2) + 32 * j + (lane & 31);
    if (n >= a.N) continue;
    const int64_t rb = a.orow_ptr[n * a.rp_mul], re = a.orow_ptr[(n + 1) * a.rp_mul];
    for (int64_t o = rb + PF_OMAX; o < re; ++o) {
      const uint32_t col = (uint32_t)a.ocol[o];
      const float d = ts_h2f(a.odelta[o]);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = min(m0 + wm * (BM / WGM) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), a.M - 1);
          acc[i][j][r] += XT<BF16>::to_f((uint16_t)ts_bld2(rx, ((uint32_t)(m * a.ldx) + col) * 2u)) * d;
        }
      }
    }
    const float b = a.bias ? XT<BF16>::to_f(a.bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * (BM / WGM) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
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
inline size_t prefill_smem() {
  constexpr int CBN = (CB && BITS == 8) ? 256 : 16;
  (void)CBN;  // the codebook is static LDS
  return (size_t)2 * (PF_BM + BN) * PF_BK * 2 + (size_t)BN * PF_OMAX * 4 + (size_t)BN * 4;
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN, int NW>
inline int launch_prefill(PrefillArgs a, hipStream_t st) {
  const size_t smem = prefill_smem<BITS, CB, BN>();
  auto kern = prefill_kernel<BITS, GS, BF16, CB, RVQ, DQ, BN, NW>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess)
      return TS_HIP_ERROR;
    attr_set = true;
  }
  a.m_tiles = ts_cdiv(a.M, PF_BM);
  a.n_tiles = ts_cdiv(a.N, BN);
  hipLaunchKernelGGL(kern, dim3((unsigned)(a.m_tiles * a.n_tiles)), dim3(64 * NW), smem, st, a);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// 256 x 128 tiles: a 256 x 256 tile with two k-steps of loads in flight does
// not fit the registers of a wave (its accumulators alone take 256).
template <int BITS, int GS, bool BF16, bool CB, bool RVQ>
inline int launch_prefill_tiles(PrefillArgs& a, hipStream_t st) {
  if (a.dqsc != nullptr) return launch_prefill<BITS, GS, BF16, CB, RVQ, true, 128, PF_NW>(a, st);
  return launch_prefill<BITS, GS, BF16, CB, RVQ, false, 128, PF_NW>(a, st);
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
