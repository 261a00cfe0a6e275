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
// Tiles of BM x BN x 64: 256 x 256 on 8 waves, two per SIMD, as a 2 x 4
// grid of 128 x 64 wave tiles (4 x 2 MFMA blocks of 32 x 32); 256 x 128 on 4
// waves, one per SIMD, 2 x 2 grid of 128 x 64; 128 x 128 on 4 waves (64 x 64
// wave tiles). A launch plan (prefill_plan) picks the tile and a split of K
// across up to 8 workgroups per tile, whose fp32 partial sums one reduction
// pass adds up. Each weight element is dequantized once per workgroup; each
// wave stores its outputs as 16-byte row chunks staged through LDS. Sized
// from gfx950 measurements: a 32x32x16 MFMA occupies a SIMD for 32 cycles;
// the LDS serves ds_read_b128 at about 190 B per cycle, ds_write_b128 at
// half that, and a 64-lane codebook lookup (ds_read_u16) costs about as much
// as a b128 read, so NF8's 256 lookups per k-step are the largest single LDS
// cost.
//   * All global reads are raw buffer loads (64-bit bases in SGPRs, 32-bit
//     offsets) into register stages: weights two k-steps ahead, x one.
//     No load the compiler tracks is conditional, so its wait counts stay
//     exact and a wait never drains younger loads.
//   * One k-step = 4 MFMA sub-steps over LDS buffer `cur` while the next
//     stage is dequantized (codebook lookup, scale, convert) into buffer
//     `cur ^ 1`. 8 waves: each sub-step reads its fragments just before its
//     MFMAs and the other wave of the SIMD covers the wait; x is stored at
//     the start of the k-step; one barrier at the end. 4 waves: fragments
//     and codebook values are read a sub-step ahead, MFMAs are interleaved
//     with the dequant work, and the barrier sits before sub-step 3.
//   * LDS tiles use a 16-byte-chunk XOR swizzle (chunk c of row r at
//     c ^ (r & 7) ^ ((r >> 3) & 1)): MFMA operand reads are conflict free on
//     gfx950's 64-bank LDS.
//   * Codebooks sit in LDS as f16 values in 32 bank-interleaved copies (one
//     32-bit slot each; lane l reads copy l % 32, in bank l % 32), so random
//     code lookups are conflict free, and each value feeds a mixed-precision
//     FMA (v_fma_mix_f32) directly. f16 keeps the NF8 grid (values in
//     [0, 255]) to 2^-11 relative, finer than the bf16 the reference's
//     kernels cast it to.
//   * Outliers: each weight row is dequantized by two threads (32 columns
//     of a k-step each) that walk the row's outliers in column order (a derived
//     column-sorted table) and adds each delta into the element it has just
//     written with an LDS packed add (ds_pk_add_bf16 / _f16), i.e.
//     w = cast(cast(w) + cast(delta)), as modules.py:918 folds them into the
//     dense W. The next entry is loaded a k-step ahead; a second outlier of the
//     same row in one k-step waits for its load (a synchronous load the
//     compiler does not track, so the common path never drains).
#pragma once
#include <algorithm>
#include <mutex>
#include <type_traits>

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
  // K split across workgroups (k_split > 1): workgroup (tile, s) covers
  // k-steps [s KT / k_split, (s + 1) KT / k_split) and stores its fp32 sums
  // to part[s][M][N] (row stride N); splitk_reduce adds them up, with the
  // bias, into y.
  float* part;
  int32_t k_split;
  int32_t bm, bn;  // the launch's tile (host side: the kernel has it as template arguments)
  // byte extents of the buffers read through buffer resources (all < 2^31)
  uint32_t x_bytes, p_bytes, meta_elems, dqm_bytes, s2_bytes, ocs_bytes;
};

constexpr int PF_BM = 256;
constexpr int PF_BK = 64;
constexpr uint32_t PF_NO_COL = 0xffffu;  // column of the "no more outliers" entry
constexpr int PF_CUS = 256;              // MI355X compute units
constexpr int PF_SPLIT_MAX = 8;          // K splits per tile at most
constexpr int PF_SPLIT_MIN_KT = 8;       // k-steps per split at least
#ifndef PF_NW_WIDE
#define PF_NW_WIDE 8  // waves per workgroup of the 256 x 256 tile
#endif

// Two floats -> packed (lo, hi) bf16/f16 pair, round to nearest even
// (v_cvt_pk_bf16_f32 on gfx950).
template <bool BF16>
TS_DEV uint32_t to_pair(float lo, float hi) {
  const ts_f32x2 v = {lo, hi};
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ts_bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ts_f16x2));
}

// LDS offset (in uint16 elements) of 16-byte chunk c of row r in a [rows][64]
// tile. gfx950 serves ds_read_b128 16 lanes at a time over 64 banks (256 B):
// the MFMA operand reads (lanes 0-15 = rows r..r+15, one chunk column) are
// conflict free when rows r and r + 8, which share r & 7 and the bank half
// given by r & 1, land on different chunk positions, hence the (r >> 3) term
// (measured: 40 % more b128 read throughput than c ^ (r & 7) alone).
TS_DEV int swz(int r, int c) { return r * PF_BK + ((c ^ (r & 7) ^ ((r >> 3) & 1)) << 3); }

// Synchronous 32-bit global load for the rare path of the outlier walk (a
// second outlier of one row within one k-step). Issued from inline asm with
// its own wait, so that the compiler sees no load in the branch: a load it
// tracks inside a divergent branch makes it wait for every outstanding load
// (vmcnt(0)) where the branches join, which drained the weight and x
// prefetches on every k-step.
TS_DEV uint32_t ts_load_sync(const uint32_t* p) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}

// Workgroup index -> tile index, so that the workgroups one XCD runs (the
// hardware deals workgroups out to the 8 XCDs round robin) take consecutive
// tiles: the 256-row M tiles of one weight tile then share that XCD's L2.
TS_DEV int64_t xcd_tile(int64_t b, int64_t n) {
  const int64_t x = b & 7, i = b >> 3;
  const int64_t q = n >> 3, r = n & 7;  // XCD x runs q + (x < r) workgroups
  return x * q + min(x, r) + i;
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN, int NW, int BM>
__global__ __launch_bounds__(64 * NW, 1) void prefill_kernel(const PrefillArgs a_in) {
  constexpr int BK = PF_BK, NT = 64 * NW;
  constexpr int WN = NW / 2;                    // waves along N (two along M)
  constexpr int TM = BM / 64;                   // 32-row blocks per wave along M (BM / 2 rows)
  constexpr int TN = BN / (32 * WN);            // 32-column blocks per wave along N
  constexpr int TPR = NT / BN;                  // threads per weight row (1 or 2)
  constexpr int CPT = BK / TPR;                 // weight codes per thread per k-step (64 or 32)
  constexpr int C8 = CPT / 8;                   // 8-code chunks per thread per k-step
  constexpr int SB = RVQ ? 4 : BITS;            // stage-1 bits
  constexpr int WB = CPT * SB / 8;              // stage-1 packed bytes per thread per k-step
  constexpr int WW = WB / 4;                    // ... in dwords
  constexpr int WW2 = RVQ ? CPT / 16 : 1;       // stage-2 dwords (16 two-bit codes each)
  constexpr int NGT = CPT > GS ? CPT / GS : 1;  // groups a thread's codes span in a k-step
  constexpr int CBN = CB ? (1 << BITS) : 1;
  constexpr int CBC = 32;                       // codebook copies: lane l reads copy l % 32 (bank l % 32)
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
  uint32_t* cbs = reinterpret_cast<uint32_t*>(Bs + 2 * BN * BK);  // [CBN][CBC] f16 in the low half

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // wave (wm, wn) of the 2 x WN grid
  const uint32_t cb_lane = lane % CBC;

  // the K splits of a tile are consecutive workgroup indices
  const int P = a.k_split;
  const int64_t lin = xcd_tile(blockIdx.x, a.m_tiles * a.n_tiles * P);
  const int64_t tile = lin / P;
  const int split = (int)(lin - tile * P);
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
  // this workgroup's k-steps: kt0 .. kt0 + KT - 1 (k-step indices below are
  // relative to kt0)
  const int KT_all = (int)(a.K / BK);
  const int kt0 = (int)(((int64_t)split * KT_all) / P);
  const int KT = (int)(((int64_t)(split + 1) * KT_all) / P) - kt0;

  // ---- raw load stage (registers only; nothing computes on the data here) --
  struct Stage {
    uint32_t w[WW];
    uint32_t w2[WW2];
    uint32_t sc[NGT], gc[NGT];  // DQ codes, or f16 scale / gmin bits
    uint32_t sm[NGT], gm[NGT];  // DQ (meta_scale, meta_min) f16 pairs
    uint32_t s2[NGT];           // RVQ stage-2 (scale, gmin) f16 bits
  };
  // x: thread tid owns chunk column tid & 7 of rows tid / 8 + (NT / 8) i. Rows
  // past M and chunks whose columns lie past `cols` are read at offsets past
  // the buffer's extent (bit 31 set for the latter), which the buffer load
  // returns as zeros; those rows are never stored.
  ts_u32x4 X[XCH];
  const uint32_t xbase = (uint32_t)((m0 + (tid >> 3)) * a.ldx) * 2u + (tid & 7) * 16u;
  const uint32_t xstep = (uint32_t)((NT / 8) * a.ldx * 2);
  const int xcol = (tid & 7) * 8;
  auto load_x = [&](int kt, ts_u32x4* xr) {
    kt = kt0 + min(kt, KT - 1);
    const uint32_t kb = (uint32_t)kt * (BK * 2);
    const uint32_t oob = (kt * BK + xcol < a.cols) ? 0u : 0x80000000u;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int64_t m = m0 + (tid >> 3) + (NT / 8) * i;
      xr[i] = ts_bld16s(rx, (m < a.M ? xbase + i * xstep : 0x7fffffffu) | oob, kb);
    }
  };
  auto store_x = [&](int buf, const ts_u32x4* xr) {
    uint16_t* Ab = As + buf * BM * BK;
#pragma unroll
    for (int i = 0; i < XCH; ++i)
      *reinterpret_cast<ts_u32x4*>(Ab + swz((tid >> 3) + (NT / 8) * i, tid & 7)) = xr[i];
  };
  auto load_stage = [&](int kt, Stage& S) {
    kt = kt0 + min(kt, KT - 1);  // a stage past the end re-reads the last k-step (never used)
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
    float s[NGT], g[NGT], s2[NGT], gg[NGT];  // gg: g + stage-2 gmin (RVQ)
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
        Q.gg[t] = Q.g[t] + ts_h2f((uint16_t)(S.s2[t] >> 16));
      }
    }
  };
  // The dequant of a stage runs in NPART parts (part p covers chunks
  // [p * C8 / NPART, (p + 1) * C8 / NPART)). With a codebook, lookup() reads a part's
  // code values from LDS as f16 pairs one sub-step before finish() scales,
  // converts and writes them, so the reads are in flight under MFMAs.
  // Uniform codes are converted inside finish().
  constexpr int NPART = NW > 4 ? 4 : 3;                  // dequant parts per stage
  constexpr int MAXP = CB ? (C8 + NPART - 1) / NPART : 1;  // chunks in the largest part
  struct Codes {
    ts_f16x2 v[MAXP][4];
  };
  const _Float16* cbh = reinterpret_cast<const _Float16*>(cbs) + 2 * cb_lane;
  auto cbval = [&](uint32_t c) { return cbh[c * (2 * CBC)]; };
  auto lookup = [&](const Stage& S, int p, Codes& C) {
    if constexpr (CB) {
#pragma unroll
      for (int c8 = 0; c8 < C8; ++c8) {
        if (!(c8 >= p * C8 / NPART && c8 < (p + 1) * C8 / NPART)) continue;
        ts_f16x2* cv = C.v[c8 - p * C8 / NPART];
        uint32_t c[8];
        if constexpr (SB == 8) {
#pragma unroll
          for (int e = 0; e < 8; ++e) c[e] = (S.w[2 * c8 + (e >> 2)] >> (8 * (e & 3))) & 0xffu;
        } else if constexpr (SB == 4) {
#pragma unroll
          for (int e = 0; e < 8; ++e) c[e] = (S.w[c8] >> (4 * e)) & 15u;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) c[e] = (S.w[c8 >> 1] >> (16 * (c8 & 1) + 2 * e)) & 3u;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cv[e].x = cbval(c[2 * e]);
          cv[e].y = cbval(c[2 * e + 1]);
        }
      }
    }
  };
  auto finish = [&](const Stage& S, const Scales& Q, int p, const Codes& C, int buf) {
    uint16_t* Bb = Bs + buf * BN * BK;
#pragma unroll
    for (int c8 = 0; c8 < C8; ++c8) {
      if (!(c8 >= p * C8 / NPART && c8 < (p + 1) * C8 / NPART)) continue;
      constexpr int GC = GS / 8;  // chunks per group
      const int t = NGT > 1 ? c8 / GC : 0;
      const float sc = Q.s[t], gm = Q.g[t];
      float cv[8];
      if constexpr (CB) {
        const ts_f16x2* h = C.v[c8 - p * C8 / NPART];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cv[2 * e] = (float)h[e].x;
          cv[2 * e + 1] = (float)h[e].y;
        }
      } else if constexpr (SB == 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[e] = (float)((S.w[2 * c8 + (e >> 2)] >> (8 * (e & 3))) & 0xffu);
      } else if constexpr (SB == 4) {
        uint32_t lo = S.w[c8] & 0x0f0f0f0fu, hi = (S.w[c8] >> 4) & 0x0f0f0f0fu;
        asm volatile("" : "+v"(lo), "+v"(hi));  // keeps the byte-select conversions (v_cvt_f32_ubyteN)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cv[2 * e] = (float)((lo >> (8 * e)) & 0xffu);
          cv[2 * e + 1] = (float)((hi >> (8 * e)) & 0xffu);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[e] = (float)((S.w[c8 >> 1] >> (16 * (c8 & 1) + 2 * e)) & 3u);
      }
      float v[8];
      if constexpr (RVQ) {
        // both stages in one affine per element, c1 s + (c2 s2 + (g + g2)):
        // byte 0 of q[k] holds stage-2 code k and byte 1 code k + 4, so each
        // conversion is a byte-select one (v_cvt_f32_ubyteN)
        const uint32_t d2 = S.w2[c8 >> 1] >> (16 * (c8 & 1));
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = (d2 >> (2 * k)) & 0x0303u;
        asm volatile("" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float c2 = (float)((q[e & 3] >> (8 * (e >> 2))) & 0xffu);
          v[e] = __builtin_fmaf(cv[e], sc, __builtin_fmaf(c2, Q.s2[t], Q.gg[t]));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(cv[e], sc, gm);
      }
      ts_u32x4 pk;
      pk.x = to_pair<BF16>(v[0], v[1]);
      pk.y = to_pair<BF16>(v[2], v[3]);
      pk.z = to_pair<BF16>(v[4], v[5]);
      pk.w = to_pair<BF16>(v[6], v[7]);
      *reinterpret_cast<ts_u32x4*>(Bb + swz(wr, wpart * C8 + c8)) = pk;
    }
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
    const uint32_t k0 = (uint32_t)(kt0 + kt) * BK;
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
      if (en_stale) {  // second entry in one k-step
        const uint32_t v = ts_load_sync(a.ocs + min(ptr, oend - 1));
        en = ptr < oend ? v : PF_NO_COL;
      }
      e = en;
      ++ptr;
      en_stale = true;
    }
  };
  // unconditional (also without outliers: roc is then a valid 4-byte dummy)
  auto fetch_outlier = [&]() { tld = oload(min(ptr, oend > 0 ? oend - 1 : 0u)); };

  // ---- prologue --------------------------------------------------------------
  // The row's outlier range is loaded first (unconditionally, through a
  // buffer resource that reads zeros without outliers): its dependent chain
  // (range -> first entry -> next entry) then overlaps the stage loads
  // instead of starting after they land.
  const __amdgpu_buffer_rsrc_t rop = ts_rsrc(a.orow_ptr, a.has_out ? (uint32_t)(4 * (a.N + 1)) : 4u);
  const int64_t orow = min(n0 + wr, a.N);  // a row past N has an empty range
  const uint32_t rb0 = ts_bld4(rop, (uint32_t)(4 * orow));
  const uint32_t re0 = ts_bld4(rop, (uint32_t)(4 * min(orow + 1, a.N)));
  Stage S0, S1;
  load_x(0, X);
  load_stage(0, S0);
  load_stage(1, S1);
  if constexpr (CB) {
    // 16-byte chunks of 4 copies: chunk i holds copies of entry i / (CBC / 4);
    // every thread runs the same trip count (a trailing thread rewrites the
    // last chunk with the same value), so no load sits behind a branch
    constexpr int CH = CBN * CBC / 4;
#pragma unroll
    for (int k = 0; k < (CH + NT - 1) / NT; ++k) {
      const int i = min(tid + k * NT, CH - 1);
      const uint32_t h = ts_f2h(a.codebook[i / (CBC / 4)]);
      *reinterpret_cast<ts_u32x4*>(cbs + 4 * i) = ts_u32x4{h, h, h, h};
    }
  }
  if (a.has_out) {
    uint32_t rb = rb0;
    oend = re0;
    if (kt0 > 0) {
      // a later K split starts at the row's first entry with column >=
      // kt0 * BK: count the entries before it among the next 16 (one round
      // trip), and search the rest of a longer row by bisection
      const uint32_t kb = (uint32_t)kt0 * BK;
      uint32_t below = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t v = oload(min(rb + j, oend > 0 ? oend - 1 : 0u));
        below += (rb + j < oend && (v & 0xffffu) < kb) ? 1u : 0u;
      }
      rb += below;
      if (below == 16) {
        uint32_t hi = oend;
        while (rb < hi) {
          const uint32_t mid = rb + (hi - rb) / 2;
          if ((a.ocs[mid] & 0xffffu) < kb) rb = mid + 1;
          else hi = mid;
        }
      }
    }
    e = rb < oend ? a.ocs[rb] : PF_NO_COL;
    ptr = rb + 1;
    tld = oload(min(ptr, oend > 0 ? oend - 1 : 0u));
  }
  ts_lds_barrier();  // codebook copies
  {
    Scales Q;
    scales(S0, Q);
#pragma unroll
    for (int p = 0; p < NPART; ++p) {
      Codes C;
      lookup(S0, p, C);
      finish(S0, Q, p, C, 0);
    }
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
      F.b[j] = *reinterpret_cast<const ts_u32x4*>(Bb + swz(wn * (BN / WN) + 32 * j + (lane & 31), c));
  };
  auto mfma = [&](const Frag& F) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = ts_mfma32x32x16<BF16>(F.a[i], F.b[j], acc[i][j]);
  };

  // Interleave a sub-step's 16 (TM * TN) MFMAs with the LDS reads, VALU work
  // and LDS writes around them, so the matrix core is fed while the rest
  // issues (one wave per SIMD: a wave stalled on a wait leaves it idle).
  auto interleave = [&]() {
    if constexpr (NW > 4) return;  // two waves per SIMD: the hardware interleaves them
#pragma unroll
    for (int i = 0; i < TM * TN; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
    }
  };
  if constexpr (NW > 4) {
    // Two waves per SIMD: each sub-step reads its fragments just before its
    // MFMAs and the dequant parts follow without look-ahead (the other wave
    // on the SIMD covers the waits); one barrier at the end of the k-step.
    // (An explicit ping-pong, the two waves of a SIMD alternating between
    // memory and MFMA phases separated by barriers, measured slower.)
    load_x(1, X);
    auto kstep8 = [&](int kt, Stage& S) {
      const int cur = kt & 1, nxt = cur ^ 1;
      // x of kt + 1 (loaded a k-step ago) goes to nxt first, which no wave
      // reads until after this k-step's barrier; X then takes kt + 2.
      store_x(nxt, X);
      load_x(kt + 2, X);
      Scales Q;
      scales(S, Q);
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) {
        Frag F;
        Codes C;
        lookup(S, sub, C);
        read_frag(cur, sub, F);
        mfma(F);
        finish(S, Q, sub, C, nxt);
      }
      fold_outliers(kt + 1, nxt);
      fetch_outlier();
      load_stage(kt + 3, S);
      ts_lds_barrier();
    };
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
      kstep8(kt, S1);
      kstep8(kt + 1, S0);
    }
    if (kt < KT) kstep8(kt, S1);
  } else {
  Frag F0, F1;
  Codes CA, CB2;
  read_frag(0, 0, F0);
  lookup(S1, 0, CA);
  // One k-step (S = stage kt + 1, Sn = stage kt + 2). x for k-step kt + 1 is
  // loaded into X; S is dequantized into buffer nxt over sub-steps 0-2 (part
  // 0's codes were looked up in the previous k-step) and refilled with
  // k-step kt + 3; X is stored to nxt; barrier; sub-step 3 runs on fragments
  // already in registers while the next k-step's first fragments and part 0
  // of Sn's codes are read.
  auto kstep = [&](int kt, Stage& S, const Stage& Sn) {
    const int cur = kt & 1, nxt = cur ^ 1;
    Scales Q;
    load_x(kt + 1, X);
    scales(S, Q);
    read_frag(cur, 1, F1);
    lookup(S, 1, CB2);
    mfma(F0);
    finish(S, Q, 0, CA, nxt);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 2, F0);
    lookup(S, 2, CA);
    mfma(F1);
    finish(S, Q, 1, CB2, nxt);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    read_frag(cur, 3, F1);
    mfma(F0);
    finish(S, Q, 2, CA, nxt);
    store_x(nxt, X);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    fold_outliers(kt + 1, nxt);
    fetch_outlier();
    load_stage(kt + 3, S);
    ts_lds_barrier();
    read_frag(nxt, 0, F0);
    lookup(Sn, 0, CA);
    mfma(F1);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
  };
  // two k-steps per iteration (the stages alternate), one exit
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    kstep(kt, S1, S0);
    kstep(kt + 1, S0, S1);
  }
  if (kt < KT) kstep(kt, S1, S0);
  }

  // ---- epilogue: bias, cast, store (a K split: its fp32 sums) ---------------
  // A lane's accumulators are 16 values of one output column (rows
  // 8 (r >> 2) + 4 (lane >> 5) + (r & 3) of a 32-row block): stored as they
  // are, every store instruction writes one 2- or 4-byte element per lane.
  // Each wave instead stages one 32 x 32 TN block at a time in a private LDS
  // region (the operand buffers are free once every wave is past the
  // barrier) and stores whole 16-byte row chunks. Outputs whose rows are not
  // 16-byte aligned take the element-wise path.
  const bool f32out = P > 1 || a.y_dtype == TS_F32;
  const int esz = f32out ? 4 : 2;
  char* const dst_base =
      P > 1 ? reinterpret_cast<char*>(a.part + (int64_t)split * a.M * a.N) : static_cast<char*>(a.y);
  const int64_t ld = P > 1 ? a.N : a.ldy;
  const int64_t mw = m0 + wm * (BM / 2), nw = n0 + wn * (BN / WN);  // the wave's first row and column
  if ((reinterpret_cast<uintptr_t>(dst_base) & 15) == 0 && (ld * esz) % 16 == 0) {
    constexpr int SC = 32 * TN;  // columns of a wave block
    constexpr int SS = SC + 8;   // staged row stride in elements: rows r and r + 4 sit 32 banks apart
    static_assert(NW * 32 * SS * 4 <= 2 * (BM + BN) * PF_BK * 2, "staging fits the operand buffers");
    ts_lds_barrier();  // every wave is past its last operand read
    char* const stage = reinterpret_cast<char*>(smem) + wave * (32 * SS * 4);
    float bv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = nw + 32 * j + (lane & 31);
      bv[j] = (P == 1 && a.bias && n < a.N) ? XT<BF16>::to_f(a.bias[n]) : 0.f;
    }
    // ESZ: bytes per staged element (4: fp32 partials or output, 2: bf16/f16)
    auto blocks = [&](auto esz_c) {
      constexpr int ESZ = decltype(esz_c)::value;
      constexpr int CPR = SC * ESZ / 16;  // 16-byte chunks per row
      constexpr int EPC = 16 / ESZ;       // elements per chunk
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), col = 32 * j + (lane & 31);
            const float v = acc[i][j][r] + bv[j];
            if constexpr (ESZ == 4) reinterpret_cast<float*>(stage)[row * SS + col] = v;
            else reinterpret_cast<uint16_t*>(stage)[row * SS + col] = XT<BF16>::from_f(v);
          }
        }
        // (one wave's LDS accesses complete in order: the reads see the
        // writes above, and the next block's writes come after these reads)
#pragma unroll
        for (int k = 0; k < 32 * CPR / 64; ++k) {
          const int c = lane + 64 * k;
          const int row = c / CPR, ch = c % CPR;
          const int64_t m = mw + 32 * i + row, n = nw + ch * EPC;
          if (m >= a.M) continue;
          const ts_u32x4 v = *reinterpret_cast<const ts_u32x4*>(stage + row * SS * ESZ + ch * 16);
          char* const dst = dst_base + (m * ld + n) * ESZ;
          if (n + EPC <= a.N) {
            *reinterpret_cast<ts_u32x4*>(dst) = v;
          } else {  // the last chunk of a ragged row
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            for (int e = 0; e < EPC && n + e < a.N; ++e) {
              if constexpr (ESZ == 4) reinterpret_cast<uint32_t*>(dst)[e] = w[e];
              else reinterpret_cast<uint16_t*>(dst)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
      }
    };
    if (f32out) blocks(std::integral_constant<int, 4>{});
    else blocks(std::integral_constant<int, 2>{});
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = nw + 32 * j + (lane & 31);
    if (n >= a.N) continue;
    const float b = (P == 1 && a.bias) ? XT<BF16>::to_f(a.bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = mw + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= a.M) continue;
        const float v = acc[i][j][r] + b;
        char* const dst = dst_base + (m * ld + n) * esz;
        if (f32out) *reinterpret_cast<float*>(dst) = v;
        else *reinterpret_cast<uint16_t*>(dst) = XT<BF16>::from_f(v);
      }
    }
  }
}

template <int BITS, bool CB, int BN, int BM>
constexpr size_t prefill_smem() {
  constexpr int CBN = CB ? (1 << BITS) : 0;
  return (size_t)2 * (BM + BN) * PF_BK * 2 + (size_t)CBN * 32 * 4;
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN, int NW, int BM = PF_BM>
inline int launch_prefill(PrefillArgs a, hipStream_t st) {
  constexpr size_t smem = prefill_smem<BITS, CB, BN, BM>();
  static_assert(smem <= 160 * 1024, "LDS budget (160 KB per CU)");
  auto kern = prefill_kernel<BITS, GS, BF16, CB, RVQ, DQ, BN, NW, BM>;
  static std::once_flag flags[64];
  static bool ok[64];
  if (!ts_set_smem_once(reinterpret_cast<const void*>(kern), smem, flags, ok)) return TS_HIP_ERROR;
  a.m_tiles = ts_cdiv(a.M, BM);
  a.n_tiles = ts_cdiv(a.N, BN);
  if (a.k_split < 1 || a.k_split > a.K / PF_BK || (a.k_split > 1 && !a.part)) return TS_BAD_ARG;
  hipLaunchKernelGGL(kern, dim3((unsigned)(a.m_tiles * a.n_tiles * a.k_split)), dim3(64 * NW), smem, st, a);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// Launch shape of the prefill kernel for an M x N x K product of a layer
// with `bits`-bit codes (cb: with a codebook): the tile (256 x 256 on 8
// waves, 256 x 128 on 4, 128 x 128 on 4) and the number of workgroups K is
// split across per tile (1-8, at least 8 k-steps each). The choice comes from
// an estimate fitted on MI355X to forced sweeps (618 launches: 4 layer shapes
// x NF4 / NF8 x M = 256-2048 x every tile x 1-8 splits; 5 % rms error):
//   workgroups per CU (rounded up)
//     x (k-steps per split x the tile's k-step time + 2.3 us of prologue and
//        epilogue), k-step times 2.05 / 1.4 / 1.12 us;
//     two 128 x 128 workgroups whose LDS fits one CU together share it at
//     1.4x the time of one;
//   + with splits: the fp32 partial sums' HBM traffic (k_split * M * N * 4
//     bytes written and read, at 5.7 TB/s) and 7.5 us for the reduction
//     pass.
// The incumbent is the tile that fills the CUs unsplit (256 x 256 when those
// tiles do, else 256 x 128, or 128 x 128 when 256 x 128 tiles would leave
// CUs idle and 128 x 128 tiles fit one round); another choice must be
// estimated 3 % faster. Splits pay where tiles are few (narrow layers or
// small M: 4096 x 14336 at M = 256 has 32 tiles of 256 x 128 for 256 CUs)
// and where they let the 256 x 256 tile fill the CUs (the same layer at M =
// 2048: 128 such tiles, two splits). The partials stay below the GEMM
// library path's workspace (rows x cols x 2 + 32 MB). split_ok = false (no
// workspace for the partials): the best unsplit tile.
struct PrefillPlan {
  int bm, bn;
  int64_t tiles;
  int splits;
};
inline PrefillPlan prefill_plan(int64_t M, int64_t N, int64_t K, int bits, bool cb, bool split_ok = true) {
  struct Shape {
    int bm, bn;
    double tk;  // us per k-step of one workgroup
  };
  constexpr Shape shapes[3] = {{256, 256, 2.05}, {256, 128, 1.4}, {128, 128, 1.12}};
  int inc;  // the incumbent shape
  if (ts_cdiv(M, 256) * ts_cdiv(N, 256) >= PF_CUS) inc = 0;
  else if (ts_cdiv(M, 256) * ts_cdiv(N, 128) < PF_CUS && ts_cdiv(M, 128) * ts_cdiv(N, 128) <= PF_CUS) inc = 2;
  else inc = 1;
  // (the LDS size of prefill_smem<bits, cb, 128, 128>; registers allow two
  // such workgroups per CU, but not two of the larger tiles)
  const size_t lds128 = (size_t)2 * 256 * PF_BK * 2 + (cb ? ((size_t)1 << bits) * 32 * 4 : 0);
  const int64_t KT = K / PF_BK;
  const double cap = (double)N * (double)K * 2 + (double)(32 << 20);
  auto estimate = [&](const Shape& sh, int s) {
    const int64_t tiles = ts_cdiv(M, sh.bm) * ts_cdiv(N, sh.bn);
    const bool pair = sh.bm == 128 && 2 * lds128 <= 160 * 1024;
    const int64_t wpc = ts_cdiv(tiles * s, PF_CUS);
    const double rounds = pair ? (double)(wpc / 2) * 1.4 + (double)(wpc % 2) : (double)wpc;
    double t = rounds * ((double)ts_cdiv(KT, s) * sh.tk + 2.3);
    if (s > 1) t += ((double)s * M * N * 8 + (double)M * N * 2) * 1e6 / 5.7e12 + 7.5;
    return t;
  };
  PrefillPlan p{shapes[inc].bm, shapes[inc].bn, ts_cdiv(M, shapes[inc].bm) * ts_cdiv(N, shapes[inc].bn), 1};
  double best = estimate(shapes[inc], 1);
  for (int i = 0; i < 3; ++i) {
    for (int s = 1; s <= (split_ok ? PF_SPLIT_MAX : 1); ++s) {
      if (s > 1 && (KT / s < PF_SPLIT_MIN_KT || (double)s * M * N * 4 >= cap)) break;
      if (i == inc && s == 1) continue;
      const double t = estimate(shapes[i], s);
      if (t < 0.97 * best) {
        best = t;
        p = PrefillPlan{shapes[i].bm, shapes[i].bn, ts_cdiv(M, shapes[i].bm) * ts_cdiv(N, shapes[i].bn), s};
      }
    }
  }
  return p;
}
inline size_t prefill_part_bytes(const PrefillPlan& p, int64_t M, int64_t N) {
  return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * 4 : 0;
}

// y = sum of the K splits' fp32 sums (+ bias), cast to y's dtype.
int launch_splitk_reduce(const PrefillArgs& a, bool bf16, hipStream_t st);

// a.bm / a.bn / a.part / a.k_split: the caller's plan (k_split = 1 without
// workspace)
template <int BITS, int GS, bool BF16, bool CB, bool RVQ>
inline int launch_prefill_tiles(PrefillArgs& a, hipStream_t st) {
  const bool dq = a.dqsc != nullptr;
  int rc;
  if (a.bn == 256) {
    rc = dq ? launch_prefill<BITS, GS, BF16, CB, RVQ, true, 256, PF_NW_WIDE>(a, st)
            : launch_prefill<BITS, GS, BF16, CB, RVQ, false, 256, PF_NW_WIDE>(a, st);
  } else if (a.bm == 128) {
    rc = dq ? launch_prefill<BITS, GS, BF16, CB, RVQ, true, 128, 4, 128>(a, st)
            : launch_prefill<BITS, GS, BF16, CB, RVQ, false, 128, 4, 128>(a, st);
  } else {
    rc = dq ? launch_prefill<BITS, GS, BF16, CB, RVQ, true, 128, 4>(a, st)
            : launch_prefill<BITS, GS, BF16, CB, RVQ, false, 128, 4>(a, st);
  }
  if (rc == TS_OK && a.k_split > 1) rc = launch_splitk_reduce(a, BF16, st);
  return rc;
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
