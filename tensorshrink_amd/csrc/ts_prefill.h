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
// Tile: 256 x BN x 64 per workgroup of 4 waves (2 x 2), each wave 128 x BN/2
// as 4 x BN/64 MFMA 32x32 blocks; one wave per SIMD.
//   * Raw global loads (x chunks, packed codes, scale / double-quant metadata)
//     go into two register stages and are issued two k-steps ahead, all
//     unconditional (addresses clamped into valid memory), so the compiler's
//     wait counts stay exact and a k-step only waits for the stage it
//     dequantizes. Nothing computes on loaded data in the load phase.
//   * Each k-step runs 4 MFMA sub-steps on LDS buffer `cur`, each followed by
//     a quarter of the next k-step's dequant (and x copy) into buffer
//     `cur ^ 1`, so the VALU work overlaps the matrix core; one LDS-only
//     barrier per k-step (a __syncthreads would drain the prefetch).
//   * LDS tiles use a 16-byte-chunk XOR swizzle (chunk c of row r at
//     c ^ (r & 7)): both the tile writes and the MFMA operand reads are
//     bank-conflict free.
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
constexpr int PF_OMAX = 64;  // outliers per tile row staged in LDS

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

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN>
__global__ __launch_bounds__(256, 1) void prefill_kernel(const PrefillArgs a_in) {
  constexpr int BM = PF_BM, BK = PF_BK;
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int A_CHUNKS = BM * 8 / 256;      // 16-byte x chunks per thread per k-step
  constexpr int CPT = BN * BK / 256;          // weight codes per thread per k-step
  constexpr int TPR = BK / CPT;               // threads per weight row
  constexpr int WB = CPT * BITS / 8;          // packed bytes per thread per k-step
  constexpr int WB2 = RVQ ? CPT / 4 : 0;      // RVQ stage-2 bytes
  constexpr int C8 = CPT / 8;                 // 8-code chunks per thread per k-step
  constexpr int NGT = CPT >= GS ? CPT / GS : 1;  // groups a thread's codes span in a k-step
  constexpr int CBN = (CB && BITS == 8) ? 256 : 16;
  static_assert(C8 % 4 == 0 || C8 == 2, "dequant chunks per sub-step");
  static_assert(WB % 4 == 0, "packed chunk");
  extern __shared__ __align__(16) unsigned char smem[];

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
  float* cbs = reinterpret_cast<float*>(Bs + 2 * BN * BK);      // codebook
  uint32_t* ol = reinterpret_cast<uint32_t*>(cbs + CBN);        // [BN][OMAX] col | f16 delta << 16
  int32_t* ocnt = reinterpret_cast<int32_t*>(ol + BN * PF_OMAX);  // [BN] outliers per tile row

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

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
    const int ch = tid + i * 256;
    xoff[i] = (uint32_t)(min(m0 + (ch >> 3), a.M - 1) * a.ldx) * 2u + (ch & 7) * 16u;
  }
  auto load_x = [&](int kt, ts_u32x4* xr) {
    const uint32_t kb = (uint32_t)min(kt, KT - 1) * (BK * 2);
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) xr[i] = ts_bld16(rx, xoff[i] + kb);
  };
  auto store_x = [&](int buf, int kt, const ts_u32x4* xr) {
    uint16_t* Ab = As + buf * BM * BK;
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int ch = tid + i * 256;
      const int r = ch >> 3, c = ch & 7;
      const bool inb = k0 + c * 8 < a.cols;
      *reinterpret_cast<ts_u32x4*>(Ab + swz(r, c)) = inb ? xr[i] : ts_u32x4{0u, 0u, 0u, 0u};
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
  // Moving pointer over this row's sorted outliers.
  int opos = 0;
  int oncnt = 0;  // staged outliers of this row (set after staging)
  int64_t o_begin = 0, o_count = 0;
  auto dequant_part = [&](const Stage& S, int part, int buf, int kt) {
    uint16_t* Bb = Bs + buf * BN * BK;
    const int k0 = kt * BK;
    constexpr int CP = C8 >= 4 ? C8 / 4 : 1;  // 8-code chunks per part
    if (C8 < 4 && part >= C8) return;
#pragma unroll
    for (int cc = 0; cc < CP; ++cc) {
      const int c8 = (C8 >= 4 ? part * CP : part) + cc;
      const int t = (c8 * 8) / (CPT >= GS ? GS : CPT);  // group of this chunk within the thread's codes
      const int tg = NGT > 1 ? t : 0;
      float s, gm;
      if constexpr (DQ) {  // modules.py:573-579: code * meta_scale + meta_min in float32
        s = __fadd_rn(__fmul_rn((float)S.sc[tg], ts_h2f(S.sm[tg] & 0xffffu)), ts_h2f(S.sm[tg] >> 16));
        gm = __fadd_rn(__fmul_rn((float)S.gc[tg], ts_h2f(S.gm[tg] & 0xffffu)), ts_h2f(S.gm[tg] >> 16));
      } else {
        s = ts_h2f((uint16_t)S.sc[tg]);
        gm = ts_h2f((uint16_t)S.gc[tg]);
      }
      float cv[8];
      if constexpr (BITS == 4) {
        const uint32_t d = S.w[c8];
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
        const uint32_t d = S.w[c8 >> 1] >> (16 * (c8 & 1));  // 8 codes in 16 bits
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t c = (d >> (2 * e)) & 3u;
          cv[e] = CB ? cbs[c] : (float)c;
        }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t d = S.w[2 * c8 + h];
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
    if (part == 3 && o_count > 0) {
      // fold this row's outliers that land in the thread's slice of the k-step
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
    for (int i = tid; i < CBN; i += 256) cbs[i] = a.codebook[i];
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
  for (int part = 0; part < 4; ++part) dequant_part(S0, part, 0, 0);
  store_x(0, 0, X0);
  load_stage(2, S0);
  ts_lds_barrier();

  ts_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = ts_f32x16{};

  // One k-step: x for k-step kt + 2 is issued into XL first; MFMAs on LDS
  // buffer `cur`, interleaved with the dequant of stage S (k-step kt + 1)
  // into the other buffer; S is refilled with k-step kt + 3; then x for
  // k-step kt + 1 (issued a k-step ago, in XS) goes to the other buffer.
  auto kstep = [&](int kt, Stage& S, ts_u32x4* XL, const ts_u32x4* XS) {
    const int cur = kt & 1;
    const uint16_t* Ab = As + cur * BM * BK;
    const uint16_t* Bb = Bs + cur * BN * BK;
    load_x(kt + 2, XL);
    asm volatile("" ::: "memory");  // keep the x loads here, ahead of the MFMA phase
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
      dequant_part(S, s, cur ^ 1, kt + 1);
    }
    load_stage(kt + 3, S);
    store_x(cur ^ 1, kt + 1, XS);
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
          const int64_t m = min(m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), a.M - 1);
          acc[i][j][r] += XT<BF16>::to_f((uint16_t)ts_bld2(rx, ((uint32_t)(m * a.ldx) + col) * 2u)) * d;
        }
      }
    }
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
inline size_t prefill_smem() {
  constexpr int CBN = (CB && BITS == 8) ? 256 : 16;
  return (size_t)2 * (PF_BM + BN) * PF_BK * 2 + CBN * 4 + (size_t)BN * PF_OMAX * 4 + (size_t)BN * 4;
}

template <int BITS, int GS, bool BF16, bool CB, bool RVQ, bool DQ, int BN>
inline int launch_prefill(PrefillArgs a, hipStream_t st) {
  const size_t smem = prefill_smem<BITS, CB, BN>();
  auto kern = prefill_kernel<BITS, GS, BF16, CB, RVQ, DQ, BN>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess)
      return TS_HIP_ERROR;
    attr_set = true;
  }
  a.m_tiles = ts_cdiv(a.M, PF_BM);
  a.n_tiles = ts_cdiv(a.N, BN);
  hipLaunchKernelGGL(kern, dim3((unsigned)(a.m_tiles * a.n_tiles)), dim3(256), smem, st, a);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// 256 x 128 tiles: with two k-steps of weights in flight in registers a
// 256 x 256 tile does not fit the 256 architectural VGPRs of a wave (the
// accumulators take all 256 AGPRs) and spills.
template <int BITS, int GS, bool BF16, bool CB, bool RVQ>
inline int launch_prefill_tiles(PrefillArgs& a, hipStream_t st) {
  if (a.dqsc != nullptr) return launch_prefill<BITS, GS, BF16, CB, RVQ, true, 128>(a, st);
  return launch_prefill<BITS, GS, BF16, CB, RVQ, false, 128>(a, st);
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
