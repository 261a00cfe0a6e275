// Decode (M <= 16, and up to 64 in MB blocks of 16 tokens) quantized linear:
// y[M, N] = x[M, K] W^T + outliers + bias.
//
// Replaces the reference's fused Triton GEMV/skinny-GEMM
// (triton_kernels.py:278-541, dispatched at modules.py:881-894) and its
// standalone outlier pass (triton_kernels.py:543-576, 940-941).
//
// Work unit: a tile of 16 weight rows x all of K, one workgroup of W waves
// (4, 8 or 16) per tile; wave w owns a contiguous run of the tile's group
// batches. Layers that read the same x can share a launch (DecodeGroup).
//   * MFMA f32_16x16x32 (bf16 or f16): lane l owns W row r0 + l%16 (B column)
//     and x row l%16 (A row); lane group q = l/16 owns a quarter of each group,
//     so one group is GS/32 MFMAs over that lane set. MB > 1: block tb's x
//     rows 16 tb + l%16, with the group's code-table entries read once for
//     all blocks.
//   * Each lane loads its quarter-group of packed codes with 8/16-byte loads,
//     U groups per batch, two batches in registers. A batch's per-group
//     metadata comes in a few vector loads: U scale/double-quant codes in one
//     load when the batch is aligned, and the (at most two) double-quant
//     super-groups it spans in four.
//   * Codes become bf16/f16 pairs through an LDS table indexed by the packed
//     byte (4-bit: one u32 = two codes; 2-bit: one u64 = four codes), kept in
//     bank-private copies (up to one per lane of a half-wave).
//   * The per-group affine is factorised out of the MFMA:
//         y += s[n,g] * (x . cb[c]) + gmin[n,g] * (x . 1)
//     with s/gmin in float32 (rebuilt from double-quant codes in-register,
//     modules.py:573-579). x . cb[c] runs on the matrix core; x . 1 too at
//     M > 1, while at M = 1 (one sum per group, the same for every row) it is
//     a lane reduction of the x chunks the lanes already hold.
//   * x at M = 1 comes in one 16-byte load per lane and batch, is written to
//     a wave-private LDS slot and read back per MFMA with the 16 lanes of a
//     row on one address (a broadcast read, no VALU); at M > 1 it is
//     staged once per workgroup in LDS when M*K fits, else read per MFMA from
//     global memory, with two 16-row tiles per workgroup sharing each
//     fragment when the launch is large.
//   * 4-byte quarter-group codes (2-bit group 64, 4-bit group 32) come as one
//     16-byte load per lane and a cross-row dword transpose.
//   * Per tile: the waves' partials reduced in LDS, the tile's outliers (its
//     per-tile slots) added with LDS float atomics, then bias and the
//     compute-dtype store.
//
// Latency rules the code follows (each was measured to matter on gfx950):
//   * kernel arguments are pinned in SGPRs at entry (one batch of scalar loads
//     instead of several dependent ones);
//   * the workgroup's barriers (x staging, code tables) come before the weight
//     stream, so no barrier waits for every wave to have issued its loads;
//   * every weight load is issued before anything waits: loads are
//     unconditional (addresses clamped into valid memory, predicates applied
//     where the value is used), since a load under a branch is followed by a
//     wait at the join;
//   * LDS barriers wait for LDS traffic only (ts_lds_barrier), never for the
//     weight loads in flight.
#pragma once
#include <utility>
#include <algorithm>

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
  uint32_t dqm_bytes;        // bytes of dqsm / dqgm (4 per super-group)
  const uint8_t* s2packed;
  int64_t s2stride;
  const uint16_t* s2scale;
  const uint16_t* s2gmin;
  const uint64_t* slots;     // per-tile outlier slots (ts_qlayer.tile_outliers), or any valid
                             // 8-byte array when cap == 0
  int32_t cap;               // slots per tile (0: no outliers; -1: DecodeCsr instead)
  const uint16_t* x;
  int64_t ldx;
  void* y;
  int64_t ldy;
  int y_dtype;
  const uint16_t* bias;      // nullptr when there is no bias
  int64_t N;
  int64_t cols;
  int64_t K;                 // padded columns
  int64_t n_groups;
  int64_t n_tiles;
  int M;
  const float* cbsrc;        // codebook (read when cb_mode == CB_DEVICE)
  int cb_mode;               // CB_UNIFORM, CB_INLINE or CB_DEVICE
  uint32_t cbq[16];          // CB_UNIFORM / CB_INLINE: entry j - cb0 in the activation type (bits in 0..15)
  float cb0;                 // the centre subtracted from cbq (0 for uniform grids and RVQ stage 1)
  const uint16_t* bias_src;  // bias, or any valid array when there is none
  int64_t bias_mul;          // 1 with a bias, else 0
};

// Several layers that read the same activations (q/k/v, gate/up) in one
// launch: the grid is the concatenation of their tiles, and each workgroup
// takes the arguments of the layer its tile belongs to.
constexpr int DEC_GMAX = 4;  // layers per launch
enum { CB_UNIFORM = 0, CB_INLINE = 1, CB_DEVICE = 2 };
// A layer without the slot table (outliers crowded into a few tiles, so the
// padded table was not built; cap == -1): each tile reads its outliers from
// the row-sorted tables through the CSR row offsets. Kept apart from
// DecodeArgs, which every workgroup copies into SGPRs at entry.
struct DecodeCsr {
  const int32_t* row_ptr;
  const int32_t* row;
  const int32_t* col;
  const uint16_t* delta;
};
struct DecodeGroup {
  DecodeArgs a[DEC_GMAX];
  int64_t tile_end[DEC_GMAX];  // cumulative tile counts
  int n;
  DecodeCsr csr[DEC_GMAX];
};

constexpr size_t DEC_XLDS_MAX = 64 * 1024;  // activations staged in LDS up to this size
enum { XM_GLOBAL = 0, XM_DMA = 1, XM_REG = 2, XM_SLOT = 3 };
// 16-byte x chunks per thread with XM_REG: 4 with 8 or 16 waves (x up to
// 32 / 64 KB: a 14336- / 28672-wide row at M = 1), else 2.
constexpr int xreg_chunks(int w) { return w >= 8 ? 4 : 2; }

// v_writelane_b32 of v[J] into lane J of q for every J (lane selects are
// inline constants; the values come from SGPRs)
template <int J>
TS_DEV void ts_writelane(int& q, uint32_t v) {
  asm("v_writelane_b32 %0, %1, %2" : "+v"(q) : "s"(v), "I"(J));
}
template <int... J>
TS_DEV void ts_writelanes(int& q, const uint32_t* v, std::integer_sequence<int, J...>) {
  (ts_writelane<J>(q, v[J]), ...);
}

template <bool BF16>
TS_DEV uint32_t pack2(float lo, float hi) {
  return (uint32_t)XT<BF16>::from_f(lo) | ((uint32_t)XT<BF16>::from_f(hi) << 16);
}

template <int NB>
struct Bytes {
  uint32_t d[(NB + 3) / 4];
};

// NB bytes (1, 2, 4, 8, 16 or 32) from an NB-aligned address, one or two loads.
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

// v moved within a 16-lane row by DPP control CTRL (every source lane valid).
template <int CTRL>
TS_DEV float ts_dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// v[l] + v[l ^ 32] and v[l] + v[l ^ 16] on every lane.
TS_DEV float ts_sum_x32(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto p = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
}
TS_DEV float ts_sum_x16(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto p = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  return __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
}

TS_DEV uint32_t byte_of(const uint32_t* d, int i) { return (d[i >> 2] >> (8 * (i & 3))) & 0xffu; }
TS_DEV uint32_t half_of(const uint32_t* d, int i) { return (d[i >> 1] >> (16 * (i & 1))) & 0xffffu; }

// Bank-private copies of a code table. REP = 32 asks for one copy per lane of
// a half-wave (conflict-free lookups, 32 KB for a 4-bit table) where one
// workgroup fills a CU (16 waves); with fewer waves per workgroup several
// workgroups share the CU's LDS and get fewer copies.
constexpr int dec_rep(int rep, int w) { return rep >= 32 ? (w >= 16 ? 32 : (w >= 8 ? 16 : 4)) : rep; }
// With x in per-wave slots (XM_SLOT) the LDS holds the tables and 1 KB per wave: four 4-wave
// workgroups per CU fit 16 copies each.
// M = 1 launches of 8 or 16 waves (one or two workgroups per CU) lay the
// 4-bit code table out in 256-byte rows (see the kernel)
constexpr bool dec_t4w(int bits, bool rvq, int xm, int w) { return bits == 4 && !rvq && xm == 3 && w >= 8; }
constexpr int dec_rep_x(int rep, int w, int xm) { return (xm == 3 && rep >= 32 && w == 4) ? 16 : dec_rep(rep, w); }

template <int BITS, int GS, bool RVQ>
struct DecGeom {
  static constexpr int GB = GS * BITS / 8;  // packed bytes per row per group
  static constexpr int LB = GB / 4;         // bytes per lane per group
  static constexpr int GB2 = GS / 4;        // RVQ stage-2 bytes per row per group
  static constexpr int LB2 = GB2 / 4;
  static constexpr int U0 = (LB + (RVQ ? LB2 : 0)) > 0 ? 64 / (LB + (RVQ ? LB2 : 0)) : 8;
  // largest groups per batch (~64 B of codes per lane), a power of two in [1, 8]
  static constexpr int UMAX = U0 >= 8 ? 8 : (U0 >= 4 ? 4 : (U0 >= 2 ? 2 : 1));
};

// W: waves per workgroup (4, 8 or 16), all on the same tile, each owning a
// contiguous run of its batches of U groups. NB = 1 or 2: every wave has at
// most NB batches and the kernel is straight-line code (with NB = 1 no second
// batch is loaded at all). The host spreads a tile over more waves when there
// are few tiles, so a small layer still has several waves per SIMD to hide
// LDS and MFMA latency. NB = 0 (LOOP) streams longer runs through the two
// register buffers.
// XM: where the A operand (x) comes from: XM_GLOBAL reads it from global
// memory per MFMA (x too large for LDS); XM_REG stages it in LDS through
// registers (at most xreg_chunks(W) 16-byte chunks per thread); XM_DMA stages it
// with direct global->LDS loads. XM_REG keeps the compiler's wait counts
// exact, so a wave computes its first batch while the second is in flight;
// with direct-to-LDS loads pending the compiler treats the load counter as
// out of order and its first wait drains everything. XM_SLOT (M = 1): no
// workgroup staging; each batch brings its x columns in one load per lane
// (CPM columns), lane 16 q + s holding the chunk that MFMA (u, j) = (s / NMF,
// s % NMF) of lane group q needs; the wave writes them to its own LDS slot
// and each MFMA reads its chunk back on one address per 16-lane row (DPP row
// broadcasts of the chunks, the earlier design, cost 16 VALU moves per group).
// AL: the row's group count is a multiple of U, so every batch starts on a
// multiple of U in the row-major (row, group) metadata arrays and its U codes
// / scales come in one aligned vector load.
// Occupancy: at most 128 VGPRs (4 waves per SIMD, 16 per CU), so 1024 waves
// of 16-row tiles are resident at once across 256 CUs.
template <int BITS, int GS, bool BF16, bool CB8, bool RVQ, int REP, int XM, bool DQ, bool AL, int W, int U,
          int NB, int RT, int MB>
__global__ __launch_bounds__(64 * W, 4) void decode_kernel(const DecodeGroup g) {
  constexpr int NT = 64 * W;
  constexpr bool LOOP = NB == 0;
  constexpr int R = dec_rep_x(REP, W, XM);  // table copies
  constexpr bool XLDS = XM != XM_GLOBAL && XM != XM_SLOT;
  extern __shared__ __align__(16) unsigned char smem[];
  using Geo = DecGeom<BITS, GS, RVQ>;
  constexpr int GB = Geo::GB, LB = Geo::LB, GB2 = Geo::GB2, LB2 = Geo::LB2;
  static_assert(U >= 1 && U <= Geo::UMAX && (U & (U - 1)) == 0, "groups per batch");
  constexpr int NMF = (BITS == 8 && CB8) ? GS / 16 : GS / 32;  // MFMAs per group
  constexpr bool TQ = LB == 4 && !RVQ && U % 4 == 0;            // quarter-transposed code loads
  constexpr int CPM = (BITS == 8 && CB8) ? 4 : 8;              // codes per lane per MFMA
  constexpr bool USE_T4 = (BITS == 4);
  // 8- and 16-wave launches at M = 1 (one or two workgroups per CU): entry
  // b's copies sit in a 256-byte row of the table, so a lookup's byte
  // address, (b << 8) | 4 rsl, is one v_perm_b32 of the code dword instead
  // of a byte extract and an add. The staged codebook then shares the
  // partials buffer (read before the table barrier, which every partial is
  // written after), so that two 8-wave workgroups fit a CU.
  constexpr bool T4W = dec_t4w(BITS, RVQ, XM, W);
  constexpr int T4S = T4W ? 64 : R;  // table words between entries
  static_assert(!T4W || R <= 64, "4 rsl fits the address's low byte");
  constexpr bool USE_T2 = (BITS == 2) || RVQ;
  constexpr bool USE_T8 = (BITS == 8) && CB8;
  constexpr int NW8 = (U + 3) / 4;   // words holding U bytes
  constexpr int NW16 = (U + 1) / 2;  // words holding U halves
  constexpr int NSC = AL ? (DQ ? NW8 : NW16) : U;

  // Every kernel argument is fetched here, in one batch of scalar loads, and
  // made opaque so the compiler keeps it in SGPRs. Otherwise it re-fetches
  // arguments lazily (they are invariant loads) in several dependent
  // batches, each a memory round trip on every workgroup's critical path.
  const int64_t bid = blockIdx.x;
  int li = 0;
#pragma unroll
  for (int i = 1; i < DEC_GMAX; ++i) li += (i < g.n && bid >= g.tile_end[i - 1]) ? 1 : 0;
  DecodeArgs a = g.a[li];
  // RT row tiles per workgroup (tile_end counts workgroups): tiles
  // RT * (its index in the layer) + 0 .. RT - 1, computed together
  const int64_t tile = RT * (bid - (li > 0 ? g.tile_end[li > 0 ? li - 1 : 0] : 0));
#define TS_PG(f) ts_pin_global(a.f)
#define TS_PS(f) ts_pin_scalar(a.f)
  TS_PG(packed); TS_PG(scale); TS_PG(gmin); TS_PG(dqsc); TS_PG(dqsm); TS_PG(dqgc); TS_PG(dqgm); TS_PG(x); TS_PG(y);
  TS_PG(slots); TS_PG(cbsrc); TS_PG(bias_src);
  TS_PS(pstride); TS_PS(dq_gs); TS_PS(dqm_bytes); TS_PS(ldx); TS_PS(ldy); TS_PS(N); TS_PS(cols); TS_PS(K); TS_PS(n_groups);
  TS_PS(n_tiles); TS_PS(M); TS_PS(cb_mode); TS_PS(cap); TS_PS(bias_mul); TS_PS(y_dtype); TS_PS(cb0);
#pragma unroll
  for (int j = 0; j < 16; ++j) TS_PS(cbq[j]);
  if constexpr (RVQ) { TS_PG(s2packed); TS_PS(s2stride); TS_PG(s2scale); TS_PG(s2gmin); }
#undef TS_PG
#undef TS_PS

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int q = lane >> 4;
  const int rsl = lane & (R - 1);
  const uint32_t rsl4 = 4u * (uint32_t)rsl;

  // ---- LDS carve-up ------------------------------------------------------
  unsigned char* sp = smem;
  uint32_t* t4 = nullptr;
  uint2* t2 = nullptr;
  uint32_t* t8 = nullptr;
  if constexpr (USE_T4) { t4 = reinterpret_cast<uint32_t*>(sp); sp += 256 * T4S * 4; }
  if constexpr (USE_T2) { t2 = reinterpret_cast<uint2*>(sp); sp += 256 * R * 8; }
  if constexpr (USE_T8) { t8 = reinterpret_cast<uint32_t*>(sp); sp += 256 * R * 4; }
  float* red = reinterpret_cast<float*>(sp);       // [MB][RT][W][64][4]
  sp += MB * RT * W * 64 * 4 * 4;
  float* cbs = T4W ? red : reinterpret_cast<float*>(sp);  // [256] staged codebook
  if constexpr (!T4W) sp += 256 * 4;
  // XM_SLOT: each wave's x slot (64 lanes x 16 bytes)
  uint16_t* xw = reinterpret_cast<uint16_t*>(sp) + wave * 512;
  if constexpr (XM == XM_SLOT) sp += W * 1024;
  uint16_t* xs = reinterpret_cast<uint16_t*>(sp);  // [M][K] staged activations (XLDS)

  // ---- per-wave share of every tile ----------------------------------------
  // The row's T batches of U groups are split into contiguous runs, one per
  // wave; every wave steps nb batches (a short run's extra batch is dead).
  // (32-bit index math: groups per row and tile counts are far below 2^31.)
  const int G = (int)a.n_groups;
  const int T = (G + U - 1) / U;
  const int g_lo = U * ((T * wave) / W);
  const int g_hi = min(G, U * ((T * (wave + 1)) / W));
  const int nb = (T + W - 1) / W;
  const uint16_t* xrow_lds = xs + min(n, a.M - 1) * a.K;          // this lane's x row (staged)
  const uint16_t* xrow_glb = a.x + (int64_t)min(n, a.M - 1) * a.ldx;  // this lane's x row (global)
  constexpr uint32_t ONE = XT<BF16>::ONE;
  const ts_u32x4 ones = CB8 ? ts_u32x4{ONE, ONE, ONE, ONE}
                            : ts_u32x4{ONE | (ONE << 16), ONE | (ONE << 16), ONE | (ONE << 16), ONE | (ONE << 16)};

  // Raw loads only: nothing here consumes loaded data, so issuing a batch
  // never waits on memory.
  struct Batch {
    Bytes<LB> w[TQ ? 1 : U];
    ts_u32x4 wq[TQ ? U / 4 : 1];    // TQ: whole groups, one per lane quarter
    Bytes<(LB2 > 0 ? LB2 : 1)> w2[U];
    uint32_t sc[NSC], gc[NSC];      // DQ codes (bytes), or f16 scale / gmin bits
    uint32_t smA, smB, gmA, gmB;    // DQ (meta_scale, meta_min) f16 pairs of the two super-groups
    int split;                      // groups u < split use the first super-group
    uint32_t s2s[RVQ ? (AL ? NW16 : U) : 1], s2g[RVQ ? (AL ? NW16 : U) : 1];  // RVQ stage-2 f16 bits
    uint32_t live;                  // bit u set when group u of the batch exists
    ts_u32x4 xv;                    // XM_SLOT: this lane's x chunk of the batch
  };

  // TQ (4-byte quarter-groups: 2-bit group 64, 4-bit group 32): each lane
  // loads one whole 16-byte group of its row, the group gb + 4 h + q of its
  // lane quarter q, and the four quarters of a row swap pieces at compute
  // time (a 4 x 4 transpose of dwords across the wave's four 16-lane rows,
  // two v_permlane32_swap + two v_permlane16_swap), which leaves lane q with
  // quarter q of groups gb + 4 h .. + 3: one 16-byte load instead of four
  // 4-byte ones.
  auto load_batch_of = [&](const DecodeArgs& A, int64_t tile, int b, Batch& B) {
    const int gb = g_lo + b * U;
    const bool any = gb < g_hi;
    // a dead batch (past the wave's run) reads the tile's first row at one
    // address per load: one cache line, never used
    const int64_t r = any ? min(tile * 16 + n, A.N - 1) : min(tile * 16, A.N - 1);
    const uint8_t* wp = A.packed + r * A.pstride + (any ? q * LB : 0);
    const int gb0 = any ? gb : g_lo;  // a dead batch re-reads the wave's first groups
    if constexpr (XM == XM_SLOT) {
      // chunk of group gb0 + s / NMF, columns (NMF q + s % NMF) * CPM .. + CPM of it
      const int sl = lane & 15;
      const int col = (gb0 + sl / NMF) * GS + (NMF * q + sl % NMF) * CPM;
      const bool use = sl < U * NMF && col < A.cols;
      if constexpr (CPM == 8) {
        const ts_u32x4 v = ts_ld16(A.x + min(col, (int)A.cols - 8));
        B.xv = use ? v : ts_u32x4{0u, 0u, 0u, 0u};
      } else {
        const ts_u32x2 v = ts_ld8(A.x + min(col, (int)A.cols - 4));
        B.xv = use ? ts_u32x4{v.x, v.y, 0u, 0u} : ts_u32x4{0u, 0u, 0u, 0u};
      }
    }
    int gg[U];
    B.live = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = gb + u < g_hi;
      B.live |= live ? (1u << u) : 0u;
      gg[u] = live ? gb + u : gb0;
    }
    if constexpr (TQ) {
      const uint8_t* rowp = A.packed + r * A.pstride;
#pragma unroll
      for (int h = 0; h < U / 4; ++h) {
        const int gq = gb + 4 * h + q;
        B.wq[h] = ts_ld16(rowp + (int64_t)((any && gq < g_hi) ? gq : gb0) * GB);
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) B.w[u] = load_bytes<LB>(wp + (int64_t)gg[u] * GB);
    }
    const int64_t rowg = r * G;
    if constexpr (RVQ) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        B.w2[u] = load_bytes<LB2>(A.s2packed + r * A.s2stride + q * LB2 + (int64_t)gg[u] * GB2);
      if constexpr (AL) {
        const Bytes<2 * U> vs = load_bytes<2 * U>(reinterpret_cast<const uint8_t*>(A.s2scale + rowg + gb0));
        const Bytes<2 * U> vg = load_bytes<2 * U>(reinterpret_cast<const uint8_t*>(A.s2gmin + rowg + gb0));
#pragma unroll
        for (int i = 0; i < NW16; ++i) { B.s2s[i] = vs.d[i]; B.s2g[i] = vg.d[i]; }
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) { B.s2s[u] = A.s2scale[rowg + gg[u]]; B.s2g[u] = A.s2gmin[rowg + gg[u]]; }
      }
    }
    if constexpr (DQ) {
      if constexpr (AL) {
        const Bytes<U> vs = load_bytes<U>(A.dqsc + rowg + gb0);
        const Bytes<U> vg = load_bytes<U>(A.dqgc + rowg + gb0);
#pragma unroll
        for (int i = 0; i < NW8; ++i) { B.sc[i] = vs.d[i]; B.gc[i] = vg.d[i]; }
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) { B.sc[u] = A.dqsc[rowg + gg[u]]; B.gc[u] = A.dqgc[rowg + gg[u]]; }
      }
      // The batch's live groups are consecutive, so they span at most two
      // super-groups (dq_gs >= U is checked on the host).
      const int nlive = max(1, min(U, g_hi - gb));
      const uint32_t f0 = (uint32_t)(rowg + gb0);
      const uint32_t sup0 = f0 / A.dq_gs;
      const uint32_t sup1 = (f0 + (uint32_t)(any ? nlive - 1 : 0)) / A.dq_gs;
      B.split = (int)min((uint32_t)U, (sup0 + 1) * A.dq_gs - f0);
      // super-groups sup0 and sup0 + 1 in one 8-byte buffer load per array
      // (raw: nothing here consumes it). sup1 is sup0 or sup0 + 1, and when
      // it is sup0 every live group is below split, so B is never read (past
      // the last super-group the buffer load returns zeros).
      (void)sup1;
      const ts_u32x2 sm = ts_bld8(ts_rsrc(A.dqsm, A.dqm_bytes), 4u * sup0);
      const ts_u32x2 gv = ts_bld8(ts_rsrc(A.dqgm, A.dqm_bytes), 4u * sup0);
      B.smA = sm.x;
      B.smB = sm.y;
      B.gmA = gv.x;
      B.gmB = gv.y;
    } else {
      if constexpr (AL) {
        const Bytes<2 * U> vs = load_bytes<2 * U>(reinterpret_cast<const uint8_t*>(A.scale + rowg + gb0));
        const Bytes<2 * U> vg = load_bytes<2 * U>(reinterpret_cast<const uint8_t*>(A.gmin + rowg + gb0));
#pragma unroll
        for (int i = 0; i < NW16; ++i) { B.sc[i] = vs.d[i]; B.gc[i] = vg.d[i]; }
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) { B.sc[u] = A.scale[rowg + gg[u]]; B.gc[u] = A.gmin[rowg + gg[u]]; }
      }
      B.smA = B.smB = B.gmA = B.gmB = 0u;
      B.split = U;
    }
  };

  auto load_batch = [&](int64_t tile, int b, Batch& B) { load_batch_of(a, tile, b, B); };

  // Codebook tables (4-bit, and 2-bit outside RVQ) hold cb[c] - c0, c0 the
  // middle of the codebook's range, and the offset term takes gmin + c0 s:
  // the same affine, with the bf16 rounding of the table entries halved for
  // codebooks on [0, 2^b - 1] (NF, Lloyd-Max). Uniform grids keep c0 = 0.
  constexpr bool CENTER = !RVQ && (BITS == 4 || BITS == 2);
  float c0 = 0.f;
  // float32 (scale, gmin + c0 scale) of group u of a batch
  auto group_affine = [&](const Batch& B, int u, float& s_, float& gm_) {
    if constexpr (DQ) {  // modules.py:573-579: code * meta_scale + meta_min in float32
      const float cs = (float)(AL ? byte_of(B.sc, u) : B.sc[u]);
      const float cg = (float)(AL ? byte_of(B.gc, u) : B.gc[u]);
      const uint32_t ms = u < B.split ? B.smA : B.smB;
      const uint32_t mg = u < B.split ? B.gmA : B.gmB;
      s_ = __fadd_rn(__fmul_rn(cs, ts_h2f(ms & 0xffffu)), ts_h2f(ms >> 16));
      gm_ = __fadd_rn(__fmul_rn(cg, ts_h2f(mg & 0xffffu)), ts_h2f(mg >> 16));
    } else {
      s_ = ts_h2f((uint16_t)(AL ? half_of(B.sc, u) : B.sc[u]));
      gm_ = ts_h2f((uint16_t)(AL ? half_of(B.gc, u) : B.gc[u]));
    }
    if constexpr (CENTER) gm_ = __builtin_fmaf(c0, s_, gm_);
  };

  auto compute_batch = [&](int b, const Batch& B, ts_f32x4* yacc) {
    // M = 1: the batch's x chunks go to this wave's LDS slot once; each MFMA
    // then reads its chunk back with the 16 lanes of a row on one address (a
    // broadcast read), instead of moving it with DPP (VALU) per MFMA. Reads
    // of the previous batch were issued before this write (in-order LDS).
    if constexpr (XM == XM_SLOT) {
      if constexpr (CPM == 8) *reinterpret_cast<ts_u32x4*>(xw + lane * 8) = B.xv;
      else *reinterpret_cast<ts_u32x2*>(xw + lane * 4) = ts_u32x2{B.xv.x, B.xv.y};
    }
    // M = 1: the gmin term's x . 1 sums, one per group and the same for every
    // row, from the chunks the lanes already hold instead of one MFMA per
    // chunk against ones: each lane sums its chunk (dot2 with ones, fp32),
    // DPP sums the NMF lanes of a (group, lane quarter) segment and two
    // permlane swaps sum the four quarters, so lane u * NMF ends with group
    // u's total.
    float xsum = 0.f;
    if constexpr (XM == XM_SLOT) {
      auto dot1 = [&](uint32_t v, float c) {
        if constexpr (BF16)
          return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ts_bf16x2, v),
                                                 __builtin_bit_cast(ts_bf16x2, 0x3f803f80u), c, false);
        else
          return __builtin_amdgcn_fdot2(__builtin_bit_cast(ts_f16x2, v), __builtin_bit_cast(ts_f16x2, 0x3c003c00u), c,
                                        false);
      };
      xsum = dot1(B.xv.y, dot1(B.xv.x, 0.f));
      if constexpr (CPM == 8) xsum = dot1(B.xv.w, dot1(B.xv.z, xsum));
      if constexpr (NMF >= 2) xsum += ts_dpp_f<0xB1>(xsum);   // quad_perm [1,0,3,2]
      if constexpr (NMF >= 4) xsum += ts_dpp_f<0x4E>(xsum);   // quad_perm [2,3,0,1]
      if constexpr (NMF >= 8) xsum += ts_dpp_f<0x141>(xsum);  // row_half_mirror
      if constexpr (NMF >= 16) xsum += ts_dpp_f<0x140>(xsum); // row_mirror
      xsum = ts_sum_x16(ts_sum_x32(xsum));
    }
    // the batch's code dwords per group (TQ: after the quarter transpose)
    uint32_t wt[TQ ? U : 1];
    if constexpr (TQ) {
#pragma unroll
      for (int h = 0; h < U / 4; ++h) {
        uint32_t d0 = B.wq[h].x, d1 = B.wq[h].y, d2 = B.wq[h].z, d3 = B.wq[h].w;
        auto p02 = __builtin_amdgcn_permlane32_swap(d0, d2, false, false);
        auto p13 = __builtin_amdgcn_permlane32_swap(d1, d3, false, false);
        auto p01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
        auto p23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
        wt[4 * h + 0] = p01[0];
        wt[4 * h + 1] = p01[1];
        wt[4 * h + 2] = p23[0];
        wt[4 * h + 3] = p23[1];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = g_lo + b * U + u;
      const uint32_t* wd = TQ ? &wt[u] : B.w[TQ ? 0 : u].d;
      if (!((B.live >> u) & 1u)) break;  // wave-uniform
      float s_, gm_;
      group_affine(B, u, s_, gm_);
      // Phase 1: every LDS read of the group (x operands and code-table
      // entries) is issued before the first MFMA, so the reads overlap
      // instead of each MFMA waiting out one LDS round trip.
      const int c0 = g * GS + q * (GS / 4);
      ts_u32x4 xa[NMF], bv[NMF], bv2[RVQ ? NMF : 1];
#pragma unroll
      for (int j = 0; j < NMF; ++j) {
        const int col = c0 + j * CPM;
        // A-operand row n >= M only feeds output rows that are never stored,
        // so those lanes read row M - 1 (no predicate, one base per lane).
        if constexpr (CPM == 8) {
          if constexpr (XM == XM_SLOT) {
            xa[j] = *reinterpret_cast<const ts_u32x4*>(xw + (16 * q + u * NMF + j) * 8);
          } else if constexpr (XLDS) {
            xa[j] = *reinterpret_cast<const ts_u32x4*>(xrow_lds + col);
          } else if constexpr (MB == 1) {
            const ts_u32x4 v = ts_ld16(xrow_glb + min(col, (int)a.cols - 8));
            xa[j] = col < a.cols ? v : ts_u32x4{0u, 0u, 0u, 0u};
          }
        } else if constexpr (XM == XM_SLOT || XLDS || MB == 1) {
          ts_u32x2 v;
          if constexpr (XM == XM_SLOT) {
            v = *reinterpret_cast<const ts_u32x2*>(xw + (16 * q + u * NMF + j) * 4);
          } else if constexpr (XLDS) {
            v = *reinterpret_cast<const ts_u32x2*>(xrow_lds + col);
          } else {
            const ts_u32x2 l = ts_ld8(xrow_glb + min(col, (int)a.cols - 4));
            v = col < a.cols ? l : ts_u32x2{0u, 0u};
          }
          // (x_k, x_k) pairs so one (hi, lo) table word multiplies x_k twice.
          xa[j] = ts_u32x4{__builtin_amdgcn_perm(v.x, v.x, 0x05040100u), __builtin_amdgcn_perm(v.x, v.x, 0x07060302u),
                           __builtin_amdgcn_perm(v.y, v.y, 0x05040100u), __builtin_amdgcn_perm(v.y, v.y, 0x07060302u)};
        }
        if constexpr (T4W) {
          // byte t of code dword j to address byte 1, 4 rsl to byte 0: the
          // LDS byte address itself (the table is at offset 0 of the
          // workgroup's LDS, which the launch checks: no static LDS)
          using lds_u32 = const __attribute__((address_space(3))) uint32_t;
          auto lk = [&](uint32_t sel) {
            return *reinterpret_cast<lds_u32*>((uintptr_t)__builtin_amdgcn_perm(wd[j], rsl4, sel));
          };
          bv[j] = ts_u32x4{lk(0x0c0c0400u), lk(0x0c0c0500u), lk(0x0c0c0600u), lk(0x0c0c0700u)};
        } else if constexpr (BITS == 4) {
          const int b0 = 4 * j;
          bv[j] = ts_u32x4{t4[byte_of(wd, b0 + 0) * R + rsl], t4[byte_of(wd, b0 + 1) * R + rsl],
                           t4[byte_of(wd, b0 + 2) * R + rsl], t4[byte_of(wd, b0 + 3) * R + rsl]};
        } else if constexpr (BITS == 2) {
          const uint2 e0 = t2[byte_of(wd, 2 * j + 0) * R + rsl];
          const uint2 e1 = t2[byte_of(wd, 2 * j + 1) * R + rsl];
          bv[j] = ts_u32x4{e0.x, e0.y, e1.x, e1.y};
        } else if constexpr (CB8) {
          bv[j] = ts_u32x4{t8[byte_of(wd, 4 * j + 0) * R + rsl], t8[byte_of(wd, 4 * j + 1) * R + rsl],
                           t8[byte_of(wd, 4 * j + 2) * R + rsl], t8[byte_of(wd, 4 * j + 3) * R + rsl]};
        } else {
          uint32_t pr[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float f0 = (float)byte_of(wd, 8 * j + 2 * t);
            const float f1 = (float)byte_of(wd, 8 * j + 2 * t + 1);
            if constexpr (BF16)
              pr[t] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0),
                                            0x07060302u);
            else
              pr[t] = pack2<false>(f0, f1);
          }
          bv[j] = ts_u32x4{pr[0], pr[1], pr[2], pr[3]};
        }
        if constexpr (RVQ) {
          const uint2 e0 = t2[byte_of(B.w2[u].d, 2 * j + 0) * R + rsl];
          const uint2 e1 = t2[byte_of(B.w2[u].d, 2 * j + 1) * R + rsl];
          bv2[j] = ts_u32x4{e0.x, e0.y, e1.x, e1.y};
        }
      }
      float s2_ = 0.f, g2_ = 0.f;
      if constexpr (RVQ) {
        s2_ = ts_h2f((uint16_t)(AL ? half_of(B.s2s, u) : B.s2s[u]));
        g2_ = ts_h2f((uint16_t)(AL ? half_of(B.s2g, u) : B.s2g[u]));
      }
      // Phase 2: the group's MFMAs (ax: per-row sums of x over the group),
      // for each block of 16 tokens (MB > 1: x of block tb read from global
      // memory here; the code-table entries above serve every block).
#pragma unroll
      for (int tb = 0; tb < MB; ++tb) {
        if constexpr (MB > 1) {
          const uint16_t* xr = a.x + (int64_t)min(16 * tb + n, a.M - 1) * a.ldx;
#pragma unroll
          for (int j = 0; j < NMF; ++j) {
            const int col = c0 + j * CPM;
            if constexpr (CPM == 8) {
              const ts_u32x4 v = ts_ld16(xr + min(col, (int)a.cols - 8));
              xa[j] = col < a.cols ? v : ts_u32x4{0u, 0u, 0u, 0u};
            } else {
              const ts_u32x2 l = ts_ld8(xr + min(col, (int)a.cols - 4));
              const ts_u32x2 v = col < a.cols ? l : ts_u32x2{0u, 0u};
              xa[j] = ts_u32x4{__builtin_amdgcn_perm(v.x, v.x, 0x05040100u),
                               __builtin_amdgcn_perm(v.x, v.x, 0x07060302u),
                               __builtin_amdgcn_perm(v.y, v.y, 0x05040100u),
                               __builtin_amdgcn_perm(v.y, v.y, 0x07060302u)};
            }
          }
        }
        ts_f32x4 aw = {0.f, 0.f, 0.f, 0.f};
        ts_f32x4 ax = {0.f, 0.f, 0.f, 0.f};
        ts_f32x4 aw2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NMF; ++j) {
          aw = ts_mfma16x16x32<BF16>(xa[j], bv[j], aw);
          if constexpr (XM != XM_SLOT) ax = ts_mfma16x16x32<BF16>(xa[j], ones, ax);
          if constexpr (RVQ) aw2 = ts_mfma16x16x32<BF16>(xa[j], bv2[j], aw2);
        }
        if constexpr (XM == XM_SLOT)
          ax[0] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, xsum), u * NMF));
        // M = 1 (XM_SLOT): only element 0 of lanes 0-15 (token 0) is stored
        constexpr int NI = XM == XM_SLOT ? 1 : 4;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          float v = yacc[tb][i];
          v = __builtin_fmaf(s_, aw[i], v);
          v = __builtin_fmaf(gm_, ax[i], v);
          if constexpr (RVQ) {
            v = __builtin_fmaf(s2_, aw2[i], v);
            v = __builtin_fmaf(g2_, ax[i], v);
          }
          yacc[tb][i] = v;
        }
      }
    }
  };

  // RT = 2 (4-bit codes, x read from global memory): the same groups of two
  // row tiles; each x fragment is loaded once for both tiles' MFMAs and the
  // x.1 sums are shared, which halves x's bytes per weight byte (at M > 8 x
  // is 4x the weights per MFMA).
  auto compute_batch2 = [&](int b, const Batch& B0, const Batch& B1, ts_f32x4& y0, ts_f32x4& y1) {
    if constexpr (RT == 2 && BITS == 4 && !RVQ && XM == XM_GLOBAL && !TQ) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int g = g_lo + b * U + u;
        if (!((B0.live >> u) & 1u)) break;  // wave-uniform; both tiles share the groups
        float s0, gm0, s1, gm1;
        group_affine(B0, u, s0, gm0);
        group_affine(B1, u, s1, gm1);
        const int c0 = g * GS + q * (GS / 4);
        ts_u32x4 xa[NMF], bv0[NMF], bv1[NMF];
#pragma unroll
        for (int j = 0; j < NMF; ++j) {
          const int col = c0 + j * CPM;
          const ts_u32x4 v = ts_ld16(xrow_glb + min(col, (int)a.cols - 8));
          xa[j] = col < a.cols ? v : ts_u32x4{0u, 0u, 0u, 0u};
          const int b0 = 4 * j;
          bv0[j] = ts_u32x4{t4[byte_of(B0.w[u].d, b0 + 0) * R + rsl], t4[byte_of(B0.w[u].d, b0 + 1) * R + rsl],
                            t4[byte_of(B0.w[u].d, b0 + 2) * R + rsl], t4[byte_of(B0.w[u].d, b0 + 3) * R + rsl]};
          bv1[j] = ts_u32x4{t4[byte_of(B1.w[u].d, b0 + 0) * R + rsl], t4[byte_of(B1.w[u].d, b0 + 1) * R + rsl],
                            t4[byte_of(B1.w[u].d, b0 + 2) * R + rsl], t4[byte_of(B1.w[u].d, b0 + 3) * R + rsl]};
        }
        ts_f32x4 aw0 = {0.f, 0.f, 0.f, 0.f}, aw1 = {0.f, 0.f, 0.f, 0.f}, ax = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NMF; ++j) {
          aw0 = ts_mfma16x16x32<BF16>(xa[j], bv0[j], aw0);
          aw1 = ts_mfma16x16x32<BF16>(xa[j], bv1[j], aw1);
          ax = ts_mfma16x16x32<BF16>(xa[j], ones, ax);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = y0[i];
          v = __builtin_fmaf(s0, aw0[i], v);
          y0[i] = __builtin_fmaf(gm0, ax[i], v);
          float w = y1[i];
          w = __builtin_fmaf(s1, aw1[i], w);
          y1[i] = __builtin_fmaf(gm1, ax[i], w);
        }
      }
    }
  };

  // ---- one tile per workgroup, batches double-buffered ----------------------
  if (tile >= a.n_tiles) return;
  const int64_t r0 = tile * 16;
  ts_f32x4 yacc[MB];
#pragma unroll
  for (int tb = 0; tb < MB; ++tb) yacc[tb] = ts_f32x4{0.f, 0.f, 0.f, 0.f};

  // Every load of the tile is issued up front, none depending on another: x
  // chunks, the codebook, both weight batches, the tile's outlier slots and
  // the bias.
  // x -> LDS ([M][K] bf16/f16).
  // XM_DMA: direct global->LDS loads, each wave instruction moving one 1 KB
  // chunk (16 B per lane, lane-contiguous). Lanes past the end of x read a
  // clamped (valid) address; their bytes land in the padded tail of the
  // buffer or in the column padding, which is zeroed below. The issue loop is
  // unrolled to a compile-time bound with uniform predicates.
  // XM_REG: XRC 16-byte chunks per thread into registers, stored to
  // LDS once every load of the tile is issued.
  // (32-bit arithmetic: with x staged, M * K * 2 <= DEC_XLDS_MAX.)
  const uint32_t kK = (uint32_t)a.K;
  const uint32_t xchunks = XM == XM_DMA ? ((uint32_t)a.M * kK * 2u + 1023u) / 1024u : 0u;
  constexpr int XCW = XM == XM_DMA ? (int)((DEC_XLDS_MAX / 1024 + W - 1) / W) : 0;  // max chunks per wave
  if constexpr (XM == XM_DMA) {
#pragma unroll
    for (int i = 0; i < XCW; ++i) {
      const uint32_t c = (uint32_t)(wave + i * W);
      if (c < xchunks) {
        const uint32_t e = c * 512u + (uint32_t)lane * 8u;
        const uint32_t m = min(e / kK, (uint32_t)a.M - 1u);
        const uint32_t k = min(e - (e / kK) * kK, (uint32_t)a.cols - 8u);
        __builtin_amdgcn_global_load_lds(a.x + (int64_t)m * a.ldx + k,
                                         (__attribute__((address_space(3))) void*)(xs + c * 512u), 16, 0, 0);
      }
    }
  }
  const uint32_t kch = kK / 8u;                                   // 16-byte chunks per x row
  const uint32_t xch8 = XM == XM_REG ? (uint32_t)a.M * kch : 1u;  // chunks of x
  constexpr int XRC = xreg_chunks(W);
  ts_u32x4 xr[XM == XM_REG ? XRC : 1];
  if constexpr (XM == XM_REG) {
#pragma unroll
    for (int i = 0; i < XRC; ++i) {
      const uint32_t c = min((uint32_t)(tid + i * NT), xch8 - 1u);
      const uint32_t m = c / kch;
      const uint32_t k = min((c - m * kch) * 8u, (uint32_t)a.cols - 8u);
      xr[i] = ts_ld16(a.x + (int64_t)m * a.ldx + k);
    }
  }
  constexpr int NCB = 1 << (RVQ ? 4 : BITS);
  // Codebooks of at most 16 entries and uniform grids come as launch
  // arguments (cbq), already centred and rounded to the activation type, so
  // the 2- and 4-bit tables are built from them directly: lane j < 16 of qv
  // holds entry j and each table word gathers its entries with ds_bpermute.
  // No staging store, barrier or rounding sits before the weight stream. A
  // device codebook (and the 8-bit table) is staged in cbs first.
  const bool argcb = a.cb_mode != CB_DEVICE && !USE_T8;  // the same for the whole workgroup
  const int cbi = tid & 255;  // staged codebook slot (every writer of a slot writes the same value)
  // Codebook value of slot cbi. The device read is the only load behind a
  // (uniform) branch: on the other paths no load is issued there, and the
  // wait at its use then covers exactly the x loads issued before it, which
  // that point needs anyway.
  float cbv = (float)cbi;  // uniform grid
  if (a.cb_mode == CB_DEVICE) cbv = a.cbsrc[cbi < NCB ? cbi : 0];

  // unconditional store (threads tid, tid + 256, ... write the same value to
  // slot tid % 256): a store under `tid < NCB` would let the compiler sink
  // the codebook load next to it and wait there for every load issued before.
  cbs[cbi] = cbv;
  int qv = 0;
  if (argcb) ts_writelanes(qv, a.cbq, std::make_integer_sequence<int, 16>{});
  // entry j of the argument codebook (every lane of the wave active)
  auto cq = [&](int j) { return (uint32_t)__builtin_amdgcn_ds_bpermute(j << 2, qv); };
  if constexpr (XM == XM_REG) {
    // unconditional stores (a thread past the end rewrites the last chunk
    // with the same bytes): a store under a predicate would let the compiler
    // sink its load next to it, past the weight loads, and drain them there
#pragma unroll
    for (int i = 0; i < XRC; ++i) {
      const uint32_t c = min((uint32_t)(tid + i * NT), xch8 - 1u);
      const uint32_t m = c / kch, k = (c - m * kch) * 8u;
      *reinterpret_cast<ts_u32x4*>(xs + m * kK + k) = k < (uint32_t)a.cols ? xr[i] : ts_u32x4{0u, 0u, 0u, 0u};
    }
  }
  if constexpr (XM == XM_DMA) {
    // Each wave waits for its own chunks before the barrier (reading one word
    // of the last one back makes the compiler emit the wait). The compiler's
    // wait-count model treats direct-to-LDS loads as completing out of order
    // with ordinary loads, so this wait also covers the weight loads issued
    // after them; compute needs those next anyway, and no load in this kernel
    // depends on another, so nothing else is serialised behind it.
    uint32_t last = 0;
    if ((uint32_t)wave < xchunks) {
      const uint32_t c_last = (uint32_t)wave + ((xchunks - 1u - (uint32_t)wave) / W) * W;
      last = reinterpret_cast<const uint32_t*>(xs)[c_last * 256u + (uint32_t)lane];
    }
    asm volatile("" ::"v"(last));
    if (kK > (uint32_t)a.cols) {  // column padding: x is zero there
      __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): all of this wave's chunks landed
      // a row's padding may sit in another wave's chunk: zero it only once
      // every wave's chunks have landed, or a late chunk overwrites the zeros
      ts_lds_barrier();
      const uint32_t padw = kK - (uint32_t)a.cols;
      for (uint32_t e = tid; e < (uint32_t)a.M * padw; e += NT) {
        const uint32_t m = e / padw;
        xs[m * kK + (uint32_t)a.cols + (e - m * padw)] = 0;
      }
    }
  }
  // x staging (XM_REG, XM_DMA) and the staged codebook are read across waves
  if (XM == XM_REG || XM == XM_DMA || !argcb) ts_lds_barrier();
  if constexpr (CENTER) {
    if (argcb) c0 = a.cb0;
    else if (a.cb_mode != CB_UNIFORM) c0 = 0.5f * (cbs[0] + cbs[NCB - 1]);
  }
  // entry b's R copies are contiguous: 16-byte stores of four (u32 entries)
  // or two (u64 entries) copies at a time. Every loop below runs whole waves
  // (256 R entries, a multiple of 64 per step), as the gathers need.
  if constexpr (USE_T4 && !USE_T2 && R % 4 == 0) {
    if (argcb) {
      for (int e = 4 * tid; e < 256 * R; e += 4 * NT) {
        const int b = e / R;
        const uint32_t v = cq(b & 15) | (cq(b >> 4) << 16);
        *reinterpret_cast<ts_u32x4*>(t4 + b * T4S + (e - b * R)) = ts_u32x4{v, v, v, v};
      }
    } else {
      for (int e = 4 * tid; e < 256 * R; e += 4 * NT) {
        const int b = e / R;
        const uint32_t v = pack2<BF16>(cbs[b & 15] - c0, cbs[b >> 4] - c0);
        *reinterpret_cast<ts_u32x4*>(t4 + b * T4S + (e - b * R)) = ts_u32x4{v, v, v, v};
      }
    }
  } else if constexpr (USE_T8 && R % 4 == 0) {
    for (int e = 4 * tid; e < 256 * R; e += 4 * NT) {
      const float v = cbs[e / R];
      const uint16_t hb = XT<BF16>::from_f(v);
      const uint16_t lb = XT<BF16>::from_f(v - XT<BF16>::to_f(hb));
      const uint32_t w = (uint32_t)hb | ((uint32_t)lb << 16);
      *reinterpret_cast<ts_u32x4*>(t8 + e) = ts_u32x4{w, w, w, w};
    }
  } else if constexpr (USE_T2 && !USE_T4 && R % 2 == 0) {
    if (argcb) {
      for (int e = 2 * tid; e < 256 * R; e += 2 * NT) {
        const int b = e / R;
        const uint32_t lo = cq(b & 3) | (cq((b >> 2) & 3) << 16), hi = cq((b >> 4) & 3) | (cq(b >> 6) << 16);
        *reinterpret_cast<ts_u32x4*>(t2 + e) = ts_u32x4{lo, hi, lo, hi};
      }
    } else {
      for (int e = 2 * tid; e < 256 * R; e += 2 * NT) {
        const int b = e / R;
        float v[4];
        for (int j = 0; j < 4; ++j) v[j] = cbs[(b >> (2 * j)) & 3] - c0;  // a 2-bit layer's codebook
        const uint32_t lo = pack2<BF16>(v[0], v[1]), hi = pack2<BF16>(v[2], v[3]);
        *reinterpret_cast<ts_u32x4*>(t2 + e) = ts_u32x4{lo, hi, lo, hi};
      }
    }
  } else
  for (int e = tid; e < 256 * R; e += NT) {
    const int b = e / R;
    if constexpr (USE_T4)
      t4[b * T4S + (e - b * R)] =
          argcb ? cq(b & 15) | (cq(b >> 4) << 16) : pack2<BF16>(cbs[b & 15] - c0, cbs[b >> 4] - c0);
    if constexpr (USE_T2) {
      // RVQ stage 2 is always a uniform grid; a 2-bit layer uses its codebook.
      if (!RVQ && argcb) {
        t2[e] = make_uint2(cq(b & 3) | (cq((b >> 2) & 3) << 16), cq((b >> 4) & 3) | (cq(b >> 6) << 16));
      } else {
        float v[4];
        for (int j = 0; j < 4; ++j) {
          const int c = (b >> (2 * j)) & 3;
          v[j] = RVQ ? (float)c : cbs[c] - c0;
        }
        t2[e] = make_uint2(pack2<BF16>(v[0], v[1]), pack2<BF16>(v[2], v[3]));
      }
    }
    if constexpr (USE_T8) {
      const float v = cbs[b];
      const uint16_t hb = XT<BF16>::from_f(v);
      const uint16_t lb = XT<BF16>::from_f(v - XT<BF16>::to_f(hb));
      t8[e] = (uint32_t)hb | ((uint32_t)lb << 16);
    }
  }
  ts_lds_barrier();

  // Offset of (token m, tile row) in a wave's partials: block m / 16 of
  // [MB][W][64][4], lane row + 16 (m % 16 / 4), element m % 4 (the MFMA's D
  // layout).
  auto pidx = [&](int m, uint32_t row) {
    return (m >> 4) * (W * 256) + (int)(row + 16 * ((m & 15) >> 2)) * 4 + (m & 3);
  };
  // The tile's outliers through the CSR row offsets (csr layers), added into
  // the wave's partials rw like the slots: the tile's rows own one
  // contiguous range of the row-sorted tables.
  auto add_csr = [&](const DecodeArgs& A, int64_t t, float* rw) {
    const DecodeCsr& C = g.csr[li];
    const int64_t r_lo = t * 16;
    const int32_t b = C.row_ptr[min(r_lo, A.N)], e = C.row_ptr[min(r_lo + 16, A.N)];
    for (int32_t i = b + tid; i < e; i += NT) {
      const uint32_t row = (uint32_t)(C.row[i] - r_lo), col = (uint32_t)C.col[i];
      const float d = ts_h2f(C.delta[i]);
      for (int m = 0; m < A.M; ++m) {
        const float xv = XLDS ? XT<BF16>::to_f(xs[m * A.K + col]) : XT<BF16>::to_f(A.x[(int64_t)m * A.ldx + col]);
        atomicAdd(&rw[pidx(m, row)], xv * d);
      }
    }
  };

  if constexpr (RT == 2) {
    static_assert(NB == 1 && XM == XM_GLOBAL && BITS == 4 && !RVQ && !TQ, "two row tiles: 4-bit, x from global");
    const int capm1 = max(a.cap - 1, 0);
    auto load_slot = [&](int64_t t, int i) { return a.slots[t * max(a.cap, 0) + min(i, capm1)]; };
    auto load_bias = [&](int64_t t) { return a.bias_src[min(t * 16 + ((tid >> 2) & 15), a.N - 1) * a.bias_mul]; };
    // reduce the waves' partials of tile t (buffers of parity par), outliers,
    // bias, store; the same steps as the single-tile epilogue below
    auto epilogue = [&](int64_t t, const ts_f32x4& yv, uint64_t slot0, uint16_t bias_v, int par) {
      float* rd = red + par * (W * 64 * 4);
      *reinterpret_cast<ts_f32x4*>(rd + (wave * 64 + lane) * 4) = yv;
      if (a.cap > 0) {  // into this wave's own partials, as in the single-tile epilogue
        float* rw = rd + wave * 64 * 4;
        auto add_slot = [&](uint64_t v) {
          const uint32_t dbits = (uint32_t)(v >> 48);
          if (dbits == 0u) return;
          const uint32_t col = (uint32_t)v, row = (uint32_t)(v >> 32) & 0xffffu;
          const float d = ts_h2f((uint16_t)dbits);
          for (int m = 0; m < a.M; ++m)
            atomicAdd(&rw[(row + 16 * (m >> 2)) * 4 + (m & 3)], XT<BF16>::to_f(a.x[(int64_t)m * a.ldx + col]) * d);
        };
        if (tid < a.cap) add_slot(slot0);
        for (int i = tid + NT; i < a.cap; i += NT) add_slot(a.slots[t * a.cap + i]);
      } else if (a.cap < 0) {
        add_csr(a, t, rd + wave * 64 * 4);
      }
      ts_lds_barrier();
      if (tid < 256) {
        const int l = tid >> 2, i = tid & 3;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) acc += rd[(w * 64 + l) * 4 + i];
        const int m = 4 * (l >> 4) + i, nn = l & 15;
        const int64_t r = t * 16 + nn;
        if (m < a.M && r < a.N) {
          if (a.bias_mul) acc += XT<BF16>::to_f(bias_v);
          const int64_t off = (int64_t)m * a.ldy + r;
          if (a.y_dtype == TS_F32) reinterpret_cast<float*>(a.y)[off] = acc;
          else if (a.y_dtype == TS_BF16) reinterpret_cast<uint16_t*>(a.y)[off] = ts_f2bf(acc);
          else reinterpret_cast<uint16_t*>(a.y)[off] = ts_f2h(acc);
        }
      }
      // (the second tile's epilogue uses the other half of red, so these
      // reads need no barrier behind them)
    };
    // a missing second tile re-reads the first and is not stored
    const bool live1 = tile + 1 < a.n_tiles;
    const int64_t t1 = live1 ? tile + 1 : tile;
    Batch bufA, bufB;
    load_batch(tile, 0, bufA);
    load_batch(t1, 0, bufB);
    const uint64_t s00 = load_slot(tile, tid), s10 = load_slot(t1, tid);
    const uint16_t b0v = load_bias(tile), b1v = load_bias(t1);
    asm volatile("" ::: "memory");
    ts_f32x4 y1 = {0.f, 0.f, 0.f, 0.f};
    compute_batch2(0, bufA, bufB, yacc[0], y1);
    epilogue(tile, yacc[0], s00, b0v, 0);
    if (live1) epilogue(t1, y1, s10, b1v, 1);
    return;
  }

  // ---- epilogue of one tile: reduce the waves' partials, outliers, bias, store
  // The tile's outliers are added into this wave's own partials, which it has
  // just written (a wave's LDS operations complete in order), so the single
  // barrier before the cross-wave sum covers them too. Entry of token m, row
  // nn: lane nn + 16 (m / 4), element m % 4 (the MFMA's D layout). rb: the
  // partials buffer ([W][64][4]).
  auto epilogue_of = [&](const DecodeArgs& A, int64_t t, const ts_f32x4* yv, uint64_t slot0, uint16_t bias_v,
                         float* rb) {
#pragma unroll
    for (int tb = 0; tb < MB; ++tb) *reinterpret_cast<ts_f32x4*>(rb + tb * (W * 256) + (wave * 64 + lane) * 4) = yv[tb];
    if (A.cap > 0) {
      // slot = col | (row in tile) << 32 | f16 delta << 48; a zero delta (an
      // unused slot) adds nothing and is skipped
      float* rw = rb + wave * 64 * 4;
      auto add_slot = [&](uint64_t v) {
        const uint32_t dbits = (uint32_t)(v >> 48);
        if (dbits == 0u) return;
        const uint32_t col = (uint32_t)v, row = (uint32_t)(v >> 32) & 0xffffu;
        const float d = ts_h2f((uint16_t)dbits);
        for (int m = 0; m < A.M; ++m) {
          const float xv = XLDS ? XT<BF16>::to_f(xs[m * A.K + col]) : XT<BF16>::to_f(A.x[(int64_t)m * A.ldx + col]);
          atomicAdd(&rw[pidx(m, row)], xv * d);
        }
      };
      if (tid < A.cap) add_slot(slot0);
      for (int i = tid + NT; i < A.cap; i += NT) add_slot(A.slots[t * A.cap + i]);  // rare: > NT in a tile
    } else if (A.cap < 0) {
      add_csr(A, t, rb + wave * 64 * 4);
    }
    ts_lds_barrier();
    // the tile's 16 x 16 MB (token m, row nn) outputs: the thread that sums
    // one over the waves also adds the bias and stores it (thread tid takes
    // outputs tid + k NT, all of row nn = (tid / 4) % 16, whose bias it holds)
    for (int e = tid; e < 256 * MB; e += NT) {
      const int tb = e >> 8, l = (e >> 2) & 63, i = e & 3;
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) acc += rb[tb * (W * 256) + (w * 64 + l) * 4 + i];
      const int m = 16 * tb + 4 * (l >> 4) + i, nn = l & 15;
      const int64_t r = t * 16 + nn;
      if (m < A.M && r < A.N) {
        if (A.bias_mul) acc += XT<BF16>::to_f(bias_v);
        const int64_t off = (int64_t)m * A.ldy + r;
        if (A.y_dtype == TS_F32) reinterpret_cast<float*>(A.y)[off] = acc;
        else if (A.y_dtype == TS_BF16) reinterpret_cast<uint16_t*>(A.y)[off] = ts_f2bf(acc);
        else reinterpret_cast<uint16_t*>(A.y)[off] = ts_f2h(acc);
      }
    }
  };

  // The weight stream starts only now, after the workgroup's barriers: a
  // barrier behind it would wait until every wave had issued all its loads,
  // which under a full memory pipeline is most of the stream, and no wave
  // could compute before then. From here on each wave computes a batch as
  // soon as its own loads land.
  Batch bufA, bufB;
  load_batch(tile, 0, bufA);
  if constexpr (NB != 1) load_batch(tile, 1, bufB);  // (a dead batch when nb == 1)
  // This tile's outlier slots sit at a fixed address (no dependent load):
  // each thread takes slot tid; more (rare: over NT in a tile) are read in
  // the epilogue. Indices past cap read a valid slot whose value is dropped.
  const int64_t sbase = tile * max(a.cap, 0);
  const int capm1 = max(a.cap - 1, 0);
  const uint64_t slot0 = a.slots[sbase + min(tid, capm1)];
  // bias of the output this thread stores (16 rows x M; entry 0 of a valid
  // array when there is no bias)
  const uint16_t bias_v = a.bias_src[min(r0 + ((tid >> 2) & 15), a.N - 1) * a.bias_mul];
  // every load above stays here (the compiler would otherwise sink batch B's
  // loads into its conditional compute step and drain the counter there)
  asm volatile("" ::: "memory");

  // Two register buffers, bound statically (a runtime-indexed pair would live
  // in scratch memory). Without LOOP both were issued in the prologue (the
  // second is dead when nb == 1) and the compiler waits for exactly the one
  // being consumed. With LOOP each is refilled right after its batch is
  // consumed, unconditionally (a batch past the end reads one uniform cache
  // line and is never used), so every path into a compute step has issued
  // the same loads in the same order.
  if constexpr (!LOOP) {
    compute_batch(0, bufA, yacc);
    if constexpr (NB == 2) {
      if (nb > 1) compute_batch(1, bufB, yacc);
    }
  } else {
    for (int b = 0; b < nb; b += 2) {
      compute_batch(b, bufA, yacc);
      load_batch(tile, b + 2, bufA);
      if (b + 1 >= nb) break;
      compute_batch(b + 1, bufB, yacc);
      load_batch(tile, b + 3, bufB);
    }
  }

  epilogue_of(a, tile, yacc, slot0, bias_v, red);
}

template <int BITS, bool CB8, bool RVQ, int REP, int XM, int W, int RT, int MB = 1>
inline size_t decode_smem(int M, int64_t K, bool xlds) {
  constexpr int R = dec_rep_x(REP, W, XM);
  constexpr bool T4W = dec_t4w(BITS, RVQ, XM, W);  // the kernel's wide table rows
  size_t s = 0;
  if (BITS == 4) s += 256 * (T4W ? 64 : R) * 4;
  if (BITS == 2 || RVQ) s += 256 * R * 8;
  if (BITS == 8 && CB8) s += 256 * R * 4;
  s += (size_t)MB * RT * W * 64 * 16;
  if (!T4W) s += 256 * 4;  // staged codebook (inside the partials with T4W)
  if (XM == XM_SLOT) s += (size_t)W * 1024;
  if (xlds) s += ((size_t)M * K * 2 + 1023) / 1024 * 1024;  // whole 1 KB chunks
  return s;
}

template <int BITS, int GS, bool BF16, bool CB8, bool RVQ, int REP, int XM, bool DQ, bool AL, int W, int U,
          int NB, int RT = 1, int MB = 1>
inline int launch_decode_x(const DecodeGroup& g_in, hipStream_t st) {
  // RT row tiles per workgroup: tile_end becomes the cumulative workgroup count
  DecodeGroup g = g_in;
  if constexpr (RT > 1) {
    int64_t acc = 0;
    for (int l = 0; l < g.n; ++l) {
      acc += (g.a[l].n_tiles + RT - 1) / RT;
      g.tile_end[l] = acc;
    }
  }
  const DecodeArgs& a = g.a[0];
  const size_t smem = decode_smem<BITS, CB8, RVQ, REP, XM, W, RT, MB>(a.M, a.K, XM != XM_GLOBAL && XM != XM_SLOT);
  auto kern = decode_kernel<BITS, GS, BF16, CB8, RVQ, REP, XM, DQ, AL, W, U, NB, RT, MB>;
  static std::once_flag flags[64];
  static bool ok[64];
  constexpr bool T4W = dec_t4w(BITS, RVQ, XM, W);  // table addressed from LDS offset 0
  if (!ts_set_smem_once(reinterpret_cast<const void*>(kern), 160 * 1024, flags, ok, T4W)) return TS_HIP_ERROR;
  // one workgroup per 16-row tile; tiles beyond the resident capacity are
  // scheduled by the hardware as workgroups retire
  hipLaunchKernelGGL(kern, dim3((unsigned)g.tile_end[g.n - 1]), dim3(64 * W), smem, st, g);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// Shape of a launch: W waves per tile, U groups per batch.
struct DecShape {
  int W, U;
  bool ok;
};

// U is the largest batch (fewest loads per payload byte). W: the smallest in
// {4, 8, 16} that covers a row in two batches per wave, raised (fewer batches
// per wave, so less serial compute per wave) while the launch stays within
// one resident round of 4096 waves (16 per CU at <= 128 VGPRs) and no wave
// would be idle. ok == false: the row is too long, stream it (LOOP).
inline DecShape decode_shape(int64_t n_tiles, int64_t G, int umax) {
  const int64_t T = (G + umax - 1) / umax;  // batches per row
  int w = 4;
  while (w < 16 && (T + w - 1) / w > 2) w *= 2;
  if ((T + w - 1) / w > 2) return {16, umax, false};
  while (w < 16 && 2 * w <= T && n_tiles * 2 * w <= 4096) w *= 2;
  return {w, umax, true};
}

// Picks the variant: x staged in LDS when it fits, aligned metadata loads
// when every batch is aligned, and the straight-line shape above; the rest
// (x too large for LDS, unaligned metadata, rows longer than 32 batches of
// the largest U) stream through the looping kernel.
// The layers of a group share bits, group size, K, M, codebook kind and
// double-quant kind (the caller checks); the launch shape is chosen for the
// group's total tile count.
template <int BITS, int GS, bool BF16, bool CB8, bool RVQ, int REP>
inline int launch_decode(const DecodeGroup& g, hipStream_t st) {
  constexpr int UMAX = DecGeom<BITS, GS, RVQ>::UMAX;
  constexpr int UMB = UMAX >= 2 ? UMAX / 2 : 1;  // batches of the multi-block (M > 16) launches: registers
  const DecodeArgs& a = g.a[0];
  const bool xfit = (size_t)a.M * a.K * 2 <= DEC_XLDS_MAX;
  const bool dq = a.dqsc != nullptr;
  for (int l = 0; l < g.n; ++l)
    if (dq && g.a[l].dq_gs < (uint32_t)UMAX) return TS_NOT_COVERED;  // a batch would span > 2 super-groups
  auto aligned_ptr = [](const void* p, size_t al) { return (reinterpret_cast<uintptr_t>(p) % al) == 0; };
  // aligned for batches of u groups: whole batches per row, and metadata base
  // pointers aligned for u-wide (codes) / 2u-wide (f16) vector loads, in
  // every layer
  auto aligned = [&](int u) {
    bool al = a.n_groups % u == 0;
    for (int l = 0; l < g.n; ++l) {
      const DecodeArgs& b = g.a[l];
      if (dq) al = al && aligned_ptr(b.dqsc, u) && aligned_ptr(b.dqgc, u);
      else al = al && aligned_ptr(b.scale, 2 * u) && aligned_ptr(b.gmin, 2 * u);
      if (RVQ) al = al && aligned_ptr(b.s2scale, 2 * u) && aligned_ptr(b.s2gmin, 2 * u);
    }
    return al;
  };
  const DecShape sh = decode_shape(g.tile_end[g.n - 1], a.n_groups, UMAX);
  // x from global memory at M > 1 with at least half a resident round of
  // waves: two row tiles per workgroup share each x fragment (4-bit codes),
  // W the smallest of {4, 8, 16} that gives one batch per wave
  constexpr bool RT2_OK = BITS == 4 && !RVQ && !CB8 && DecGeom<BITS, GS, RVQ>::LB != 4;
  const int64_t T1 = (a.n_groups + UMAX - 1) / UMAX;
  const int w_rt = T1 <= 4 ? 4 : (T1 <= 8 ? 8 : (T1 <= 16 ? 16 : 0));
  const bool rt2_shape = RT2_OK && a.M > 1 && w_rt > 0 && aligned(UMAX) &&
                         ((g.tile_end[g.n - 1] + 1) / 2) * w_rt >= 2048;
  // x staged in LDS when it fits, except for 4-bit codes at M >= 3 on the
  // launches that read it from L2 faster (two row tiles per workgroup, or
  // 8-wave straight-line): 14336 x 4096 at M = 8 21.9 -> 18.6 us, 4096 x 4096
  // at M = 6 8.0 -> 7.0 us (2- and 8-bit layers, and 4-bit layers that would
  // take the looping kernel, keep staging)
  const bool xlds = xfit && !(RT2_OK && a.M > 2 && (rt2_shape || (sh.ok && sh.W == 8 && aligned(UMAX))));
  const bool rt2 = rt2_shape && !xlds;
  // x through registers when xreg_chunks(w) chunks per thread hold it
  auto xreg = [&](int w) { return xlds && (int64_t)a.M * a.K / 8 <= (int64_t)xreg_chunks(w) * 64 * w; };
  // M = 1: x through per-wave LDS slots when a batch's (group, MFMA) pairs fit
  // the 16 lanes of a row
  constexpr bool SLOT_OK = UMAX * ((BITS == 8 && CB8) ? GS / 16 : GS / 32) <= 16;
  const bool slot = SLOT_OK && a.M == 1;
  const bool one = (a.n_groups + UMAX - 1) / UMAX <= sh.W;  // one batch per wave
#define TS_DEC(XMV, DQV, ALV, WV, UV, LP) \
  return launch_decode_x<BITS, GS, BF16, CB8, RVQ, REP, XMV, DQV, ALV, WV, UV, (LP) ? 0 : 2>(g, st)
#define TS_DEC1(XMV, DQV, ALV, WV, UV) \
  return launch_decode_x<BITS, GS, BF16, CB8, RVQ, REP, XMV, DQV, ALV, WV, UV, 1>(g, st)
#define TS_DECMB(DQV, ALV, MBV)                                                                      \
  do {                                                                                               \
    if (g.tile_end[g.n - 1] > 512)                                                                   \
      return launch_decode_x<BITS, GS, BF16, CB8, RVQ, REP, XM_GLOBAL, DQV, ALV, 4, UMB, 0, 1, MBV>(g, st); \
    return launch_decode_x<BITS, GS, BF16, CB8, RVQ, REP, XM_GLOBAL, DQV, ALV, 16, UMB, 0, 1, MBV>(g, st);  \
  } while (0)
#define TS_DECRT(DQV, WV) \
  return launch_decode_x<BITS, GS, BF16, CB8, RVQ, REP, XM_GLOBAL, DQV, true, WV, UMAX, 1, 2>(g, st)
#define TS_DEC_ALL(DQV)                                                          \
  do {                                                                           \
    const bool alm = aligned(UMAX);                                              \
    if (a.M > 16) { /* blocks of 16 tokens share each code-table read */          \
      if (a.M > 64) return TS_NOT_COVERED;                                       \
      if (a.M <= 32) {                                                           \
        if (alm) TS_DECMB(DQV, true, 2);                                         \
        TS_DECMB(DQV, false, 2);                                                 \
      }                                                                          \
      if (alm) TS_DECMB(DQV, true, 4);                                           \
      TS_DECMB(DQV, false, 4);                                                   \
    }                                                                            \
    if constexpr (SLOT_OK) {                                                      \
      if (slot && sh.ok && alm) {                                                 \
        if (sh.W == 4) {                                                         \
          if (one) TS_DEC1(XM_SLOT, DQV, true, 4, UMAX);                          \
          TS_DEC(XM_SLOT, DQV, true, 4, UMAX, false);                             \
        }                                                                        \
        if (sh.W == 8) {                                                         \
          if (one) TS_DEC1(XM_SLOT, DQV, true, 8, UMAX);                          \
          TS_DEC(XM_SLOT, DQV, true, 8, UMAX, false);                             \
        }                                                                        \
        if (one) TS_DEC1(XM_SLOT, DQV, true, 16, UMAX);                           \
        TS_DEC(XM_SLOT, DQV, true, 16, UMAX, false);                              \
      }                                                                          \
      if (slot && alm) TS_DEC(XM_SLOT, DQV, true, 16, UMAX, true);                 \
    }                                                                            \
    if constexpr (RT2_OK) {                                                      \
      if (rt2) {                                                                 \
        if (w_rt == 4) TS_DECRT(DQV, 4);                                         \
        if (w_rt == 8) TS_DECRT(DQV, 8);                                         \
        TS_DECRT(DQV, 16);                                                       \
      }                                                                          \
    }                                                                            \
    if (xlds && sh.ok && alm) {                                                  \
      if (sh.W == 4) {                                                           \
        if (xreg(4)) TS_DEC(XM_REG, DQV, true, 4, UMAX, false);                  \
        TS_DEC(XM_DMA, DQV, true, 4, UMAX, false);                               \
      }                                                                          \
      if (sh.W == 8) {                                                           \
        if (xreg(8)) TS_DEC(XM_REG, DQV, true, 8, UMAX, false);                  \
        TS_DEC(XM_DMA, DQV, true, 8, UMAX, false);                               \
      }                                                                          \
      if (xreg(16)) TS_DEC(XM_REG, DQV, true, 16, UMAX, false);                  \
      TS_DEC(XM_DMA, DQV, true, 16, UMAX, false);                                \
    }                                                                            \
    /* x from L2 on launches whose rows fit two batches per wave of 8: the */   \
    /* straight-line kernel (config 1 at M = 16: 12.4 -> 11.7 us) */           \
    if (!xlds && sh.ok && alm && sh.W == 8) {                                    \
      if (one) TS_DEC1(XM_GLOBAL, DQV, true, 8, UMAX);                           \
      TS_DEC(XM_GLOBAL, DQV, true, 8, UMAX, false);                              \
    }                                                                            \
    if (xlds && alm) TS_DEC(XM_DMA, DQV, true, 16, UMAX, true);                  \
    if (xlds) TS_DEC(XM_DMA, DQV, false, 16, UMAX, true);                        \
    if (alm) TS_DEC(XM_GLOBAL, DQV, true, 16, UMAX, true);                       \
    TS_DEC(XM_GLOBAL, DQV, false, 16, UMAX, true);                               \
  } while (0)
  if (dq) TS_DEC_ALL(true);
  TS_DEC_ALL(false);
#undef TS_DEC_ALL
#undef TS_DECRT
#undef TS_DECMB
#undef TS_DEC1
#undef TS_DEC
}

// Per-(bit width, group size) launchers, one translation unit each
// (ts_decode_b<bits>_g<gs>.hip).
int decode_b2_g64(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b2_g128(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b2_g256(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b4_g32(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b4_g64(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b4_g128(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b4_g256(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b6_g64(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b6_g128(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b8_g32(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b8_g64(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);
int decode_b8_g128(const ts_qlayer* L, DecodeGroup& g, bool bf16, hipStream_t st);

}  // namespace ts
