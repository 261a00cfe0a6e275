// GOAP quantize (codec.py:453-675; GPU twin gpu_quantize.py:52-166).
//
// Top-k outliers must come out in torch.topk's CPU order (codec.py:534), which
// for k*64 <= n is libstdc++'s heap selection: make_heap over the first k
// (|w|, index) pairs, then for every later element in index order, if it beats
// the heap top it replaces the top and sifts down; finally sort_heap. Ties at
// the threshold are resolved by that heap history, not by index.
//
// An element i >= k can only enter the heap if |w_i| exceeds the k-th largest
// value of the prefix [0, i). The GPU computes, for prefixes ending at k*2^s,
// a histogram lower bound of that value and compacts every element above the
// bound of its segment (plus [0, k)), in index order. Replaying the heap over
// this candidate stream gives the same heap as over the full array, because
// the dropped elements are exactly no-ops of the replay. The replay itself is
// sequential and runs on the host (ts_topk_select).
#include <algorithm>
#include <cmath>
#include <vector>

#include "ts_common.h"

namespace ts {

constexpr int HBITS = 12;            // histogram bins on |w| float bits [30:19]
constexpr int HBINS = 1 << HBITS;
constexpr int HSHIFT = 31 - HBITS;
constexpr int CHUNK = 4096;          // elements per workgroup in the scans
constexpr int HCHUNK = 16 * CHUNK;   // elements per workgroup in the histogram pass

TS_DEV float load_w(const void* w, int dt, int64_t i) {
  if (dt == TS_F16) return ts_h2f(static_cast<const uint16_t*>(w)[i]);
  if (dt == TS_BF16) return ts_bf2f(static_cast<const uint16_t*>(w)[i]);
  return static_cast<const float*>(w)[i];
}

// Segment s >= 1 covers [k*2^(s-1), k*2^s); segment 0 covers [0, k).
static int n_segments(int64_t n, int64_t k) {
  int s = 1;
  int64_t start = k;
  while (start < n) { ++s; start = (start > (INT64_MAX >> 1)) ? n : start * 2; }
  return s;
}
TS_DEV int seg_of(int64_t i, int64_t k) {
  if (i < k) return 0;
  int s = 1;
  int64_t end = 2 * k;
  while (i >= end) { ++s; end *= 2; }
  return s;
}
TS_DEV int64_t seg_end(int s, int64_t k) { return s == 0 ? k : (k << s); }

// Segment of i for i inside a chunk whose first element is in segment s0
// ending at e0: almost always s0, so the loop only runs at boundaries.
TS_DEV int seg_in_chunk(int64_t i, int s0, int64_t e0, int64_t k) { return i < e0 ? s0 : seg_of(i, k); }

struct TopkWS {
  uint32_t* hist;    // [S][HBINS]
  uint32_t* thr;     // [S] float bits of the lower bound used by segment s
  uint32_t* counts;  // [n_chunks + 1] candidates per chunk, then exclusive offsets
  int S;
  int64_t n_chunks;
};

static size_t align256(size_t b) { return (b + 255) / 256 * 256; }

static TopkWS carve_topk(void* ws, int64_t n, int64_t k) {
  TopkWS t;
  t.S = n_segments(n, k);
  t.n_chunks = ts_cdiv(n, CHUNK);
  char* p = static_cast<char*>(ws);
  t.hist = reinterpret_cast<uint32_t*>(p);
  p += align256((size_t)t.S * HBINS * 4);
  t.thr = reinterpret_cast<uint32_t*>(p);
  p += align256((size_t)t.S * 4);
  t.counts = reinterpret_cast<uint32_t*>(p);
  return t;
}

size_t topk_ws_bytes(int64_t n, int64_t k) {
  const int S = n_segments(n, k);
  return align256((size_t)S * HBINS * 4) + align256((size_t)S * 4) + align256((size_t)(ts_cdiv(n, CHUNK) + 1) * 4);
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

TS_DEV uint32_t abs_bits(const void* w, int dt, int64_t i) {
  return __builtin_bit_cast(uint32_t, load_w(w, dt, i)) & 0x7fffffffu;
}

// Per-segment histograms of |w|. A chunk touches few segments; the first two
// go through an LDS histogram, the rest straight to global atomics. Chunks of
// HCHUNK elements: clearing and flushing the 2 x HBINS LDS bins costs about
// as much as 4096 elements' counting, so a workgroup counts 64 K of them.
__global__ __launch_bounds__(256) void topk_hist_kernel(const void* w, int dt, int64_t n, int64_t k, uint32_t* hist) {
  __shared__ uint32_t lh[2][HBINS];
  const int64_t c0 = (int64_t)blockIdx.x * HCHUNK;
  const int64_t c1 = min(c0 + (int64_t)HCHUNK, n);
  const int s0 = seg_of(c0, k);
  const int64_t e0 = seg_end(s0, k);
  for (int i = threadIdx.x; i < 2 * HBINS; i += blockDim.x) (&lh[0][0])[i] = 0;
  __syncthreads();
  for (int64_t i = c0 + threadIdx.x; i < c1; i += blockDim.x) {
    const uint32_t b = abs_bits(w, dt, i) >> HSHIFT;
    const int s = seg_in_chunk(i, s0, e0, k);
    if (s - s0 < 2) atomicAdd(&lh[s - s0][b], 1u);
    else atomicAdd(&hist[(int64_t)s * HBINS + b], 1u);
  }
  __syncthreads();
  const int S_total = seg_of(n - 1, k) + 1;
  for (int j = 0; j < 2; ++j) {
    if (s0 + j >= S_total) break;
    for (int b = threadIdx.x; b < HBINS; b += blockDim.x) {
      const uint32_t c = lh[j][b];
      if (c) atomicAdd(&hist[(int64_t)(s0 + j) * HBINS + b], c);
    }
  }
}

// thr[s] for s >= 1 = lower edge of the bin holding the k-th largest value of
// the prefix made of segments 0..s-1.
__global__ __launch_bounds__(256) void topk_thr_kernel(const uint32_t* hist, int S, int64_t k, uint32_t* thr) {
  __shared__ uint32_t cum[HBINS];
  __shared__ uint64_t part[256];
  __shared__ int found;
  constexpr int PER = HBINS / 256;
  for (int b = threadIdx.x; b < HBINS; b += blockDim.x) cum[b] = 0;
  if (threadIdx.x == 0) thr[0] = 0;
  __syncthreads();
  for (int s = 1; s < S; ++s) {
    for (int b = threadIdx.x; b < HBINS; b += blockDim.x) cum[b] += hist[(int64_t)(s - 1) * HBINS + b];
    __syncthreads();
    // suffix sums: part[t] = count in bins [t*PER, HBINS)
    uint64_t mine = 0;
    for (int j = 0; j < PER; ++j) mine += cum[threadIdx.x * PER + j];
    part[threadIdx.x] = mine;
    if (threadIdx.x == 0) found = -1;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t acc = 0;
      int b_found = 0;
      for (int t = 255; t >= 0; --t) {
        if (acc + part[t] >= (uint64_t)k) {
          for (int b = t * PER + PER - 1; b >= t * PER; --b) {
            acc += cum[b];
            if (acc >= (uint64_t)k) { b_found = b; break; }
          }
          break;
        }
        acc += part[t];
      }
      thr[s] = (uint32_t)b_found << HSHIFT;
    }
    __syncthreads();
  }
}

TS_DEV bool is_candidate(const void* w, int dt, int64_t i, int64_t k, const uint32_t* thr, int s0, int64_t e0) {
  if (i < k) return true;
  // Bit patterns of non-negative floats order as the values do, and NaN
  // patterns lie above +inf: NaN, which the selection ranks first, stays in.
  return abs_bits(w, dt, i) > thr[seg_in_chunk(i, s0, e0, k)];
}

__global__ __launch_bounds__(256) void topk_count_kernel(const void* w, int dt, int64_t n, int64_t k,
                                                         const uint32_t* thr, uint32_t* counts) {
  __shared__ uint32_t tot;
  if (threadIdx.x == 0) tot = 0;
  __syncthreads();
  const int64_t c0 = (int64_t)blockIdx.x * CHUNK;
  const int64_t c1 = min(c0 + (int64_t)CHUNK, n);
  const int s0 = seg_of(c0, k);
  const int64_t e0 = seg_end(s0, k);
  uint32_t c = 0;
  for (int64_t i = c0 + threadIdx.x; i < c1; i += blockDim.x) c += is_candidate(w, dt, i, k, thr, s0, e0) ? 1u : 0u;
  atomicAdd(&tot, c);
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = tot;
}

// Exclusive scan of counts[0..n) in place, total in counts[n]. One workgroup.
__global__ __launch_bounds__(1024) void scan_counts_kernel(uint32_t* counts, int64_t n) {
  __shared__ uint64_t part[1024];
  const int64_t per = ts_cdiv(n, 1024);
  const int64_t b0 = threadIdx.x * per, b1 = min(b0 + per, n);
  uint64_t s = 0;
  for (int64_t i = b0; i < b1; ++i) s += counts[i];
  part[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t acc = 0;
    for (int t = 0; t < 1024; ++t) { const uint64_t v = part[t]; part[t] = acc; acc += v; }
    counts[n] = (uint32_t)acc;
  }
  __syncthreads();
  uint64_t acc = part[threadIdx.x];
  for (int64_t i = b0; i < b1; ++i) { const uint32_t v = counts[i]; counts[i] = (uint32_t)acc; acc += v; }
}

// Order-preserving compaction: rounds of 256 consecutive elements, ballot
// prefix inside each wave, wave offsets through LDS.
__global__ __launch_bounds__(256) void topk_write_kernel(const void* w, int dt, int64_t n, int64_t k,
                                                         const uint32_t* thr, const uint32_t* offsets,
                                                         int64_t* cidx, float* cval) {
  __shared__ uint32_t wsum[4];
  const int64_t c0 = (int64_t)blockIdx.x * CHUNK;
  const int64_t c1 = min(c0 + (int64_t)CHUNK, n);
  uint32_t base = offsets[blockIdx.x];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int s0 = seg_of(c0, k);
  const int64_t e0 = seg_end(s0, k);
  for (int64_t r = c0; r < c1; r += blockDim.x) {
    const int64_t i = r + threadIdx.x;
    const bool live = i < c1;
    const bool cand = live && is_candidate(w, dt, i, k, thr, s0, e0);
    const uint64_t bal = __ballot(cand);
    const uint32_t pre = __popcll(bal & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    if (lane == 0) wsum[wv] = __popcll(bal);
    __syncthreads();
    uint32_t wo = 0;
    for (int j = 0; j < wv; ++j) wo += wsum[j];
    const uint32_t tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (cand) {
      const uint32_t pos = base + wo + pre;
      cidx[pos] = i;
      cval[pos] = __builtin_bit_cast(float, abs_bits(w, dt, i));
    }
    base += tot;
    __syncthreads();
  }
}

int topk_count(const ts_qinput* in, int64_t k, void* ws, size_t ws_bytes, int64_t* n_cand, hipStream_t st) {
  const int64_t n = in->rows * in->cols;
  if (k <= 0 || k >= n) return TS_BAD_ARG;
  if (ws_bytes < topk_ws_bytes(n, k)) return TS_WORKSPACE;
  TopkWS t = carve_topk(ws, n, k);
  hipLaunchKernelGGL(fill_u32_kernel, dim3(256), dim3(256), 0, st, t.hist, (int64_t)t.S * HBINS, 0u);
  TS_CHECK_LAUNCH();
  hipLaunchKernelGGL(topk_hist_kernel, dim3((unsigned)ts_cdiv(n, HCHUNK)), dim3(256), 0, st, in->w, in->w_dtype, n, k,
                     t.hist);
  TS_CHECK_LAUNCH();
  hipLaunchKernelGGL(topk_thr_kernel, dim3(1), dim3(256), 0, st, t.hist, t.S, k, t.thr);
  TS_CHECK_LAUNCH();
  hipLaunchKernelGGL(topk_count_kernel, dim3((unsigned)t.n_chunks), dim3(256), 0, st, in->w, in->w_dtype, n, k,
                     t.thr, t.counts);
  TS_CHECK_LAUNCH();
  hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(1024), 0, st, t.counts, t.n_chunks);
  TS_CHECK_LAUNCH();
  uint32_t total = 0;
  if (hipMemcpyAsync(&total, t.counts + t.n_chunks, 4, hipMemcpyDeviceToHost, st) != hipSuccess) return TS_HIP_ERROR;
  if (hipStreamSynchronize(st) != hipSuccess) return TS_HIP_ERROR;
  *n_cand = total;
  return TS_OK;
}

int topk_write(const ts_qinput* in, int64_t k, void* ws, int64_t* cidx, float* cval, hipStream_t st) {
  const int64_t n = in->rows * in->cols;
  TopkWS t = carve_topk(ws, n, k);
  hipLaunchKernelGGL(topk_write_kernel, dim3((unsigned)t.n_chunks), dim3(256), 0, st, in->w, in->w_dtype, n, k,
                     t.thr, t.counts, cidx, cval);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// ---------------------------------------------------------------------------
// Host: exact replay of torch.topk's CPU selection over a candidate stream.
// ---------------------------------------------------------------------------
typedef std::pair<float, int64_t> elem_t;
static bool topk_cmp(const elem_t& x, const elem_t& y) {
  return (std::isnan(x.first) && !std::isnan(y.first)) || (x.first > y.first);
}

// The same heap steps as libstdc++'s __heap_select / __adjust_heap /
// __push_heap / __sort_heap (the steps std::partial_sort runs, and with them
// torch.topk on the CPU), on one 64-bit word per entry: the value's float
// bits above a 32-bit index. A level of the sift is then one 16-byte sibling
// pair, a float compare and a select (no branch to mispredict), with the
// grandchildren prefetched. Valid when no value is NaN (the comparator is
// then `a > b`) and every index fits 32 bits; every move, tie and order is
// that of the std:: calls.
struct PackedHeap {
  uint64_t* h;
  static inline float val(uint64_t e) { return __builtin_bit_cast(float, (uint32_t)(e >> 32)); }
  // __adjust_heap(first, hole, len, x) followed by __push_heap.
  inline void adjust(int64_t hole, int64_t len, uint64_t x) {
    const int64_t top = hole;
    int64_t child = hole;
    while (child < (len - 1) / 2) {
      child = 2 * (child + 1);
      const uint64_t r = h[child], l = h[child - 1];
      const bool left = val(r) > val(l);  // comp(first[child], first[child - 1]), comp = greater
      child -= left;
      h[hole] = left ? l : r;
      hole = child;
      __builtin_prefetch(h + 4 * hole + 3);
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
      child = 2 * (child + 1);
      h[hole] = h[child - 1];
      hole = child - 1;
    }
    const float xv = val(x);
    int64_t parent = (hole - 1) / 2;
    while (hole > top && val(h[parent]) > xv) {  // comp(first[parent], value)
      h[hole] = h[parent];
      hole = parent;
      parent = (hole - 1) / 2;
    }
    h[hole] = x;
  }
};

static void topk_heap_packed(const int64_t* cidx, const float* cval, int64_t nc, int64_t k, int64_t* out_idx,
                             float* out_val) {
  auto pack = [](float v, int64_t i) { return (uint64_t)__builtin_bit_cast(uint32_t, v) << 32 | (uint32_t)i; };
  std::vector<uint64_t> buf((size_t)k);
  PackedHeap H{buf.data()};
  uint64_t* h = H.h;
  for (int64_t j = 0; j < k; ++j) h[j] = pack(cval[j], cidx[j]);
  // __make_heap
  if (k >= 2) {
    for (int64_t parent = (k - 2) / 2;; --parent) {
      H.adjust(parent, k, h[parent]);
      if (parent == 0) break;
    }
  }
  // __heap_select: an element beating the top (comp(e, first): e > top)
  // replaces it through __pop_heap(first, middle, e) = __adjust_heap(first, 0, k, e)
  float topv = PackedHeap::val(h[0]);
  for (int64_t j = k; j < nc; ++j) {
    const float e = cval[j];
    if (e > topv) {
      H.adjust(0, k, pack(e, cidx[j]));
      topv = PackedHeap::val(h[0]);
    }
  }
  // __sort_heap: repeatedly __pop_heap(first, last - 1, last - 1)
  for (int64_t last = k; last > 1; --last) {
    const uint64_t x = h[last - 1];
    h[last - 1] = h[0];
    H.adjust(0, last - 1, x);
  }
  for (int64_t j = 0; j < k; ++j) {
    out_idx[j] = (int64_t)(uint32_t)h[j];
    out_val[j] = PackedHeap::val(h[j]);
  }
}

// The same heap steps again, with the keys and the indices in separate arrays:
// the sift's dependent loads then touch only the keys (for k = 234 881,
// 470 KB of 16-bit keys instead of 1.9 MB of packed words, so the deep
// levels stay in the core's L2), and the index moves are plain stores. The
// keys are order-preserving codes of non-negative values: f16 or bf16 bits
// when every value is exactly one, else the float bits; non-negative floats
// and their bit patterns compare alike (no -0.0, no NaN: the caller checks).
enum KeyKind { KEY_F16, KEY_BF16, KEY_F32 };

template <typename KT>
struct SplitHeap {
  KT* key;
  uint32_t* ix;
  // __adjust_heap(first, hole, len, x) followed by __push_heap, as PackedHeap
  inline void adjust(int64_t hole, int64_t len, KT xk, uint32_t xi) {
    const int64_t top = hole;
    int64_t child = hole;
    while (child < (len - 1) / 2) {
      child = 2 * (child + 1);
      const KT r = key[child], l = key[child - 1];
      const bool left = r > l;  // comp(first[child], first[child - 1]), comp = greater
      child -= left;
      key[hole] = left ? l : r;
      ix[hole] = ix[child];
      hole = child;
      __builtin_prefetch(key + 4 * hole + 3);  // grandchildren
      __builtin_prefetch(key + 8 * hole + 7);  // great-grandchildren
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
      child = 2 * (child + 1);
      key[hole] = key[child - 1];
      ix[hole] = ix[child - 1];
      hole = child - 1;
    }
    int64_t parent = (hole - 1) / 2;
    while (hole > top && key[parent] > xk) {  // comp(first[parent], value)
      key[hole] = key[parent];
      ix[hole] = ix[parent];
      hole = parent;
      parent = (hole - 1) / 2;
    }
    key[hole] = xk;
    ix[hole] = xi;
  }
};

template <typename KT, KeyKind KK>
static void topk_heap_split(const int64_t* cidx, const float* cval, int64_t nc, int64_t k, int64_t* out_idx,
                            float* out_val) {
  auto enc = [](float v) -> KT {
    if constexpr (KK == KEY_F16) return __builtin_bit_cast(uint16_t, (_Float16)v);
    else if constexpr (KK == KEY_BF16) return (uint16_t)(__builtin_bit_cast(uint32_t, v) >> 16);
    else return __builtin_bit_cast(uint32_t, v);
  };
  auto dec = [](KT x) -> float {
    if constexpr (KK == KEY_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)x);
    else if constexpr (KK == KEY_BF16) return __builtin_bit_cast(float, (uint32_t)x << 16);
    else return __builtin_bit_cast(float, (uint32_t)x);
  };
  std::vector<KT> kb((size_t)k);
  std::vector<uint32_t> ib((size_t)k);
  SplitHeap<KT> H{kb.data(), ib.data()};
  KT* key = H.key;
  uint32_t* ix = H.ix;
  for (int64_t j = 0; j < k; ++j) {
    key[j] = enc(cval[j]);
    ix[j] = (uint32_t)cidx[j];
  }
  if (k >= 2) {  // __make_heap
    for (int64_t parent = (k - 2) / 2;; --parent) {
      H.adjust(parent, k, key[parent], ix[parent]);
      if (parent == 0) break;
    }
  }
  KT top = key[0];  // __heap_select
  for (int64_t j = k; j < nc; ++j) {
    const KT e = enc(cval[j]);
    if (e > top) {
      H.adjust(0, k, e, (uint32_t)cidx[j]);
      top = key[0];
    }
  }
  for (int64_t last = k; last > 1; --last) {  // __sort_heap
    const KT xk = key[last - 1];
    const uint32_t xi = ix[last - 1];
    key[last - 1] = key[0];
    ix[last - 1] = ix[0];
    H.adjust(0, last - 1, xk, xi);
  }
  for (int64_t j = 0; j < k; ++j) {
    out_idx[j] = (int64_t)ix[j];
    out_val[j] = dec(key[j]);
  }
}

// Which split-heap keys the stream allows; false: some value is negative,
// -0.0 or NaN (the packed float heap then runs).
static bool split_key_kind(const float* cval, int64_t nc, KeyKind* kind) {
  bool f16 = true, bf16 = true;
  for (int64_t j = 0; j < nc; ++j) {
    const float v = cval[j];
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u >> 31) || std::isnan(v)) return false;
    f16 = f16 && (float)(_Float16)v == v;
    bf16 = bf16 && (u & 0xffffu) == 0;
  }
  *kind = f16 ? KEY_F16 : (bf16 ? KEY_BF16 : KEY_F32);
  return true;
}

int topk_select(const int64_t* cidx, const float* cval, int64_t nc, int64_t n, int64_t k, int64_t* out_idx,
                float* out_val) {
  if (k <= 0 || k > n || nc < k) return TS_BAD_ARG;
  if (k * 64 <= n) {
    for (int64_t i = 0; i < k; ++i)
      if (cidx[i] != i) return TS_BAD_ARG;  // the stream must start with [0, k)
    bool packable = n <= (int64_t)UINT32_MAX + 1;
    for (int64_t j = 0; j < nc && packable; ++j) packable = !std::isnan(cval[j]);
    if (packable) {
      KeyKind kk;
      if (!split_key_kind(cval, nc, &kk)) topk_heap_packed(cidx, cval, nc, k, out_idx, out_val);
      else if (kk == KEY_F16) topk_heap_split<uint16_t, KEY_F16>(cidx, cval, nc, k, out_idx, out_val);
      else if (kk == KEY_BF16) topk_heap_split<uint16_t, KEY_BF16>(cidx, cval, nc, k, out_idx, out_val);
      else topk_heap_split<uint32_t, KEY_F32>(cidx, cval, nc, k, out_idx, out_val);
      return TS_OK;
    }
    // __heap_select: make_heap(first k); for later elements beating the top,
    // __pop_heap(first, middle, it) == write it at slot k, pop_heap over k+1.
    std::vector<elem_t> h((size_t)k + 1);
    for (int64_t i = 0; i < k; ++i) {
      if (cidx[i] != i) return TS_BAD_ARG;  // the stream must start with [0, k)
      h[i] = elem_t(cval[i], cidx[i]);
    }
    std::make_heap(h.begin(), h.begin() + k, topk_cmp);
    for (int64_t j = k; j < nc; ++j) {
      const elem_t e(cval[j], cidx[j]);
      if (topk_cmp(e, h[0])) {
        h[k] = e;
        std::pop_heap(h.begin(), h.begin() + k + 1, topk_cmp);
      }
    }
    std::sort_heap(h.begin(), h.begin() + k, topk_cmp);
    for (int64_t i = 0; i < k; ++i) { out_idx[i] = h[i].second; out_val[i] = h[i].first; }
    return TS_OK;
  }
  // nth_element regime: needs the full array in index order.
  if (nc != n) return TS_BAD_ARG;
  std::vector<elem_t> q((size_t)n);
  for (int64_t i = 0; i < n; ++i) q[i] = elem_t(cval[i], cidx[i]);
  std::nth_element(q.begin(), q.begin() + k - 1, q.end(), topk_cmp);
  std::sort(q.begin(), q.begin() + k - 1, topk_cmp);
  for (int64_t i = 0; i < k; ++i) { out_idx[i] = q[i].second; out_val[i] = q[i].first; }
  return TS_OK;
}

// ---------------------------------------------------------------------------
// Group encode: clamp, per-(row, group) min/max, scale, codes, packing.
// ---------------------------------------------------------------------------
struct GroupArgs {
  const void* w;
  int dt;
  int64_t rows, cols, padded_cols, n_groups;
  int bits, gs;
  float t;
  int clamp;
  const float* cb;  // sorted f32 grid or null
  int cb_len;
  uint8_t* packed;
  int64_t pstride;
  uint16_t* scale16;
  uint16_t* gmin16;
  float* scale32;
  float* gmin32;
};

// NaN-propagating min / max, as torch's amin/amax and numpy's min/max
// (codec.py:566-567, 395-396); equal to fminf / fmaxf when neither is NaN.
TS_DEV float nan_min(float a, float b) { return a != a ? a : (b != b ? b : fminf(a, b)); }
TS_DEV float nan_max(float a, float b) { return a != a ? a : (b != b ? b : fmaxf(a, b)); }
// max(x, lo) keeping NaN, as torch's clamp(min=) and numpy's maximum do.
TS_DEV float nan_floor(float x, float lo) { return x != x ? x : fmaxf(x, lo); }

TS_DEV float load_clamped(const GroupArgs& a, int64_t r, int64_t c) {
  const int64_t src = c < a.cols ? c : a.cols - 1;  // pad with the last column (codec.py:555-560)
  float v = load_w(a.w, a.dt, r * a.cols + src);
  // flat.clamp_(-t, t) (codec.py:543): NaN stays NaN, and a NaN bound (t is
  // the top-k minimum, NaN once a NaN weight is among the top k) makes every
  // element NaN.
  if (a.clamp) v = a.t != a.t ? a.t : (v != v ? v : fminf(fmaxf(v, -a.t), a.t));
  return v;
}

TS_DEV uint32_t assign_code(float v, int levels, const float* mids, int n_mids) {
  // NaN: torch.searchsorted sorts it after every mid (the last code after
  // the clamp, codec.py:371-372); the uniform grid's round/clamp/uint8 cast
  // gives 0 on the reference's CPU.
  if (v != v) return mids ? (uint32_t)n_mids : 0u;
  if (!mids) {
    float c = rintf(v);
    c = fminf(fmaxf(c, 0.f), (float)levels);
    return (uint32_t)c;
  }
  // searchsorted(mids, v, side='left') = number of mids strictly below v.
  int lo = 0, hi = n_mids;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (mids[mid] < v) lo = mid + 1;
    else hi = mid;
  }
  return (uint32_t)lo;
}

// One thread per 8 consecutive (padded) columns; a group is gs/8 adjacent lanes.
template <int GL>  // lanes per group = gs / 8
__global__ __launch_bounds__(256) void quant_groups_kernel(const GroupArgs a) {
#pragma clang fp contract(off)
  __shared__ float mids[255];
  const int n_mids = a.cb ? a.cb_len - 1 : 0;
  for (int i = threadIdx.x; i < n_mids; i += blockDim.x) mids[i] = (a.cb[i] + a.cb[i + 1]) / 2.0f;
  __syncthreads();
  const int64_t r = blockIdx.y;
  const int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;  // 8-column chunk
  const int64_t c0 = j * 8;
  const bool live = c0 < a.padded_cols;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = load_clamped(a, r, live ? c0 + e : a.cols - 1);
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) { mn = nan_min(mn, v[e]); mx = nan_max(mx, v[e]); }
#pragma unroll
  for (int o = 1; o < GL; o <<= 1) {
    mn = nan_min(mn, __shfl_xor(mn, o, 64));
    mx = nan_max(mx, __shfl_xor(mx, o, 64));
  }
  const int levels = (1 << a.bits) - 1;
  float scale = (mx - mn) / (float)levels;
  scale = nan_floor(scale, 1e-8f);
  if (!live) return;
  uint32_t code[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q = (v[e] - mn) / scale;
    code[e] = assign_code(q, levels, a.cb ? mids : nullptr, n_mids);
  }
  uint8_t* prow = a.packed + r * a.pstride;
  if (a.bits == 4) {
    uint32_t p = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) p |= code[e] << (4 * e);
    *reinterpret_cast<uint32_t*>(prow + c0 / 2) = p;
  } else if (a.bits == 2) {
    uint32_t p = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) p |= code[e] << (2 * e);
    *reinterpret_cast<uint16_t*>(prow + c0 / 4) = (uint16_t)p;
  } else {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) { lo |= code[e] << (8 * e); hi |= code[e + 4] << (8 * e); }
    *reinterpret_cast<ts_u32x2*>(prow + c0) = ts_u32x2{lo, hi};
  }
  if ((threadIdx.x & (GL - 1)) == 0) {
    const int64_t g = c0 / a.gs;
    a.scale16[r * a.n_groups + g] = ts_f2h(scale);
    a.gmin16[r * a.n_groups + g] = ts_f2h(mn);
    if (a.scale32) { a.scale32[r * a.n_groups + g] = scale; a.gmin32[r * a.n_groups + g] = mn; }
  }
}

TS_DEV void or_code(uint8_t* base, int64_t byte, int sh, uint32_t code) {
  uint32_t* word = reinterpret_cast<uint32_t*>(base + (byte & ~(int64_t)3));
  atomicOr(word, code << (sh + 8 * (int)(byte & 3)));
}

// Any group size: one thread per (row, group), serial. Also writes the dummy
// packing column(s) the codec appends when padded_cols is not a multiple of
// the codes per byte (codec.py:613-632).
__global__ void quant_groups_generic_kernel(const GroupArgs a) {
#pragma clang fp contract(off)
  __shared__ float mids[255];
  const int n_mids = a.cb ? a.cb_len - 1 : 0;
  for (int i = threadIdx.x; i < n_mids; i += blockDim.x) mids[i] = (a.cb[i] + a.cb[i + 1]) / 2.0f;
  __syncthreads();
  const int64_t id = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (id >= a.rows * a.n_groups) return;
  const int64_t r = id / a.n_groups, g = id % a.n_groups;
  const int64_t c0 = g * a.gs;
  float mn = load_clamped(a, r, c0), mx = mn;
  for (int e = 1; e < a.gs; ++e) { const float v = load_clamped(a, r, c0 + e); mn = nan_min(mn, v); mx = nan_max(mx, v); }
  const int levels = (1 << a.bits) - 1;
  float scale = (mx - mn) / (float)levels;
  scale = nan_floor(scale, 1e-8f);
  uint8_t* prow = a.packed + r * a.pstride;
  const int per = 8 / a.bits;  // codes per byte
  uint32_t last = 0;
  for (int e = 0; e < a.gs; ++e) {
    const int64_t c = c0 + e;
    const float q = (load_clamped(a, r, c) - mn) / scale;
    const uint32_t code = assign_code(q, levels, a.cb ? mids : nullptr, n_mids);
    last = code;
    if (a.bits == 8) { prow[c] = (uint8_t)code; continue; }
    // A byte can hold codes of two groups (odd group sizes), so codes are
    // OR-ed into zeroed 32-bit words with atomics.
    or_code(a.packed, r * a.pstride + c / per, (int)(c % per) * a.bits, code);
  }
  if (g == a.n_groups - 1 && a.bits != 8) {
    // dummy columns duplicating the last code up to the byte boundary
    for (int64_t c = a.padded_cols; c % per != 0; ++c) {
      or_code(a.packed, r * a.pstride + c / per, (int)(c % per) * a.bits, last);
    }
  }
  a.scale16[r * a.n_groups + g] = ts_f2h(scale);
  a.gmin16[r * a.n_groups + g] = ts_f2h(mn);
  if (a.scale32) { a.scale32[r * a.n_groups + g] = scale; a.gmin32[r * a.n_groups + g] = mn; }
}

int quantize_groups(const ts_qinput* in, const ts_group_opts* o, uint8_t* packed, int64_t pstride, uint16_t* s16,
                    uint16_t* g16, float* s32, float* g32, hipStream_t st) {
  GroupArgs a{};
  a.w = in->w;
  a.dt = in->w_dtype;
  a.rows = in->rows;
  a.cols = in->cols;
  a.bits = o->bits;
  a.gs = o->group_size;
  a.padded_cols = ts_cdiv(in->cols, o->group_size) * o->group_size;
  a.n_groups = a.padded_cols / o->group_size;
  a.t = o->threshold;
  a.clamp = o->clamp;
  a.cb = o->codebook;
  a.cb_len = o->codebook ? o->codebook_len : 0;
  a.packed = packed;
  a.pstride = pstride;
  a.scale16 = s16;
  a.gmin16 = g16;
  a.scale32 = s32;
  a.gmin32 = g32;
  if (a.cb_len > 256) return TS_BAD_ARG;
  const int gl = a.gs / 8;
  const int64_t align = a.bits == 8 ? 8 : (a.bits == 4 ? 4 : 2);
  const bool fast = (a.gs % 8 == 0) && gl >= 1 && gl <= 64 && (gl & (gl - 1)) == 0 && (pstride % align == 0);
  if (fast) {
    dim3 grid((unsigned)ts_cdiv(a.padded_cols / 8, 256), (unsigned)a.rows);
    switch (gl) {
      case 1: hipLaunchKernelGGL(quant_groups_kernel<1>, grid, dim3(256), 0, st, a); break;
      case 2: hipLaunchKernelGGL(quant_groups_kernel<2>, grid, dim3(256), 0, st, a); break;
      case 4: hipLaunchKernelGGL(quant_groups_kernel<4>, grid, dim3(256), 0, st, a); break;
      case 8: hipLaunchKernelGGL(quant_groups_kernel<8>, grid, dim3(256), 0, st, a); break;
      case 16: hipLaunchKernelGGL(quant_groups_kernel<16>, grid, dim3(256), 0, st, a); break;
      case 32: hipLaunchKernelGGL(quant_groups_kernel<32>, grid, dim3(256), 0, st, a); break;
      default: hipLaunchKernelGGL(quant_groups_kernel<64>, grid, dim3(256), 0, st, a); break;
    }
  } else {
    // generic path ORs codes into zeroed packed words
    if (hipMemsetAsync(packed, 0, (size_t)pstride * a.rows, st) != hipSuccess) return TS_HIP_ERROR;
    hipLaunchKernelGGL(quant_groups_generic_kernel, dim3((unsigned)ts_cdiv(a.rows * a.n_groups, 256)), dim3(256), 0,
                       st, a);
  }
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// Normalized value at flat position p of the padded [rows, padded_cols]
// tensor, computed exactly as quant_groups_kernel does (Lloyd-Max sample).
__global__ void lm_sample_kernel(const GroupArgs a, const int64_t* idx, int64_t n, float* out) {
#pragma clang fp contract(off)
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t p = idx[i];
  const int64_t r = p / a.padded_cols, c = p % a.padded_cols;
  const int64_t g = c / a.gs;
  const float v = load_clamped(a, r, c);
  out[i] = (v - a.gmin32[r * a.n_groups + g]) / a.scale32[r * a.n_groups + g];
}

int lm_sample(const ts_qinput* in, const ts_group_opts* o, const float* s32, const float* g32, const int64_t* idx,
              int64_t n, float* out, hipStream_t st) {
  GroupArgs a{};
  a.w = in->w;
  a.dt = in->w_dtype;
  a.rows = in->rows;
  a.cols = in->cols;
  a.gs = o->group_size;
  a.padded_cols = ts_cdiv(in->cols, o->group_size) * o->group_size;
  a.n_groups = a.padded_cols / o->group_size;
  a.t = o->threshold;
  a.clamp = o->clamp;
  a.scale32 = const_cast<float*>(s32);
  a.gmin32 = const_cast<float*>(g32);
  if (n <= 0) return TS_OK;
  hipLaunchKernelGGL(lm_sample_kernel, dim3((unsigned)ts_cdiv(n, 256)), dim3(256), 0, st, a, idx, n, out);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// ---------------------------------------------------------------------------
// Host Lloyd-Max fit (codec.py:320-361) with the reference's float32 order.
// ---------------------------------------------------------------------------
int lloyd_max_fit_host(const float* x, int64_t m, const float* init, int32_t n_levels, int32_t iters, float* out) {
#pragma clang fp contract(off)
  if (m <= 0 || n_levels <= 0) return TS_BAD_ARG;
  std::vector<float> cent(init, init + n_levels), cs(n_levels), mids(n_levels > 1 ? n_levels - 1 : 1);
  std::vector<int64_t> order(n_levels);
  std::vector<float> newc(n_levels), cnt(n_levels);
  for (int it = 0; it < iters; ++it) {
    for (int i = 0; i < n_levels; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return cent[a] < cent[b]; });
    for (int i = 0; i < n_levels; ++i) cs[i] = cent[order[i]];
    for (int i = 0; i + 1 < n_levels; ++i) mids[i] = (cs[i] + cs[i + 1]) / 2.0f;
    std::fill(newc.begin(), newc.end(), 0.f);
    std::fill(cnt.begin(), cnt.end(), 0.f);
    for (int64_t j = 0; j < m; ++j) {
      int64_t a = 0;
      if (n_levels > 1) a = std::lower_bound(mids.begin(), mids.begin() + (n_levels - 1), x[j]) - mids.begin();
      const int64_t c = order[a];
      newc[c] = newc[c] + x[j];
      cnt[c] = cnt[c] + 1.0f;
    }
    for (int i = 0; i < n_levels; ++i) {
      const bool empty = cnt[i] == 0.f;
      const float d = cnt[i] < 1.0f ? 1.0f : cnt[i];
      newc[i] = empty ? cent[i] : newc[i] / d;
    }
    cent = newc;
  }
  std::sort(cent.begin(), cent.end());
  std::copy(cent.begin(), cent.end(), out);
  return TS_OK;
}

// ---------------------------------------------------------------------------
// Double quantization (codec.py:380-417). One workgroup per super-group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dq_kernel(const uint16_t* vals, int64_t n, int dqgs, uint8_t* codes,
                                                 uint16_t* meta, uint16_t* recon) {
#pragma clang fp contract(off)
  __shared__ float smn[256], smx[256];
  const int64_t base = (int64_t)blockIdx.x * dqgs;
  float mn = INFINITY, mx = -INFINITY;
  for (int i = threadIdx.x; i < dqgs; i += blockDim.x) {
    const int64_t f = base + i;
    const float v = ts_h2f(vals[f < n ? f : n - 1]);
    mn = nan_min(mn, v);
    mx = nan_max(mx, v);
  }
  smn[threadIdx.x] = mn;
  smx[threadIdx.x] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      smn[threadIdx.x] = nan_min(smn[threadIdx.x], smn[threadIdx.x + s]);
      smx[threadIdx.x] = nan_max(smx[threadIdx.x], smx[threadIdx.x + s]);
    }
    __syncthreads();
  }
  mn = smn[0];
  mx = smx[0];
  float ms = (mx - mn) / 255.0f;
  ms = nan_floor(ms, 1e-8f);
  const uint16_t ms16 = ts_f2h(ms), mn16 = ts_f2h(mn);
  if (threadIdx.x == 0) { meta[2 * blockIdx.x] = ms16; meta[2 * blockIdx.x + 1] = mn16; }
  const float msr = ts_h2f(ms16), mnr = ts_h2f(mn16);
  for (int i = threadIdx.x; i < dqgs; i += blockDim.x) {
    const int64_t f = base + i;
    const float v = ts_h2f(vals[f < n ? f : n - 1]);
    float c = rintf((v - mn) / ms);
    c = fminf(fmaxf(c, 0.f), 255.f);
    codes[f] = (uint8_t)c;
    if (f < n && recon) recon[f] = ts_f2h(c * msr + mnr);
  }
}

int double_quantize(const uint16_t* v, int64_t n, int64_t dqgs, uint8_t* codes, uint16_t* meta, uint16_t* recon,
                    hipStream_t st) {
  if (n <= 0 || dqgs <= 0) return TS_BAD_ARG;
  const int64_t ns = ts_cdiv(n, dqgs);
  hipLaunchKernelGGL(dq_kernel, dim3((unsigned)ns), dim3(256), 0, st, v, n, (int)dqgs, codes, meta, recon);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

// ---------------------------------------------------------------------------
// RVQ residual (codec.py:703-707) and squared-error sums (codec.py:850-857).
// ---------------------------------------------------------------------------
TS_DEV float base_value_q(const ts_qlayer& L, int64_t row, int64_t col) {
#pragma clang fp contract(off)
  const uint8_t* p = L.packed + row * L.packed_stride;
  const uint32_t c = (p[col >> 1] >> (4 * (col & 1))) & 15u;
  const int64_t flat = row * L.n_groups + col / L.group_size;
  float s, gm;
  if (L.dq_scale_codes) {
    const int64_t sup = flat / L.dq_group_size;
    s = (float)L.dq_scale_codes[flat] * ts_h2f(L.dq_scale_meta[2 * sup]) + ts_h2f(L.dq_scale_meta[2 * sup + 1]);
    gm = (float)L.dq_gmin_codes[flat] * ts_h2f(L.dq_gmin_meta[2 * sup]) + ts_h2f(L.dq_gmin_meta[2 * sup + 1]);
  } else {
    s = ts_h2f(L.scale[flat]);
    gm = ts_h2f(L.gmin[flat]);
  }
  return (float)c * s + gm;
}

__global__ void rvq_residual_kernel(const void* w, int dt, const ts_qlayer L, float* res) {
#pragma clang fp contract(off)
  const int64_t row = blockIdx.y;
  for (int64_t col = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; col < L.cols;
       col += (int64_t)gridDim.x * blockDim.x)
    res[row * L.cols + col] = load_w(w, dt, row * L.cols + col) - base_value_q(L, row, col);
}

__global__ void rvq_residual_outlier_kernel(const void* w, int dt, const int32_t* idx, const uint16_t* val, int64_t n,
                                            float* res) {
#pragma clang fp contract(off)
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  const int64_t f = idx[o];
  res[f] = load_w(w, dt, f) - ts_h2f(val[o]);
}

int rvq_residual(const ts_qinput* in, const ts_qlayer* L, const int32_t* idx, const uint16_t* val, int64_t n,
                 float* res, hipStream_t st) {
  dim3 grid((unsigned)std::min<int64_t>(ts_cdiv(in->cols, 256), 64), (unsigned)in->rows);
  hipLaunchKernelGGL(rvq_residual_kernel, grid, dim3(256), 0, st, in->w, in->w_dtype, *L, res);
  TS_CHECK_LAUNCH();
  if (n > 0) {
    hipLaunchKernelGGL(rvq_residual_outlier_kernel, dim3((unsigned)ts_cdiv(n, 256)), dim3(256), 0, st, in->w,
                       in->w_dtype, idx, val, n, res);
    TS_CHECK_LAUNCH();
  }
  return TS_OK;
}

__global__ __launch_bounds__(256) void sq_err_kernel(const void* w, int dt, const void* d, int ddt, int64_t n,
                                                     double* sums) {
  __shared__ double s0[256], s1[256];
  double a = 0, b = 0;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const double x = load_w(w, dt, i);
    const double y = load_w(d, ddt, i);
    a += (x - y) * (x - y);
    b += x * x;
  }
  s0[threadIdx.x] = a;
  s1[threadIdx.x] = b;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) { s0[threadIdx.x] += s0[threadIdx.x + s]; s1[threadIdx.x] += s1[threadIdx.x + s]; }
    __syncthreads();
  }
  if (threadIdx.x == 0) { atomicAdd(&sums[0], s0[0]); atomicAdd(&sums[1], s1[0]); }
}

int sq_error_sums(const ts_qinput* in, const void* d, int ddt, double* sums, hipStream_t st) {
  const int64_t n = in->rows * in->cols;
  if (hipMemsetAsync(sums, 0, 16, st) != hipSuccess) return TS_HIP_ERROR;
  hipLaunchKernelGGL(sq_err_kernel, dim3((unsigned)std::min<int64_t>(ts_cdiv(n, 256), 2048)), dim3(256), 0, st,
                     in->w, in->w_dtype, d, ddt, n, sums);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

__global__ void gather_f16_kernel(const void* w, int dt, const int64_t* idx, int64_t n, uint16_t* out) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = ts_f2h(load_w(w, dt, idx[i]));
}

int gather_f16(const void* w, int dt, const int64_t* idx, int64_t n, uint16_t* out, hipStream_t st) {
  if (n <= 0) return TS_OK;
  hipLaunchKernelGGL(gather_f16_kernel, dim3((unsigned)ts_cdiv(n, 256)), dim3(256), 0, st, w, dt, idx, n, out);
  TS_CHECK_LAUNCH();
  return TS_OK;
}

}  // namespace ts
