// Shared device helpers for the gfx950 GOAP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/tensorshrink_hip.h"

#define TS_DEV __device__ __forceinline__

typedef __bf16 ts_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 ts_f16x8 __attribute__((ext_vector_type(8)));
typedef float ts_f32x4 __attribute__((ext_vector_type(4)));
typedef float ts_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t ts_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t ts_u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 ts_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 ts_f16x2 __attribute__((ext_vector_type(2)));
typedef float ts_f32x2 __attribute__((ext_vector_type(2)));
typedef short ts_s16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// scalar conversions (IEEE, round to nearest even, subnormals kept)
// ---------------------------------------------------------------------------
TS_DEV float ts_h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
TS_DEV uint16_t ts_f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
TS_DEV float ts_bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
TS_DEV uint16_t ts_f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Activation element type: bf16 or f16 storage as uint16_t.
template <bool BF16> struct XT;
template <> struct XT<true> {
  static TS_DEV float to_f(uint16_t v) { return ts_bf2f(v); }
  static TS_DEV uint16_t from_f(float f) { return ts_f2bf(f); }
  static constexpr uint32_t ONE = 0x3f80u;
};
template <> struct XT<false> {
  static TS_DEV float to_f(uint16_t v) { return ts_h2f(v); }
  static TS_DEV uint16_t from_f(float f) { return ts_f2h(f); }
  static constexpr uint32_t ONE = 0x3c00u;
};

// D[16x16] += A[16x32] * B[32x16]. Lane l holds A row l%16, B column l%16,
// k = 8*(l/16) + i for element i, and D[4*(l/16) + i][l%16] (checked on gfx950).
template <bool BF16>
TS_DEV ts_f32x4 ts_mfma16x16x32(ts_u32x4 a, ts_u32x4 b, ts_f32x4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(ts_bf16x8, a),
                                                   __builtin_bit_cast(ts_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(ts_f16x8, a),
                                                  __builtin_bit_cast(ts_f16x8, b), c, 0, 0, 0);
}

// D[32x32] += A[32x16] * B[16x32]. Lane l holds A row l%32, B column l%32,
// k = 8*(l/32) + i, and D[8*(i/4) + 4*(l/32) + i%4][l%32] (checked on gfx950).
template <bool BF16>
TS_DEV ts_f32x16 ts_mfma32x32x16(ts_u32x4 a, ts_u32x4 b, ts_f32x16 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(ts_bf16x8, a),
                                                   __builtin_bit_cast(ts_bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(ts_f16x8, a),
                                                  __builtin_bit_cast(ts_f16x8, b), c, 0, 0, 0);
}

// Non-temporal-free plain 16-byte global load (compiles to global_load_dwordx4).
TS_DEV ts_u32x4 ts_ld16(const void* p) { return *reinterpret_cast<const ts_u32x4*>(p); }
TS_DEV ts_u32x2 ts_ld8(const void* p) { return *reinterpret_cast<const ts_u32x2*>(p); }
TS_DEV uint32_t ts_ld4(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Raw buffer resource over `bytes` bytes at `base` (stride 0, gfx9 dword 3).
// Loads through it take a 32-bit byte offset in one VGPR (the 64-bit base
// stays in SGPRs) and return zero at offsets past `bytes` instead of faulting.
TS_DEV __amdgpu_buffer_rsrc_t ts_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
TS_DEV ts_u32x4 ts_bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(ts_u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Same, with a wave-uniform byte offset `soff` added in the scalar offset field.
TS_DEV ts_u32x4 ts_bld16s(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_bit_cast(ts_u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, 0));
}
TS_DEV ts_u32x2 ts_bld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(ts_u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
TS_DEV uint32_t ts_bld4(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
TS_DEV uint32_t ts_bld2(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }
TS_DEV uint32_t ts_bld1(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0); }

// Kernel-argument pinning. The compiler treats kernel arguments as invariant
// loads and re-fetches them lazily, in dependent batches of scalar loads (each
// a memory round trip) wherever SGPR pressure is high. Passing a value
// through an empty asm makes it opaque, so it is fetched once, up front, and
// kept in SGPRs. Pointers are pinned in the global address space so that
// accesses through them stay global (not flat) instructions.
template <typename T>
TS_DEV void ts_pin_scalar(T& v) {
  asm volatile("" : "+s"(v));
}
template <typename T>
TS_DEV void ts_pin_global(T*& p) {
  auto g = (__attribute__((address_space(1))) T*)p;
  asm volatile("" : "+s"(g));
  p = (T*)g;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS ops
// (lgkmcnt(0)) but not for its in-flight global loads, unlike __syncthreads,
// whose workgroup fence drains vmcnt. The empty asm statements keep the
// compiler from moving memory accesses across it.
TS_DEV void ts_lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt=63, expcnt=7, lgkmcnt=0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Host-side helpers shared by the entry points.
#define TS_CHECK_LAUNCH()                                   \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return TS_HIP_ERROR; \
  } while (0)

__host__ __device__ inline int64_t ts_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Raises a kernel's dynamic LDS limit once per device, thread safe: each
// caller owns a flags/ok pair of 64 entries (one per device ordinal).
// lds_at_zero: the kernel addresses its dynamic LDS from offset 0, so it
// must have no static LDS (checked once, like the attribute).
inline bool ts_set_smem_once(const void* kern, size_t smem, std::once_flag* flags, bool* ok,
                             bool lds_at_zero = false) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::call_once(flags[dev], [&] {
    ok[dev] = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) == hipSuccess;
    if (ok[dev] && lds_at_zero) {
      hipFuncAttributes fa{};
      ok[dev] = hipFuncGetAttributes(&fa, kern) == hipSuccess && fa.sharedSizeBytes == 0;
    }
  });
  return ok[dev];
}
