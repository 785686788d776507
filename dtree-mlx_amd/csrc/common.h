// Shared device helpers for the gfx950 DTree verify kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/dtree_hip.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

namespace dtree {

// ---- host-side error plumbing ---------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_check(hipError_t e, const char* what);

#define DTREE_REQUIRE(cond, msg)                         \
  do {                                                   \
    if (!(cond)) return ::dtree::fail(DTREE_E_ARG, msg); \
  } while (0)

#define DTREE_LAUNCH_CHECK(what) \
  do {                           \
    int _rc = ::dtree::hip_check(hipGetLastError(), what); \
    if (_rc) return _rc;         \
  } while (0)

// ---- numeric helpers ---------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);                      // round to nearest even
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ u32x4_t ld_u32x4(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// Streaming (read-once) load: weights are not reused within a step, keep them
// out of the way of activations and partials in L2 / MALL.
__device__ __forceinline__ u32x4_t ld_u32x4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Row of 32x32 MFMA accumulator register r held by a lane in half h (= lane/32):
// D[row][col] with col = lane % 32.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// Agent-scope release/acquire around split-K / split-KV partials.
__device__ __forceinline__ void fence_release() { __threadfence(); }
__device__ __forceinline__ void fence_acquire() { __threadfence(); }

}  // namespace dtree
