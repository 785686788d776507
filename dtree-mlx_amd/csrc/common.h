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
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

namespace dtree {

// ---- host-side error plumbing ---------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_check(hipError_t e, const char* what);
bool off_xcd_test();  // DTREE_TEST_OFF_XCD=1: exercise the cross-XCD exchange paths
int attn_spin_limit();  // polls of a bounded cross-workgroup wait (DTREE_TEST_SPIN_LIMIT lowers it)

#define DTREE_REQUIRE(cond, msg)                         \
  do {                                                   \
    if (!(cond)) return ::dtree::fail(DTREE_E_ARG, msg); \
  } while (0)

#define DTREE_LAUNCH_CHECK(what) \
  do {                           \
    int _rc = ::dtree::hip_check(hipGetLastError(), what); \
    if (_rc) return _rc;         \
  } while (0)

// ---- KV cache pages ------------------------------------------------------------
// One (page, kv head) block holds DTREE_PAGE = 64 positions x D dims of K and
// of V, bf16, each in the order the attention MFMAs read them, so that one
// 16-byte load per lane of a wavefront reads one contiguous kilobyte:
// * K: the A operand of S^T = K Q^T (32 keys x 16 dims per fragment, lane
//   (r, h) = 32 h + r holds dims 8h .. 8h+7 of its key). Fragment (key half b,
//   dim step j) is the kilobyte b * (D/16) + j, so the 32 keys of a half page
//   are one contiguous run; lane r of it holds slot 32 b + pi(r), pi = swap
//   bits 2 and 3, the key order in which the S^T registers of a lane half form
//   runs of eight consecutive keys for the P.V step.
// * V: the A operand of O^T = V^T P^T (32 dims x 16 keys per fragment, lane
//   (r, h) holds slots 8h .. 8h+7 of its dim). Fragment (key step st of 16
//   slots, dim block db) is the kilobyte st * (D/32) + db.
__host__ __device__ __forceinline__ int kv_pi(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
__host__ __device__ __forceinline__ int kv_k_off(int slot, int d, int D) {
  return ((((slot >> 5) * (D >> 4) + (d >> 4)) * 64 + ((d >> 3) & 1) * 32 + kv_pi(slot & 31)) << 3) + (d & 7);
}
__host__ __device__ __forceinline__ int kv_v_off(int slot, int d, int D) {
  return ((((slot >> 4) * (D >> 5) + (d >> 5)) * 64 + ((slot >> 3) & 1) * 32 + (d & 31)) << 3) + (slot & 7);
}

// ---- numeric helpers ---------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even (NaN stays NaN): gfx950's
// v_cvt_pk_bf16_f32, reached through the vector conversion.
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)(pack_bf2(f, 0.f) & 0xffffu); }

// 2^x with the bare v_exp_f32 (no denormal range fix-up): callers pass x <= 0
// where results below 2^-126 only ever scale down a sum.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ u32x4_t ld_u32x4(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }

// Streaming (read-once) load: weights are not reused within a step, keep them
// out of the way of activations and partials in L2 / MALL.
__device__ __forceinline__ u32x4_t ld_u32x4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// ---- ranged buffer loads for register rings ------------------------------
// A load through a raw buffer resource at a byte offset >= its size returns
// zero without touching memory. A ring that refills its slots this way issues
// the same number of loads on every path, whatever the remaining trip count,
// so the compiler can wait for exactly the slot it consumes (vmcnt(N) with N
// loads still in flight) instead of for every outstanding load, which it must
// do when a refill is skipped on some path.
constexpr unsigned kOob = 0x80000000u;  // offset past any buffer here (sizes < 2 GiB)
constexpr int kNt = 2;                  // cache policy: nontemporal (read-once weights)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t buf_ld(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x4_t buf_ld_stream(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kNt);
}
__device__ __forceinline__ uint32_t buf_ld32(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ float buf_ldf(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// fp16 operands (v_mfma_f32_32x32x16_f16), fp32 accumulate.
__device__ __forceinline__ f32x16_t mfma32_f16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                0, 0, 0);
}

// fp32 pair -> fp16 pair, round to nearest even.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}
__device__ __forceinline__ uint16_t f2h(float f) { return (uint16_t)(pack_h2(f, 0.f) & 0xffffu); }
__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// Activations for the next GEMM, 4 or 8 consecutive values at element oi:
// DTREE_W_TILED_F16 (h16) -> one fp16 plane; else bf16 hi + bf16 lo (lo =
// bf16(v - hi), skipped when lo is null).
__device__ __forceinline__ void store_act4(uint16_t* hi, uint16_t* lo, size_t oi, const float (&y)[4], bool h16) {
  if (h16) {
    *reinterpret_cast<u32x2_t*>(hi + oi) = u32x2_t{pack_h2(y[0], y[1]), pack_h2(y[2], y[3])};
    return;
  }
  float rl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rl[i] = y[i] - bf2f(f2bf(y[i]));
  *reinterpret_cast<u32x2_t*>(hi + oi) = u32x2_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3])};
  if (lo) *reinterpret_cast<u32x2_t*>(lo + oi) = u32x2_t{pack_bf2(rl[0], rl[1]), pack_bf2(rl[2], rl[3])};
}
__device__ __forceinline__ void store_act8(uint16_t* hi, uint16_t* lo, size_t oi, const float (&y)[8], bool h16) {
  if (h16) {
    *reinterpret_cast<u32x4_t*>(hi + oi) =
        u32x4_t{pack_h2(y[0], y[1]), pack_h2(y[2], y[3]), pack_h2(y[4], y[5]), pack_h2(y[6], y[7])};
    return;
  }
  float rr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rr[i] = y[i] - bf2f(f2bf(y[i]));
  *reinterpret_cast<u32x4_t*>(hi + oi) =
      u32x4_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]), pack_bf2(y[6], y[7])};
  if (lo)
    *reinterpret_cast<u32x4_t*>(lo + oi) =
        u32x4_t{pack_bf2(rr[0], rr[1]), pack_bf2(rr[2], rr[3]), pack_bf2(rr[4], rr[5]), pack_bf2(rr[6], rr[7])};
}

// 8 consecutive elements of one 16-byte load as fp32: fp16 (h16: the
// DTREE_W_TILED_F16 layout) or bf16 (every other layout).
__device__ __forceinline__ void unpack8(u32x4_t w, bool h16, float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t b = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu);
    v[i] = h16 ? h2f((uint16_t)b) : __uint_as_float(b << 16);
  }
}

// bf16 pair -> fp16 pair. Exact for every bf16 value of magnitude in
// [2^-14, 65504] (fp16 has more significand bits than bf16); smaller ones
// round to fp16's 2^-24 grid, larger ones saturate to +-65504.
__device__ __forceinline__ uint32_t bf2_to_h2(uint32_t w) {
  const float lo = __builtin_amdgcn_fmed3f(__uint_as_float(w << 16), -65504.f, 65504.f);
  const float hi = __builtin_amdgcn_fmed3f(__uint_as_float(w & 0xffff0000u), -65504.f, 65504.f);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}
__device__ __forceinline__ u32x4_t bf8_to_h8(u32x4_t v) {
  return u32x4_t{bf2_to_h2(v[0]), bf2_to_h2(v[1]), bf2_to_h2(v[2]), bf2_to_h2(v[3])};
}

// ---- cross-lane reductions without LDS round trips -------------------------
// DPP moves within 16-lane rows plus one ds_swizzle across the two rows of a
// 32-lane half. Every lane of a 32-lane half ends with the half's total.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ int swz_xor16_i(int v) {
  // bitmask mode: and_mask 0x1F, or_mask 0, xor_mask 0x10 (groups of 32 lanes)
  return __builtin_amdgcn_ds_swizzle(v, 0x401F);
}
__device__ __forceinline__ float swz_xor16(float v) {
  return __builtin_bit_cast(float, swz_xor16_i(__builtin_bit_cast(int, v)));
}
// a + (the same lane's value in the other 16-lane row of its 32-lane half),
// with v_permlane16_swap (a VALU lane exchange, no LDS round trip). Written
// as one asm sequence: the compiler's own lowering of the builtin, when both
// swapped registers hold the same value and the two results are added, adds
// the first result to itself (checked on the device), so it is not used.
// The s_nop covers the VALU-write to permlane-read hazard, as the compiler
// places it.
__device__ __forceinline__ float row_pair_sum(float a) {
  float b;
  asm volatile("v_mov_b32 %1, %0\n\ts_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_add_f32 %0, %0, %1"
               : "+v"(a), "=&v"(b));
  return a;
}
__device__ __forceinline__ float row_sum32(float a) {
  a += dpp<0xB1>(a);   // lane ^ 1
  a += dpp<0x4E>(a);   // lane ^ 2
  a += dpp<0x141>(a);  // half-row mirror: the other quad of 8 lanes
  a += dpp<0x140>(a);  // row mirror: the other 8 lanes of 16
  return a + swz_xor16(a);  // the other 16-lane row
}

// (max, first index on ties): a total order, so a reduction's result does not
// depend on how candidates are paired.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& v, int& i) {
  argmax_merge(v, i, dpp<CTRL>(v), dpp_i<CTRL>(i));
}
// (max, first index on ties) over TN lanes (32: each half-wave, 64: the wave).
template <int TN>
__device__ __forceinline__ void lane_argmax(float& v, int& i) {
  argmax_dpp<0xB1>(v, i);
  argmax_dpp<0x4E>(v, i);
  argmax_dpp<0x141>(v, i);
  argmax_dpp<0x140>(v, i);
  argmax_merge(v, i, swz_xor16(v), swz_xor16_i(i));
  if constexpr (TN == 64) argmax_merge(v, i, __shfl_xor(v, 32), __shfl_xor(i, 32));
}

// Parent index of tree node t as a kernel may use it: parents precede their
// children (dtree_runtime.py:125-130), so anything outside [0, t) (a tree the
// host did not validate) is read as the root's parent -1, which keeps every
// per-node access in bounds and every ancestor walk finite.
__device__ __forceinline__ int valid_parent(int p, int t) { return (p >= 0 && p < t) ? p : -1; }

// Row of 32x32 MFMA accumulator register r held by a lane in half h (= lane/32):
// D[row][col] with col = lane % 32.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// Per-row RMSNorm statistics (sums of x^2 over each 32-column tile) are laid
// out [rows/32][tiles][32]: every 32-row block is one contiguous [tiles][32]
// array, so kernels that work on one 32-row block address it directly.
__device__ __forceinline__ size_t ss_index(int t, int m, int tiles) {
  return ((size_t)(m >> 5) * tiles + t) * 32 + (m & 31);
}
// LM-head candidates (per workgroup, per row) are laid out [rows/32][blocks][32]
// the same way.
__device__ __forceinline__ size_t cand_index(int blk, int m, int blocks) {
  return ((size_t)(m >> 5) * blocks + blk) * 32 + (m & 31);
}

// Element (row r, column k) of a DTREE_W_TILED matrix with `width` columns:
// [rows/32][width/64][4][64][8], lane l = r%32 + 32*((k%64)/32) of load i.
__device__ __forceinline__ size_t tiled_index(int r, int k, int width) {
  const int l = (r & 31) + 32 * ((k & 63) >> 5);
  const int i = (k & 31) >> 3, e = k & 7;
  return (((size_t)(r >> 5) * (width >> 6) + (k >> 6)) * 4 + i) * 512 + (size_t)l * 8 + e;
}

// Cross-workgroup hand-off of partial results without cache maintenance.
// A device-scope __threadfence() writes back and invalidates the whole L2 of
// the XCD (buffer_wbl2 / buffer_inv) and costs tens of microseconds when every
// workgroup issues it. Partials are instead written and read with
// agent-coherent (sc1) accesses; the producer waits for its stores to be
// acknowledged (s_waitcnt) before the workgroup's counter increment, and the
// last workgroup to arrive reads every partial coherently.
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores_done() { __builtin_amdgcn_s_waitcnt(0); }
// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS (and
// scalar) operations, not for its global loads and stores, which
// __syncthreads() drains as a workgroup-scope fence. Loads issued before it
// stay in flight; stores (e.g. cache rows nobody in the workgroup reads back)
// retire in the background.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ int arrive(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_counter(int* counter) {
  __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int arrive_add(int* counter, int v) {
  return __hip_atomic_fetch_add(counter, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCD placement. Workgroups are dispatched round-robin over the 8 XCDs
// (blockIdx % 8); a workgroup checks its own with HW_REG_XCC_ID. Cross-
// workgroup exchanges write through (sc1) and read from the local L2 (sc0)
// only when every party is confirmed on the same XCD; an arrival from a
// workgroup off its expected XCD adds kForeign to the counter.
constexpr int kXcds = 8;
constexpr int kForeign = 1 << 16;
constexpr int kSc0 = 1;   // cache policy sc0: coherent within one XCD (read from its L2)
constexpr int kSc1 = 16;  // cache policy sc1: coherent across the XCDs' L2s (written through / read past them)
__device__ __forceinline__ int xcc_id() {
  return __builtin_amdgcn_s_getreg(20 | (3 << 11));  // HW_REG_XCC_ID, bits [3:0]
}

// Tree-attention workspace layout shared by both attention designs:
//   [0, 4 KiB)           header: error word (bytes 0..3), the flag exchange's
//                        epoch table location (bytes 8..15), split counters
//                        from byte 64
//   [4 KiB, + ll bytes)  flag exchange of the per-head kernel (rows_padded 32
//                        only): one epoch word per query head, then
//                        kAttnLLSplits slots per head; neither design's
//                        partials ever land here, so a flag word only ever
//                        holds a flag
//   then                 the design's own partials
// A slot is 512 bytes of (row max, flag, row sum, flag) for 32 query rows,
// then one 2 KiB unit per (32-dim block, 8-dim group): two runs of 64 lanes x
// 16 bytes of (value, flag) pairs (a lane's values 0, 1, then its 2, 3).
constexpr size_t kAttnWsHeader = 4096;
constexpr int kAttnLLSplits = 8;
__host__ __device__ constexpr unsigned attn_ll_slot_bytes(int D) { return 512u + 4u * (unsigned)(D / 32) * 2048u; }
__host__ __device__ constexpr size_t attn_ll_epoch_bytes(int Hq) { return ((size_t)Hq * 4 + 255) & ~(size_t)255; }
__host__ __device__ constexpr size_t attn_ll_bytes(int Hq, int D, int rows_padded) {
  return rows_padded == 32 ? attn_ll_epoch_bytes(Hq) + (size_t)Hq * kAttnLLSplits * attn_ll_slot_bytes(D) : 0;
}

}  // namespace dtree
