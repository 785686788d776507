// Context K/V append of the DFlash drafter: the target hidden rows handed to
// the drafter become keys and values of every drafter layer
// (DFlashAttention.precompute_context_kv, draft.py:186-206): k = RoPE(k_norm(
// k_proj(h))) at the cache's running offset, v = v_proj(h), appended to
// either an mlx KVCache (draft.py:206) or the sink + window context cache
// (ContextOnlyDraftKVCache.append_context, draft.py:67-110).
//
// The projections come from the skinny GEMM (fp32 rows [k heads | v heads]);
// this kernel does the per-head RMSNorm and rotation and writes bf16 rows into
// the paged cache layout of the tree attention (K [page][head][64][D], V^T
// [page][head][D][64]).
#include "common.h"

namespace dtree {
namespace {

constexpr int kHeadDim = 128;  // 64 lanes x 2 dims: lane l holds the RoPE pair (l, l + 64)

// One wavefront per (row, kv head); every branch below is uniform over the
// wavefront, so a wave either exits whole or runs its reduction whole.
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ kv, int ld, int n_rows,
                                                        int first_pos, const uint16_t* __restrict__ k_norm, float eps,
                                                        int Hkv, float base, int sink, int window, uint16_t* kp,
                                                        uint16_t* vp, const int32_t* __restrict__ page_table) {
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (wave >= n_rows * Hkv) return;
  const int r = wave / Hkv, g = wave % Hkv;
  const int pos = first_pos + r;
  int slot = pos;
  if (window > 0 && pos >= sink) {
    // Ring slots sink .. sink + window - 1 hold the newest `window` positions;
    // a row that a later row of this call replaces is not written at all.
    if (pos + window <= first_pos + n_rows - 1) return;
    slot = sink + (pos - sink) % window;
  }
  const float* krow = kv + (size_t)r * ld + g * kHeadDim;
  const float* vrow = kv + (size_t)r * ld + (Hkv + g) * kHeadDim;
  float k1 = krow[lane], k2 = krow[lane + 64];
  if (k_norm) {
    float ss = k1 * k1 + k2 * k2;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    const float rs = rsqrtf(ss * (1.0f / kHeadDim) + eps);
    k1 *= rs * bf2f(k_norm[lane]);
    k2 *= rs * bf2f(k_norm[lane + 64]);
  }
  // angle = position * base^(-2i/D) in fp64, as the RoPE table of the tree rows
  const double inv = exp(-log((double)base) * (2.0 * lane) / (double)kHeadDim);
  const double ang = (double)pos * inv;
  const float cs = (float)cos(ang), sn = (float)sin(ang);
  const float y1 = k1 * cs - k2 * sn, y2 = k1 * sn + k2 * cs;
  const int page = page_table[slot / DTREE_PAGE], off = slot % DTREE_PAGE;
  // (page, head) block in the attention kernels' fragment order (kv_k_off / kv_v_off)
  const size_t blk = (size_t)(page * Hkv + g) * DTREE_PAGE * kHeadDim;
  kp[blk + kv_k_off(off, lane, kHeadDim)] = f2bf(y1);
  kp[blk + kv_k_off(off, lane + 64, kHeadDim)] = f2bf(y2);
  vp[blk + kv_v_off(off, lane, kHeadDim)] = f2bf(vrow[lane]);
  vp[blk + kv_v_off(off, lane + 64, kHeadDim)] = f2bf(vrow[lane + 64]);
}

}  // namespace
}  // namespace dtree

using namespace dtree;

extern "C" int dtree_kv_append(const float* kv, int32_t ld_kv, int32_t n_rows, int32_t first_position,
                               const uint16_t* k_norm, float eps, int32_t num_kv_heads, int32_t head_dim,
                               float rope_base, int32_t sink, int32_t window, uint16_t* k_pages, uint16_t* v_pages,
                               const int32_t* page_table, int32_t capacity, hipStream_t stream) {
  DTREE_REQUIRE(head_dim == kHeadDim, "kv_append: head_dim must be 128");
  DTREE_REQUIRE(num_kv_heads > 0 && num_kv_heads <= 64 && ld_kv >= 2 * num_kv_heads * head_dim,
                "kv_append: num_kv_heads / ld_kv");
  DTREE_REQUIRE(n_rows >= 0 && first_position >= 0 && sink >= 0 && window >= 0, "kv_append: negative size");
  DTREE_REQUIRE(n_rows <= (1 << 24) && first_position <= (1 << 30) - n_rows && sink <= (1 << 30) - window,
                "kv_append: size");
  // Every slot written must lie in the positions the page table covers.
  DTREE_REQUIRE(window > 0 ? sink + window <= capacity : first_position + n_rows <= capacity,
                "kv_append: rows beyond the cache capacity");
  DTREE_REQUIRE(rope_base > 0.f, "kv_append: rope_base");
  if (n_rows == 0) return DTREE_OK;
  DTREE_REQUIRE(kv && k_pages && v_pages && page_table, "kv_append: null pointer");
  const int waves = n_rows * num_kv_heads;
  kv_append_kernel<<<(waves + 3) / 4, 256, 0, stream>>>(kv, ld_kv, n_rows, first_position, k_norm, eps,
                                                        num_kv_heads, rope_base, sink, window, k_pages, v_pages,
                                                        page_table);
  DTREE_LAUNCH_CHECK("kv_append launch");
  return DTREE_OK;
}
