// Per-step kernels around the layer stack: embedding gather (+ first RMSNorm
// fold and RoPE table), vocab-argmax reduction + greedy accept walk, KV/hidden
// compaction, and the final RMSNorm output.
#include "common.h"

namespace dtree {

// RoPE table for the tree rows: angle = position * base^(-2i/D) in fp64, so
// positions in the thousands keep full fp32 accuracy in cos / sin.
__device__ __forceinline__ void rope_entry(const DtreeStepDesc* desc, int e, int rows, int half, float base,
                                           float* cos_out, float* sin_out) {
  if (e >= rows * half) return;
  const int m = e / half, i = e % half;
  const int pos = m < desc->num_nodes ? desc->positions[m] : 0;
  const double inv = exp(-log((double)base) * (2.0 * i) / (2.0 * half));
  const double ang = (double)pos * inv;
  cos_out[e] = (float)cos(ang);
  sin_out[e] = (float)sin(ang);
}

__global__ __launch_bounds__(256) void rope_table_kernel(const DtreeStepDesc* desc, int rows, int half, float base,
                                                         float* cos_out, float* sin_out) {
  rope_entry(desc, blockIdx.x * 256 + threadIdx.x, rows, half, base, cos_out, sin_out);
}

// x[m][:] = E[tokens[m]] (rows >= L zero), xg = bf16(x * g), per-tile sums of x^2.
// Blocks [0, H/256) gather; the remaining blocks fill the RoPE table.
// Element (row, col) of an embedding in DTREE_W_Q4G64 layout, dequantised:
// scale * q + bias of the row's group col / 64.
__device__ __forceinline__ float q4_element(const uint32_t* words, const uint32_t* sb, int row, int col, int H) {
  const int nkb = H >> 6, kb = col >> 6, kk = col & 63;
  const int l = (row & 31) + 32 * (kk >> 5), i = (kk & 31) >> 3, e = kk & 7;
  const size_t blk = (size_t)(row >> 5) * nkb + kb;
  const uint32_t w = words[(blk * 64 + l) * 4 + i];
  const float q = (float)((w >> ((e & 1) * 16 + 4 * (e >> 1))) & 0xFu);
  const uint32_t pr = sb[blk * 32 + (row & 31)];
  return __uint_as_float(pr << 16) * q + __uint_as_float(pr & 0xffff0000u);
}

// Thread = one hidden column over all rows: x[m] = E[tokens[m]], xg = split(x * g),
// ss = per-32-column sums of x^2. Rows go in batches of 32 whose loads are all
// issued before any use.
__global__ __launch_bounds__(256) void embed_kernel(const DtreeStepDesc* desc, const uint16_t* emb, int layout,
                                                    const uint16_t* emb_sb, int V, int H,
                                                    const uint16_t* g, int MP, float* x, uint16_t* xg,
                                                    uint16_t* xg_lo, int xg_tiled, float* ss,
                                                    int half, float base, float* cos_out, float* sin_out,
                                                    int gather_blocks) {
  if ((int)blockIdx.x >= gather_blocks) {
    rope_entry(desc, (blockIdx.x - gather_blocks) * 256 + threadIdx.x, MP, half, base, cos_out, sin_out);
    return;
  }
  const int col = blockIdx.x * 256 + threadIdx.x;
  const int n = threadIdx.x & 31;
  const bool in = col < H;
  const int L = min(desc->num_nodes, MP);
  const float gw = in ? bf2f(g[col]) : 0.f;
  for (int m0 = 0; m0 < MP; m0 += 32) {
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int m = m0 + j;
      v[j] = 0.f;
      if (in && m < L) {
        const int tok = desc->tokens[m];
        if (tok >= 0 && tok < V) {  // out-of-range ids embed as zero
          if (layout == DTREE_W_Q4G64)
            v[j] = q4_element(reinterpret_cast<const uint32_t*>(emb), reinterpret_cast<const uint32_t*>(emb_sb), tok,
                              col, H);
          else
            v[j] = bf2f(emb[layout == DTREE_W_TILED ? tiled_index(tok, col, H) : (size_t)tok * H + col]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int m = m0 + j;
      if (m >= MP) break;
      if (in) {
        x[(size_t)m * H + col] = v[j];
        const float vg = v[j] * gw;
        const uint16_t hi = f2bf(vg);
        const size_t xi = xg_tiled ? tiled_index(m, col, H) : (size_t)m * H + col;
        xg[xi] = hi;
        if (xg_lo) xg_lo[xi] = f2bf(vg - bf2f(hi));
      }
      const float sq = row_sum32(v[j] * v[j]);  // this 32-column tile
      if (in && n == 0) ss[ss_index(col >> 5, m, (H + 31) >> 5)] = sq;
    }
  }
}

__device__ __forceinline__ void argmax_merge2(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

// One workgroup: reduce the LM-head candidates per tree row (wavefront
// butterflies, first index on ties), then walk the tree from the root while
// the target's argmax at the current node is the token of one of its
// children (dtree_runtime.py:195-208).
__global__ __launch_bounds__(256) void walk_kernel(DtreeStepDesc* desc, const int2* cand, int nblocks, int MP,
                                                   int* result) {
  __shared__ int post[DTREE_MAX_NODES];
  const int L = min(max(desc->num_nodes, 1), min(MP, DTREE_MAX_NODES));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int m = wave; m < L; m += 4) {
    float v = -__builtin_huge_valf();
    int idx = 0x7fffffff;
    for (int b = lane; b < nblocks; b += 64) {
      const int2 cv = cand[cand_index(b, m, nblocks)];
      argmax_merge2(v, idx, __int_as_float(cv.x), cv.y);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(v, o);
      const int oi = __shfl_xor(idx, o);
      argmax_merge2(v, idx, ov, oi);
    }
    if (lane == 0) post[m] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc[DTREE_MAX_NODES];
    int n = 1, cur = 0;
    acc[0] = 0;
    int nxt = post[0];
    for (;;) {
      // child_maps[cur][token] keeps the last node inserted with that token.
      int found = -1;
      for (int t = L - 1; t > cur; --t)
        if (desc->parents[t] == cur && desc->tokens[t] == nxt) {
          found = t;
          break;
        }
      if (found < 0) break;
      cur = found;
      acc[n++] = cur;
      nxt = post[cur];
    }
    desc->n_accepted = n;
    desc->bonus_token = nxt;
    for (int i = 0; i < n; ++i) desc->accepted[i] = acc[i];
    if (result) {
      result[0] = n;
      result[1] = nxt;
      result[2] = L;
      for (int i = 0; i < n; ++i) result[3 + i] = acc[i];
    }
  }
  __syncthreads();
  for (int m = threadIdx.x; m < L; m += 256) {
    desc->posterior[m] = post[m];
    if (result) result[3 + DTREE_MAX_NODES + m] = post[m];
  }
}

// Blocks [0, layers*Hkv): K rows of one (layer, kv head); next layers*Hkv
// blocks: V^T columns; one more block: hidden-state select. Kept rows are
// read into LDS before any is written, so the in-place move is safe.
__global__ __launch_bounds__(256) void compact_kernel(const DtreeStepDesc* desc, uint16_t* kp, uint16_t* vp,
                                                      size_t layer_stride, int layers, int Hkv, int D,
                                                      const int* page_table, const uint16_t* hid_in, int hid_w,
                                                      uint16_t* hid_out) {
  __shared__ uint16_t buf[DTREE_MAX_NODES * 128];
  __shared__ int acc[DTREE_MAX_NODES];
  const int n = min(max(desc->n_accepted, 0), DTREE_MAX_NODES), P = desc->past_length, L = desc->num_nodes;
  for (int i = threadIdx.x; i < n; i += 256) acc[i] = desc->accepted[i];
  __syncthreads();
  const int nkv = layers * Hkv;
  const int b = blockIdx.x;
  if (b >= 2 * nkv) {
    if (!hid_out) return;
    for (int e = threadIdx.x; e < n * hid_w; e += 256) {
      const int j = e / hid_w, col = e % hid_w;
      hid_out[(size_t)j * hid_w + col] = hid_in[(size_t)acc[j] * hid_w + col];
    }
    return;
  }
  if (n >= L) return;  // every tree row kept in place (adapters.py:654-655)
  const int layer = (b % nkv) / Hkv, g = (b % nkv) % Hkv;
  const bool is_v = b >= nkv;
  uint16_t* pool = (is_v ? vp : kp) + layer_stride * layer;
  // One kept row = D values; rows staged through LDS in D/128 passes.
  for (int d0 = 0; d0 < D; d0 += 128) {
    const int dw = min(128, D - d0);
    for (int e = threadIdx.x; e < n * dw; e += 256) {
      const int j = e / dw, d = d0 + e % dw;
      const int pos = P + acc[j];
      const int page = page_table[pos / DTREE_PAGE], off = pos % DTREE_PAGE;
      const size_t idx = is_v ? ((size_t)(page * Hkv + g) * D + d) * DTREE_PAGE + off
                              : ((size_t)(page * Hkv + g) * DTREE_PAGE + off) * D + d;
      buf[j * 128 + (d - d0)] = pool[idx];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n * dw; e += 256) {
      const int j = e / dw, d = d0 + e % dw;
      const int pos = P + j;
      const int page = page_table[pos / DTREE_PAGE], off = pos % DTREE_PAGE;
      const size_t idx = is_v ? ((size_t)(page * Hkv + g) * D + d) * DTREE_PAGE + off
                              : ((size_t)(page * Hkv + g) * DTREE_PAGE + off) * D + d;
      pool[idx] = buf[j * 128 + (d - d0)];
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void rownorm_kernel(const float* x, int ldx, int MP, int H, const float* ss,
                                                      int ss_tiles, const uint16_t* w, float eps, uint16_t* out,
                                                      int ld_out) {
  __shared__ float rs[128];
  if ((int)threadIdx.x < MP) {
    float s = 0.f;
    for (int t = 0; t < ss_tiles; ++t) s += ss[ss_index(t, threadIdx.x, ss_tiles)];
    rs[threadIdx.x] = rsqrtf(s / (float)H + eps);
  }
  __syncthreads();
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= H) return;
  const float gw = bf2f(w[col]);
  for (int m = 0; m < MP; ++m) out[(size_t)m * ld_out + col] = f2bf(x[(size_t)m * ldx + col] * rs[m] * gw);
}

__global__ __launch_bounds__(256) void tile_weight_kernel(const uint16_t* src, uint16_t* dst, int n, int k) {
  const size_t total = (size_t)n * k / 8;
  for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < total; v += (size_t)gridDim.x * 256) {
    const int r = (int)(v / (k / 8)), k0 = (int)(v % (k / 8)) * 8;  // 8 consecutive columns of one row
    *reinterpret_cast<u32x4_t*>(dst + tiled_index(r, k0, k)) = *reinterpret_cast<const u32x4_t*>(src + (size_t)r * k + k0);
  }
}

}  // namespace dtree

using namespace dtree;

extern "C" int dtree_tile_weight(const uint16_t* src, uint16_t* dst, int32_t n, int32_t k, hipStream_t stream) {
  DTREE_REQUIRE(src && dst && src != dst, "tile_weight: pointers");
  DTREE_REQUIRE(n > 0 && k > 0 && n % 32 == 0 && k % 64 == 0, "tile_weight: n % 32 and k % 64");
  const size_t total = (size_t)n * k / 8;
  const int grid = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  tile_weight_kernel<<<grid, 256, 0, stream>>>(src, dst, n, k);
  DTREE_LAUNCH_CHECK("tile_weight launch");
  return DTREE_OK;
}

extern "C" int dtree_rope_table(const DtreeStepDesc* desc, int32_t rows_padded, int32_t head_dim, float rope_base,
                                float* rope_cos, float* rope_sin, hipStream_t stream) {
  DTREE_REQUIRE(desc && rope_cos && rope_sin, "rope_table: null pointer");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= DTREE_MAX_NODES, "rope_table: rows_padded");
  DTREE_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "rope_table: head_dim");
  const int n = rows_padded * head_dim / 2;
  rope_table_kernel<<<(n + 255) / 256, 256, 0, stream>>>(desc, rows_padded, head_dim / 2, rope_base, rope_cos,
                                                          rope_sin);
  DTREE_LAUNCH_CHECK("rope_table launch");
  return DTREE_OK;
}

extern "C" int dtree_embed(const DtreeStepDesc* desc, const uint16_t* embed, int32_t embed_layout,
                           const uint16_t* embed_scales, int32_t vocab, int32_t hidden,
                           const uint16_t* norm_w, int32_t rows_padded, float* x, uint16_t* xg, uint16_t* xg_lo,
                           int32_t xg_layout, float* ss, int32_t head_dim, float rope_base,
                           float* rope_cos, float* rope_sin, hipStream_t stream) {
  DTREE_REQUIRE(desc && embed && norm_w && x && xg && ss, "embed: null pointer");
  DTREE_REQUIRE(hidden > 0 && hidden % 32 == 0, "embed: hidden must be a multiple of 32");
  DTREE_REQUIRE(vocab > 0, "embed: vocab");
  DTREE_REQUIRE(embed_layout == DTREE_W_ROWMAJOR ||
                    ((embed_layout == DTREE_W_TILED || embed_layout == DTREE_W_Q4G64) && hidden % 64 == 0 &&
                     vocab % 32 == 0),
                "embed: layout");
  DTREE_REQUIRE(embed_layout != DTREE_W_Q4G64 || embed_scales, "embed: q4 embedding needs embed_scales");
  DTREE_REQUIRE(xg_layout == DTREE_W_ROWMAJOR || (xg_layout == DTREE_W_TILED && hidden % 64 == 0), "embed: xg layout");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= DTREE_MAX_NODES && rows_padded % 32 == 0, "embed: rows_padded");
  const int gather = (hidden + 255) / 256;
  int rope_blocks = 0;
  if (rope_cos && rope_sin) {
    DTREE_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "embed: head_dim");
    rope_blocks = (rows_padded * head_dim / 2 + 255) / 256;
  }
  embed_kernel<<<gather + rope_blocks, 256, 0, stream>>>(desc, embed, embed_layout, embed_scales, vocab, hidden,
                                                          norm_w, rows_padded, x, xg, xg_lo,
                                                          xg_layout == DTREE_W_TILED, ss, head_dim / 2, rope_base,
                                                          rope_cos, rope_sin, gather);
  DTREE_LAUNCH_CHECK("embed launch");
  return DTREE_OK;
}

extern "C" int dtree_accept_walk(DtreeStepDesc* desc, const void* candidates, int32_t num_candidate_blocks,
                                 int32_t rows_padded, int32_t* result, hipStream_t stream) {
  DTREE_REQUIRE(desc && candidates, "accept_walk: null pointer");
  DTREE_REQUIRE(num_candidate_blocks > 0, "accept_walk: num_candidate_blocks");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= DTREE_MAX_NODES, "accept_walk: rows_padded");
  walk_kernel<<<1, 256, 0, stream>>>(desc, reinterpret_cast<const int2*>(candidates), num_candidate_blocks,
                                     rows_padded, result);
  DTREE_LAUNCH_CHECK("accept_walk launch");
  return DTREE_OK;
}

extern "C" int dtree_compact(const DtreeStepDesc* desc, uint16_t* k_pages, uint16_t* v_pages, size_t layer_stride,
                             int32_t layers, int32_t num_kv_heads, int32_t head_dim, const int32_t* page_table,
                             const uint16_t* hidden_in, int32_t hidden_width, uint16_t* hidden_out,
                             hipStream_t stream) {
  DTREE_REQUIRE(desc && page_table, "compact: null pointer");
  DTREE_REQUIRE(layers >= 0 && num_kv_heads > 0 && head_dim > 0, "compact: shape");
  DTREE_REQUIRE(layers == 0 || (k_pages && v_pages), "compact: null cache");
  DTREE_REQUIRE(!hidden_out || (hidden_in && hidden_width > 0), "compact: hidden_in / hidden_width");
  const int grid = 2 * layers * num_kv_heads + 1;
  compact_kernel<<<grid, 256, 0, stream>>>(desc, k_pages, v_pages, layer_stride, layers, num_kv_heads, head_dim,
                                           page_table, hidden_in, hidden_width, hidden_out);
  DTREE_LAUNCH_CHECK("compact launch");
  return DTREE_OK;
}

extern "C" int dtree_rownorm(const float* x, int32_t ldx, int32_t rows_padded, int32_t hidden, const float* ss_in,
                             int32_t ss_tiles, const uint16_t* w, float eps, uint16_t* out, int32_t ld_out,
                             hipStream_t stream) {
  DTREE_REQUIRE(x && ss_in && w && out, "rownorm: null pointer");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= 128 && hidden > 0, "rownorm: shape");
  rownorm_kernel<<<(hidden + 255) / 256, 256, 0, stream>>>(x, ldx, rows_padded, hidden, ss_in, ss_tiles, w, eps, out,
                                                           ld_out);
  DTREE_LAUNCH_CHECK("rownorm launch");
  return DTREE_OK;
}
