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

// Stores 8 consecutive columns of row m of the layer input: x = v (fp32),
// xg = v * g in xg's layout (DTREE_W_TILED_F16: one fp16 plane; else bf16 hi,
// optional lo), and the row's sum of x^2 over the
// 32-column tile, added over the tile's 4 threads (a lane quad) with DPP.
// Every thread of the wavefront calls it (the DPP needs all lanes); `in`
// marks the threads that own a column group.
__device__ __forceinline__ void fold_store8(const float (&v)[8], bool in, int m, int col, const uint16_t* g, int H,
                                            float* x, uint16_t* xg, uint16_t* xg_lo, int xg_layout, float* ss) {
  if (in) {
    const u32x4_t gwv = ld_u32x4(g + col);
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      y[i] = v[i] * __uint_as_float((i & 1) ? (gwv[i >> 1] & 0xffff0000u) : (gwv[i >> 1] << 16));
    float* xr = x + (size_t)m * H + col;
    *reinterpret_cast<f32x4_t*>(xr) = f32x4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4_t*>(xr + 4) = f32x4_t{v[4], v[5], v[6], v[7]};
    const size_t xi = xg_layout != DTREE_W_ROWMAJOR ? tiled_index(m, col, H) : (size_t)m * H + col;
    store_act8(xg, xg_lo, xi, y, xg_layout == DTREE_W_TILED_F16);
  }
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sq += v[i] * v[i];
  sq += dpp<0xB1>(sq);  // the 4 threads of a 32-column tile (a lane quad; rows hold whole quads)
  sq += dpp<0x4E>(sq);
  if (in && (col & 31) == 0) ss[ss_index(col >> 5, m, H >> 5)] = sq;
}

// Thread = 8 consecutive hidden columns of one row (one 16-byte load of the
// embedding row): x[m] = E[tokens[m]] (rows >= L zero), then fold_store8.
// Blocks [0, gather_blocks) gather; the remaining blocks fill the RoPE table.
__global__ __launch_bounds__(256) void embed_kernel(const DtreeStepDesc* desc, const uint16_t* emb, int layout,
                                                    const uint16_t* emb_sb, int V, int H,
                                                    const uint16_t* g, int MP, float* x, uint16_t* xg,
                                                    uint16_t* xg_lo, int xg_layout, float* ss,
                                                    int half, float base, float* cos_out, float* sin_out,
                                                    int gather_blocks) {
  if ((int)blockIdx.x >= gather_blocks) {
    rope_entry(desc, (blockIdx.x - gather_blocks) * 256 + threadIdx.x, MP, half, base, cos_out, sin_out);
    return;
  }
  const int per_row = H >> 3;
  const int gt = blockIdx.x * 256 + threadIdx.x;
  const bool in = gt < MP * per_row;
  const int m = in ? gt / per_row : 0, col = in ? (gt % per_row) * 8 : 0;
  const int L = min(desc->num_nodes, MP);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
  if (in && m < L) {
    const int tok = desc->tokens[m];
    if (tok >= 0 && tok < V) {  // out-of-range ids embed as zero
      if (layout == DTREE_W_Q4G64) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = q4_element(reinterpret_cast<const uint32_t*>(emb), reinterpret_cast<const uint32_t*>(emb_sb), tok,
                            col + i, H);
      } else {
        const bool tl = layout != DTREE_W_ROWMAJOR;  // tiled bf16, or tiled fp16 (TILED_F16)
        unpack8(ld_u32x4(emb + (tl ? tiled_index(tok, col, H) : (size_t)tok * H + col)), layout == DTREE_W_TILED_F16,
                v);
      }
    }
  }
  fold_store8(v, in, m, col, g, H, x, xg, xg_lo, xg_layout, ss);
}

// Gather + fold for a token array of any length (prompt prefill): row m < n
// embeds tokens[m], rows n .. MP - 1 are zero.
__global__ __launch_bounds__(256) void embed_tokens_kernel(const int32_t* tokens, int n, const uint16_t* emb,
                                                           int layout, const uint16_t* emb_sb, int V, int H,
                                                           const uint16_t* g, int MP, float* x, uint16_t* xg,
                                                           uint16_t* xg_lo, int xg_layout, float* ss) {
  const int per_row = H >> 3;
  const long long gt = (long long)blockIdx.x * 256 + threadIdx.x;
  const bool in = gt < (long long)MP * per_row;
  const int m = in ? (int)(gt / per_row) : 0, col = in ? (int)(gt % per_row) * 8 : 0;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
  if (in && m < n) {
    const int tok = tokens[m];
    if (tok >= 0 && tok < V) {
      if (layout == DTREE_W_Q4G64) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = q4_element(reinterpret_cast<const uint32_t*>(emb), reinterpret_cast<const uint32_t*>(emb_sb), tok,
                            col + i, H);
      } else {
        const bool tl = layout != DTREE_W_ROWMAJOR;  // tiled bf16, or tiled fp16 (TILED_F16)
        unpack8(ld_u32x4(emb + (tl ? tiled_index(tok, col, H) : (size_t)tok * H + col)), layout == DTREE_W_TILED_F16,
                v);
      }
    }
  }
  fold_store8(v, in, m, col, g, H, x, xg, xg_lo, xg_layout, ss);
}

// The same layer-input fold for rows handed over by the caller (the DFlash
// drafter's noise embedding, draft.py:355-364): x[m] = rows[m] (bf16, rows
// >= n_rows zero), then fold_store8.
__global__ __launch_bounds__(256) void rows_in_kernel(const uint16_t* rows, int ld_rows, int n_rows, const uint16_t* g,
                                                      int MP, int H, float* x, uint16_t* xg, uint16_t* xg_lo,
                                                      int xg_layout, float* ss) {
  const int per_row = H >> 3;
  const int gt = blockIdx.x * 256 + threadIdx.x;
  const bool in = gt < MP * per_row;
  const int m = in ? gt / per_row : 0, col = in ? (gt % per_row) * 8 : 0;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
  if (in && m < n_rows) {
    const u32x4_t w = ld_u32x4(rows + (size_t)m * ld_rows + col);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
  }
  fold_store8(v, in, m, col, g, H, x, xg, xg_lo, xg_layout, ss);
}


// One workgroup: reduce the LM-head candidates per tree row (wavefront
// butterflies, first index on ties), then walk the tree from the root while
// the target's argmax at the current node is the token of one of its
// children (dtree_runtime.py:195-208).
constexpr int kWalkThreads = 1024;  // 16 waves, 16 candidate loads each in flight
__global__ __launch_bounds__(kWalkThreads) void walk_kernel(DtreeStepDesc* desc, const int2* cand, int nblocks, int MP,
                                                   int* result) {
  __shared__ int post[DTREE_MAX_NODES];
  __shared__ int par_s[DTREE_MAX_NODES], tok_s[DTREE_MAX_NODES];
  const int L = min(max(desc->num_nodes, 1), min(MP, DTREE_MAX_NODES));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // The walk reads parents and tokens from LDS (one load per node here).
  for (int m = threadIdx.x; m < L; m += kWalkThreads) {
    par_s[m] = valid_parent(desc->parents[m], m);
    tok_s[m] = desc->tokens[m];
  }
  // Candidates of one 32-row block are [blocks][32] pairs, 256 bytes per
  // workgroup. Thread t = 16 s + j reads the 16 bytes of rows 2j, 2j + 1 of
  // workgroups s, s + S, s + 2S, ... (S = threads / 16), so each wave load
  // covers 1 KB contiguous; the four lanes of a wave that share j, then the
  // waves, are merged ((max, first index) is a total order, so the pairing
  // does not matter).
  constexpr int kW = kWalkThreads / 64;
  __shared__ float red_v[kW][32];
  __shared__ int red_i[kW][32];
  constexpr int kBatch = 16384 / kWalkThreads;  // loads in flight per thread (one batch covers 1024 workgroups)
  const int j = threadIdx.x & 15, s0 = threadIdx.x >> 4;
  for (int r0 = 0; r0 < L; r0 += 32) {
    const __amdgpu_buffer_rsrc_t crs = buf_rsrc(cand + cand_index(0, r0, nblocks), (unsigned)nblocks * 256u);
    float v0 = -__builtin_huge_valf(), v1 = v0;
    int i0 = 0x7fffffff, i1 = i0;
    for (int b0 = s0; b0 < nblocks; b0 += (kWalkThreads / 16) * kBatch) {
      u32x4_t w[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int b = b0 + (kWalkThreads / 16) * k;
        w[k] = buf_ld(crs, b < nblocks ? (unsigned)(b * 256 + j * 16) : kOob);
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (b0 + (kWalkThreads / 16) * k < nblocks) {
          argmax_merge(v0, i0, __uint_as_float(w[k][0]), (int)w[k][1]);
          argmax_merge(v1, i1, __uint_as_float(w[k][2]), (int)w[k][3]);
        }
      }
    }
    argmax_merge(v0, i0, swz_xor16(v0), swz_xor16_i(i0));
    argmax_merge(v1, i1, swz_xor16(v1), swz_xor16_i(i1));
    argmax_merge(v0, i0, __shfl_xor(v0, 32), __shfl_xor(i0, 32));
    argmax_merge(v1, i1, __shfl_xor(v1, 32), __shfl_xor(i1, 32));
    if (lane < 16) {
      red_v[wave][2 * lane] = v0;
      red_i[wave][2 * lane] = i0;
      red_v[wave][2 * lane + 1] = v1;
      red_i[wave][2 * lane + 1] = i1;
    }
    __syncthreads();
    if (threadIdx.x < 32 && r0 + (int)threadIdx.x < L) {
      const int m = threadIdx.x;
      float bv = red_v[0][m];
      int bi = red_i[0][m];
#pragma unroll
      for (int w2 = 1; w2 < kW; ++w2) argmax_merge(bv, bi, red_v[w2][m], red_i[w2][m]);
      post[r0 + m] = bi;
    }
    __syncthreads();
  }
  // The walk on wave 0: at each step every lane tests its nodes against
  // (parent cur, token nxt) and a ballot picks the largest match, i.e. the
  // last node inserted with that token (child_maps semantics). cur strictly
  // increases, so the walk ends within L steps.
  __shared__ int acc_s[DTREE_MAX_NODES];
  __shared__ int walk_n;
  if (wave == 0) {
    int n = 1, cur = 0, nxt = post[0];
    if (lane == 0) acc_s[0] = 0;
    for (;;) {
      int found = -1;
      for (int base = ((L - 1) >> 6) << 6; base >= 0 && found < 0; base -= 64) {
        const int t = base + lane;
        const bool hit = t > cur && t < L && par_s[t] == cur && tok_s[t] == nxt;
        const unsigned long long m = __ballot(hit);
        if (m) found = base + 63 - __builtin_clzll(m);
      }
      if (found < 0) break;
      cur = found;
      if (lane == 0) acc_s[n] = cur;
      ++n;
      nxt = post[cur];
    }
    if (lane == 0) {
      walk_n = n;
      desc->n_accepted = n;
      desc->bonus_token = nxt;
      if (result) {
        result[0] = n;
        result[1] = nxt;
        result[2] = L;
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < walk_n; i += kWalkThreads) {
    desc->accepted[i] = acc_s[i];
    if (result) result[3 + i] = acc_s[i];
  }
  for (int m = threadIdx.x; m < L; m += kWalkThreads) {
    desc->posterior[m] = post[m];
    if (result) result[3 + DTREE_MAX_NODES + m] = post[m];
  }
}

// Blocks [0, layers*Hkv): K rows of one (layer, kv head); next layers*Hkv
// blocks: V^T columns; kHidBlocks more blocks: hidden-state select. Kept rows are
// read into LDS before any is written, so the in-place move is safe. The
// page and slot of every source (P + accepted[j]) and destination (P + j)
// position are looked up once per block; K rows move in 16-byte pieces, and
// V^T (positions contiguous within a dim) is walked position-fastest, so a
// wave's reads and writes of one dim touch one or two 128-byte lines.
constexpr int kHidBlocks = 16;  // blocks of the compaction's hidden-state select

__global__ __launch_bounds__(256) void compact_kernel(const DtreeStepDesc* desc, uint16_t* kp, uint16_t* vp,
                                                      size_t layer_stride, int layers, int Hkv, int D,
                                                      const int* page_table, const uint16_t* hid_in, int hid_w,
                                                      uint16_t* hid_out) {
  __shared__ u32x4_t buf[DTREE_MAX_NODES * 16];  // 32 KB: n rows x 128 dims (bf16) per pass
  __shared__ int acc[DTREE_MAX_NODES];
  __shared__ int src_row[DTREE_MAX_NODES], dst_row[DTREE_MAX_NODES];  // page * 64 + slot
  const int n = min(max(desc->n_accepted, 0), DTREE_MAX_NODES), P = desc->past_length, L = desc->num_nodes;
  const int nkv = layers * Hkv;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  if (t < n) {
    const int a = desc->accepted[t];
    acc[t] = a;
    if (b < 2 * nkv) {
      const int ps = P + a, pd = P + t;
      src_row[t] = page_table[ps / DTREE_PAGE] * DTREE_PAGE + ps % DTREE_PAGE;
      dst_row[t] = page_table[pd / DTREE_PAGE] * DTREE_PAGE + pd % DTREE_PAGE;
    }
  }
  __syncthreads();
  if (b >= 2 * nkv) {
    // hidden select over kHidBlocks blocks, 16-byte pieces (hid_w % 8 == 0)
    if (!hid_out) return;
    const int nch = hid_w / 8;
    for (int e = (b - 2 * nkv) * 256 + t; e < n * nch; e += kHidBlocks * 256) {
      const int j = e / nch, ch = e % nch;
      *reinterpret_cast<u32x4_t*>(hid_out + (size_t)j * hid_w + 8 * ch) =
          *reinterpret_cast<const u32x4_t*>(hid_in + (size_t)acc[j] * hid_w + 8 * ch);
    }
    return;
  }
  if (n >= L) return;  // every tree row kept in place (adapters.py:654-655)
  const int layer = (b % nkv) / Hkv, g = (b % nkv) % Hkv;
  if (b < nkv) {
    // K of position (page, slot): dims 8c .. 8c+7 are one 16-byte run at
    // kv_k_off(slot, 8c) in the (page, head) block.
    uint16_t* pool = kp + layer_stride * layer;
    for (int d0 = 0; d0 < D; d0 += 128) {
      const int dw = min(128, D - d0), nch = dw / 8;  // 16-byte pieces per row this pass
      for (int e = t; e < n * nch; e += 256) {
        const int j = e / nch, ch = e % nch, r = src_row[j];
        const size_t idx = (size_t)((r / DTREE_PAGE) * Hkv + g) * DTREE_PAGE * D + kv_k_off(r % DTREE_PAGE, d0 + 8 * ch, D);
        buf[j * 16 + ch] = *reinterpret_cast<const u32x4_t*>(pool + idx);
      }
      __syncthreads();
      for (int e = t; e < n * nch; e += 256) {
        const int j = e / nch, ch = e % nch, r = dst_row[j];
        const size_t idx = (size_t)((r / DTREE_PAGE) * Hkv + g) * DTREE_PAGE * D + kv_k_off(r % DTREE_PAGE, d0 + 8 * ch, D);
        *reinterpret_cast<u32x4_t*>(pool + idx) = buf[j * 16 + ch];
      }
      __syncthreads();
    }
    return;
  }
  // V of (dim d, position (page, slot)) at kv_v_off(slot, d) of the (page, head) block.
  uint16_t* pool = vp + layer_stride * layer;
  uint16_t* vb = reinterpret_cast<uint16_t*>(buf);
  for (int d0 = 0; d0 < D; d0 += 128) {
    const int dw = min(128, D - d0);
    for (int e = t; e < n * dw; e += 256) {
      const int d = d0 + e / n, j = e % n, r = src_row[j];
      vb[(d - d0) * n + j] = pool[(size_t)((r / DTREE_PAGE) * Hkv + g) * DTREE_PAGE * D + kv_v_off(r % DTREE_PAGE, d, D)];
    }
    __syncthreads();
    for (int e = t; e < n * dw; e += 256) {
      const int d = d0 + e / n, j = e % n, r = dst_row[j];
      pool[(size_t)((r / DTREE_PAGE) * Hkv + g) * DTREE_PAGE * D + kv_v_off(r % DTREE_PAGE, d, D)] = vb[(d - d0) * n + j];
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

// bf16 row-major -> tiled, bf16 or (H) fp16 elements: every bf16 of
// magnitude 2^-17 .. 65504 converts to fp16 exactly; smaller ones round to
// fp16's 2^-24 grid (nearest even), larger ones saturate to +-65504.
template <bool H>
__global__ __launch_bounds__(256) void tile_weight_kernel(const uint16_t* src, uint16_t* dst, int n, int k) {
  const size_t total = (size_t)n * k / 8;
  for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < total; v += (size_t)gridDim.x * 256) {
    const int r = (int)(v / (k / 8)), k0 = (int)(v % (k / 8)) * 8;  // 8 consecutive columns of one row
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(src + (size_t)r * k + k0);
    if constexpr (H) {
      float f[8];
      unpack8(w, false, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = __builtin_amdgcn_fmed3f(f[i], -65504.f, 65504.f);
      *reinterpret_cast<u32x4_t*>(dst + tiled_index(r, k0, k)) =
          u32x4_t{pack_h2(f[0], f[1]), pack_h2(f[2], f[3]), pack_h2(f[4], f[5]), pack_h2(f[6], f[7])};
    } else {
      *reinterpret_cast<u32x4_t*>(dst + tiled_index(r, k0, k)) = w;
    }
  }
}

}  // namespace dtree

using namespace dtree;

extern "C" int dtree_tile_weight(const uint16_t* src, uint16_t* dst, int32_t n, int32_t k, hipStream_t stream) {
  DTREE_REQUIRE(src && dst && src != dst, "tile_weight: pointers");
  DTREE_REQUIRE(n > 0 && k > 0 && n % 32 == 0 && k % 64 == 0, "tile_weight: n % 32 and k % 64");
  const size_t total = (size_t)n * k / 8;
  const int grid = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  tile_weight_kernel<false><<<grid, 256, 0, stream>>>(src, dst, n, k);
  DTREE_LAUNCH_CHECK("tile_weight launch");
  return DTREE_OK;
}

extern "C" int dtree_tile_weight_f16(const uint16_t* src, uint16_t* dst, int32_t n, int32_t k, hipStream_t stream) {
  DTREE_REQUIRE(src && dst && src != dst, "tile_weight_f16: pointers");
  DTREE_REQUIRE(n > 0 && k > 0 && n % 32 == 0 && k % 64 == 0, "tile_weight_f16: n % 32 and k % 64");
  const size_t total = (size_t)n * k / 8;
  const int grid = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  tile_weight_kernel<true><<<grid, 256, 0, stream>>>(src, dst, n, k);
  DTREE_LAUNCH_CHECK("tile_weight_f16 launch");
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
                    ((embed_layout == DTREE_W_TILED || embed_layout == DTREE_W_TILED_F16 ||
                      embed_layout == DTREE_W_Q4G64) && hidden % 64 == 0 && vocab % 32 == 0),
                "embed: layout");
  DTREE_REQUIRE(embed_layout != DTREE_W_Q4G64 || embed_scales, "embed: q4 embedding needs embed_scales");
  DTREE_REQUIRE(xg_layout == DTREE_W_ROWMAJOR ||
                    ((xg_layout == DTREE_W_TILED || xg_layout == DTREE_W_TILED_F16) && hidden % 64 == 0),
                "embed: xg layout");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= DTREE_MAX_NODES && rows_padded % 32 == 0, "embed: rows_padded");
  DTREE_REQUIRE(((uintptr_t)embed & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && ((uintptr_t)x & 15) == 0 &&
                    ((uintptr_t)xg & 15) == 0 && ((uintptr_t)xg_lo & 15) == 0,
                "embed: embed, norm_w, x, xg and xg_lo must be 16-byte aligned");
  const int gather = (rows_padded * (hidden / 8) + 255) / 256;
  int rope_blocks = 0;
  if (rope_cos && rope_sin) {
    DTREE_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "embed: head_dim");
    rope_blocks = (rows_padded * head_dim / 2 + 255) / 256;
  }
  embed_kernel<<<gather + rope_blocks, 256, 0, stream>>>(desc, embed, embed_layout, embed_scales, vocab, hidden,
                                                          norm_w, rows_padded, x, xg, xg_lo,
                                                          xg_layout, ss, head_dim / 2, rope_base,
                                                          rope_cos, rope_sin, gather);
  DTREE_LAUNCH_CHECK("embed launch");
  return DTREE_OK;
}

extern "C" int dtree_embed_tokens(const int32_t* tokens, int32_t n, const uint16_t* embed, int32_t embed_layout,
                                  const uint16_t* embed_scales, int32_t vocab, int32_t hidden, const uint16_t* norm_w,
                                  int32_t rows_padded, float* x, uint16_t* xg, uint16_t* xg_lo, int32_t xg_layout,
                                  float* ss, hipStream_t stream) {
  DTREE_REQUIRE(tokens && embed && norm_w && x && xg && ss, "embed_tokens: null pointer");
  DTREE_REQUIRE(hidden > 0 && hidden % 64 == 0, "embed_tokens: hidden must be a multiple of 64");
  DTREE_REQUIRE(vocab > 0 && vocab % 32 == 0, "embed_tokens: vocab");
  DTREE_REQUIRE(embed_layout == DTREE_W_ROWMAJOR || embed_layout == DTREE_W_TILED ||
                    embed_layout == DTREE_W_TILED_F16 || embed_layout == DTREE_W_Q4G64,
                "embed_tokens: layout");
  DTREE_REQUIRE(embed_layout != DTREE_W_Q4G64 || embed_scales, "embed_tokens: q4 embedding needs embed_scales");
  DTREE_REQUIRE(xg_layout == DTREE_W_ROWMAJOR || xg_layout == DTREE_W_TILED || xg_layout == DTREE_W_TILED_F16,
                "embed_tokens: xg layout");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded % 32 == 0 && rows_padded <= (1 << 20) && n >= 0 && n <= rows_padded,
                "embed_tokens: rows_padded (a multiple of 32) and n <= rows_padded");
  DTREE_REQUIRE(((uintptr_t)embed & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && ((uintptr_t)x & 15) == 0 &&
                    ((uintptr_t)xg & 15) == 0 && ((uintptr_t)xg_lo & 15) == 0,
                "embed_tokens: embed, norm_w, x, xg and xg_lo must be 16-byte aligned");
  const long long threads = (long long)rows_padded * (hidden / 8);
  embed_tokens_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(
      tokens, n, embed, embed_layout, embed_scales, vocab, hidden, norm_w, rows_padded, x, xg, xg_lo,
      xg_layout, ss);
  DTREE_LAUNCH_CHECK("embed_tokens launch");
  return DTREE_OK;
}

extern "C" int dtree_rows_in(const uint16_t* rows, int32_t ld_rows, int32_t n_rows, const uint16_t* norm_w,
                             int32_t rows_padded, int32_t hidden, float* x, uint16_t* xg, uint16_t* xg_lo,
                             int32_t xg_layout, float* ss, hipStream_t stream) {
  DTREE_REQUIRE(rows && norm_w && x && xg && ss, "rows_in: null pointer");
  DTREE_REQUIRE(hidden > 0 && hidden % 64 == 0, "rows_in: hidden must be a multiple of 64");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= DTREE_MAX_NODES && rows_padded % 32 == 0, "rows_in: rows_padded");
  DTREE_REQUIRE(n_rows >= 0 && n_rows <= rows_padded, "rows_in: n_rows");
  DTREE_REQUIRE(ld_rows >= hidden && ld_rows % 8 == 0, "rows_in: ld_rows (>= hidden, a multiple of 8)");
  DTREE_REQUIRE(xg_layout == DTREE_W_ROWMAJOR || xg_layout == DTREE_W_TILED || xg_layout == DTREE_W_TILED_F16,
                "rows_in: xg layout");
  DTREE_REQUIRE(((uintptr_t)rows & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && ((uintptr_t)x & 15) == 0 &&
                    ((uintptr_t)xg & 15) == 0 && ((uintptr_t)xg_lo & 15) == 0,
                "rows_in: rows, norm_w, x, xg and xg_lo must be 16-byte aligned");
  const int grid = (rows_padded * (hidden / 8) + 255) / 256;
  rows_in_kernel<<<grid, 256, 0, stream>>>(rows, ld_rows, n_rows, norm_w, rows_padded, hidden, x, xg, xg_lo,
                                           xg_layout, ss);
  DTREE_LAUNCH_CHECK("rows_in launch");
  return DTREE_OK;
}

extern "C" int dtree_accept_walk(DtreeStepDesc* desc, const void* candidates, int32_t num_candidate_blocks,
                                 int32_t rows_padded, int32_t* result, hipStream_t stream) {
  DTREE_REQUIRE(desc && candidates, "accept_walk: null pointer");
  DTREE_REQUIRE(num_candidate_blocks > 0 && num_candidate_blocks <= (1 << 20), "accept_walk: num_candidate_blocks");
  DTREE_REQUIRE(rows_padded > 0 && rows_padded <= DTREE_MAX_NODES, "accept_walk: rows_padded");
  walk_kernel<<<1, kWalkThreads, 0, stream>>>(desc, reinterpret_cast<const int2*>(candidates), num_candidate_blocks,
                                     rows_padded, result);
  DTREE_LAUNCH_CHECK("accept_walk launch");
  return DTREE_OK;
}

extern "C" int dtree_compact(const DtreeStepDesc* desc, uint16_t* k_pages, uint16_t* v_pages, size_t layer_stride,
                             int32_t layers, int32_t num_kv_heads, int32_t head_dim, const int32_t* page_table,
                             const uint16_t* hidden_in, int32_t hidden_width, uint16_t* hidden_out,
                             hipStream_t stream) {
  DTREE_REQUIRE(desc && page_table, "compact: null pointer");
  DTREE_REQUIRE(layers >= 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 32 == 0, "compact: shape (head_dim a multiple of 32)");
  DTREE_REQUIRE(layers == 0 || (k_pages && v_pages), "compact: null cache");
  DTREE_REQUIRE(!hidden_out || (hidden_in && hidden_width > 0 && hidden_width % 8 == 0 &&
                                 ((uintptr_t)hidden_in & 15) == 0 && ((uintptr_t)hidden_out & 15) == 0),
                "compact: hidden_in / hidden_width (a multiple of 8, 16-byte aligned rows)");
  const int grid = 2 * layers * num_kv_heads + kHidBlocks;
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
