// Skinny bf16 GEMM for tree verification: Y[M<=128, N] = X[M, K] * W[N, K]^T.
//
// The verify step multiplies ~25 tree rows by every weight matrix of the
// model, so each launch is a pure weight stream (26 FLOP/B, far under the
// bf16 MFMA ridge): the design goal is HBM bandwidth, not MFMA throughput.
//
// Work split
//   * A column tile is 32*NB weight rows. A workgroup (4 waves) owns one tile
//     and a K range; its waves interleave 64-wide K blocks so one iteration of
//     the workgroup reads 512 contiguous bytes of every weight row.
//   * Lane (c = lane%32, h = lane/32) loads 64 contiguous bytes of weight row
//     c of each of the NB 32-row blocks (K offset 32h within the block) with
//     streaming loads, and the same K slice of activation row c. Element group
//     j of both operands feeds MFMA j (v_mfma_f32_32x32x16_bf16), so A and B
//     see the same K permutation and 4 MFMAs sum exactly the block's 64 K
//     values. One activation fragment serves NB weight blocks.
//   * Activations may arrive as a split pair x = hi + lo (both bf16, about
//     16 significant bits together); both halves are multiplied with the same
//     weight fragment. The weights stay bf16, so HBM traffic is unchanged and
//     the MFMA work doubles, which the bandwidth-bound kernel absorbs.
//   * Waves reduce through LDS in a fixed order. With split_k > 1 the K range
//     is split over workgroups; each writes its partial tile, and the last to
//     arrive (device-scope counter) sums all partials in split order, so the
//     result does not depend on arrival order. All splits of a tile are
//     mapped to one XCD (workgroups go round-robin over the 8 XCDs), so the
//     partials stay in that XCD's L2.
//   * Epilogues fuse the RMSNorm row scale (norm weight folded into the
//     producer's X), residual add, SwiGLU, and the per-32-column sum of
//     squares the next RMSNorm needs; they emit split hi/lo outputs (one
//     fp16 plane for the DTREE_W_TILED_F16 layout).
//   * H (DTREE_W_TILED_F16): fp16 weights and one fp16 activation plane run
//     the fp16 MFMA once per weight fragment; the other tiled paths keep bf16
//     weights with the activation pair (two bf16 MFMAs) and q4 dequantises to
//     bf16.
#include "common.h"

namespace dtree {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

struct GemmParams {
  const uint16_t* x; const uint16_t* x_lo; int ldx;
  const uint16_t* w; int n, k;
  const uint16_t* w_sb;  // q4: (scale, bias) pairs
  int S, kb_per_split, ntiles;
  const float* ss_in; int ss_tiles; float inv_norm_dim; float eps;
  float* out_f32; int ld_out_f32;
  uint16_t* out_bf16; uint16_t* out_lo; int ld_out_bf16; int out_tiled;
  int out_h16;  // outputs in DTREE_W_TILED_F16: one fp16 plane
  const uint16_t* next_norm;
  float* ss_out;
  uint16_t* hidden_out; int ld_hidden;
  float* part; int* counters;
  // stream-K schedule: T = (n/64) * (k/64) units over G workgroups
  int T, G; unsigned part_bytes;
  // ranged ring loads (32 tiled rows): bytes of w, w_sb and one x plane
  unsigned w_bytes, sb_bytes, x_bytes;
  int off_xcd;  // test hook: treat every workgroup as off its expected XCD
  // LM-head mode of the one-pass q4 kernel: optional fp32 logits [rows][n]
  // and per-(workgroup, row) argmax candidates over lm_blocks workgroups
  float* lm_logits;
  int2* lm_cand;
  int lm_blocks;
  int spin;  // polls of a bounded wait for other workgroups (q4 one-pass K parts)
};

// Index of element (m, col) of a bf16 output with `ld` columns.
__device__ __forceinline__ size_t out_index(int tiled, int m, int col, int ld) {
  return tiled ? tiled_index(m, col, ld) : (size_t)m * ld + col;
}

// An activation for the next GEMM: one fp16 value (h16: DTREE_W_TILED_F16), or
// bf16 hi + bf16 lo (lo = bf16(v - hi)).
__device__ __forceinline__ void split_store(uint16_t* hi, uint16_t* lo, size_t idx, float v, int h16) {
  if (h16) {
    hi[idx] = f2h(v);
    return;
  }
  const uint16_t h = f2bf(v);
  hi[idx] = h;
  if (lo) lo[idx] = f2bf(v - bf2f(h));
}

// Partial product of one tile (32*NB columns) over K blocks [kb0, kb1); the
// waves' tiles are summed into red[0 .. MB*32*32*NB) laid out [row][col].
// TILED: W is stored in the kernel's consumption order (DTREE_W_TILED), so
// every load instruction of a wave reads one contiguous kilobyte.
template <int MB, int NB, int U, bool LO, bool TILED, bool H = false>
__device__ __forceinline__ void wg_tile(const uint16_t* __restrict__ x, const uint16_t* __restrict__ xlo, int ldx,
                                        const uint16_t* __restrict__ w, int K, int tile, int kb0, int kb1,
                                        float* red) {
  constexpr int TN = 32 * NB;
  const int lane = threadIdx.x & 63;
  // Wave index in a scalar register: the K loop below is then uniform
  // control flow with scalar branches instead of an exec-masked loop.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 31, h = lane >> 5;
  f32x16_t acc[NB][MB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nb][mb][r] = 0.f;

  // Row-major: lane (c, h) reads row tile*TN + nb*32 + c, K offset 64*kk + 32h.
  // Tiled ([N/32][K/64][4][64][8]): the 32-row x 64-K block (r32, kk) is 2048
  // contiguous elements; load i of lane l reads elements (64*i + l)*8 .. +8
  // of it, which hold the same K values as the row-major load.
  const int nkb = K >> 6;
  const uint16_t* wp = TILED ? w + (size_t)tile * NB * nkb * 2048 + lane * 8 : w + (size_t)(tile * TN + c) * K + 32 * h;
  const size_t wnb = TILED ? (size_t)nkb * 2048 : (size_t)32 * K;  // next 32-row weight block
  const size_t wkb = TILED ? 2048 : 64;                            // next K block
  const int wi = TILED ? 512 : 8;                     // next 16-byte load of a lane
  // Activations use the same layout as the weights (tiled: [MP/32][K/64]
  // blocks of 2048 elements, so each activation load is one contiguous KB too).
  const uint16_t* xp = TILED ? x + lane * 8 : x + (size_t)c * ldx + 32 * h;
  const uint16_t* xq = LO ? (TILED ? xlo + lane * 8 : xlo + (size_t)c * ldx + 32 * h) : nullptr;
  const size_t xmb = TILED ? (size_t)nkb * 2048 : (size_t)32 * ldx;  // next 32-row activation block
  // Software pipeline over this wave's n K blocks (kb0 + wave + 4j): while
  // block j is multiplied, block j+1's weights are already in flight in the
  // other register set. Per block the activations are loaded first and the
  // weight prefetch second, so waiting for the activations (loads retire in
  // issue order) never waits for the prefetch. The loop runs whole pairs of
  // blocks (A then B register set) plus an optional single tail block, so
  // every prefetch is used on every path and cannot be sunk out of place; a
  // prefetch past the end re-reads a 64-byte slice of the (L2-resident)
  // activations instead of weights.
  const int kfirst = kb0 + wave;
  const int n = kfirst < kb1 ? (kb1 - kfirst + kWaves - 1) / kWaves : 0;
  if (n > 0) {
    u32x4_t wa[NB][4], wb[NB][4];
    auto load_w = [&](u32x4_t (&dst)[NB][4], int j) {
      const bool real = j < n;
      const int kk = kfirst + kWaves * j;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint16_t* src = real ? wp + nb * wnb + (size_t)kk * wkb : xp;
        const int step = real ? wi : 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[nb][i] = ld_u32x4_stream(src + step * i);
      }
    };
    auto step = [&](const u32x4_t (&wc)[NB][4], u32x4_t (&wn)[NB][4], int j, bool prefetch) {
      const int kk = kfirst + kWaves * j;
      u32x4_t xv[MB][4], xl[MB][4];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const size_t off = (size_t)mb * xmb + (size_t)kk * wkb + (size_t)wi * i;
          xv[mb][i] = ld_u32x4(xp + off);
          if (LO) xl[mb][i] = ld_u32x4(xq + off);
        }
      // Fixed issue order: activations, then the weight prefetch, then MFMAs.
      __builtin_amdgcn_sched_barrier(0);
      if (prefetch) load_w(wn, j + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if constexpr (H) {  // fp16 weights, one fp16 activation plane
              acc[nb][mb] = mfma32_f16(xv[mb][i], wc[nb][i], acc[nb][mb]);
            } else {
              acc[nb][mb] = mfma32(xv[mb][i], wc[nb][i], acc[nb][mb]);
              if (LO) acc[nb][mb] = mfma32(xl[mb][i], wc[nb][i], acc[nb][mb]);
            }
          }
    };
    load_w(wa, 0);
    int j = 0;
    for (; j + 2 <= n; j += 2) {
      step(wa, wb, j, true);      // block j+1 is always real here
      step(wb, wa, j + 1, true);  // block j+2 may be past the end (dummy)
    }
    if (j < n) step(wa, wb, j, false);
  }

  // Waves 1..3 park their tiles in LDS; wave 0 adds them in wave order, so
  // the sum is independent of timing, then publishes the tile at red[0..).
  constexpr int TE = MB * 32 * TN;
  if (wave > 0) {
    float* my = red + (wave - 1) * TE;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) my[(mb * 32 + acc_row(r, h)) * TN + nb * 32 + c] = acc[nb][mb][r];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int wv = 0; wv < kWaves - 1; ++wv)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[nb][mb][r] += red[wv * TE + (mb * 32 + acc_row(r, h)) * TN + nb * 32 + c];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(mb * 32 + acc_row(r, h)) * TN + nb * 32 + c] = acc[nb][mb][r];
  }
  __syncthreads();
}

// RMSNorm row scale rs[m] = rsqrt(sum_t ss_in[t][m] * inv_dim + eps) (1 when
// ss_in is null) with every thread of the workgroup: thread (part, m) owns
// tiles part, part + kThreads/MP, ...; ss_issue puts its first kSsBatch loads
// in flight at once (issue them before other long loads: loads retire in
// order), ss_finish adds the rest, and the parts are added in a fixed order.
// ss_finish contains one barrier; callers barrier again before reading rs.
constexpr int kSsBatch = 16;

template <int MB>
__device__ __forceinline__ void ss_issue(const float* ss_in, int ss_tiles, float (&v)[kSsBatch]) {
  constexpr int MP = MB * 32, TPR = kThreads / MP;
  const int m = threadIdx.x % MP, part = threadIdx.x / MP;
  // Ranged loads (zero past the statistics, or everywhere without them), so
  // the same loads go out on every path and a later ring of loads can be
  // waited on slot by slot.
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(ss_in, ss_in ? (unsigned)(ss_tiles * MP * 4) : 0u);
#pragma unroll
  for (int i = 0; i < kSsBatch; ++i) {
    const int t = part + i * TPR;
    v[i] = buf_ldf(r, t < ss_tiles ? (unsigned)(ss_index(t, m, ss_tiles) * 4) : kOob);
  }
}

template <int MB>
__device__ __forceinline__ void ss_finish(const float* ss_in, int ss_tiles, float inv_dim, float eps,
                                          const float (&v)[kSsBatch], float* rs, float* scratch) {
  constexpr int MP = MB * 32, TPR = kThreads / MP;
  const int m = threadIdx.x % MP, part = threadIdx.x / MP;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kSsBatch; ++i) s += v[i];
  if (ss_in) {
    for (int base = kSsBatch * TPR; base < ss_tiles; base += kSsBatch * TPR) {
      float w[kSsBatch];
#pragma unroll
      for (int i = 0; i < kSsBatch; ++i) {
        const int t = base + part + i * TPR;
        w[i] = t < ss_tiles ? ss_in[ss_index(t, m, ss_tiles)] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < kSsBatch; ++i) s += w[i];
    }
  }
  scratch[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x < MP) {
    float r = 1.f;
    if (ss_in) {
      float tot = 0.f;
      for (int q = 0; q < TPR; ++q) tot += scratch[q * MP + threadIdx.x];
      r = rsqrtf(tot * inv_dim + eps);
    }
    rs[threadIdx.x] = r;
  }
}

template <int MB>
__device__ __forceinline__ void row_scale(const float* ss_in, int ss_tiles, float inv_dim, float eps, float* rs,
                                          float* scratch) {
  float v[kSsBatch];
  ss_issue<MB>(ss_in, ss_tiles, v);
  ss_finish<MB>(ss_in, ss_tiles, inv_dim, eps, v, rs, scratch);
}

// Epilogue of one finished tile held in LDS as red[row * TN + col] (row scale
// rs[] applied here). Element e of the tile: row e / TN, column e % TN; with
// TN in {32, 64} and 256 threads a 32-column group of one row is held by 32
// consecutive lanes.
// Residual rows of one output tile for the residual epilogue (thread t holds
// elements t, t + kThreads, ... of the [MP][TN] tile) and, last, the next
// RMSNorm weight of its column; all loads in flight together (callers issue
// them before other waits to overlap the round trip).
// tid: the thread's index within the kThreads threads that run the
// epilogue (threadIdx.x, or its offset inside a 256-thread group of a larger
// workgroup).
template <int MP, int TN>
__device__ __forceinline__ void residual_issue(const GemmParams& p, int tile, float (&xo)[MP * TN / kThreads + 1],
                                               int tid = threadIdx.x) {
  const int col = tile * TN + tid % TN;
#pragma unroll
  for (int i = 0; i < MP * TN / kThreads; ++i)
    xo[i] = p.out_f32[(size_t)((tid + i * kThreads) / TN) * p.ld_out_f32 + col];
  xo[MP * TN / kThreads] = bf2f(p.next_norm[col]);  // the next RMSNorm's weight
}

template <int MP, int TN, int EPI>
__device__ __forceinline__ void tile_epilogue(const GemmParams& p, const float* red, const float* rs, int tile,
                                              const float* xpre = nullptr, int tid = threadIdx.x) {
  constexpr int TE = MP * TN;
  if constexpr (EPI == DTREE_EPI_STORE_F32) {
    // (columns past p.n: the long-M GEMM's last tile when n % 128 == 64)
    for (int e = tid; e < TE; e += kThreads) {
      const int m = e / TN, n = e % TN;
      if (tile * TN + n < p.n) p.out_f32[(size_t)m * p.ld_out_f32 + tile * TN + n] = red[e] * rs[m];
    }
  } else if constexpr (EPI == DTREE_EPI_STORE_BF16) {
    for (int e = tid; e < TE; e += kThreads) {
      const int m = e / TN, n = e % TN;
      split_store(p.out_bf16, p.out_lo, out_index(p.out_tiled, m, tile * TN + n, p.ld_out_bf16), red[e] * rs[m],
                  p.out_h16);
    }
  } else if constexpr (EPI == DTREE_EPI_RESIDUAL) {
    constexpr int IT = TE / kThreads;
    const int n = tid % TN;
    const int col = tile * TN + n;
    float xo[IT + 1];
    if (xpre) {
#pragma unroll
      for (int i = 0; i <= IT; ++i) xo[i] = xpre[i];
    } else {
      residual_issue<MP, TN>(p, tile, xo, tid);
    }
    const float g = xo[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int e = tid + i * kThreads;
      const int m = e / TN;
      float* xp = p.out_f32 + (size_t)m * p.ld_out_f32 + col;
      const float xv = xo[i] + red[e];
      *xp = xv;
      split_store(p.out_bf16, p.out_lo, out_index(p.out_tiled, m, col, p.ld_out_bf16), xv * g, p.out_h16);
      if (p.hidden_out) p.hidden_out[(size_t)m * p.ld_hidden + col] = f2bf(xv);
      // sum of x^2 over this 32-column tile (the 32 lanes of a half-wave)
      const float sq = row_sum32(xv * xv);
      if ((n & 31) == 0) p.ss_out[ss_index(col >> 5, m, p.n >> 5)] = sq;
    }
  } else if constexpr (EPI == DTREE_EPI_SWIGLU) {
    // Each 32-column group = 16 gate rows then 16 up rows of 16 FFN features.
    for (int e = tid; e < MP * TN / 2; e += kThreads) {
      const int m = e / (TN / 2), f = e % (TN / 2);
      const int sb = f >> 4, j = f & 15;
      const float gt = red[m * TN + sb * 32 + j] * rs[m];
      const float up = red[m * TN + sb * 32 + 16 + j] * rs[m];
      split_store(p.out_bf16, p.out_lo, out_index(p.out_tiled, m, tile * (TN / 2) + f, p.ld_out_bf16),
                  silu_f(gt) * up, p.out_h16);
    }
  }

}

template <int MB, int NB, int U, bool LO, bool TILED, int EPI, bool H = false>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams p) {
  constexpr int MP = MB * 32;
  constexpr int TN = 32 * NB;
  constexpr int TE = MP * TN;  // tile elements
  __shared__ float red[(kWaves - 1) * TE];
  __shared__ float rs[MP];
  __shared__ float rs_scratch[kThreads];
  __shared__ int is_last;

  int tile, s;
  if (p.S == 1) {
    tile = blockIdx.x;
    s = 0;
  } else {
    const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
    tile = (j / p.S) * 8 + xcd;
    s = j % p.S;
  }
  if (tile >= p.ntiles) return;
  const int nkb = p.k >> 6;
  const int kb0 = s * p.kb_per_split;
  const int kb1 = min(kb0 + p.kb_per_split, nkb);

  wg_tile<MB, NB, U, LO, TILED, H>(p.x, p.x_lo, p.ldx, p.w, p.k, tile, kb0, kb1, red);

  if (p.S > 1) {
    float* mine = p.part + ((size_t)tile * p.S + s) * TE;
    for (int e = threadIdx.x; e < TE; e += kThreads) st_coherent(mine + e, red[e]);
    wait_stores_done();
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&p.counters[tile]) == p.S - 1);
    __syncthreads();
    if (!is_last) return;
    // Splits' loads kPb at a time (agent-coherent, past the L2), added in
    // split order.
    constexpr int kPb = 8;
    const __amdgpu_buffer_rsrc_t prs =
        buf_rsrc(p.part + (size_t)tile * p.S * TE, (unsigned)((size_t)p.S * TE * sizeof(float)));
    for (int e = threadIdx.x; e < TE; e += kThreads) {
      float v = 0.f;
      for (int q0 = 0; q0 < p.S; q0 += kPb) {
        float pv[kPb];
#pragma unroll
        for (int z = 0; z < kPb; ++z) {
          const unsigned off = q0 + z < p.S ? (unsigned)(((q0 + z) * TE + e) * 4) : kOob;
          pv[z] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)off, 0, kSc1));
        }
#pragma unroll
        for (int z = 0; z < kPb; ++z)
          if (q0 + z < p.S) v += pv[z];
      }
      red[e] = v;
    }
    if (threadIdx.x == 0) reset_counter(&p.counters[tile]);
  }
  row_scale<MB>(p.ss_in, p.ss_tiles, p.inv_norm_dim, p.eps, rs, rs_scratch);
  __syncthreads();

  tile_epilogue<MP, TN, EPI>(p, red, rs, tile);
}


// ---- stream-K GEMM for 32 rows (tiled operands) ------------------------------
//
// The weight stream of the whole launch is cut evenly across the grid: unit u
// = (64-column block b = u / nkb, 64-wide K block kb = u % nkb), 8 KB of
// weights; workgroup g owns units [g*T/G, (g+1)*T/G), one workgroup per CU, so
// every CU streams the same number of bytes whatever the matrix shape. The
// four waves take contiguous quarters of that range and keep kSkDepth units
// (weights and activation hi/lo) in flight in registers. A wave's per-block
// accumulator goes to LDS when its block changes; the workgroup then adds its
// four waves per block and, when other workgroups share the block, publishes
// one partial tile (agent-coherent stores to slot g + b, which is unique per
// (workgroup, block) pair because ranges are ordered). The last workgroup to
// arrive at a block sums the partials in workgroup order (deterministic) and
// runs the shared tile epilogue.
constexpr int kSkMaxBlocks = 4;  // 64-column blocks one workgroup may touch
constexpr int kSkDepth = 4;      // units in flight per wave
constexpr int kSkMaxGrid = 1024; // CU-count bound used for workspace sizing

// q4 nibble pair j of a repacked word -> two bf16 holding 128 + q (exact: the
// bf16 with bits 0x4300 | q is 128 + q for q < 128), K order (2j, 2j+1).
// The mask and the exponent bits are brought into registers by (pure, hence
// shared) asm moves: with both in registers each pair is one v_and_or_b32
// (a VOP3 instruction, which takes no literal operand on this target) after
// its shift, where literal operands cost a v_and and a v_or.
__device__ __forceinline__ u32x4_t q4_pairs(uint32_t w) {
  uint32_t m, e;
  asm("s_mov_b32 %0, 0x000f000f" : "=s"(m));
  asm("v_mov_b32 %0, 0x43004300" : "=v"(e));
  return u32x4_t{(w & m) | e, ((w >> 4) & m) | e, ((w >> 8) & m) | e, ((w >> 12) & m) | e};
}

// ---- q4 helpers for 32 rows ----------------------------------------------------
// One q4 group (64 K) of two 32-column blocks: fresh MFMA sums of x (128 + q),
// then acc += s * sums + (b - 128 s) * sum(x) per (row, column). sum(x) (the
// affine bias term and the 128 offset of the nibble encoding need it) comes
// from the same registers: an MFMA of the group's activations against bf16
// ones gives sum_k x per row in the accumulator layout.
template <bool LO>
__device__ __forceinline__ void q4_group(const u32x4_t (&xv)[2][4], const u32x4_t (&wq)[2],
                                            const uint32_t (&sb)[2], f32x16_t (&acc)[2]) {
  const u32x4_t ones = u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  f32x16_t xs;
#pragma unroll
  for (int r = 0; r < 16; ++r) xs[r] = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xs = mfma32(xv[0][i], ones, xs);
    if (LO) xs = mfma32(xv[1][i], ones, xs);
  }
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    f32x16_t au;
#pragma unroll
    for (int r = 0; r < 16; ++r) au[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4_t bq = q4_pairs(wq[nb][i]);
      au = mfma32(xv[0][i], bq, au);
      if (LO) au = mfma32(xv[1][i], bq, au);
    }
    const float sc = __uint_as_float(sb[nb] << 16);
    const float cf = __uint_as_float(sb[nb] & 0xffff0000u) - 128.f * sc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = fmaf(cf, xs[r], fmaf(sc, au[r], acc[nb][r]));
  }
}

// q4 counterpart of wg_tile for 32 rows and 64 columns (two 32-row blocks):
// the tile over all K, waves interleaving groups, a 4-deep register ring of
// (q4 words, scale/bias, activations), LDS reduction of the four waves into
// red[row * 64 + col] in wave order.
template <bool LO>
__device__ __forceinline__ void wg_tile_q4(const uint16_t* __restrict__ x, const uint16_t* __restrict__ xlo,
                                           const uint32_t* __restrict__ wq, const uint32_t* __restrict__ wsb,
                                           int K, int tile, float* red) {
  constexpr int TN = 64, TE = 32 * TN, D = 4;
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nkb = K >> 6;
  const int n = wave < nkb ? (nkb - wave + kWaves - 1) / kWaves : 0;  // groups wave, wave + 4, ...
  f32x16_t acc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0.f;
  u32x4_t wr[D][2], xr[D][2][4];
  uint32_t sbr[D][2];
  auto issue = [&](int s, int j) {
    if (j < n) {
      const int kb = wave + kWaves * j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xr[s][0][i] = ld_u32x4(x + (size_t)kb * 2048 + lane * 8 + 512 * i);
        if (LO) xr[s][1][i] = ld_u32x4(xlo + (size_t)kb * 2048 + lane * 8 + 512 * i);
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const size_t blk = (size_t)(2 * tile + nb) * nkb + kb;
        wr[s][nb] = ld_u32x4_stream(wq + blk * 256 + lane * 4);
        sbr[s][nb] = wsb[blk * 32 + c];
      }
    }
  };
#pragma unroll
  for (int s = 0; s < D; ++s) issue(s, s);
  for (int j0 = 0; j0 < n; j0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int j = j0 + s;
      if (j < n) {
        __builtin_amdgcn_sched_barrier(0);
        q4_group<LO>(xr[s], wr[s], sbr[s], acc);
        __builtin_amdgcn_sched_barrier(0);
        issue(s, j + D);
      }
    }
  }
  if (wave > 0) {
    float* my = red + (wave - 1) * TE;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) my[acc_row(r, h) * TN + nb * 32 + c] = acc[nb][r];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int wv = 0; wv < kWaves - 1; ++wv)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[nb][r] += red[wv * TE + acc_row(r, h) * TN + nb * 32 + c];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[acc_row(r, h) * TN + nb * 32 + c] = acc[nb][r];
  }
  __syncthreads();
}


__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(float* part, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(part, 0, (int)bytes, 0x00020000);
}
// Stream-K ranges in XCD order. Workgroups are dispatched round-robin over
// the XCDs (blockIdx % 8; each workgroup checks its own with HW_REG_XCC_ID),
// so logical range g = (blockIdx % 8) * (G / 8) + blockIdx / 8 puts the
// consecutive ranges that share a column block on one XCD. A partial tile
// is always written through (sc1), and read from that XCD's L2 (sc0) when
// its writers and reader are all confirmed on the same XCD.
__device__ __forceinline__ int sk_logical(int bid, int G) {
  return G % kXcds == 0 ? (bid % kXcds) * (G / kXcds) + bid / kXcds : bid;
}

// One round of partial-tile loads for block b: the partials of workgroups
// q0 .. min(q0 + kRedBatch, q_end) - 1 (slot q + b), elements 8t .. 8t+7, as
// (16-byte, 16-byte) pairs; slots past the last read zero (ranged loads) and
// are not added. Sole-owner blocks pass q_end = q0 and load nothing.
constexpr int kRedBatch = 8;
template <int AUX>
__device__ __forceinline__ void partials_issue(__amdgpu_buffer_rsrc_t prs, int b, int q0, int q_end, int t,
                                               u32x4_t (&v)[kRedBatch][2]) {
  constexpr int TE = 32 * 64;
#pragma unroll
  for (int z = 0; z < kRedBatch; ++z) {
    const unsigned off = q0 + z < q_end ? (unsigned)(((q0 + z + b) * TE + 8 * t) * 4) : kOob;
    v[z][0] = __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, 0, AUX);
    v[z][1] = __builtin_amdgcn_raw_buffer_load_b128(prs, (int)(off + 16), 0, AUX);
  }
}
__device__ __forceinline__ void partials_add(const u32x4_t (&v)[kRedBatch][2], int n, f32x4_t& s0, f32x4_t& s1) {
#pragma unroll
  for (int z = 0; z < kRedBatch; ++z) {
    if (z < n) {
      s0 += __builtin_bit_cast(f32x4_t, v[z][0]);
      s1 += __builtin_bit_cast(f32x4_t, v[z][1]);
    }
  }
}

// RING units in flight per wave, at most MAXB column blocks per workgroup.
template <bool LO, int EPI, bool Q4, int RING, int MAXB, bool H = false>
__device__ __forceinline__ void sk_gemm_body(const GemmParams& p) {
  constexpr int TN = 64, TE = 32 * TN;
  __shared__ float acc_lds[MAXB * kWaves * TE];  // [local block][wave][row][col]
  __shared__ float rs[32];
  __shared__ float rs_scratch[kThreads];
  __shared__ int last_flag[kSkMaxBlocks], first_q[kSkMaxBlocks], pieces[kSkMaxBlocks];
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = p.G, T = p.T, nkb = p.k >> 6;
  // Logical range g in XCD order (see sk_logical): the workgroups that share
  // a column block run on one XCD; `native` confirms the placement.
  const bool xcd_order = G % kXcds == 0;
  const int g = sk_logical(blockIdx.x, G);
  const bool native = xcd_order && !p.off_xcd && xcc_id() == (int)(blockIdx.x % kXcds);
  const int U0 = (int)((long long)g * T / G), U1 = (int)((long long)(g + 1) * T / G);
  if (U0 >= U1) return;
  const int b_first = U0 / nkb, b_last = (U1 - 1) / nkb;
  const int nloc = b_last - b_first + 1;  // <= MAXB (host-checked)
  if (nloc > MAXB) return;
  // The row scale's loads go out before the weight stream (loads retire in
  // order, so waiting for them later does not wait for the stream).
  float ssv[kSsBatch];
  ss_issue<1>(p.ss_in, p.ss_tiles, ssv);

  // ---- stream this wave's quarter of the range ----
  const int R = U1 - U0;
  const int a0 = U0 + wave * R / kWaves, a1 = U0 + (wave + 1) * R / kWaves;
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(p.x, p.x_bytes), xlrs = buf_rsrc(p.x_lo, LO ? p.x_bytes : 0u);
  const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(p.w, p.w_bytes), sbrs = buf_rsrc(p.w_sb, Q4 ? p.sb_bytes : 0u);
  // Ring of in-flight units: bf16 weights (2 blocks x 4 loads) or q4 words
  // (2 blocks x 1 load) + (scale, bias) per block; activations hi/lo. A slot
  // past the wave's range is refilled with ranged loads that return zero, so
  // every refill issues the same loads (see kOob) and is never consumed.
  u32x4_t wr[RING][2][Q4 ? 1 : 4], xr[RING][2][4];
  uint32_t sbr[RING][2];
  auto issue = [&](int s, int u) {
    const bool ok = u < a1;
    const int b = u / nkb, kb = u - b * nkb;
    const unsigned xo = ok ? (unsigned)(kb * 2048 + lane * 8) * 2u : kOob;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xr[s][0][i] = buf_ld(xrs, xo + 1024u * i);
      if (LO) xr[s][1][i] = buf_ld(xlrs, xo + 1024u * i);
    }
    if constexpr (Q4) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const unsigned blk = (unsigned)((2 * b + nb) * nkb + kb);
        wr[s][nb][0] = buf_ld_stream(wrs, ok ? (blk * 256u + lane * 4) * 4u : kOob);
        sbr[s][nb] = buf_ld32(sbrs, ok ? (blk * 32u + c) * 4u : kOob);
      }
    } else {
      const unsigned w0 = ok ? (unsigned)(((2 * b) * nkb + kb) * 2048 + lane * 8) * 2u : kOob;
      const unsigned w1 = ok ? w0 + (unsigned)nkb * 4096u : kOob;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wr[s][0][i] = buf_ld_stream(wrs, w0 + 1024u * i);
        wr[s][1][i] = buf_ld_stream(wrs, w1 + 1024u * i);
      }
    }
  };
  f32x16_t acc[2];
  auto zero = [&]() {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nb][r] = 0.f;
  };
  // Per-wave accumulator -> LDS [row][col] of (local block, wave); written
  // once per pair because a wave's units of one block are contiguous.
  auto dump = [&](int b) {
    float* d = acc_lds + ((b - b_first) * kWaves + wave) * TE;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) d[acc_row(r, h) * TN + nb * 32 + c] = acc[nb][r];
  };
  zero();
  int cur = a0 < a1 ? a0 / nkb : -1;
#pragma unroll
  for (int s = 0; s < RING; ++s) issue(s, a0 + s);
  // The accumulator slots are cleared while the first units are in flight.
  for (int e = threadIdx.x; e < nloc * kWaves * TE / 4; e += kThreads)
    reinterpret_cast<f32x4_t*>(acc_lds)[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  ss_finish<1>(p.ss_in, p.ss_tiles, p.inv_norm_dim, p.eps, ssv, rs, rs_scratch);
  for (int ub = a0; ub < a1; ub += RING) {
#pragma unroll
    for (int s = 0; s < RING; ++s) {
      const int u = ub + s;
      if (u < a1) {
        const int b = u / nkb;
        if (b != cur) {
          dump(cur);
          zero();
          cur = b;
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (Q4) {
          u32x4_t wq2[2] = {wr[s][0][0], wr[s][1][0]};
          q4_group<LO>(xr[s], wq2, sbr[s], acc);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
              if constexpr (H) {
                acc[nb] = mfma32_f16(xr[s][0][i], wr[s][nb][i], acc[nb]);
              } else {
                acc[nb] = mfma32(xr[s][0][i], wr[s][nb][i], acc[nb]);
                if (LO) acc[nb] = mfma32(xr[s][1][i], wr[s][nb][i], acc[nb]);
              }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      issue(s, u + RING);
    }
  }
  if (cur >= 0) dump(cur);
  __syncthreads();

  // ---- per block: add the four waves; publish or finish ----
  const __amdgpu_buffer_rsrc_t prs = part_rsrc(p.part, p.part_bytes);
  const int t = threadIdx.x;  // owns tile elements 8t .. 8t+7
  // Workgroup whose range holds unit u (T * G < 2^31, host-checked).
  auto owner = [&](int u) { return (int)(((unsigned)(u + 1) * (unsigned)G + (unsigned)(T - 1)) / (unsigned)T) - 1; };
  bool any_shared = false;
  int sole = 0;  // bit j: this workgroup owns local block j alone
  // The residual rows of the first two blocks go out now (a workgroup spans
  // at most two blocks at the usual shapes): their round trip overlaps the
  // publish and the arrival below.
  constexpr int IT = TE / kThreads;
  float xo0[IT + 1], xo1[IT + 1];
  if constexpr (EPI == DTREE_EPI_RESIDUAL) {
    residual_issue<32, TN>(p, b_first, xo0);
    if (nloc > 1) residual_issue<32, TN>(p, b_first + 1, xo1);
  }
  for (int j = 0; j < nloc; ++j) {
    const int b = b_first + j;
    const int gf = owner(b * nkb), gl = owner((b + 1) * nkb - 1);
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const f32x4_t* src = reinterpret_cast<const f32x4_t*>(acc_lds + (j * kWaves + w) * TE + 8 * t);
      s0 += src[0];
      s1 += src[1];
    }
    if (gf == gl) {
      // Sole owner: keep the sum in this block's wave-0 slot for the epilogue
      // (each thread rewrites only the elements it just read).
      f32x4_t* dst = reinterpret_cast<f32x4_t*>(acc_lds + (j * kWaves) * TE + 8 * t);
      dst[0] = s0;
      dst[1] = s1;
      sole |= 1 << j;
    } else {
      any_shared = true;
      const int off = ((g + b) * TE + 8 * t) * 4;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, s0), prs, off, 0, kSc1);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, s1), prs, off + 16, 0, kSc1);
    }
  }
  // Epilogue of local block j (its tile summed in LDS): residual rows from the
  // early loads for the first two blocks (selected by value, so the arrays
  // stay in registers).
#define DTREE_SK_EPILOGUE(j)                                                                \
  do {                                                                                      \
    float xj[IT + 1];                                                                       \
    if constexpr (EPI == DTREE_EPI_RESIDUAL) {                                              \
      if ((j) >= 2) {                                                                       \
        residual_issue<32, TN>(p, b_first + (j), xj);                                       \
      } else {                                                                              \
        _Pragma("unroll") for (int i = 0; i <= IT; ++i) xj[i] = (j) == 0 ? xo0[i] : xo1[i]; \
      }                                                                                     \
    }                                                                                       \
    tile_epilogue<32, TN, EPI>(p, acc_lds + ((j) * kWaves) * TE, rs, b_first + (j),         \
                               EPI == DTREE_EPI_RESIDUAL ? xj : nullptr);                   \
  } while (0)
  // Blocks owned alone wait for nobody: their epilogues run while the shared
  // blocks' partial stores are being acknowledged.
  if (sole) {
    __syncthreads();
    for (int j = 0; j < nloc; ++j)
      if ((sole >> j) & 1) DTREE_SK_EPILOGUE(j);
  }
  if (any_shared) wait_stores_done();
  __syncthreads();
  if (t < nloc) {
    const int b = b_first + t;
    const int gf = owner(b * nkb), gl = owner((b + 1) * nkb - 1);
    // last_flag: 0 not last (or owned alone, finished above); 1 last, partials
    // read past L2 (sc1); 2 last, every contributor ran on this XCD, partials
    // read from its L2 (sc0).
    int last = 0;
    if (gf != gl) {
      // Arrival count in the low half, workgroups off their XCD in the high.
      const int old = arrive_add(&p.counters[b], native ? 1 : 1 + kForeign);
      last = 0;
      if ((old & (kForeign - 1)) == gl - gf) {
        const int Gx = G / kXcds;
        const bool local = native && old < kForeign && gf / Gx == gl / Gx;
        last = local ? 2 : 1;
        reset_counter(&p.counters[b]);
      }
    }
    last_flag[t] = last;
    first_q[t] = gf;
    pieces[t] = last && gf != gl ? gl - gf + 1 : 0;
  }
  __syncthreads();

  // The blocks this workgroup finishes, in order. The first round of the next
  // block's partials is in flight during the current block's epilogue.
  auto flag = [&](int j) { return __builtin_amdgcn_readfirstlane(last_flag[j]); };
  auto next_last = [&](int j) {
    for (++j; j < nloc && !flag(j); ++j) {}
    return j;
  };
  u32x4_t pv[kRedBatch][2];
  auto issue_partials = [&](int j, int q0) {
    const int q_end = __builtin_amdgcn_readfirstlane(first_q[j]) + __builtin_amdgcn_readfirstlane(pieces[j]);
    if (flag(j) == 2) partials_issue<kSc0>(prs, b_first + j, q0, q_end, t, pv);
    else partials_issue<kSc1>(prs, b_first + j, q0, q_end, t, pv);
  };
  int j = next_last(-1);
  if (j < nloc) issue_partials(j, __builtin_amdgcn_readfirstlane(first_q[j]));
  while (j < nloc) {
    const int np = __builtin_amdgcn_readfirstlane(pieces[j]);
    const int jn = next_last(j);
    float* red = acc_lds + (j * kWaves) * TE;
    if (np > 0) {
      const int q0 = __builtin_amdgcn_readfirstlane(first_q[j]);
      f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
      partials_add(pv, np < kRedBatch ? np : kRedBatch, s0, s1);
      for (int q = kRedBatch; q < np; q += kRedBatch) {  // more than kRedBatch contributors
        issue_partials(j, q0 + q);
        partials_add(pv, np - q < kRedBatch ? np - q : kRedBatch, s0, s1);
      }
      reinterpret_cast<f32x4_t*>(red + 8 * t)[0] = s0;
      reinterpret_cast<f32x4_t*>(red + 8 * t)[1] = s1;
    }
    if (jn < nloc) issue_partials(jn, __builtin_amdgcn_readfirstlane(first_q[jn]));
    __syncthreads();
    DTREE_SK_EPILOGUE(j);
    j = jn;
  }
#undef DTREE_SK_EPILOGUE
}

template <bool LO, int EPI, bool Q4, bool H = false>
__global__ __launch_bounds__(kThreads) void sk_gemm_kernel(GemmParams p) {
  sk_gemm_body<LO, EPI, Q4, kSkDepth, kSkMaxBlocks, H>(p);
}

// q4 at two waves per SIMD: a 3-deep ring and at most two column blocks per
// workgroup (half the accumulator LDS) let two workgroups share a CU. q4
// units are issue-bound (nibble unpacking, MFMA chain and scale/bias
// epilogue in one instruction stream), so a second wave per SIMD pays on
// the large shapes.
template <bool LO, int EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void sk2_gemm_kernel(GemmParams p) {
  sk_gemm_body<LO, EPI, true, 3, 2>(p);
}

// ---- q4 GEMM over 64-128 rows in one pass -------------------------------------
//
// For the 65-node trees of the 9B-shaped step (96 rows) the 32-row q4 kernels
// stream and dequantise the weights once per 32-row block. This kernel makes
// one pass: a workgroup owns a tile of CW 64-column blocks and one part of K,
// with one wave per (K lane kl, row block rb, column block cb): 64 * CW * MB
// * KI threads (KI = 2 K lanes for CW 2, else 1). Per step the workgroup
// stages the next KI groups' activations (all row blocks, hi and lo planes;
// 4 KB per row block and plane) in LDS with coalesced 16-byte loads, double
// buffered and prefetched a step ahead in registers, so each activation byte is loaded
// once per workgroup and read from LDS by the CW waves that use it. A wave
// holds one 32 x 64 accumulator, so two or three waves share each SIMD and
// one wave's scale/bias arithmetic overlaps another's MFMAs. Per group a wave
// dequantises its column block's q4 words (128 + q as bf16, exact), runs
// the MFMAs of its row block, and takes sum(x) per row (for the affine bias
// and the 128 offset) from an MFMA of the activations against bf16 ones, as
// in the 32-row kernels. The K lanes are added in LDS in lane order; the
// parts of a tile are added by the last part to arrive, in part order
// (deterministic), which then runs the shared tile epilogue per 64-column
// block.
template <bool LO, int MB, int CW>
struct Q4mShape {
  static constexpr int KI = CW == 2 ? 2 : 1;             // K lanes (CW 2, 3 or 4)
  static constexpr int NPL = LO ? 2 : 1;                 // activation planes
  static constexpr int MP = MB * 32;                     // rows
  static constexpr int THREADS = 64 * CW * MB * KI;      // one wave per (kl, rb, cb); q4m_threads
  static constexpr int CHUNKS = KI * MB * NPL;           // 4 KB activation chunks per step
  static constexpr int STAGE_BYTES = CHUNKS * 4096;
  static constexpr int PIECES = CHUNKS * 256;            // 16-byte staging pieces per step
  static constexpr int LOADS = (PIECES + THREADS - 1) / THREADS;  // per thread
  static constexpr int TILE_FLOATS = CW * MP * 64;       // one part's output tile
  static constexpr int RED_BYTES = KI * TILE_FLOATS * 4;
  static constexpr int LDS_BYTES = 2 * STAGE_BYTES > RED_BYTES ? 2 * STAGE_BYTES : RED_BYTES;
};
constexpr int kQ4mDepth = 2;   // weight groups in flight per wave
constexpr int kQ4mMaxParts = 8;  // K parts per tile (remote partials of a pair fit one round of 8 loads)
constexpr int kQ4mSpin = 2048;   // polls (about a microsecond each) before an owner leaves its pairs to the last arriver
constexpr int kQ4mCtrInts = 32;  // counter words per tile: published, released, 16 pair claims (+ padding)
// Epilogue of the one-pass q4 kernel as the fused LM head (not a GEMM
// epilogue of the C ABI): row scale, optional fp32 logits, and per row the
// (largest logit, first index) of the tile as the workgroup's candidate.
constexpr int kEpiLmArgmax = 16;

constexpr int q4m_threads(int mb, int cw) { return 64 * cw * mb * (cw == 2 ? 2 : 1); }

template <bool LO, int EPI, int MB, int CW>
__global__ __launch_bounds__(q4m_threads(MB, CW)) void q4m_gemm_kernel(GemmParams p) {
  using Sh = Q4mShape<LO, MB, CW>;
  constexpr int KI = Sh::KI, NPL = Sh::NPL, MP = Sh::MP, D = kQ4mDepth, NT = Sh::THREADS;
  static_assert(D == 2, "the loop's issue order assumes two weight groups in flight");
  constexpr int TF = Sh::TILE_FLOATS;
  static_assert(EPI != kEpiLmArgmax || NT == 8 * MP, "LM-head epilogue: 8 threads per row");
  __shared__ __align__(16) unsigned char lds[Sh::LDS_BYTES];
  __shared__ float rs[MP];
  __shared__ float rs_scratch[NT];
  const int t = threadIdx.x, lane = t & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int cw = wave % CW, rb = (wave / CW) % MB, kl = wave / (CW * MB);
  const int nkb = p.k >> 6, nblk = p.n >> 6, P = p.S;
  const int tile = blockIdx.x / P, part = blockIdx.x % P;
  const int g0 = (int)((long long)part * nkb / P), g1 = (int)((long long)(part + 1) * nkb / P);
  const int nsteps = (g1 - g0 + KI - 1) / KI;
  const int cb = tile * CW + cw;
  const bool cb_ok = cb < nblk;
  if constexpr (EPI == kEpiLmArgmax) {
    // the candidate grid is wider than the vocab's tiles: the rest report
    // empty candidates
    if (tile * CW >= nblk) {
      if (t < MP) p.lm_cand[cand_index(blockIdx.x, t, p.lm_blocks)] = make_int2(__float_as_int(-__builtin_huge_valf()), 0x7fffffff);
      return;
    }
  }

  // The row scale's loads go out first (loads retire in order). Threads past
  // the first kThreads load and add tiles the final sum never reads.
  float ssv[kSsBatch];
  ss_issue<MB>(p.ss_in, p.ss_tiles, ssv);

  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(p.x, p.x_bytes), xlrs = buf_rsrc(p.x_lo, LO ? p.x_bytes : 0u);
  const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(p.w, p.w_bytes), sbrs = buf_rsrc(p.w_sb, p.sb_bytes);
  // Activation staging: piece j of thread t is piece t + j * NT of the step,
  // i.e. bytes 16 * (piece % 256) of chunk q = piece / 256 = (K lane kk, row
  // block rq, plane pl). Groups past the part read zero (ranged loads) and
  // are never used.
  u32x4_t xpre[Sh::LOADS];
  auto x_issue = [&](int st) {
#pragma unroll
    for (int j = 0; j < Sh::LOADS; ++j) {
      const int piece = min(t + j * NT, Sh::PIECES - 1), q = piece >> 8, tq = piece & 255;
      const int kk = q / (MB * NPL), rq = (q / NPL) % MB, pl = q % NPL;
      const int kb = g0 + st * KI + kk;
      const unsigned off = kb < g1 ? (unsigned)(rq * nkb + kb) * 4096u + 16u * tq : kOob;
      xpre[j] = pl == 0 ? buf_ld(xrs, off) : buf_ld(xlrs, off);
    }
  };
  auto x_store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < Sh::LOADS; ++j)
      if (Sh::LOADS * NT == Sh::PIECES || t + j * NT < Sh::PIECES)
        *reinterpret_cast<u32x4_t*>(lds + buf * Sh::STAGE_BYTES + 16 * (t + j * NT)) = xpre[j];
  };
  // Weight ring: group j of this wave is kb = g0 + kl + KI * j; two 32-column
  // halves (nb) of q4 words (1 KB each) and their (scale, bias) words.
  u32x4_t wr[D][2];
  uint32_t sbr[D][2];
  auto w_issue = [&](int s, int j) {
    const int kb = g0 + kl + KI * j;
    const bool ok = cb_ok && kb < g1;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const unsigned blk = (unsigned)((2 * cb + nb) * nkb + kb);
      wr[s][nb] = buf_ld_stream(wrs, ok ? (blk * 256u + lane * 4) * 4u : kOob);
      sbr[s][nb] = buf_ld32(sbrs, ok ? (blk * 32u + c) * 4u : kOob);
    }
  };
  f32x16_t acc[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0.f;
  const u32x4_t ones = u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const int xbase = ((kl * MB + rb) * NPL) * 4096 + lane * 16;
  auto compute = [&](int s, int buf) {
    u32x4_t xv[NPL][4];
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xv[pl][i] = *reinterpret_cast<const u32x4_t*>(lds + buf * Sh::STAGE_BYTES + xbase + pl * 4096 + i * 1024);
    f32x16_t xs;
#pragma unroll
    for (int r = 0; r < 16; ++r) xs[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int pl = 0; pl < NPL; ++pl) xs = mfma32(xv[pl][i], ones, xs);
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      f32x16_t au;
#pragma unroll
      for (int r = 0; r < 16; ++r) au[r] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4_t bq = q4_pairs(wr[s][nb][i]);
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) au = mfma32(xv[pl][i], bq, au);
      }
      const float sc = __uint_as_float(sbr[s][nb] << 16);
      const float cf = __uint_as_float(sbr[s][nb] & 0xffff0000u) - 128.f * sc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nb][r] = fmaf(cf, xs[r], fmaf(sc, au[r], acc[nb][r]));
    }
  };

  // Prologue in the loop's issue order (a step's activations, then a weight
  // group), so the loads in flight at the loop's head are those of any
  // later iteration: w(0), x(1), w(1).
  x_issue(0);
  w_issue(0, 0);
  ss_finish<MB>(p.ss_in, p.ss_tiles, p.inv_norm_dim, p.eps, ssv, rs, rs_scratch);
  x_store(0);
  x_issue(1);
#pragma unroll
  for (int s = 1; s < D; ++s) w_issue(s, s);
  __syncthreads();
  // Step st: compute from LDS buffer st & 1, store step st + 1's activations
  // (issued a step ago) into the other buffer, issue step st + 2's, then
  // refill the weight slot with group st + D. A wave's loads return in issue
  // order: storing step st + 1 waits for the loads issued before it, i.e.
  // up to the weights of group st + D - 2 = st (D = 2), which the step's
  // compute needs anyway, issued two steps ago. Every step issues the same
  // loads (ranged loads past the part return zero and are never used) so the
  // loop body has one pattern of loads in flight; a step guarded as a whole
  // made the compiler wait for every load (vmcnt(0)) inside the compute.
  // (Weights issued before the activations made every step wait for the
  // weights issued one step earlier; D = 3 with two activation steps in
  // flight measured no faster and spills at 128 rows.)
  for (int st0 = 0; st0 < nsteps; st0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int st = st0 + s;
      if (cb_ok && g0 + st * KI + kl < g1) {
        __builtin_amdgcn_sched_barrier(0);
        compute(s, st & 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      x_store((st + 1) & 1);
      x_issue(st + 2);
      w_issue(s, st + D);
      __syncthreads();
    }
  }

  // ---- K lanes, then parts ----
  float* red = reinterpret_cast<float*>(lds);  // [kl][cb][row][64]
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      red[((kl * CW + cw) * MP + rb * 32 + acc_row(r, h)) * 64 + nb * 32 + c] = acc[nb][r];
  __syncthreads();
  if constexpr (KI > 1) {
    for (int e4 = t; e4 < TF / 4; e4 += NT) {
      f32x4_t v = reinterpret_cast<const f32x4_t*>(red)[e4];
#pragma unroll
      for (int k2 = 1; k2 < KI; ++k2) v += reinterpret_cast<const f32x4_t*>(red + k2 * TF)[e4];
      reinterpret_cast<f32x4_t*>(red)[e4] = v;
    }
    __syncthreads();
  }
  const int nvalid = min(CW, nblk - tile * CW);  // column blocks of this tile inside n
  if constexpr (EPI == kEpiLmArgmax) {
    // One part per tile (the host launches the LM head with S = 1). 8
    // consecutive threads per row (NT = 8 * MP): each scans every 8th column
    // of the tile, then the 8 lanes reduce (max, first index on ties).
    const int m = t >> 3, q8 = t & 7;
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int cc = q8; cc < nvalid * 64; cc += 8) {
      const float v = red[((cc >> 6) * MP + m) * 64 + (cc & 63)] * rs[m];
      const int idx = tile * CW * 64 + cc;
      if (p.lm_logits) p.lm_logits[(size_t)m * p.n + idx] = v;
      argmax_merge(bv, bi, v, idx);
    }
    argmax_dpp<0xB1>(bv, bi);   // lane ^ 1
    argmax_dpp<0x4E>(bv, bi);   // lane ^ 2
    argmax_dpp<0x141>(bv, bi);  // half-row mirror: the other quad of the 8
    if (q8 == 0) p.lm_cand[cand_index(blockIdx.x, m, p.lm_blocks)] = make_int2(__float_as_int(bv), bi);
    return;
  } else {
  // The tile's output is cut into NPAIR (64-column block j, 32-row block r2)
  // pairs, i = j * MB + r2, each 32 x 64 floats contiguous in red and in a
  // published partial (blocks are [cb][row][64]).
  constexpr int NPAIR = CW * MB;
  static_assert(NPAIR <= 16, "pair masks and claim words");
  unsigned valid = 0;
#pragma unroll
  for (int i = 0; i < NPAIR; ++i)
    if (i / MB < nvalid) valid |= 1u << i;
  // The m-th pair of a mask (m < popcount), by a scan over the static pairs.
  auto nth_pair = [&](unsigned mask, int m) {
    int res = 0;
#pragma unroll
    for (int i = 0; i < NPAIR; ++i)
      if ((mask >> i) & 1u) {
        if (m == 0) res = i;
        --m;
      }
    return res;
  };
  auto pair_f4 = [&](int i) { return ((i / MB) * MP + 32 * (i % MB)) * 16; };  // f32x4 offset in red
  // Epilogue of the pairs in `todo`. The tile epilogue is written for
  // kThreads threads and one pair, outputs shifted by the row block (32-row
  // blocks are contiguous in both output layouts; statistics are per 32-row
  // block). The m-th pair of the mask goes to 256-thread group m % NG, each
  // group with the residual rows of all its pairs in flight before its first
  // epilogue (a remainder of threads past the last full group idles).
  constexpr int NG = NT / kThreads, PG = (NPAIR + NG - 1) / NG;
  constexpr int EIT = 32 * 64 / kThreads;
  const int grp = t / kThreads, gt = t % kThreads;
  auto pair_params = [&](int r2) {
    const int R = 32 * r2;
    GemmParams q = p;
    if (q.out_f32) q.out_f32 += (size_t)R * q.ld_out_f32;
    if (q.out_bf16) q.out_bf16 += (size_t)R * q.ld_out_bf16;
    if (q.out_lo) q.out_lo += (size_t)R * q.ld_out_bf16;
    if (q.hidden_out) q.hidden_out += (size_t)R * q.ld_hidden;
    if (q.ss_out) q.ss_out += (size_t)r2 * (q.n >> 5) * 32;
    return q;
  };
  auto epilogue = [&](unsigned todo) {
    const int cnt = __builtin_popcount(todo);
    if (grp >= NG) return;
    float xo[PG][EIT + 1];
    if constexpr (EPI == DTREE_EPI_RESIDUAL) {
#pragma unroll
      for (int k = 0; k < PG; ++k) {
        const int m = grp + NG * k;
        if (m < cnt) {
          const int i = nth_pair(todo, m);
          residual_issue<32, 64>(pair_params(i % MB), tile * CW + i / MB, xo[k], gt);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < PG; ++k) {
      const int m = grp + NG * k;
      if (m < cnt) {
        const int i = nth_pair(todo, m), j = i / MB, r2 = i % MB;
        tile_epilogue<32, 64, EPI>(pair_params(r2), red + (j * MP + 32 * r2) * 64, rs + 32 * r2, tile * CW + j,
                                   EPI == DTREE_EPI_RESIDUAL ? xo[k] : nullptr, gt);
      }
    }
  };
  if (P == 1) {
    epilogue(valid);
    return;
  }
  // ---- K parts: distributed combine ----
  // Every part publishes its whole partial tile (written through), waits for
  // the acknowledgement and counts itself on the tile's publication word.
  // Pair i belongs to part i % P. An owner other than the last part to
  // arrive polls the publication word (bounded) and, once every part has
  // published, claims its pairs; the last arriver needs no wait. A pair's
  // partials are added in part order (the sum does not depend on who adds
  // them), then the pair's epilogue runs. The last arriver finally claims
  // every pair it does not own, so pairs whose owner gave up waiting are
  // still combined (by it); a claim word counts 1 or 2 claims, and the first
  // claimer combines. Each part counts itself once more on the release word
  // after its last use of the tile's words; the last to release clears them
  // for the next launch. No part waits unboundedly: a give-up costs time,
  // never a result.
  const __amdgpu_buffer_rsrc_t prs = part_rsrc(p.part, p.part_bytes);
  const unsigned tile_base = (unsigned)tile * (unsigned)P * (unsigned)(TF * 4);
  {
    const unsigned mine = tile_base + (unsigned)part * (unsigned)(TF * 4);
    const int nf4 = nvalid * MP * 16;  // valid floats / 4
    for (int e4 = t; e4 < nf4; e4 += NT)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, reinterpret_cast<const f32x4_t*>(red)[e4]),
                                             prs, (int)(mine + 16u * e4), 0, kSc1);
  }
  wait_stores_done();
  __syncthreads();
  int* const ctr = p.counters + tile * kQ4mCtrInts;  // [0] published, [1] released, [2 + i] claims of pair i
  unsigned own = 0;
#pragma unroll
  for (int i = 0; i < NPAIR; ++i)
    if (i % P == part) own |= 1u << i;
  own &= valid;
  auto release = [&]() {
    if (arrive(ctr + 1) == P - 1) {
      reset_counter(ctr);
      reset_counter(ctr + 1);
#pragma unroll
      for (int i = 0; i < NPAIR; ++i) reset_counter(ctr + 2 + i);
    }
  };
  // Wave 0 runs the protocol: lane 0 arrives and polls, lane i claims pair i.
  __shared__ unsigned s_todo, s_islast;
  if (wave == 0) {
    int last_l = 0, seen_l = 0;
    if (lane == 0) {
      last_l = arrive(ctr) == P - 1;
      if (!last_l && own) {
        for (int it = 0; it <= p.spin; ++it) {
          if (it > 0) __builtin_amdgcn_s_sleep(1);
          if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= P) {
            seen_l = 1;
            break;
          }
        }
      }
    }
    const bool lst = __builtin_amdgcn_readfirstlane(last_l) != 0, seen = __builtin_amdgcn_readfirstlane(seen_l) != 0;
    // The last arriver's own pairs: nobody else claims them (its closing
    // claims skip them).
    unsigned todo = lst ? own : 0u;
    if (!lst && seen) {
      const bool won = lane < NPAIR && ((own >> lane) & 1u) && arrive(ctr + 2 + lane) == 0;
      todo = (unsigned)__builtin_amdgcn_ballot_w64(won);
    }
    if (lane == 0) {
      if (!lst) release();  // after this wave's claims have returned
      s_todo = todo;
      s_islast = lst;
    }
  }
  __syncthreads();
  const bool last = s_islast != 0;
  // Sum the partials of the pairs in `todo` into red, in part order. Items
  // are (m-th pair of todo, f32x4 e4 of the pair's 512); a thread takes R =
  // 8 / (P - 1) items per round, items t + (round * R + r) * NT, with all
  // their remote partials in flight (8 loads, ranged loads for the rest).
  auto sum_pairs = [&](unsigned todo) {
    const int cnt = __builtin_popcount(todo), items = cnt * 512;
    const int per = P - 1, R = 8 / per;  // P <= kQ4mMaxParts = 8
    // slot z holds remote part qq(z) of item r(z) (wave-uniform tables)
    int zr[8], zq[8];
    {
      int r = 0, qq = 0;
#pragma unroll
      for (int z = 0; z < 8; ++z) {
        zr[z] = r;
        zq[z] = qq < part ? qq : qq + 1;
        if (++qq == per) {
          qq = 0;
          ++r;
        }
      }
    }
    for (int it0 = t; it0 < items; it0 += R * NT) {
      int loc[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int item = it0 + r * NT;
        loc[r] = r < R && item < items ? pair_f4(nth_pair(todo, item >> 9)) + (item & 511) : -1;
      }
      u32x4_t pv[8];
#pragma unroll
      for (int z = 0; z < 8; ++z) {
        int l = -1;
#pragma unroll
        for (int r = 0; r < 8; ++r)
          if (zr[z] == r) l = loc[r];
        const unsigned off = l >= 0 ? tile_base + (unsigned)zq[z] * (TF * 4) + 16u * (unsigned)l : kOob;
        pv[z] = __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, 0, kSc1);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        if (loc[r] < 0) continue;
        const f32x4_t own_v = reinterpret_cast<const f32x4_t*>(red)[loc[r]];
        f32x4_t v = {0.f, 0.f, 0.f, 0.f};
        bool added = false;
#pragma unroll
        for (int z = 0; z < 8; ++z) {
          if (zr[z] != r) continue;
          if (!added && zq[z] > part) {
            v += own_v;
            added = true;
          }
          v += __builtin_bit_cast(f32x4_t, pv[z]);
        }
        if (!added) v += own_v;
        reinterpret_cast<f32x4_t*>(red)[loc[r]] = v;
      }
    }
  };
  unsigned todo = s_todo;
  if (todo) {
    sum_pairs(todo);
    __syncthreads();
    epilogue(todo);
  }
  if (!last) return;
  __syncthreads();  // every thread has read s_todo
  if (wave == 0) {
    const bool won = lane < NPAIR && (((valid & ~own) >> lane) & 1u) && arrive(ctr + 2 + lane) == 0;
    const unsigned got = (unsigned)__builtin_amdgcn_ballot_w64(won);
    if (lane == 0) {
      release();
      s_todo = got;
    }
  }
  __syncthreads();
  todo = s_todo;
  if (todo) {
    sum_pairs(todo);
    __syncthreads();
    epilogue(todo);
  }
  }
}

// ---- LM head: persistent over vocab tiles, per-row running argmax --------
struct LmParams {
  const uint16_t* x; const uint16_t* x_lo; int ldx;
  const uint16_t* w; int vocab, k;
  const uint16_t* w_sb;  // q4: (scale, bias) pairs
  int ntiles;
  const float* ss_in; int ss_tiles; float inv_norm_dim; float eps;
  float* logits;
  int2* cand;  // (value bits, index) per (row, workgroup), see cand_index
  int cand_blocks;
};



template <int MB, int NB, int U, bool LO, bool TILED, bool Q4, bool H = false>
__global__ __launch_bounds__(kThreads) void lmhead_kernel(LmParams p) {
  constexpr int MP = MB * 32;
  constexpr int TN = 32 * NB;
  constexpr int TE = MP * TN;
  constexpr int IT = TE / kThreads;  // rows handled per thread
  __shared__ float red[(kWaves - 1) * TE];
  __shared__ float rs[MP];
  __shared__ float rs_scratch[kThreads];
  static_assert(!Q4 || (MB == 1 && NB == 2), "q4 LM head: 32 rows, 64-column tiles");
  row_scale<MB>(p.ss_in, p.ss_tiles, p.inv_norm_dim, p.eps, rs, rs_scratch);
  float bv[IT];
  int bi[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    bv[i] = -__builtin_huge_valf();
    bi[i] = 0x7fffffff;
  }
  const int nkb = p.k >> 6;
  const int n = threadIdx.x % TN;
  for (int tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    __syncthreads();
    if constexpr (Q4)
      wg_tile_q4<LO>(p.x, p.x_lo, reinterpret_cast<const uint32_t*>(p.w), reinterpret_cast<const uint32_t*>(p.w_sb),
                     p.k, tile, red);
    else
      wg_tile<MB, NB, U, LO, TILED, H>(p.x, p.x_lo, p.ldx, p.w, p.k, tile, 0, nkb, red);
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int e = threadIdx.x + i * kThreads;
      const int m = e / TN;
      float v = red[e] * rs[m];
      int idx = tile * TN + n;
      if (p.logits) p.logits[(size_t)m * p.vocab + idx] = v;
      lane_argmax<TN>(v, idx);
      argmax_merge(bv[i], bi[i], v, idx);
    }
  }
  if (n == 0) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int m = (threadIdx.x + i * kThreads) / TN;
      p.cand[cand_index(blockIdx.x, m, p.cand_blocks)] = make_int2(__float_as_int(bv[i]), bi[i]);
    }
  }
}

// Tile width per row block count: two 32-row weight blocks share one
// activation fragment for up to 64 rows; wider row blocks keep one.
template <int MB> struct Cfg;
template <> struct Cfg<1> { static constexpr int NB = 2, U = 2; };
template <> struct Cfg<2> { static constexpr int NB = 2, U = 1; };
template <> struct Cfg<3> { static constexpr int NB = 1, U = 1; };
template <> struct Cfg<4> { static constexpr int NB = 1, U = 1; };

static int tile_cols(int rows_padded) { return rows_padded <= 64 ? 64 : 32; }

static int lmhead_grid(int ntiles) { return ntiles < 1024 ? ntiles : 1024; }

// Split-K only while the grid stays within one workgroup per CU (256) and
// every split keeps at least 16 K blocks: each split costs a partial-tile
// round trip through memory at the end, so splitting pays only where it
// brings otherwise idle CUs into the weight stream.
static int auto_split(int ntiles, int nkb) {
  int s = 1;
  while ((s + 1) * ntiles <= 256 && nkb / (s + 1) >= 16) ++s;
  return s;
}

template <int MB, bool LO, bool TILED, bool H = false>
static void launch_gemm_lo(const GemmParams& p, int epi, int blocks, hipStream_t st) {
  constexpr int NB = Cfg<MB>::NB, U = Cfg<MB>::U;
  switch (epi) {
    case DTREE_EPI_STORE_F32:
      gemm_kernel<MB, NB, U, LO, TILED, DTREE_EPI_STORE_F32, H><<<blocks, kThreads, 0, st>>>(p);
      break;
    case DTREE_EPI_RESIDUAL:
      gemm_kernel<MB, NB, U, LO, TILED, DTREE_EPI_RESIDUAL, H><<<blocks, kThreads, 0, st>>>(p);
      break;
    case DTREE_EPI_SWIGLU:
      gemm_kernel<MB, NB, U, LO, TILED, DTREE_EPI_SWIGLU, H><<<blocks, kThreads, 0, st>>>(p);
      break;
    default:
      gemm_kernel<MB, NB, U, LO, TILED, DTREE_EPI_STORE_BF16, H><<<blocks, kThreads, 0, st>>>(p);
      break;
  }
}

template <int MB>
static void launch_gemm(const GemmParams& p, int epi, int blocks, hipStream_t st, bool tiled, bool h16) {
  if (h16) {
    launch_gemm_lo<MB, false, true, true>(p, epi, blocks, st);
  } else if (p.x_lo) {
    if (tiled) launch_gemm_lo<MB, true, true>(p, epi, blocks, st);
    else launch_gemm_lo<MB, true, false>(p, epi, blocks, st);
  } else {
    if (tiled) launch_gemm_lo<MB, false, true>(p, epi, blocks, st);
    else launch_gemm_lo<MB, false, false>(p, epi, blocks, st);
  }
}

template <int MB>
static void launch_lm(const LmParams& p, int grid, hipStream_t st, bool tiled, bool h16) {
  constexpr int NB = Cfg<MB>::NB, U = Cfg<MB>::U;
  if (h16) {
    lmhead_kernel<MB, NB, U, false, true, false, true><<<grid, kThreads, 0, st>>>(p);
  } else if (p.x_lo) {
    if (tiled) lmhead_kernel<MB, NB, U, true, true, false><<<grid, kThreads, 0, st>>>(p);
    else lmhead_kernel<MB, NB, U, true, false, false><<<grid, kThreads, 0, st>>>(p);
  } else {
    if (tiled) lmhead_kernel<MB, NB, U, false, true, false><<<grid, kThreads, 0, st>>>(p);
    else lmhead_kernel<MB, NB, U, false, false, false><<<grid, kThreads, 0, st>>>(p);
  }
}

static void launch_lm_q4(const LmParams& p, int grid, hipStream_t st) {
  if (p.x_lo) lmhead_kernel<1, 2, 2, true, true, true><<<grid, kThreads, 0, st>>>(p);
  else lmhead_kernel<1, 2, 2, false, true, true><<<grid, kThreads, 0, st>>>(p);
}

// Workspace = a fixed counter region (so GEMMs of different shapes can share
// one workspace without one's partials landing on another's counters) followed
// by the split-K partial tiles.
constexpr size_t kCounterBytes = 65536;  // 16384 column tiles

// Stream-K grid: one workgroup per CU, more only when a workgroup's range
// would touch more than kSkMaxBlocks column blocks.
static int sk_grid(int T, int nkb, int cus) {
  int G = T < cus ? T : cus;
  const int need = (T + 3 * nkb - 1) / (3 * nkb);  // <= kSkMaxBlocks column blocks per workgroup
  return G > need ? G : need;
}

// q4 two-per-CU grid (sk2_gemm_kernel) for large unit counts: two
// workgroups per CU, more only when a range would touch more than two
// column blocks; 0 when the shape keeps one workgroup per CU.
static int sk2_grid(int T, int nkb, int cus) {
  if (T < 20 * cus) return 0;
  const int G = T < 2 * cus ? T : 2 * cus;
  const int need = (T + nkb - 1) / nkb;  // ranges of <= nkb units touch <= 2 blocks
  return G > need ? G : need;
}

static size_t sk_workspace_bytes(int n, int k, int cus) {
  const int nkb = k / 64, nblk = n / 64, T = nblk * nkb;
  const int g1 = sk_grid(T, nkb, cus), g2 = sk2_grid(T, nkb, cus);
  return kCounterBytes + (size_t)((g1 > g2 ? g1 : g2) + nblk) * 32 * 64 * sizeof(float);
}

// q4 one-pass plan for 64-128 rows (q4m_gemm_kernel): CW 64-column blocks per
// workgroup (4 when the tiles still cover half the CUs, else 2), and K parts
// so that tiles x parts stays within the CU count of the current device (one
// workgroup per CU: the LDS staging and K-lane reduction take 64-128 KB), at
// most kQ4mMaxParts (a tile's parts then run at once, so the owners' bounded
// waits for each other's partials end early). Workspace sizing and launch both plan for the current device. DTREE_Q4M_CW and
// DTREE_Q4M_PARTS override the choice; DTREE_Q4M=0 sends these shapes back to
// one 32-row pass per row block.
struct Q4mPlan {
  int cw, parts, tiles;
};
static int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}
static bool q4m_enabled() {
  static const int on = env_int("DTREE_Q4M", 1);
  return on != 0;
}
static Q4mPlan q4m_plan(int n, int k, int cus) {
  const int nblk = n / 64, nkb = k / 64;
  static const int cw_env = env_int("DTREE_Q4M_CW", 0), parts_env = env_int("DTREE_Q4M_PARTS", 0);
  auto plan_for = [&](int cw) {
    Q4mPlan q{};
    q.cw = cw;
    q.tiles = (nblk + cw - 1) / cw;
    const int ki = cw == 2 ? 2 : 1;
    int parts = parts_env > 0 ? parts_env : cus / q.tiles;
    const int max_parts = nkb / ki;  // at least one step of groups per part
    if (parts > max_parts) parts = max_parts;
    if (parts > kQ4mMaxParts) parts = kQ4mMaxParts;
    if (parts < 1) parts = 1;
    q.parts = parts;
    return q;
  };
  if (cw_env >= 2 && cw_env <= 4) return plan_for(cw_env);
  Q4mPlan pl = plan_for((nblk % 4 == 0 && 2 * (nblk / 4) >= cus) ? 4 : 2);
  // Three column blocks per workgroup when that fills at least an eighth more
  // of the CUs (the 9B-shaped gate/up: 384 blocks are 192 tiles of 2 or 96 of
  // 4 in two parts, 192 workgroups; 128 tiles of 3 in two parts fill 256).
  const Q4mPlan p3 = plan_for(3);
  if (p3.tiles * p3.parts >= pl.tiles * pl.parts + cus / 8) pl = p3;
  return pl;
}
static size_t q4m_workspace_bytes(int rows, int n, int k, int cus) {
  const Q4mPlan pl = q4m_plan(n, k, cus);
  if (pl.parts <= 1) return kCounterBytes;
  return kCounterBytes + (size_t)pl.tiles * pl.parts * pl.cw * rows * 64 * sizeof(float);
}

template <bool LO, int MB, int CW>
static void launch_q4m_mb(const GemmParams& p, int epi, int grid, hipStream_t st) {
  switch (epi) {
    case DTREE_EPI_STORE_F32: q4m_gemm_kernel<LO, DTREE_EPI_STORE_F32, MB, CW><<<grid, Q4mShape<LO, MB, CW>::THREADS, 0, st>>>(p); break;
    case DTREE_EPI_RESIDUAL: q4m_gemm_kernel<LO, DTREE_EPI_RESIDUAL, MB, CW><<<grid, Q4mShape<LO, MB, CW>::THREADS, 0, st>>>(p); break;
    case DTREE_EPI_SWIGLU: q4m_gemm_kernel<LO, DTREE_EPI_SWIGLU, MB, CW><<<grid, Q4mShape<LO, MB, CW>::THREADS, 0, st>>>(p); break;
    default: q4m_gemm_kernel<LO, DTREE_EPI_STORE_BF16, MB, CW><<<grid, Q4mShape<LO, MB, CW>::THREADS, 0, st>>>(p); break;
  }
}
template <bool LO, int CW>
static void launch_q4m_cw(const GemmParams& p, int epi, int mb, int grid, hipStream_t st) {
  switch (mb) {
    case 2: launch_q4m_mb<LO, 2, CW>(p, epi, grid, st); break;
    case 3: launch_q4m_mb<LO, 3, CW>(p, epi, grid, st); break;
    default: launch_q4m_mb<LO, 4, CW>(p, epi, grid, st); break;
  }
}
template <bool LO>
static void launch_q4m_lm(const GemmParams& p, int mb, int grid, hipStream_t st) {
  switch (mb) {
    case 1: q4m_gemm_kernel<LO, kEpiLmArgmax, 1, 4><<<grid, kThreads, 0, st>>>(p); break;
    case 2: q4m_gemm_kernel<LO, kEpiLmArgmax, 2, 4><<<grid, kThreads * 2, 0, st>>>(p); break;
    case 3: q4m_gemm_kernel<LO, kEpiLmArgmax, 3, 4><<<grid, kThreads * 3, 0, st>>>(p); break;
    default: q4m_gemm_kernel<LO, kEpiLmArgmax, 4, 4><<<grid, kThreads * 4, 0, st>>>(p); break;
  }
}
static void launch_q4m(const GemmParams& p, int epi, int mb, int cw, int grid, hipStream_t st) {
  if (p.x_lo) {
    if (cw == 4) launch_q4m_cw<true, 4>(p, epi, mb, grid, st);
    else if (cw == 3) launch_q4m_cw<true, 3>(p, epi, mb, grid, st);
    else launch_q4m_cw<true, 2>(p, epi, mb, grid, st);
  } else {
    if (cw == 4) launch_q4m_cw<false, 4>(p, epi, mb, grid, st);
    else if (cw == 3) launch_q4m_cw<false, 3>(p, epi, mb, grid, st);
    else launch_q4m_cw<false, 2>(p, epi, mb, grid, st);
  }
}

static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <bool LO>
static void launch_sk2(const GemmParams& p, int epi, hipStream_t st) {
  switch (epi) {
    case DTREE_EPI_STORE_F32: sk2_gemm_kernel<LO, DTREE_EPI_STORE_F32><<<p.G, kThreads, 0, st>>>(p); break;
    case DTREE_EPI_RESIDUAL: sk2_gemm_kernel<LO, DTREE_EPI_RESIDUAL><<<p.G, kThreads, 0, st>>>(p); break;
    case DTREE_EPI_SWIGLU: sk2_gemm_kernel<LO, DTREE_EPI_SWIGLU><<<p.G, kThreads, 0, st>>>(p); break;
    default: sk2_gemm_kernel<LO, DTREE_EPI_STORE_BF16><<<p.G, kThreads, 0, st>>>(p); break;
  }
}

template <bool LO, bool Q4, bool H = false>
static void launch_sk(const GemmParams& p, int epi, hipStream_t st) {
  switch (epi) {
    case DTREE_EPI_STORE_F32: sk_gemm_kernel<LO, DTREE_EPI_STORE_F32, Q4, H><<<p.G, kThreads, 0, st>>>(p); break;
    case DTREE_EPI_RESIDUAL: sk_gemm_kernel<LO, DTREE_EPI_RESIDUAL, Q4, H><<<p.G, kThreads, 0, st>>>(p); break;
    case DTREE_EPI_SWIGLU: sk_gemm_kernel<LO, DTREE_EPI_SWIGLU, Q4, H><<<p.G, kThreads, 0, st>>>(p); break;
    default: sk_gemm_kernel<LO, DTREE_EPI_STORE_BF16, Q4, H><<<p.G, kThreads, 0, st>>>(p); break;
  }
}


// ---- data-parallel GEMM (32 tiled rows, bf16 or q4 weights) -----------------
// A workgroup owns one 32-column output tile over the whole K (KS = 1) or
// over one half of it (KS = 2). Wave w streams the K blocks w, w + 4, ... of
// its range through a kDpDepth-deep register ring (weights and both
// activation planes of kDpDepth blocks in flight), the waves' partial tiles
// are added in LDS in wave order (deterministic), and the shared tile
// epilogue runs. Each CU reads every activation block of its K range from L2
// (about twice the bytes of its weights), so a CU's load bandwidth bounds
// the one-workgroup-per-tile launch when N / 32 is well below the CU count;
// KS = 2 puts twice the workgroups on the chip, each with half the bytes.
// The two halves of a tile run as workgroups b and b + 8, which the
// round-robin dispatch places on one XCD; each publishes its partial tile
// (4 KB) written through, and the last to arrive adds the two (half 0 +
// half 1: fp32 addition is commutative, so the sum does not depend on which
// half arrives last) and runs the epilogue, reading its partner's tile from
// its own L2 when both placements are confirmed (HW_REG_XCC_ID).
constexpr int kDpDepth = 4;

// Q4: group-64 q4 weights (DTREE_W_Q4G64) in place of bf16. A K block is then
// one quantisation group, 1 KB of nibbles (one 16-byte load per lane) and 32
// scale/bias pairs per 32-column block; each group gets a fresh MFMA sum of
// x (128 + q), folded in as acc += s * sum + (b - 128 s) * sum(x), with
// sum(x) from an MFMA of the same activation registers against bf16 ones (as
// q4_group).
template <bool LO, int EPI, int KS, bool Q4, bool H = false>
__device__ __forceinline__ void dp_gemm_body(const GemmParams& p) {
  constexpr int TN = 32, TE = 32 * TN;
  constexpr int WL = Q4 ? 1 : 4;  // 16-byte weight loads per lane per K block
  __shared__ float red[kWaves * TE];
  __shared__ float rs[32];
  __shared__ float rs_scratch[kThreads];
  __shared__ int last_s;
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nkb = p.k >> 6;
  // KS > 1: blockIdx = 8 KS (tile / 8) + 8 part + tile % 8 (host: tiles % 8 == 0).
  const int bid = blockIdx.x;
  const int part = KS > 1 ? (bid >> 3) % KS : 0;
  const int tile = KS > 1 ? (bid / (8 * KS)) * 8 + (bid & 7) : bid;
  const int kb0 = part * nkb / KS, kb1 = (part + 1) * nkb / KS;
  const int nk = kb1 - kb0;
  float ssv[kSsBatch];
  ss_issue<1>(p.ss_in, p.ss_tiles, ssv);
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(p.x, p.x_bytes), xlrs = buf_rsrc(p.x_lo, LO ? p.x_bytes : 0u);
  const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(p.w, p.w_bytes);
  const __amdgpu_buffer_rsrc_t sbrs = buf_rsrc(p.w_sb, Q4 ? p.sb_bytes : 0u);
  const int n = wave < nk ? (nk - wave + kWaves - 1) / kWaves : 0;
  u32x4_t wr[kDpDepth][WL], xr[kDpDepth][2][4];
  uint32_t sbr[kDpDepth];
  // Slots past the wave's blocks are refilled with ranged loads that return
  // zero (same loads on every path, see kOob) and are never consumed.
  auto issue = [&](int s, int j) {
    const int kb = kb0 + wave + kWaves * j;
    const unsigned off = j < n ? (unsigned)(kb * 2048 + lane * 8) * 2u : kOob;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xr[s][0][i] = buf_ld(xrs, off + 1024u * i);
      if (LO) xr[s][1][i] = buf_ld(xlrs, off + 1024u * i);
    }
    if constexpr (Q4) {
      const unsigned blk = (unsigned)(tile * nkb + kb);
      wr[s][0] = buf_ld_stream(wrs, j < n ? blk * 1024u + lane * 16u : kOob);
      sbr[s] = buf_ld32(sbrs, j < n ? (blk * 32u + c) * 4u : kOob);
    } else {
      const unsigned wtile = (unsigned)(tile * nkb * 2048) * 2u;
#pragma unroll
      for (int i = 0; i < 4; ++i) wr[s][i] = buf_ld_stream(wrs, j < n ? wtile + off + 1024u * i : kOob);
    }
  };
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
  for (int s = 0; s < kDpDepth; ++s) issue(s, s);
  ss_finish<1>(p.ss_in, p.ss_tiles, p.inv_norm_dim, p.eps, ssv, rs, rs_scratch);
  for (int jb = 0; jb < n; jb += kDpDepth) {
#pragma unroll
    for (int s = 0; s < kDpDepth; ++s) {
      const int j = jb + s;
      if (j < n) {
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (Q4) {
          const u32x4_t ones = u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
          f32x16_t xs, au;
#pragma unroll
          for (int r = 0; r < 16; ++r) xs[r] = au[r] = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xs = mfma32(xr[s][0][i], ones, xs);
            if (LO) xs = mfma32(xr[s][1][i], ones, xs);
          }
          const uint32_t wq[4] = {wr[s][0][0], wr[s][0][1], wr[s][0][2], wr[s][0][3]};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4_t bq = q4_pairs(wq[i]);
            au = mfma32(xr[s][0][i], bq, au);
            if (LO) au = mfma32(xr[s][1][i], bq, au);
          }
          const float sc = __uint_as_float(sbr[s] << 16);
          const float cf = __uint_as_float(sbr[s] & 0xffff0000u) - 128.f * sc;
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] = fmaf(cf, xs[r], fmaf(sc, au[r], acc[r]));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (H) {
              acc = mfma32_f16(xr[s][0][i], wr[s][i], acc);
            } else {
              acc = mfma32(xr[s][0][i], wr[s][i], acc);
              if (LO) acc = mfma32(xr[s][1][i], wr[s][i], acc);
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      issue(s, j + kDpDepth);
    }
  }
  // The residual rows are in flight during the wave reduction (and the
  // partial exchange).
  float xo[TE / kThreads + 1];
  if constexpr (EPI == DTREE_EPI_RESIDUAL) residual_issue<32, TN>(p, tile, xo);
  // Every wave parks its tile; thread t adds elements 4t .. 4t+3 of the four
  // in wave order (the order the sum always had) into slot 0. The barriers
  // wait for LDS only: the residual rows stay in flight.
  {
    float* my = red + wave * TE;
#pragma unroll
    for (int r = 0; r < 16; ++r) my[acc_row(r, h) * TN + c] = acc[r];
  }
  lds_barrier();
  f32x4_t tsum = reinterpret_cast<const f32x4_t*>(red)[threadIdx.x];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) tsum += reinterpret_cast<const f32x4_t*>(red + w * TE)[threadIdx.x];
  reinterpret_cast<f32x4_t*>(red)[threadIdx.x] = tsum;
  lds_barrier();
  if constexpr (KS > 1) {
    // Thread t holds elements 4t .. 4t+3 of the tile; slot KS * tile + part.
    const int t = threadIdx.x;
    const bool native = !p.off_xcd && xcc_id() == (bid & 7);
    const __amdgpu_buffer_rsrc_t prs = part_rsrc(p.part, p.part_bytes);
    const f32x4_t mine = tsum;
    const int off = ((KS * tile + part) * TE + 4 * t) * 4;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, mine), prs, off, 0, kSc1);
    wait_stores_done();
    __syncthreads();
    if (t == 0) {
      const int old = arrive_add(&p.counters[tile], native ? 1 : 1 + kForeign);
      int last = 0;
      if ((old & (kForeign - 1)) == KS - 1) {
        last = native && old < kForeign ? 2 : 1;
        reset_counter(&p.counters[tile]);
      }
      last_s = last;
    }
    __syncthreads();
    const int last = __builtin_amdgcn_readfirstlane(last_s);
    if (!last) return;
    // The parts in part order (own part from registers), so the sum does not
    // depend on which part arrives last.
    u32x4_t pv[KS];
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      const int poff = q == part ? (int)kOob : ((KS * tile + q) * TE + 4 * t) * 4;
      pv[q] = last == 2 ? __builtin_amdgcn_raw_buffer_load_b128(prs, poff, 0, kSc0)
                        : __builtin_amdgcn_raw_buffer_load_b128(prs, poff, 0, kSc1);
    }
    f32x4_t sum = part == 0 ? mine : __builtin_bit_cast(f32x4_t, pv[0]);
#pragma unroll
    for (int q = 1; q < KS; ++q) sum += q == part ? mine : __builtin_bit_cast(f32x4_t, pv[q]);
    reinterpret_cast<f32x4_t*>(red)[t] = sum;
    __syncthreads();
  }
  tile_epilogue<32, TN, EPI>(p, red, rs, tile, EPI == DTREE_EPI_RESIDUAL ? xo : nullptr);
}

template <bool LO, int EPI, int KS, bool H = false>
__global__ __launch_bounds__(kThreads) void dp_gemm_kernel(GemmParams p) {
  dp_gemm_body<LO, EPI, KS, false, H>(p);
}

template <bool LO, int EPI, int KS>
__global__ __launch_bounds__(kThreads) void dpq_gemm_kernel(GemmParams p) {
  dp_gemm_body<LO, EPI, KS, true>(p);
}

template <bool LO, int KS, bool Q4, bool H = false>
static void launch_dp(const GemmParams& p, int epi, hipStream_t st) {
  const int grid = KS * (p.n / 32);
  if constexpr (Q4) {
    switch (epi) {
      case DTREE_EPI_STORE_F32: dpq_gemm_kernel<LO, DTREE_EPI_STORE_F32, KS><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_RESIDUAL: dpq_gemm_kernel<LO, DTREE_EPI_RESIDUAL, KS><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_SWIGLU: dpq_gemm_kernel<LO, DTREE_EPI_SWIGLU, KS><<<grid, kThreads, 0, st>>>(p); break;
      default: dpq_gemm_kernel<LO, DTREE_EPI_STORE_BF16, KS><<<grid, kThreads, 0, st>>>(p); break;
    }
  } else {
    switch (epi) {
      case DTREE_EPI_STORE_F32: dp_gemm_kernel<LO, DTREE_EPI_STORE_F32, KS, H><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_RESIDUAL: dp_gemm_kernel<LO, DTREE_EPI_RESIDUAL, KS, H><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_SWIGLU: dp_gemm_kernel<LO, DTREE_EPI_SWIGLU, KS, H><<<grid, kThreads, 0, st>>>(p); break;
      default: dp_gemm_kernel<LO, DTREE_EPI_STORE_BF16, KS, H><<<grid, kThreads, 0, st>>>(p); break;
    }
  }
}
template <int KS>
static void launch_dp_any(const GemmParams& p, int epi, bool q4, bool h16, hipStream_t st) {
  if (h16) return launch_dp<false, KS, false, true>(p, epi, st);
  const bool lo = p.x_lo != nullptr;
  if (q4) lo ? launch_dp<true, KS, true>(p, epi, st) : launch_dp<false, KS, true>(p, epi, st);
  else lo ? launch_dp<true, KS, false>(p, epi, st) : launch_dp<false, KS, false>(p, epi, st);
}

// ---- long-M GEMM (prompt prefill): rows a multiple of 128 --------------------
// Compute-bound: a workgroup owns a 128-row x 128-column output tile over the
// whole K. Per 64-wide K block the workgroup stages the tile's activation
// blocks (4 row blocks, hi and lo planes) and weight blocks (4 column blocks)
// in LDS, 16 bytes per thread per 4 KB block, double-buffered with one barrier
// per K block (the next block's loads are in flight during the current
// block's MFMAs). Wave w computes rows 64 (w / 2) .. + 63 x columns
// 64 (w % 2) .. + 63 as 2 x 2 MFMA 32 x 32 tiles: 32 MFMAs per K block with
// both planes. The finished tile goes through LDS to the same epilogues as
// the skinny GEMMs, applied to 128 rows.
constexpr int kLongRows = 128, kLongCols = 128;

// Q4: group-64 q4 weights (DTREE_W_Q4G64). A K block is one quantisation
// group: per 32-column block 1 KB of nibbles and 32 (scale, bias) words are
// staged; each wave's 32 x 32 tiles take a fresh MFMA sum of x (128 + q) per
// group and fold it in as acc += s * sum + (b - 128 s) * sum(x), with sum(x)
// per row block from an MFMA of the staged activations against bf16 ones.
template <bool LO, int EPI, bool Q4, bool H = false>
__device__ __forceinline__ void long_gemm_body(const GemmParams& p) {
  constexpr int NPL = LO ? 2 : 1, ABLK = 4 * NPL;
  constexpr int WBYTES = Q4 ? 4 * 1024 + 4 * 128 : 4 * 4096;            // weight bytes per stage
  constexpr int STAGE = ABLK * 4096 + WBYTES;                           // bytes per stage
  constexpr int SMEM = 2 * STAGE > kLongRows * kLongCols * 4 ? 2 * STAGE : kLongRows * kLongCols * 4;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  __shared__ float rs[kLongRows];
  const int t = threadIdx.x, lane = t & 63, c = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const int ntn = (p.n + kLongCols - 1) / kLongCols;  // the last tile may hold 64 columns (STORE_F32)
  const int mt = blockIdx.x / ntn, nt = blockIdx.x - mt * ntn;
  const int nkb = p.k >> 6;
  const int R = mt * kLongRows;
  if (t < kLongRows) {
    float r = 1.f;
    if (p.ss_in) {
      float s = 0.f;
      for (int tt = 0; tt < p.ss_tiles; ++tt) s += p.ss_in[ss_index(tt, R + t, p.ss_tiles)];
      r = rsqrtf(s * p.inv_norm_dim + p.eps);
    }
    rs[t] = r;
  }
  // Staged per thread: ABLK activation pieces, then the weight pieces (bf16:
  // 4 x 16 bytes; q4: 16 bytes of nibbles, and for t < 32 16 bytes of
  // scale / bias words).
  constexpr int NW = Q4 ? 2 : 4;
  u32x4_t ld[ABLK + NW];
  const uint32_t* wsb = reinterpret_cast<const uint32_t*>(p.w_sb);
  auto load_stage = [&](int kb) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const size_t blk = ((size_t)((R >> 5) + rb) * nkb + kb) * 2048 + 8 * t;
      ld[rb * NPL] = ld_u32x4(p.x + blk);
      if (LO) ld[rb * NPL + NPL - 1] = ld_u32x4(p.x_lo + blk);
    }
    if constexpr (Q4) {
      const int cb = nt * 4 + (t >> 6);  // this thread's 32-column block
      ld[ABLK] = cb * 32 < p.n ? ld_u32x4(reinterpret_cast<const uint32_t*>(p.w) + ((size_t)cb * nkb + kb) * 256 +
                                          4 * (t & 63))
                               : u32x4_t{0u, 0u, 0u, 0u};
      if (t < 32) {
        const int sbb = nt * 4 + (t >> 3);
        ld[ABLK + 1] = sbb * 32 < p.n ? ld_u32x4(wsb + ((size_t)sbb * nkb + kb) * 32 + 4 * (t & 7))
                                      : u32x4_t{0u, 0u, 0u, 0u};
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        ld[ABLK + cb] = (nt * 4 + cb) * 32 < p.n ? ld_u32x4(p.w + ((size_t)(nt * 4 + cb) * nkb + kb) * 2048 + 8 * t)
                                                 : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_stage = [&](int s) {
    unsigned char* st = smem + s * STAGE;
#pragma unroll
    for (int b = 0; b < ABLK; ++b) *reinterpret_cast<u32x4_t*>(st + b * 4096 + 16 * t) = ld[b];
    if constexpr (Q4) {
      // nibbles [block][lane] 16 bytes each, then (scale, bias) words [block][32]
      *reinterpret_cast<u32x4_t*>(st + ABLK * 4096 + 16 * t) = ld[ABLK];
      if (t < 32) *reinterpret_cast<u32x4_t*>(st + ABLK * 4096 + 4096 + 16 * t) = ld[ABLK + 1];
    } else {
#pragma unroll
      for (int b = 0; b < 4; ++b) *reinterpret_cast<u32x4_t*>(st + (ABLK + b) * 4096 + 16 * t) = ld[ABLK + b];
    }
  };
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int s = kb & 1;
    if (kb + 1 < nkb) load_stage(kb + 1);
    const unsigned char* st = smem + s * STAGE;
    if constexpr (Q4) {
      const u32x4_t ones = u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
      u32x4_t wq[2];
      float sc[2], cf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cb = 2 * wc + j;
        wq[j] = *reinterpret_cast<const u32x4_t*>(st + ABLK * 4096 + cb * 1024 + 16 * lane);
        const uint32_t sbw = *reinterpret_cast<const uint32_t*>(st + ABLK * 4096 + 4096 + (cb * 32 + c) * 4);
        sc[j] = __uint_as_float(sbw << 16);
        cf[j] = __uint_as_float(sbw & 0xffff0000u) - 128.f * sc[j];
      }
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        u32x4_t xa[4][NPL];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int pl = 0; pl < NPL; ++pl)
            xa[i][pl] = *reinterpret_cast<const u32x4_t*>(st + ((2 * wr + rb) * NPL + pl) * 4096 + (64 * i + lane) * 16);
        f32x16_t xs;
#pragma unroll
        for (int r = 0; r < 16; ++r) xs[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int pl = 0; pl < NPL; ++pl) xs = mfma32(xa[i][pl], ones, xs);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          f32x16_t au;
#pragma unroll
          for (int r = 0; r < 16; ++r) au[r] = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4_t bq = q4_pairs(wq[j][i]);
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl) au = mfma32(xa[i][pl], bq, au);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[rb][j][r] = fmaf(cf[j], xs[r], fmaf(sc[j], au[r], acc[rb][j][r]));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int fo = (64 * i + lane) * 16;
        u32x4_t b[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(st + (ABLK + 2 * wc + j) * 4096 + fo);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          const u32x4_t ah = *reinterpret_cast<const u32x4_t*>(st + ((2 * wr + rb) * NPL) * 4096 + fo);
          if constexpr (H) {
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[rb][j] = mfma32_f16(ah, b[j], acc[rb][j]);
          } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[rb][j] = mfma32(ah, b[j], acc[rb][j]);
          }
          if (LO) {
            const u32x4_t al = *reinterpret_cast<const u32x4_t*>(st + ((2 * wr + rb) * NPL + 1) * 4096 + fo);
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[rb][j] = mfma32(al, b[j], acc[rb][j]);
          }
        }
      }
    }
    if (kb + 1 < nkb) store_stage(s ^ 1);
    __syncthreads();
  }
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        red[(64 * wr + 32 * rb + acc_row(r, h)) * kLongCols + 64 * wc + 32 * j + c] = acc[rb][j][r];
  __syncthreads();
  // The epilogue of rows R .. R + 127, one 32-row block at a time (outputs
  // shifted by the block's first row: 32-row blocks are contiguous in both
  // layouts; statistics are per 32-row block). In one 128-row piece the
  // residual epilogue held 64 preloaded values per thread and took the kernel
  // to 320 VGPRs, one workgroup per CU for the whole K loop.
#pragma unroll 1
  for (int r2 = 0; r2 < kLongRows / 32; ++r2) {
    const int R2 = R + 32 * r2;
    GemmParams q = p;
    if (q.out_f32) q.out_f32 += (size_t)R2 * q.ld_out_f32;
    if (q.out_bf16) q.out_bf16 += (size_t)R2 * q.ld_out_bf16;
    if (q.out_lo) q.out_lo += (size_t)R2 * q.ld_out_bf16;
    if (q.hidden_out) q.hidden_out += (size_t)R2 * q.ld_hidden;
    if (q.ss_out) q.ss_out += (size_t)(R2 >> 5) * (q.n >> 5) * 32;
    tile_epilogue<32, kLongCols, EPI>(q, red + 32 * r2 * kLongCols, rs + 32 * r2, nt);
  }
}

template <bool LO, int EPI, bool H = false>
__global__ __launch_bounds__(kThreads) void long_gemm_kernel(GemmParams p) {
  long_gemm_body<LO, EPI, false, H>(p);
}

template <bool LO, int EPI>
__global__ __launch_bounds__(kThreads) void longq_gemm_kernel(GemmParams p) {
  long_gemm_body<LO, EPI, true>(p);
}

template <bool LO>
static void launch_long(const GemmParams& p, int epi, int grid, bool q4, bool h16, hipStream_t st) {
  if (h16) {
    switch (epi) {
      case DTREE_EPI_STORE_F32: long_gemm_kernel<false, DTREE_EPI_STORE_F32, true><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_RESIDUAL: long_gemm_kernel<false, DTREE_EPI_RESIDUAL, true><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_SWIGLU: long_gemm_kernel<false, DTREE_EPI_SWIGLU, true><<<grid, kThreads, 0, st>>>(p); break;
      default: long_gemm_kernel<false, DTREE_EPI_STORE_BF16, true><<<grid, kThreads, 0, st>>>(p); break;
    }
    return;
  }
  if (q4) {
    switch (epi) {
      case DTREE_EPI_STORE_F32: longq_gemm_kernel<LO, DTREE_EPI_STORE_F32><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_RESIDUAL: longq_gemm_kernel<LO, DTREE_EPI_RESIDUAL><<<grid, kThreads, 0, st>>>(p); break;
      case DTREE_EPI_SWIGLU: longq_gemm_kernel<LO, DTREE_EPI_SWIGLU><<<grid, kThreads, 0, st>>>(p); break;
      default: longq_gemm_kernel<LO, DTREE_EPI_STORE_BF16><<<grid, kThreads, 0, st>>>(p); break;
    }
    return;
  }
  switch (epi) {
    case DTREE_EPI_STORE_F32: long_gemm_kernel<LO, DTREE_EPI_STORE_F32><<<grid, kThreads, 0, st>>>(p); break;
    case DTREE_EPI_RESIDUAL: long_gemm_kernel<LO, DTREE_EPI_RESIDUAL><<<grid, kThreads, 0, st>>>(p); break;
    case DTREE_EPI_SWIGLU: long_gemm_kernel<LO, DTREE_EPI_SWIGLU><<<grid, kThreads, 0, st>>>(p); break;
    default: long_gemm_kernel<LO, DTREE_EPI_STORE_BF16><<<grid, kThreads, 0, st>>>(p); break;
  }
}

}  // namespace dtree

using namespace dtree;

// The split per-tile schedules: counters + one 32 x 32 fp32 partial per
// (tile, part), at most kDpMaxParts parts.
constexpr int kDpMaxParts = 3;
static size_t dp_pair_workspace_bytes(int n) {
  return kCounterBytes + (size_t)(n / 32) * kDpMaxParts * 32 * 32 * sizeof(float);
}

extern "C" size_t dtree_gemm_workspace_bytes(int rows_padded, int n, int k, int split_k) {
  if (rows_padded <= 0 || n <= 0 || k <= 0) return 0;
  const int tn = tile_cols(rows_padded);
  const int ntiles = (n + tn - 1) / tn, nkb = k / 64;
  const int S = split_k > 0 ? split_k : auto_split(ntiles, nkb);
  const size_t nt8 = (size_t)((ntiles + 7) / 8) * 8;
  size_t need = kCounterBytes + (S > 1 ? nt8 * S * (size_t)rows_padded * tn * sizeof(float) : 0);
  if (split_k <= 0 && rows_padded % 32 == 0) {
    // The stream-K path (tiled operands; q4 weights at any row count, one
    // 32-row pass per block) may serve this shape: size for the largest CU
    // count it plans for.
    const size_t sk = sk_workspace_bytes(n, k, kSkMaxGrid);
    if (sk > need) need = sk;
    const size_t pairs = dp_pair_workspace_bytes(n);
    if (pairs > need) need = pairs;
  }
  if (split_k <= 0 && rows_padded > 32 && rows_padded % 32 == 0 && n % 64 == 0) {
    // q4 weights at 64-128 rows take the one-pass kernel (q4m_gemm_kernel).
    const size_t q4m = q4m_workspace_bytes(rows_padded, n, k, device_cus());
    if (q4m > need) need = q4m;
  }
  return need;
}

extern "C" int dtree_gemm_bf16(const DtreeGemmArgs* a, hipStream_t stream) {
  DTREE_REQUIRE(a, "gemm: null args");
  DTREE_REQUIRE(a->x && a->w, "gemm: null x or w");
  DTREE_REQUIRE(a->rows_padded == 32 || a->rows_padded == 64 || a->rows_padded == 96 || a->rows_padded == 128,
                "gemm: rows_padded must be 32, 64, 96 or 128");
  const int tn = tile_cols(a->rows_padded);
  DTREE_REQUIRE(a->n > 0 && a->n % tn == 0, "gemm: n must be a positive multiple of 64 (32 for > 64 rows)");
  DTREE_REQUIRE(a->k > 0 && a->k % 64 == 0, "gemm: k must be a positive multiple of 64");
  DTREE_REQUIRE(a->ldx >= a->k && a->ldx % 8 == 0, "gemm: ldx must be >= k and a multiple of 8");
  const int ntiles = a->n / tn, nkb = a->k / 64;
  DTREE_REQUIRE(a->split_k >= -4, "gemm: split_k must be >= -4");
  DTREE_REQUIRE(a->split_k >= 0 || (a->w_layout != DTREE_W_ROWMAJOR && a->rows_padded == 32),
                "gemm: split_k -1 .. -4 need tiled weights and 32 rows");
  const int S = a->split_k > 0 ? a->split_k : auto_split(ntiles, nkb);
  DTREE_REQUIRE(S <= nkb, "gemm: split_k larger than the number of 64-wide K blocks");
  DTREE_REQUIRE((size_t)ntiles * sizeof(int) <= kCounterBytes, "gemm: n too large for the tile counter region");
  const int epi = a->epilogue;
  DTREE_REQUIRE(epi >= 0 && epi <= 3, "gemm: unknown epilogue");
  if (epi == DTREE_EPI_STORE_F32 || epi == DTREE_EPI_RESIDUAL)
    DTREE_REQUIRE(a->out_f32 && a->ld_out_f32 >= a->n, "gemm: out_f32 missing or ld too small");
  if (epi == DTREE_EPI_RESIDUAL)
    DTREE_REQUIRE(a->out_bf16 && a->next_norm && a->ss_out && a->ld_out_bf16 >= a->n,
                  "gemm: residual epilogue needs out_bf16, next_norm, ss_out");
  if (epi == DTREE_EPI_SWIGLU)
    DTREE_REQUIRE(a->out_bf16 && a->ld_out_bf16 >= a->n / 2, "gemm: swiglu needs out_bf16 (n/2 wide)");
  if (epi == DTREE_EPI_STORE_BF16) DTREE_REQUIRE(a->out_bf16 && a->ld_out_bf16 >= a->n, "gemm: out_bf16");
  if (a->hidden_out) DTREE_REQUIRE(a->ld_hidden >= a->n, "gemm: ld_hidden too small");
  if (a->ss_in) DTREE_REQUIRE(a->ss_tiles > 0 && a->norm_dim > 0, "gemm: ss_in needs ss_tiles and norm_dim");
  const size_t need = dtree_gemm_workspace_bytes(a->rows_padded, a->n, a->k, S);
  DTREE_REQUIRE(a->workspace && a->workspace_bytes >= need, "gemm: workspace too small");
  // fp16 path: fp16 weights and one fp16 activation plane, both TILED_F16
  const bool h16 = a->x_layout == DTREE_W_TILED_F16;
  DTREE_REQUIRE(h16 == (a->w_layout == DTREE_W_TILED_F16),
                "gemm: DTREE_W_TILED_F16 weights and activations go together (q4 weights take DTREE_W_TILED x)");

  GemmParams p{};
  p.x = a->x; p.x_lo = h16 ? nullptr : a->x_lo; p.ldx = a->ldx; p.w = a->w; p.n = a->n; p.k = a->k;
  p.S = S; p.kb_per_split = (nkb + S - 1) / S; p.ntiles = ntiles;
  p.ss_in = a->ss_in; p.ss_tiles = a->ss_tiles;
  p.inv_norm_dim = a->norm_dim > 0 ? 1.0f / (float)a->norm_dim : 1.f; p.eps = a->eps;
  p.out_f32 = a->out_f32; p.ld_out_f32 = a->ld_out_f32;
  p.out_tiled = a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16;
  p.out_h16 = a->out_layout == DTREE_W_TILED_F16;
  p.out_bf16 = a->out_bf16; p.out_lo = p.out_h16 ? nullptr : a->out_lo; p.ld_out_bf16 = a->ld_out_bf16;
  p.next_norm = a->next_norm; p.ss_out = a->ss_out;
  p.hidden_out = a->hidden_out; p.ld_hidden = a->ld_hidden;
  p.off_xcd = off_xcd_test();
  const size_t nt8 = (size_t)((ntiles + 7) / 8) * 8;
  p.counters = reinterpret_cast<int*>(a->workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) + kCounterBytes);
  const int blocks = S == 1 ? ntiles : (int)(nt8 * S);
  const bool q4 = a->w_layout == DTREE_W_Q4G64;
  const bool tiled = a->w_layout == DTREE_W_TILED || q4 || h16;
  DTREE_REQUIRE(a->w_layout == DTREE_W_ROWMAJOR || tiled, "gemm: unknown w_layout");
  if (q4 && a->rows_padded > 32 && q4m_enabled()) {
    // One pass over the q4 weights for every row block (q4m_gemm_kernel).
    DTREE_REQUIRE(a->x_layout == DTREE_W_TILED && a->ldx == a->k && a->split_k <= 0,
                  "gemm: q4 weights need tiled activations (ldx == k) and split_k 0");
    DTREE_REQUIRE(a->n % 64 == 0, "gemm: q4 weights need n % 64 == 0");
    DTREE_REQUIRE(a->w_scales && ((uintptr_t)a->w & 15) == 0 && ((uintptr_t)a->w_scales & 3) == 0,
                  "gemm: q4 weights need w (16-byte aligned) and w_scales (4-byte aligned)");
    DTREE_REQUIRE(((uintptr_t)a->x & 15) == 0 && ((uintptr_t)a->x_lo & 15) == 0,
                  "gemm: q4 activations must be 16-byte aligned");
    const size_t xb = (size_t)a->rows_padded * a->k * 2, wb = (size_t)a->n * a->k / 2;
    DTREE_REQUIRE(xb < kOob && wb < kOob, "gemm: operands must be smaller than 2 GiB");
    const int cus = device_cus();
    const Q4mPlan pl = q4m_plan(a->n, a->k, cus);
    DTREE_REQUIRE((size_t)pl.tiles * kQ4mCtrInts * sizeof(int) <= kCounterBytes,
                  "gemm: n too large for the tile counter region");
    const size_t need_m = q4m_workspace_bytes(a->rows_padded, a->n, a->k, cus);
    DTREE_REQUIRE(a->workspace_bytes >= need_m, "gemm: workspace too small for the q4 one-pass schedule");
    p.w_sb = a->w_scales;
    p.x_bytes = (unsigned)xb;
    p.w_bytes = (unsigned)wb;
    p.sb_bytes = (unsigned)((size_t)a->n * (a->k / 64) * 4);
    p.S = pl.parts;
    p.part_bytes = (unsigned)(need_m - kCounterBytes);
    p.spin = attn_spin_limit() < kQ4mSpin ? attn_spin_limit() : kQ4mSpin;
    launch_q4m(p, epi, a->rows_padded / 32, pl.cw, pl.tiles * pl.parts, stream);
    DTREE_LAUNCH_CHECK("gemm launch");
    return DTREE_OK;
  }
  if (q4 && a->rows_padded > 32) {
    // q4 weights stream through the 32-row kernels, once per 32-row block:
    // tiled activations, statistics and tiled outputs are contiguous per
    // block; row-major outputs advance by 32 rows.
    DTREE_REQUIRE(a->x_layout == DTREE_W_TILED, "gemm: q4 weights need tiled activations");
    for (int r = 0; r < a->rows_padded / 32; ++r) {
      DtreeGemmArgs b = *a;
      b.rows_padded = 32;
      const size_t xo = (size_t)r * 32 * a->k;
      b.x = a->x + xo;
      b.x_lo = a->x_lo ? a->x_lo + xo : nullptr;
      if (a->out_f32) b.out_f32 = a->out_f32 + (size_t)r * 32 * a->ld_out_f32;
      if (a->out_bf16) {
        const size_t oo = (size_t)r * 32 * a->ld_out_bf16;  // tiled: ld_out_bf16 == width
        b.out_bf16 = a->out_bf16 + oo;
        b.out_lo = a->out_lo ? a->out_lo + oo : nullptr;
      }
      if (a->hidden_out) b.hidden_out = a->hidden_out + (size_t)r * 32 * a->ld_hidden;
      if (a->ss_in) b.ss_in = a->ss_in + (size_t)r * a->ss_tiles * 32;
      if (a->ss_out) b.ss_out = a->ss_out + (size_t)r * (a->n / 32) * 32;
      const int rc = dtree_gemm_bf16(&b, stream);
      if (rc) return rc;
    }
    return DTREE_OK;
  }
  if (q4) {
    DTREE_REQUIRE(a->x_layout == DTREE_W_TILED && a->rows_padded == 32 && a->split_k <= 0,
                  "gemm: q4 weights need tiled 32-row activations and split_k 0");
    DTREE_REQUIRE(a->w_scales && ((uintptr_t)a->w & 15) == 0 && ((uintptr_t)a->w_scales & 3) == 0,
                  "gemm: q4 weights need w (16-byte aligned) and w_scales (4-byte aligned)");
  } else {
    DTREE_REQUIRE(a->x_layout == a->w_layout, "gemm: x_layout must equal w_layout (both row-major or both tiled)");
  }
  p.w_sb = a->w_scales;
  DTREE_REQUIRE(!tiled || (a->ldx == a->k && a->rows_padded % 32 == 0), "gemm: tiled x needs ldx == k");
  // Ranged ring loads address w, w_sb and the activation planes with 32-bit
  // byte offsets below kOob.
  const size_t w_bytes = q4 ? (size_t)a->n * a->k / 2 : (size_t)a->n * a->k * 2;
  DTREE_REQUIRE(w_bytes < kOob, "gemm: weight matrix must be smaller than 2 GiB");
  p.w_bytes = (unsigned)w_bytes;
  p.sb_bytes = (unsigned)((size_t)a->n * (a->k / 64) * 4);
  p.x_bytes = (unsigned)((size_t)32 * a->k * 2);
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR || a->out_layout == DTREE_W_TILED ||
                    a->out_layout == DTREE_W_TILED_F16,
                "gemm: unknown out_layout");
  if (p.out_tiled && a->out_bf16) {
    const int width = epi == DTREE_EPI_SWIGLU ? a->n / 2 : a->n;
    DTREE_REQUIRE(a->ld_out_bf16 == width && width % 64 == 0, "gemm: tiled out needs ld_out_bf16 == width, width % 64");
  }
  // Automatic choice among the 32-row tiled schedules (split_k 0), from
  // measurements on MI355X with the weights streamed from HBM:
  // * K >= 4096 over N % 256 == 0: three workgroups per tile, one per part of
  //   K, when N / 32 * 3 <= CUs (o_proj N = 2560: 11.3 vs 16.1 us stream-K;
  //   down_proj N = 2560, K = 9728: 17.2 vs 20.2 us), else two at K = 4096
  //   (N = 4096: 12.6 vs 14.8 us; at K = 12288 stream-K wins, 24.6 vs 26.2);
  // * else K <= 4096 with at most one tile per CU: one workgroup per tile over
  //   the whole K, no cross-workgroup reduction tail (QKV N = 6144: 12.5 vs
  //   14.5 us stream-K);
  // * else stream-K: more tiles than CUs (N = 10240: 18.2 vs 22.7 us one per
  //   tile) or long K on narrow N.
  // q4 weights follow the same rule (dpq_gemm_kernel), measured against the
  // stream-K q4 kernels: QKV (N 6144, K 2560, high plane only) 8.0 vs 12.1 us,
  // o_proj 10.6 vs 15.3, down_proj 15.0 vs 18.4; and at K <= 4096 they take
  // one workgroup per tile also past the CU count: the Qwen3-4B q4 step with
  // gate/up (N 19456: 608 tiles) one per tile runs 2.18 ms, 2.31 ms with the
  // two-per-CU stream-K kernel (bf16 weights keep stream-K there: 2.88 vs
  // 2.91 ms for the bf16 step).
  const int auto_cus = device_cus();
  const bool k_auto = a->split_k == 0 && tiled && a->rows_padded == 32;
  const bool pairs_auto = k_auto && a->k >= 4096 && a->n % 256 == 0 &&
                          ((a->n / 32) * 3 <= auto_cus || (a->k == 4096 && (a->n / 32) * 2 <= auto_cus));
  const bool dp_auto = k_auto && !pairs_auto && a->k <= 4096 && (a->n / 32 <= auto_cus || q4);
  if (tiled && a->rows_padded == 32 && (a->split_k == -3 || a->split_k == -4 || pairs_auto)) {
    // Two (-3) or three (-4) workgroups per tile, one per part of K (see
    // dp_gemm_kernel).
    // automatic: three parts while the grid stays within one workgroup per CU
    // (o_proj: 240 workgroups, 11.4 us; two parts 11.9 us)
    const int dp_parts = a->split_k == -4 ? 3 : a->split_k == -3 ? 2 : (a->n / 32) * 3 <= auto_cus ? 3 : 2;
    DTREE_REQUIRE(a->n % 256 == 0 && nkb >= dp_parts,
                  "gemm: split_k -3 / -4 need n % 256 == 0 and k >= 64 * parts");
    const size_t need_pairs = dp_pair_workspace_bytes(a->n);
    DTREE_REQUIRE(a->workspace_bytes >= need_pairs, "gemm: workspace too small for the paired schedule");
    p.part_bytes = (unsigned)(need_pairs - kCounterBytes);
    if (dp_parts == 3) launch_dp_any<3>(p, epi, q4, h16, stream);
    else launch_dp_any<2>(p, epi, q4, h16, stream);
    DTREE_LAUNCH_CHECK("gemm launch");
    return DTREE_OK;
  }
  if (tiled && a->rows_padded == 32 && (a->split_k == -1 || dp_auto)) {
    launch_dp_any<1>(p, epi, q4, h16, stream);
    DTREE_LAUNCH_CHECK("gemm launch");
    return DTREE_OK;
  }
  if (tiled && a->rows_padded == 32 && (a->split_k == 0 || a->split_k == -2 || q4)) {
    const int cus = device_cus();
    const int nblk = a->n / 64;
    p.T = nblk * nkb;
    const int g2 = q4 ? sk2_grid(p.T, nkb, cus < kSkMaxGrid ? cus : kSkMaxGrid) : 0;
    p.G = g2 ? g2 : sk_grid(p.T, nkb, cus < kSkMaxGrid ? cus : kSkMaxGrid);
    DTREE_REQUIRE((long long)p.T * p.G < (1LL << 31), "gemm: too many 64 x 64 units for the stream-K schedule");
    const size_t need_sk = sk_workspace_bytes(a->n, a->k, cus < kSkMaxGrid ? cus : kSkMaxGrid);
    DTREE_REQUIRE(a->workspace_bytes >= need_sk, "gemm: workspace too small for the stream-K schedule");
    p.part_bytes = (unsigned)(need_sk - kCounterBytes);
    if (q4 && g2) {
      if (p.x_lo) launch_sk2<true>(p, epi, stream);
      else launch_sk2<false>(p, epi, stream);
    } else if (q4) {
      if (p.x_lo) launch_sk<true, true>(p, epi, stream);
      else launch_sk<false, true>(p, epi, stream);
    } else if (h16) {
      launch_sk<false, false, true>(p, epi, stream);
    } else {
      if (p.x_lo) launch_sk<true, false>(p, epi, stream);
      else launch_sk<false, false>(p, epi, stream);
    }
    DTREE_LAUNCH_CHECK("gemm launch");
    return DTREE_OK;
  }
  switch (a->rows_padded) {
    case 32: launch_gemm<1>(p, epi, blocks, stream, tiled, h16); break;
    case 64: launch_gemm<2>(p, epi, blocks, stream, tiled, h16); break;
    case 96: launch_gemm<3>(p, epi, blocks, stream, tiled, h16); break;
    default: launch_gemm<4>(p, epi, blocks, stream, tiled, h16); break;
  }
  DTREE_LAUNCH_CHECK("gemm launch");
  return DTREE_OK;
}

extern "C" int dtree_gemm_long(const DtreeGemmArgs* a, hipStream_t stream) {
  DTREE_REQUIRE(a, "gemm_long: null args");
  DTREE_REQUIRE(a->x && a->w, "gemm_long: null x or w");
  const bool q4 = a->w_layout == DTREE_W_Q4G64;
  const bool h16 = a->x_layout == DTREE_W_TILED_F16;
  DTREE_REQUIRE((a->x_layout == DTREE_W_TILED && (a->w_layout == DTREE_W_TILED || q4)) ||
                    (h16 && a->w_layout == DTREE_W_TILED_F16),
                "gemm_long: tiled bf16 activations with tiled bf16 or q4 group-64 weights, or TILED_F16 both");
  DTREE_REQUIRE(!q4 || (a->w_scales && ((uintptr_t)a->w_scales & 15) == 0),
                "gemm_long: q4 weights need w_scales (16-byte aligned)");
  DTREE_REQUIRE(a->rows_padded >= kLongRows && a->rows_padded % kLongRows == 0 && a->rows_padded <= (1 << 20),
                "gemm_long: rows_padded must be a positive multiple of 128");
  const int epi = a->epilogue;
  DTREE_REQUIRE(a->n > 0 && (a->n % kLongCols == 0 || (a->n % 64 == 0 && epi == DTREE_EPI_STORE_F32)),
                "gemm_long: n must be a positive multiple of 128 (of 64 with the fp32 store epilogue)");
  DTREE_REQUIRE(a->k > 0 && a->k % 64 == 0 && a->ldx == a->k, "gemm_long: k a multiple of 64, ldx == k");
  DTREE_REQUIRE(epi >= 0 && epi <= 3, "gemm_long: unknown epilogue");
  if (epi == DTREE_EPI_STORE_F32 || epi == DTREE_EPI_RESIDUAL)
    DTREE_REQUIRE(a->out_f32 && a->ld_out_f32 >= a->n, "gemm_long: out_f32 missing or ld too small");
  if (epi == DTREE_EPI_RESIDUAL)
    DTREE_REQUIRE(a->out_bf16 && a->next_norm && a->ss_out && a->ld_out_bf16 >= a->n,
                  "gemm_long: residual epilogue needs out_bf16, next_norm, ss_out");
  if (epi == DTREE_EPI_SWIGLU)
    DTREE_REQUIRE(a->out_bf16 && a->ld_out_bf16 >= a->n / 2, "gemm_long: swiglu needs out_bf16 (n/2 wide)");
  if (epi == DTREE_EPI_STORE_BF16) DTREE_REQUIRE(a->out_bf16 && a->ld_out_bf16 >= a->n, "gemm_long: out_bf16");
  if (a->hidden_out) DTREE_REQUIRE(a->ld_hidden >= a->n, "gemm_long: ld_hidden too small");
  if (a->ss_in) DTREE_REQUIRE(a->ss_tiles > 0 && a->norm_dim > 0, "gemm_long: ss_in needs ss_tiles and norm_dim");
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR || a->out_layout == DTREE_W_TILED ||
                    a->out_layout == DTREE_W_TILED_F16,
                "gemm_long: unknown out_layout");
  if (a->out_layout != DTREE_W_ROWMAJOR && a->out_bf16) {
    const int width = epi == DTREE_EPI_SWIGLU ? a->n / 2 : a->n;
    DTREE_REQUIRE(a->ld_out_bf16 == width && width % 64 == 0,
                  "gemm_long: tiled out needs ld_out_bf16 == width, width % 64");
  }
  DTREE_REQUIRE(((uintptr_t)a->x & 15) == 0 && ((uintptr_t)a->x_lo & 15) == 0 && ((uintptr_t)a->w & 15) == 0,
                "gemm_long: x, x_lo and w must be 16-byte aligned");
  GemmParams p{};
  p.x = a->x; p.x_lo = h16 ? nullptr : a->x_lo; p.ldx = a->ldx; p.w = a->w; p.n = a->n; p.k = a->k;
  p.ss_in = a->ss_in; p.ss_tiles = a->ss_tiles;
  p.inv_norm_dim = a->norm_dim > 0 ? 1.0f / (float)a->norm_dim : 1.f; p.eps = a->eps;
  p.out_f32 = a->out_f32; p.ld_out_f32 = a->ld_out_f32;
  p.out_tiled = a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16;
  p.out_h16 = a->out_layout == DTREE_W_TILED_F16;
  p.out_bf16 = a->out_bf16; p.out_lo = p.out_h16 ? nullptr : a->out_lo; p.ld_out_bf16 = a->ld_out_bf16;
  p.next_norm = a->next_norm; p.ss_out = a->ss_out;
  p.hidden_out = a->hidden_out; p.ld_hidden = a->ld_hidden;
  const long long grid = (long long)(a->rows_padded / kLongRows) * ((a->n + kLongCols - 1) / kLongCols);
  DTREE_REQUIRE(grid < (1LL << 31), "gemm_long: grid too large");
  p.w_sb = a->w_scales;
  if (p.x_lo) launch_long<true>(p, epi, (int)grid, q4, h16, stream);
  else launch_long<false>(p, epi, (int)grid, q4, h16, stream);
  DTREE_LAUNCH_CHECK("gemm_long launch");
  return DTREE_OK;
}

extern "C" size_t dtree_lmhead_candidates_bytes(int32_t rows_padded) {
  return (size_t)1024 * rows_padded * sizeof(int2);
}

extern "C" int dtree_lmhead_candidate_blocks(int32_t vocab, int32_t rows_padded) {
  const int tn = tile_cols(rows_padded);
  return lmhead_grid(vocab / tn);
}

extern "C" int dtree_lmhead_argmax(const uint16_t* x, const uint16_t* x_lo, int32_t x_layout, int32_t ldx,
                                   int32_t rows_padded,
                                   const uint16_t* emb, int32_t emb_layout, const uint16_t* emb_scales,
                                   int32_t vocab, int32_t hidden, const float* ss_in,
                                   int32_t ss_tiles, float eps, float* logits, void* candidates,
                                   hipStream_t stream) {
  DTREE_REQUIRE(x && emb && candidates, "lmhead: null pointer");
  DTREE_REQUIRE(rows_padded == 32 || rows_padded == 64 || rows_padded == 96 || rows_padded == 128,
                "lmhead: rows_padded must be 32, 64, 96 or 128");
  const int tn = tile_cols(rows_padded);
  DTREE_REQUIRE(vocab > 0 && vocab % tn == 0, "lmhead: vocab must be a multiple of 64 (32 for > 64 rows)");
  DTREE_REQUIRE(hidden > 0 && hidden % 64 == 0 && ldx >= hidden, "lmhead: hidden must be a multiple of 64");
  LmParams p{};
  p.x = x; p.x_lo = x_lo; p.ldx = ldx; p.w = emb; p.w_sb = emb_scales; p.vocab = vocab; p.k = hidden;
  p.ntiles = vocab / tn;
  p.ss_in = ss_in; p.ss_tiles = ss_tiles; p.inv_norm_dim = 1.0f / (float)hidden; p.eps = eps;
  p.logits = logits; p.cand = reinterpret_cast<int2*>(candidates);
  const int grid = lmhead_grid(p.ntiles);
  p.cand_blocks = grid;
  DTREE_REQUIRE(emb_layout == DTREE_W_ROWMAJOR || emb_layout == DTREE_W_TILED || emb_layout == DTREE_W_TILED_F16 ||
                    emb_layout == DTREE_W_Q4G64,
                "lmhead: unknown emb_layout");
  if (emb_layout == DTREE_W_Q4G64) {
    DTREE_REQUIRE(x_layout == DTREE_W_TILED && ldx == hidden && hidden <= 4096,
                  "lmhead: q4 embedding needs tiled x and hidden <= 4096");
    DTREE_REQUIRE(emb_scales && ((uintptr_t)emb & 15) == 0, "lmhead: q4 embedding needs emb_scales");
    DTREE_REQUIRE(vocab % 64 == 0, "lmhead: q4 embedding needs vocab % 64 == 0");
    if ((vocab / 64 + 3) / 4 <= grid && q4m_enabled()) {
      // One pass over the q4 embedding for every row block: the one-pass q4
      // GEMM kernel with its LM-head epilogue, 4 64-column blocks per
      // workgroup, one workgroup per candidate block (the ones past the
      // vocab's tiles report empty candidates). Also at 32 rows, where the
      // activations staged once per K group in LDS serve the four column
      // blocks (Qwen3-4B: 103 vs 172 us for the 32-row kernel below).
      DTREE_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)x_lo & 15) == 0 && ((uintptr_t)emb_scales & 3) == 0,
                    "lmhead: q4 operands misaligned");
      const size_t xb = (size_t)rows_padded * hidden * 2, wb = (size_t)vocab * hidden / 2;
      DTREE_REQUIRE(xb < kOob && wb < kOob, "lmhead: operands must be smaller than 2 GiB");
      GemmParams g{};
      g.x = x; g.x_lo = x_lo; g.ldx = hidden; g.w = emb; g.w_sb = emb_scales; g.n = vocab; g.k = hidden;
      g.S = 1;
      g.ss_in = ss_in; g.ss_tiles = ss_tiles; g.inv_norm_dim = 1.0f / (float)hidden; g.eps = eps;
      g.x_bytes = (unsigned)xb; g.w_bytes = (unsigned)wb; g.sb_bytes = (unsigned)((size_t)vocab * (hidden / 64) * 4);
      g.lm_logits = logits; g.lm_cand = p.cand; g.lm_blocks = grid;
      if (x_lo) launch_q4m_lm<true>(g, rows_padded / 32, grid, stream);
      else launch_q4m_lm<false>(g, rows_padded / 32, grid, stream);
      DTREE_LAUNCH_CHECK("lmhead launch");
      return DTREE_OK;
    }
    // Vocabularies past the one-pass grid (more than 4 x 64 x 1024 = 262144
    // entries) or DTREE_Q4M=0: one pass of the 32-row kernel per 32-row block (tiled x,
    // statistics and candidates are contiguous per block; logits rows are
    // row-major). The kernel walks 64-column tiles; the grid stays the
    // candidate block count of this row count (workgroups past the tiles
    // write empty candidates).
    p.ntiles = vocab / 64;
    for (int r = 0; r < rows_padded / 32; ++r) {
      LmParams pb = p;
      pb.x = x + (size_t)r * 32 * hidden;
      pb.x_lo = x_lo ? x_lo + (size_t)r * 32 * hidden : nullptr;
      pb.ss_in = ss_in ? ss_in + (size_t)r * ss_tiles * 32 : nullptr;
      pb.logits = logits ? logits + (size_t)r * 32 * vocab : nullptr;
      pb.cand = p.cand + (size_t)r * grid * 32;
      launch_lm_q4(pb, grid, stream);
    }
    DTREE_LAUNCH_CHECK("lmhead launch");
    return DTREE_OK;
  }
  DTREE_REQUIRE(x_layout == emb_layout, "lmhead: x_layout must equal emb_layout");
  const bool h16 = emb_layout == DTREE_W_TILED_F16;
  const bool tiled = emb_layout == DTREE_W_TILED || h16;
  DTREE_REQUIRE(!tiled || ldx == hidden, "lmhead: tiled x needs ldx == hidden");
  if (h16) p.x_lo = nullptr;  // one fp16 plane
  switch (rows_padded) {
    case 32: launch_lm<1>(p, grid, stream, tiled, h16); break;
    case 64: launch_lm<2>(p, grid, stream, tiled, h16); break;
    case 96: launch_lm<3>(p, grid, stream, tiled, h16); break;
    default: launch_lm<4>(p, grid, stream, tiled, h16); break;
  }
  DTREE_LAUNCH_CHECK("lmhead launch");
  return DTREE_OK;
}
