// Ancestor-masked GQA tree attention over a paged bf16 KV prefix, one
// workgroup per (KV group, 32-row query block, key split).
//
// Work split
//   * A KV group's G query heads read the same keys (GQA h -> h / G,
//     qwen3_tree.py:69-76), so a workgroup owns one KV group: G waves, wave w
//     computing query head g*G + w. Each K/V chunk is loaded from HBM once
//     per workgroup into LDS and read by the G waves' MFMAs (for the Qwen3-4B
//     step: 25 tree rows x 4 heads per chunk).
//   * Keys are cut into chunks: 64-key prefix pages at head_dim 128 (32 keys,
//     half a page, at 256), and 32-key tree chunks (tree chunk t = nodes
//     32t .. 32t+31, masked with word t of each query's ancestor bitset).
//     Split 0 of a (group, query block) takes the tree chunks 0 .. rb (later
//     tree chunks hold no ancestor of a row of block rb); split s >= 1 takes
//     the prefix chunks (s-1)*cps .. s*cps - 1 below P. The mapping depends on
//     the grid only, so the first chunk's loads go out before the step
//     descriptor (which holds P and L, so one grid serves every step up to
//     max_past_length) is read; chunks run through two LDS buffers, the next
//     chunk's loads in flight while the current one is multiplied, each wave
//     keeping an online softmax.
//   * Every split publishes one partial per head (unnormalised output, row
//     max, row sum). The S workgroups of a (group, query block) then meet at
//     a device-scope counter (all of them are resident: the grid never holds
//     more workgroups than the GPU has CUs) and share the combine: unit
//     (head, 32-dim block) u goes to workgroup u mod S, whose waves read the
//     splits' 4 KB slices of that unit, merge them in LDS in wave order
//     (deterministic) and write the output rows (normalised, optionally
//     gated, as a bf16 hi / lo pair). The counter's second phase returns it
//     to zero for the next launch. The wait is bounded: a workgroup that
//     gives up sets the workspace's error word instead of hanging.
//
// MFMA use (v_mfma_f32_32x32x16_f16, fp32 accumulate), tree rows as the
// 32-wide B dimension. The cached bf16 K and V convert exactly to fp16 (fp16
// keeps more significand bits; magnitudes above 65504 saturate), and q and the
// probabilities round to fp16 (11 significant bits, against bf16's 8):
//   S^T = K Q^T : A = 32 keys x 16 dims (LDS), B = 16 dims x 32 queries
//                 (registers), so each lane owns one query column and its
//                 softmax statistics stay lane-local (plus one exchange with
//                 lane ^ 32).
//   O^T = V^T P^T: A = V^T (32 dims x 16 keys, LDS), B = P^T straight from the
//                 S^T registers: A-row rho of S^T is loaded from key rho with
//                 bits 2 and 3 swapped, so register r of a lane in half h
//                 holds key 16*(r/8) + 8*h + r%8, eight consecutive keys per
//                 PV step.
// K pages are [page][kv_head][64][D]; V pages are [page][kv_head][D][64].
#include <cstdlib>
#include <mutex>

#include "common.h"

namespace dtree {

constexpr int kMaxPast = 16384;  // longest prefix the grid is sized for
__host__ __device__ constexpr int chunk_keys(int D) { return D <= 128 ? DTREE_PAGE : DTREE_PAGE / 2; }
constexpr float kNeg = -1e30f;
constexpr float kLog2e = 1.4426950408889634f;
// Workspace header (kAttnWsHeader): error word (bytes 0..3), then one counter
// per (group, query block) from byte 64; the per-head kernel's flag exchange
// region follows, then this kernel's partials.
constexpr int kWsHeader = (int)kAttnWsHeader;
constexpr int kMaxPairs = (kWsHeader - 64) / 4;
constexpr int kCombineBatch = 4;     // split slices in flight per wave in the combine

struct AttnParams {
  const float* qkv; int ld_qkv;
  int q_stride, k_off, v_off;  // qkv row: q of head h at h*q_stride (gate at +D), k / v of group g at k_off / v_off + g*D
  const uint16_t* q_norm; const uint16_t* k_norm; float eps;
  const float* rope_cos; const float* rope_sin;
  uint16_t* kp; uint16_t* vp; const int* page_table;
  const DtreeStepDesc* desc;
  uint16_t* out; uint16_t* out_lo; int ld_out; int out_tiled;
  int out_h16;  // DTREE_W_TILED_F16 output: one fp16 plane
  int Hq, Hkv, NT;       // NT: 32-row query blocks = 32-key tree chunks
  int S, max_pchunks;    // splits per (group, query block); prefix chunks the grid is sized for
  int cps;               // prefix chunks per split
  int max_past;          // longest prefix the cache and page table hold
  float scale_log2;
  int write_cache;
  float* part; int* counters; int* err;
  int spin_limit;  // counter polls before a workgroup gives up
  int off_xcd;  // test hook: treat every workgroup as off its expected XCD
};

__device__ __forceinline__ int swap_bits23(int c) { return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1); }

// Raw operands of one head row for lane (c, h), which owns dims 16j + 8h + i:
// the fp32 values, the bf16 RMSNorm weights and the RoPE cos/sin of the first
// half of the R rotated dims, all loads issued before any use.
template <int D, int R>
struct HeadRow {
  f32x4_t x[D / 16][2];
};

// The block's 32 RoPE table rows (cos then sin, R/2 each) and the q_norm
// weight, loaded once per workgroup and shared by its waves through LDS
// (the waves' query heads use the same positions and weight).
template <int D, int R, int NT_>
struct QAux {
  static constexpr int kRope = 32 * (R / 2) * 2;  // floats
  static constexpr int kPieces = kRope / 4;       // 16-byte pieces
  static constexpr int PT = (kPieces + NT_ - 1) / NT_;
  static constexpr int kBytes = kRope * 4 + D * 2;
  f32x4_t r[PT];
  u32x4_t nw;

  __device__ __forceinline__ void issue(const AttnParams& p, int rb, int t) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int e = t + i * NT_;
      if (e < kPieces) {
        const int half = e / (kPieces / 2), o = e % (kPieces / 2);  // cos rows, then sin rows
        r[i] = *reinterpret_cast<const f32x4_t*>((half ? p.rope_sin : p.rope_cos) + 32 * rb * (R / 2) + 4 * o);
      }
    }
    if (t < D / 8) nw = p.q_norm ? ld_u32x4(p.q_norm + 8 * t) : u32x4_t{0u, 0u, 0u, 0u};
  }
  __device__ __forceinline__ void commit(unsigned char* lds, int t) const {
    f32x4_t* ro = reinterpret_cast<f32x4_t*>(lds);
#pragma unroll
    for (int i = 0; i < PT; ++i)
      if (t + i * NT_ < kPieces) ro[t + i * NT_] = r[i];
    if (t < D / 8) reinterpret_cast<u32x4_t*>(lds + kRope * 4)[t] = nw;
  }
};

template <int D, int R>
__device__ __forceinline__ void row_issue(HeadRow<D, R>& r, const float* src, int h) {
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    r.x[j][0] = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h);
    r.x[j][1] = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h + 4);
  }
}

// RMSNorm over D (sum of squares completed with the partner lane ^ 32), RoPE
// on (d, d + R/2) for d < R/2 (registers j and j + R/32 of the same lane),
// then the B-operand fragments in fp16.
template <int D, int R>
__device__ __forceinline__ void q_fragments(const HeadRow<D, R>& qr, const unsigned char* aux, bool norm, float eps,
                                            int c, int h, u32x4_t (&qf)[D / 16]) {
  constexpr int NJ = D / 16;
  const float* rope = reinterpret_cast<const float*>(aux);  // [cos | sin][32 rows][R/2]
  const uint16_t* nwl = reinterpret_cast<const uint16_t*>(aux + 32 * (R / 2) * 2 * 4);
  float v[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[j][i] = qr.x[j][0][i];
      v[j][i + 4] = qr.x[j][1][i];
    }
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
    ss += __shfl_xor(ss, 32);
    const float rs = rsqrtf(ss * (1.0f / D) + eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const u32x4_t nw = *reinterpret_cast<const u32x4_t*>(nwl + 16 * j + 8 * h);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = nw[i >> 1];
        v[j][i] *= rs * __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
      }
    }
  }
  constexpr int RJ = R / 32;
#pragma unroll
  for (int j = 0; j < RJ; ++j) {
    const f32x4_t* cr = reinterpret_cast<const f32x4_t*>(rope + c * (R / 2) + 16 * j + 8 * h);
    const f32x4_t* sr = reinterpret_cast<const f32x4_t*>(rope + (32 + c) * (R / 2) + 16 * j + 8 * h);
    const f32x4_t cs0 = cr[0], cs1 = cr[1], sn0 = sr[0], sn1 = sr[1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float cs = i < 4 ? cs0[i & 3] : cs1[i & 3], sn = i < 4 ? sn0[i & 3] : sn1[i & 3];
      const float x1 = v[j][i], x2 = v[j + RJ][i];
      v[j][i] = x1 * cs - x2 * sn;
      v[j + RJ][i] = x1 * sn + x2 * cs;
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    qf[j] = u32x4_t{pack_h2(v[j][0], v[j][1]), pack_h2(v[j][2], v[j][3]), pack_h2(v[j][4], v[j][5]),
                    pack_h2(v[j][6], v[j][7])};
}

// ---- tree K/V rows: 8 threads per node ------------------------------------
// Thread part j of a node row owns, for head_dim 128 (RoPE pairs (d, d + 64)),
// dims 8j .. 8j+7 and 64+8j .. +7; for head_dim 256 (RoPE on dims 0..63,
// pairs (d, d + 32)) dims 4j .. 4j+3, 32+4j .. +3 and the unrotated
// 64+24j .. 64+24j+23. Each RoPE pair stays in one thread; the RMSNorm sum
// of squares is completed over the row's 8 threads with DPP.
template <int D>
__device__ __forceinline__ int row8_dim(int j, int i) {
  if constexpr (D == 128) return i < 8 ? 8 * j + i : 64 + 8 * j + (i - 8);
  else return i < 4 ? 4 * j + i : (i < 8 ? 32 + 4 * j + (i - 4) : 64 + 24 * j + (i - 8));
}

template <int D>
struct Row8 {
  static constexpr int NV = D / 8;
  f32x4_t x[NV / 4];
  u32x2_t nw[NV / 4];
  f32x4_t cs[D == 128 ? 2 : 1], sn[D == 128 ? 2 : 1];
};

template <int D>
__device__ __forceinline__ void row8_issue(Row8<D>& r, const float* src, const uint16_t* norm_w, const float* cosr,
                                           const float* sinr, int j, bool aux) {
  const uint16_t* nwp = norm_w ? norm_w : reinterpret_cast<const uint16_t*>(src);
#pragma unroll
  for (int k = 0; k < Row8<D>::NV / 4; ++k) {
    const int d0 = row8_dim<D>(j, 4 * k);
    r.x[k] = *reinterpret_cast<const f32x4_t*>(src + d0);
    if (aux) r.nw[k] = *reinterpret_cast<const u32x2_t*>(nwp + d0);
  }
  if (aux) {
    if constexpr (D == 128) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        r.cs[u] = *reinterpret_cast<const f32x4_t*>(cosr + 8 * j + 4 * u);
        r.sn[u] = *reinterpret_cast<const f32x4_t*>(sinr + 8 * j + 4 * u);
      }
    } else {
      r.cs[0] = *reinterpret_cast<const f32x4_t*>(cosr + 4 * j);
      r.sn[0] = *reinterpret_cast<const f32x4_t*>(sinr + 4 * j);
    }
  }
}

template <int D>
__device__ __forceinline__ void row8_finish(const Row8<D>& r, bool norm, bool rope, float eps,
                                            float (&v)[Row8<D>::NV]) {
  constexpr int NV = Row8<D>::NV;
#pragma unroll
  for (int k = 0; k < NV / 4; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) v[4 * k + i] = r.x[k][i];
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) ss += v[i] * v[i];
    ss += dpp<0xB1>(ss);   // lane ^ 1
    ss += dpp<0x4E>(ss);   // lane ^ 2
    ss += dpp<0x141>(ss);  // the other quad of the row's 8 lanes
    const float rs = rsqrtf(ss * (1.0f / D) + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t w = r.nw[i >> 2][(i & 3) >> 1];
      v[i] *= rs * __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
    }
  }
  if (rope) {
    constexpr int NR = D == 128 ? 8 : 4;  // rotated pairs per thread
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const float cs = D == 128 ? r.cs[i >> 2][i & 3] : r.cs[0][i & 3];
      const float sn = D == 128 ? r.sn[i >> 2][i & 3] : r.sn[0][i & 3];
      const float x1 = v[i], x2 = v[NR + i];
      v[i] = x1 * cs - x2 * sn;
      v[NR + i] = x1 * sn + x2 * cs;
    }
  }
}

// Tree chunk tc into an LDS buffer (K rows [32][KS], V^T [D][VS], fp16 of
// the bf16 cache values): k = RoPE(k_norm(k)), v raw, from the fused qkv rows
// of nodes 32tc .. +31 (zero past the tree); the writer also appends the rows
// to the paged cache at positions P + node (qwen3_tree.py:146). issue() only
// reads the qkv rows, weights and RoPE table, so it can run before the step
// descriptor arrives; commit() needs P and L.
template <int D, int R, int TPS>
struct TreeStage {
  static constexpr int NTI = TPS >= 256 ? 1 : 256 / TPS;  // (node, part) units per thread
  Row8<D> kr[NTI], vr[NTI];

  __device__ __forceinline__ void issue(const AttnParams& p, int tc, int g, int ts) {
#pragma unroll
    for (int it = 0; it < NTI; ++it) {
      const int e = ts + it * TPS;
      if (e < 256) {
        const int node = 32 * tc + (e >> 3), j = e & 7;
        const float* row = p.qkv + (size_t)node * p.ld_qkv;
        row8_issue<D>(kr[it], row + p.k_off + g * D, p.k_norm, p.rope_cos + node * (R / 2),
                      p.rope_sin + node * (R / 2), j, true);
        row8_issue<D>(vr[it], row + p.v_off + g * D, nullptr, nullptr, nullptr, j, false);
      }
    }
  }

  template <int KS, int VS>
  __device__ __forceinline__ void commit(const AttnParams& p, int tc, int g, int P, int L, int ts, uint16_t* ks,
                                         uint16_t* vt, bool write) {
    constexpr int NV = D / 8;
#pragma unroll
    for (int it = 0; it < NTI; ++it) {
      const int e = ts + it * TPS;
      if (e >= 256) continue;
      const int nl = e >> 3, j = e & 7;
      const int node = 32 * tc + nl;
      float kv[NV], vv[NV];
      row8_finish<D>(kr[it], p.k_norm != nullptr, true, p.eps, kv);
      row8_finish<D>(vr[it], false, false, 0.f, vv);
      const bool live = node < L;
      uint16_t kb[NV], vb[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        kb[i] = live ? f2bf(kv[i]) : (uint16_t)0;
        vb[i] = live ? f2bf(vv[i]) : (uint16_t)0;
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        // the MFMA operands are the cached bf16 values, converted exactly to fp16
        const int d = row8_dim<D>(j, i);
        ks[nl * KS + d] = (uint16_t)(bf2_to_h2(kb[i]) & 0xffffu);
        vt[d * VS + nl] = (uint16_t)(bf2_to_h2(vb[i]) & 0xffffu);
      }
      if (write && live) {
        // Buffer stores over the layer's cache pages: per lane one row offset
        // plus the j-dependent part of the dim (dim = A(i) + B(i) j, B 4 / 8
        // or 24), the constant A(i) part in the scalar offset, so no per-dim
        // 64-bit address is held across the chunk loop. K dims come in runs of
        // four consecutive dims (8-byte stores); V^T is one 2-byte store per
        // dim (stride DTREE_PAGE).
        const int pos = P + node;
        const int page = p.page_table[pos / DTREE_PAGE], off = pos % DTREE_PAGE;
        // (one resource for the whole layer cache, uniform across the lanes;
        // a layer's pages stay below 2 GiB)
        const __amdgpu_buffer_rsrc_t kr = buf_rsrc(p.kp, 0x7ffffff0u);
        const __amdgpu_buffer_rsrc_t vr = buf_rsrc(p.vp, 0x7ffffff0u);
        const int blk = (page * p.Hkv + g) * DTREE_PAGE * D * 2;  // byte offset of the (page, head) block
        // The dims' offsets are computed here, next to their stores: j is
        // made opaque so they are not hoisted out of the chunk loop, where
        // NV of them would stay live across the MFMA registers.
        int jj = j;
        asm volatile("" : "+v"(jj));
#pragma unroll
        for (int i = 0; i < NV; i += 4) {
          // four consecutive dims from a multiple of 4: one 8-byte run of K
          const u32x2_t w = {(uint32_t)kb[i] | ((uint32_t)kb[i + 1] << 16),
                             (uint32_t)kb[i + 2] | ((uint32_t)kb[i + 3] << 16)};
          __builtin_amdgcn_raw_buffer_store_b64(w, kr, blk + 2 * kv_k_off(off, row8_dim<D>(jj, i), D), 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NV; ++i)
          __builtin_amdgcn_raw_buffer_store_b16(vb[i], vr, blk + 2 * kv_v_off(off, row8_dim<D>(jj, i), D), 0, 0);
      }
    }
  }
};

// Prefix chunk pc (CK keys of one page) into an LDS buffer: K rows and V^T
// columns in 16-byte pieces, every load of the workgroup's threads in flight
// together; keys at or past P (stale rows of the last page) are zeroed.
// The page block stores K and V in MFMA-fragment order (kv_k_off /
// kv_v_off), and the chunk's K and its V are each one contiguous run of
// kilobytes (from key half po / 32, resp. key step po / 16). Wavefront f's
// kilobyte of K is fragment (key half f / NJ, dim step j = f % NJ): lane rem
// holds key 32 (f / NJ) + pi(rem % 32) of the chunk, dims 16 j + 8 (rem / 32)
// .. +7. Its kilobyte of V is key step f / ND, dim block db = f % ND: dim
// 32 db + rem % 32, keys 16 (f / ND) + 8 (rem / 32) .. +7 of the chunk.
// issue() needs only the chunk index (the page table is read there), commit()
// needs P.
template <int D, int TPS>
struct PrefixStage {
  static constexpr int CK = chunk_keys(D);
  static constexpr int NJ = D / 16, ND = D / 32;
  static constexpr int PK = CK * D / 8 / TPS;  // 16-byte pieces of K (and of V^T) per thread
  static_assert(PK * TPS == CK * D / 8 && TPS % 64 == 0, "whole wavefronts cover the chunk");
  u32x4_t kv[PK], vv[PK];

  // Physical page of chunk pc, read through the scalar cache (pc is uniform):
  // waiting for it does not wait for the vector loads issued before it.
  __device__ __forceinline__ static int page_of(const AttnParams& p, int pc) {
    typedef const __attribute__((address_space(4))) int* const_int_ptr;  // constant address space: s_load
    return ((const_int_ptr)(uintptr_t)p.page_table)[pc * CK / DTREE_PAGE];
  }
  // The wave index (ts / 64) is uniform: the kilobyte each wavefront load
  // reads is a scalar; only the lane's 16-byte slot in it is per lane.
  __device__ __forceinline__ void issue(const AttnParams& p, int pc, int page, int g, int ts) {
    const int po = (pc * CK) % DTREE_PAGE;
    const size_t blk = (size_t)(page * p.Hkv + g) * DTREE_PAGE * D;
    const __amdgpu_buffer_rsrc_t kr = buf_rsrc(p.kp + blk, (unsigned)(DTREE_PAGE * D * 2));
    const __amdgpu_buffer_rsrc_t vr = buf_rsrc(p.vp + blk, (unsigned)(DTREE_PAGE * D * 2));
    const int w = __builtin_amdgcn_readfirstlane(ts >> 6), lo = 16 * (ts & 63);
#pragma unroll
    for (int i = 0; i < PK; ++i) {
      const int f = w + i * (TPS / 64);  // this wavefront's kilobyte of the chunk
      kv[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, lo, 1024 * ((po / 32) * NJ + f), kNt);
      vv[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, lo, 1024 * ((po / 16) * ND + f), kNt);
    }
  }

  template <int KS, int VS>
  __device__ __forceinline__ void commit(int pc, int P, int ts, uint16_t* ks, uint16_t* vt) const {
    const int kend = P - pc * CK;  // keys >= kend are past the prefix
    const int w = __builtin_amdgcn_readfirstlane(ts >> 6), rem = ts & 63;
    const int kl = kv_pi(rem & 31), hl = 8 * (rem >> 5);  // the lane's key row (pi) and 8-element half
#pragma unroll
    for (int i = 0; i < PK; ++i) {
      const int f = w + i * (TPS / 64);
      const int key = 32 * (f / NJ) + kl, kcol = 16 * (f % NJ) + hl;
      *reinterpret_cast<u32x4_t*>(ks + key * KS + kcol) = key < kend ? bf8_to_h8(kv[i]) : u32x4_t{0u, 0u, 0u, 0u};
      const int dim = 32 * (f % ND) + (rem & 31), k0 = 16 * (f / ND) + hl;
      u32x4_t v = vv[i];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo_ok = (k0 + 2 * q) < kend ? 0xffffu : 0u;
        const uint32_t hi_ok = (k0 + 2 * q + 1) < kend ? 0xffff0000u : 0u;
        v[q] &= lo_ok | hi_ok;
      }
      *reinterpret_cast<u32x4_t*>(vt + dim * VS + k0) = bf8_to_h8(v);
    }
  }
};

// One chunk of NBK 32-key blocks from LDS for this wave's head: S^T = K Q^T,
// scale and mask, online softmax update (running max m, lane-partial row sum
// l, output rescaled when the max grows), O^T += V^T P^T. TREE: key k of
// block 0 is tree node 32 tc + k, visible when bit k of the query's ancestor
// word is set; else prefix keys >= kend are masked.
// The query fragments come from QF: q(j) returns fragment j, from registers
// (QRegs) or, at head_dim 256 where registers run out, from the wave's copy in
// LDS (QLds, read one dims-step ahead like the K fragments).
template <int D>
struct QRegs {
  const u32x4_t (&qf)[D / 16];
  __device__ __forceinline__ u32x4_t operator()(int j) const { return qf[j]; }
};
struct QLds {
  const u32x4_t* q;  // this wave's fragments: [j][lane]
  int lane;
  __device__ __forceinline__ u32x4_t operator()(int j) const { return q[j * 64 + lane]; }
};

template <int D, int NBK, int KS, int VS, bool TREE, typename QF>
__device__ __forceinline__ void attend_chunk(const uint16_t* ks, const uint16_t* vt, const QF& qf,
                                             float scale_log2, int kend, uint32_t anc,
                                             bool qlive, int c, int h, float& m_run, float& l_run,
                                             f32x16_t (&o)[D / 32]) {
  constexpr int NJ = D / 16, ND = D / 32;
  f32x16_t s[NBK];
#pragma unroll
  for (int b = 0; b < NBK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[b][r] = 0.f;
  const int krow = swap_bits23(c);
  // K (and q) fragments are read one dims-step ahead of their MFMAs (not all
  // at once: registers for two waves per SIMD).
  u32x4_t a[2][NBK], qn[2];
#pragma unroll
  for (int b = 0; b < NBK; ++b) a[0][b] = *reinterpret_cast<const u32x4_t*>(ks + (32 * b + krow) * KS + 8 * h);
  qn[0] = qf(0);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (j + 1 < NJ) {
#pragma unroll
      for (int b = 0; b < NBK; ++b)
        a[(j + 1) & 1][b] = *reinterpret_cast<const u32x4_t*>(ks + (32 * b + krow) * KS + 16 * (j + 1) + 8 * h);
      qn[(j + 1) & 1] = qf(j + 1);
    }
#pragma unroll
    for (int b = 0; b < NBK; ++b) s[b] = mfma32_f16(a[j & 1][b], qn[j & 1], s[b]);
    __builtin_amdgcn_sched_barrier(0);
  }
  float bmax = kNeg;
#pragma unroll
  for (int b = 0; b < NBK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 32 * b + 16 * (r >> 3) + 8 * h + (r & 7);
      const bool ok = TREE ? (qlive && key < kend && ((anc >> key) & 1u)) : key < kend;
      s[b][r] = ok ? s[b][r] * scale_log2 : kNeg;
      bmax = fmaxf(bmax, s[b][r]);
    }
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
  const float m_new = fmaxf(m_run, bmax);
  const float alpha = fast_exp2(m_run - m_new);
  l_run *= alpha;
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
#pragma unroll
  for (int b = 0; b < NBK; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      // masked keys contribute nothing, also while every key so far is masked
      const float e = s[b][r] > 0.5f * kNeg ? fast_exp2(s[b][r] - m_new) : 0.f;
      s[b][r] = e;
      l_run += e;
    }
  m_run = m_new;
#pragma unroll
  for (int b = 0; b < NBK; ++b)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int r0 = 8 * s2;
      const u32x4_t ph = {pack_h2(s[b][r0], s[b][r0 + 1]), pack_h2(s[b][r0 + 2], s[b][r0 + 3]),
                          pack_h2(s[b][r0 + 4], s[b][r0 + 5]), pack_h2(s[b][r0 + 6], s[b][r0 + 7])};
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const u32x4_t va = *reinterpret_cast<const u32x4_t*>(vt + (32 * db + c) * VS + 32 * b + 16 * s2 + 8 * h);
        o[db] = mfma32_f16(va, ph, o[db]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Prefix chunks [c0, c1) of split s >= 1: cps consecutive chunks, cut at the
// np chunks of the prefix. The mapping depends on the grid only (not on P), so
// a split can read its page table entry and issue its first K/V loads before
// the step descriptor arrives.
__device__ __forceinline__ void split_range(int s, int cps, int np, int& c0, int& c1) {
  c0 = (s - 1) * cps;
  c1 = min(c0 + cps, np);
}

// Output rows of one (head, 32-dim block) unit from lane (c, h)'s 16 values
// (accumulator layout: register 4 gq + i = dim 32 db + 8 gq + 4 h + i of query
// row 32 rb + c): normalised, gated, stored as the bf16 hi / lo pair.
template <int D, bool GATE>
__device__ __forceinline__ void write_unit(const AttnParams& p, int hq, int db, int rb, int L, int c, int h,
                                           const float (&acc)[16], float inv) {
  const int orow = 32 * rb + c;
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int dim = 32 * db + 8 * gq + 4 * h;
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = orow < L ? acc[4 * gq + i] * inv : 0.f;
    if (GATE && orow < L) {
      // o_proj input = attention * sigmoid(gate), gate = q_proj row dims D.. of the head (qwen35_tree.py:540)
      const f32x4_t gt = *reinterpret_cast<const f32x4_t*>(p.qkv + (size_t)orow * p.ld_qkv + hq * p.q_stride + D + dim);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] *= 1.0f / (1.0f + __expf(-gt[i]));
    }
    const int col = hq * D + dim;
    const size_t oi = p.out_tiled ? tiled_index(orow, col, p.ld_out) : (size_t)orow * p.ld_out + col;
    store_act4(p.out, p.out_lo, oi, y, p.out_h16);
  }
}

template <int D, int R, bool GATE, int G>
__global__ __launch_bounds__(64 * G) void gqa_tree_attn_kernel(AttnParams p) {
  constexpr int NJ = D / 16, ND = D / 32;
  constexpr int CK = chunk_keys(D), NB = CK / 32;
  constexpr int KS = D + 8;   // LDS K row stride (bf16 / fp16 elements)
  constexpr int VS = CK + 8;  // LDS V^T row stride
  constexpr int kStage = (CK * KS + D * VS) * 2;
  constexpr int TPS = 64 * G;      // threads
  constexpr int W = G;             // waves
  constexpr int U = G * ND;        // combine units (head, 32-dim block)
  constexpr int kComb = W * 64 * 5 * 16;  // [wave][4 f32x4 + (M, T) pad][lane]
  constexpr int kLdsKV = 2 * kStage > kComb ? 2 * kStage : kComb;
  __shared__ __align__(16) unsigned char lds[kLdsKV];
  __shared__ __align__(16) unsigned char lds_aux[QAux<D, R, TPS>::kBytes];
  __shared__ int s_flag;
  // head_dim 256, split 0: each wave's query fragments live in LDS
  // ([wave][j][lane], 16 KB per wave) instead of 64 registers, which the tree
  // chunk loop (which also appends the tree K/V to the cache) otherwise
  // spills, reloading addresses from scratch on every chunk. The prefix
  // splits keep them in registers (their loop has room, and 16 more LDS reads
  // per chunk would cost more there).
  constexpr bool QL = D == 256;
  __shared__ __align__(16) u32x4_t q_lds[QL ? W * NJ * 64 : 1];

  const int pairs = p.Hkv * p.NT;
  // Workgroup (group g, query block rb, split s). u = s * Hkv + g runs over
  // groups of 8; the query blocks of one u take blockIdx u % 8 + 8 rb inside
  // its group's 8 * NT workgroups, so they share blockIdx % 8 (an XCD under
  // the round-robin dispatch) and read their K/V chunks through one L2
  // (9B-shaped layer, three query blocks: 69.0 -> 66.5 us). A last,
  // incomplete group of u takes its workgroups in (rb, u) order.
  const int nu = p.Hkv * p.S, full = nu / kXcds * kXcds * p.NT;
  int rb_u, u_s;
  if ((int)blockIdx.x < full) {
    const int grp = blockIdx.x / (kXcds * p.NT), rem = blockIdx.x % (kXcds * p.NT);
    rb_u = rem / kXcds;
    u_s = grp * kXcds + rem % kXcds;
  } else {
    const int m = nu % kXcds, b2 = blockIdx.x - full;
    rb_u = b2 / m;
    u_s = nu / kXcds * kXcds + b2 % m;
  }
  const int g = u_s % p.Hkv, s = u_s / p.Hkv, rb = rb_u;
  const int pair = rb * p.Hkv + g;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hw = wave;
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int ts = threadIdx.x;
  const int hq = g * G + hw;
  const int qrow = 32 * rb + c;
  const int S = p.S;

  // The step descriptor's P and L are read first; everything that does not
  // depend on them (the query rows and their norm / RoPE, the first chunk:
  // tree rows, or page table entry then K/V) goes out before they are used,
  // so the latencies overlap.
  u32x4_t qf[NJ];
  HeadRow<D, R> qr;
  row_issue<D, R>(qr, p.qkv + (size_t)qrow * p.ld_qkv + hq * p.q_stride, h);
  QAux<D, R, TPS> qa;
  qa.issue(p, rb, ts);
  // RoPE rows and q_norm weight into LDS, then this wave's q fragments
  auto build_q = [&](bool to_lds) {
    qa.commit(lds_aux, ts);
    __syncthreads();
    q_fragments<D, R>(qr, lds_aux, p.q_norm != nullptr, p.eps, c, h, qf);
    if constexpr (QL) {
      if (to_lds) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) q_lds[(wave * NJ + j) * 64 + lane] = qf[j];
      }
    }
  };
  const QRegs<D> q_regs{qf};
  const QLds q_mem{q_lds + wave * NJ * 64, lane};
  int P = 0, L = 0, np = 0;
  // The descriptor is read after the chunk loads are issued (its scalar wait
  // must not hold them back).
  auto read_desc = [&]() {
    P = p.desc->past_length;
    L = p.desc->num_nodes;
    np = (P + CK - 1) / CK;
  };
  // A descriptor beyond the grid's capacity leaves the output untouched (every
  // workgroup returns, so none waits at the counter); a query block past the
  // tree writes zero rows without an exchange.
  auto bail = [&]() -> bool {
    if (P < 0 || P > p.max_past || np > p.max_pchunks || L > 32 * p.NT || L < 1 || (np > 0 && S < 2)) return true;
    if (32 * rb >= L) {
      if (wave == 0) {
        float z[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) z[i] = 0.f;
        for (int u = s; u < U; u += S) write_unit<D, false>(p, g * G + u / ND, u % ND, rb, L, c, h, z, 0.f);
      }
      return true;
    }
    return false;
  };

  float m_run = kNeg, l_run = 0.f;
  f32x16_t o[ND];
  int n_items;
  // Chunks run through two LDS buffers: chunk i + 1's loads are in flight
  // while chunk i is multiplied.
  auto buf_k = [&](int i) { return reinterpret_cast<uint16_t*>(lds + (i & 1) * kStage); };
  auto buf_v = [&](int i) { return reinterpret_cast<uint16_t*>(lds + (i & 1) * kStage) + CK * KS; };
  if (s == 0) {
    // split 0: tree chunks 0 .. rb (later ones hold no ancestor of this block's rows)
    n_items = min(rb, p.NT - 1) + 1;
    TreeStage<D, R, TPS> st;
    st.issue(p, 0, g, ts);
    read_desc();
    build_q(true);
    if (bail()) return;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
    for (int it = 0; it < n_items; ++it) {
      st.template commit<KS, VS>(p, it, g, P, L, ts, buf_k(it), buf_v(it), p.write_cache && it == rb);
      if (it + 1 < n_items) st.issue(p, it + 1, g, ts);
      __syncthreads();
      const uint32_t anc = p.desc->ancestors[qrow][it];
      if constexpr (QL)
        attend_chunk<D, 1, KS, VS, true>(buf_k(it), buf_v(it), q_mem, p.scale_log2, L - 32 * it, anc, qrow < L, c,
                                         h, m_run, l_run, o);
      else
        attend_chunk<D, 1, KS, VS, true>(buf_k(it), buf_v(it), q_regs, p.scale_log2, L - 32 * it, anc, qrow < L, c,
                                         h, m_run, l_run, o);
    }
  } else {
    // split s >= 1: prefix chunks c0 .. c0 + cps - 1 (cut at the prefix's np)
    const int c0 = (s - 1) * p.cps;
    // The first chunk's loads go out on every path (a split past the prefix
    // chunks loads the last one and never commits it), so waiting for the
    // query rows issued before them does not become a wait for every load.
    const int cfirst = min(c0, p.max_pchunks - 1);  // splits s >= 1 exist only with prefix chunks
    PrefixStage<D, TPS> st;
    st.issue(p, cfirst, PrefixStage<D, TPS>::page_of(p, cfirst), g, ts);
    read_desc();
    build_q(false);
    if (bail()) return;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
    n_items = max(0, min(c0 + p.cps, np) - c0);
    for (int it = 0; it < n_items; ++it) {
      st.template commit<KS, VS>(c0 + it, P, ts, buf_k(it), buf_v(it));
      if (it + 1 < n_items) st.issue(p, c0 + it + 1, PrefixStage<D, TPS>::page_of(p, c0 + it + 1), g, ts);
      __syncthreads();
      attend_chunk<D, NB, KS, VS, false>(buf_k(it), buf_v(it), q_regs, p.scale_log2, P - (c0 + it) * CK, 0u, true, c,
                                         h, m_run, l_run, o);
    }
  }
  __syncthreads();  // the LDS buffers are reused below

  // ---- publish this split's partial, written through (sc1): per head
  // [db][gq][lane] f32x4 (accumulator registers 4 gq .. 4 gq + 3 of block db:
  // each store instruction of the wave writes one contiguous kilobyte), then
  // m[32] and l[32] ----
  constexpr int kHeadStride = ND * 64 * 16 + 64;  // floats per head
  const size_t split_floats = (size_t)G * kHeadStride;
  const unsigned part_bytes = (unsigned)((size_t)pairs * S * split_floats * sizeof(float));
  const __amdgpu_buffer_rsrc_t prs = buf_rsrc(p.part, part_bytes);
  const unsigned pair_base = (unsigned)((size_t)pair * S * split_floats * sizeof(float));
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (n_items > 0) {
    const unsigned hb = pair_base + (unsigned)(((size_t)s * split_floats + (size_t)hw * kHeadStride) * 4);
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4_t, f32x4_t{o[db][4 * gq], o[db][4 * gq + 1], o[db][4 * gq + 2],
                                                o[db][4 * gq + 3]}),
            prs, (int)(hb + (unsigned)(((db * 4 + gq) * 64 + lane) * 16)), 0, kSc1);
    if (h == 0) {
      const unsigned mo = hb + (unsigned)(ND * 64 * 16 * 4);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, m_run), prs, (int)(mo + 4 * c), 0, kSc1);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, l_tot), prs, (int)(mo + 4 * (32 + c)), 0,
                                            kSc1);
    }
  }
  wait_stores_done();
  __syncthreads();

  // ---- meet the (group, query block)'s other splits ----
  int* cnt = p.counters + pair;
  if (threadIdx.x == 0) {
    // arrivals in the low 16 bits; workgroups off their expected XCD add kForeign
    const bool native = !p.off_xcd && xcc_id() == (int)(blockIdx.x % kXcds);
    const int add = native ? 1 : 1 + kForeign;
    int v = arrive_add(cnt, add) + add;
    int it = 0;
    while ((v & (kForeign - 1)) < S && it < p.spin_limit) {
      __builtin_amdgcn_s_sleep(1);
      v = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ++it;
    }
    int flag;
    if ((v & (kForeign - 1)) < S) {
      __hip_atomic_fetch_or(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      flag = 0;
    } else {
      // all splits on this XCD (Hkv % 8 == 0 gives a pair's splits one
      // blockIdx % 8 and none was foreign): read the partials from the local L2
      flag = (v < kForeign && p.Hkv % kXcds == 0) ? 2 : 1;
    }
    s_flag = flag;
  }
  __syncthreads();
  const int flag = s_flag;

  if (flag) {
    // ---- combine: unit u = (head u / ND, dim block u % ND) ----
    // k waves of one workgroup share a unit (k = the power of two <= W that
    // spreads the U units over the S * W waves), wave wl of the group reading
    // splits wl, wl + k, ...; groups of k waves take units gi, gi + S * W / k, ..
    int k = 1;
    while (2 * k <= W && 2 * k * U <= S * W) k *= 2;
    const int gpw = W / k;                       // wave groups per workgroup
    const int gi = s * gpw + wave / k, wl = wave % k;
    const int stride = S * gpw;
    const int rounds = (U + stride - 1) / stride;
    f32x4_t* xc = reinterpret_cast<f32x4_t*>(lds);  // [wave][5][lane]
    for (int rd = 0; rd < rounds; ++rd) {
      const int u = gi + rd * stride;
      const bool has_unit = u < U;
      const int uh = has_unit ? u / ND : 0, udb = has_unit ? u % ND : 0;
      float Ms = kNeg, T = 0.f;
      f32x4_t acc[4];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) acc[gq] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int sp0 = wl; has_unit && sp0 < S; sp0 += k * kCombineBatch) {
        f32x4_t v[kCombineBatch][4];
        float mm[kCombineBatch], ll[kCombineBatch];
#pragma unroll
        for (int b = 0; b < kCombineBatch; ++b) {
          const int sp = sp0 + k * b;
          bool has = sp < S;
          if (has && sp > 0) {
            int a0, a1;
            split_range(sp, p.cps, np, a0, a1);
            has = a1 > a0;
          }
          const unsigned hb =
              has ? pair_base + (unsigned)(((size_t)sp * split_floats + (size_t)uh * kHeadStride) * 4) : kOob;
          const unsigned mo = hb + (has ? (unsigned)(ND * 64 * 16 * 4) : 0u);
          float mv, lv;
          if (flag == 2) {
            mv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(mo + 4 * c), 0, kSc0));
            lv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(mo + 4 * (32 + c)), 0, kSc0));
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
              v[b][gq] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                  prs, (int)(hb + (unsigned)(((udb * 4 + gq) * 64 + lane) * 16)), 0, kSc0));
          } else {
            mv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(mo + 4 * c), 0, kSc1));
            lv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(mo + 4 * (32 + c)), 0, kSc1));
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
              v[b][gq] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                  prs, (int)(hb + (unsigned)(((udb * 4 + gq) * 64 + lane) * 16)), 0, kSc1));
          }
          mm[b] = has ? mv : kNeg;
          ll[b] = has ? lv : 0.f;
        }
        float gm = Ms;
#pragma unroll
        for (int b = 0; b < kCombineBatch; ++b) gm = fmaxf(gm, mm[b]);
        const float rsc = fast_exp2(Ms - gm);
        T *= rsc;
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) acc[gq] *= rsc;
#pragma unroll
        for (int b = 0; b < kCombineBatch; ++b) {
          const float w = mm[b] > 0.5f * kNeg ? fast_exp2(mm[b] - gm) : 0.f;
          T += w * ll[b];
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) acc[gq] += w * v[b][gq];
        }
        Ms = gm;
      }
      // merge the group's k waves in wave order
      if (k > 1) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) xc[(wave * 5 + gq) * 64 + lane] = acc[gq];
        xc[(wave * 5 + 4) * 64 + lane] = f32x4_t{Ms, T, 0.f, 0.f};
        __syncthreads();
      }
      if (has_unit && wl == 0) {
        float y[16], tot;
        if (k > 1) {
          float M = kNeg;
          for (int w = wave; w < wave + k; ++w) M = fmaxf(M, xc[(w * 5 + 4) * 64 + lane][0]);
          tot = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) y[i] = 0.f;
          for (int w = wave; w < wave + k; ++w) {
            const f32x4_t mt = xc[(w * 5 + 4) * 64 + lane];
            const float f = mt[0] > 0.5f * kNeg ? fast_exp2(mt[0] - M) : 0.f;
            tot += f * mt[1];
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const f32x4_t x = xc[(w * 5 + gq) * 64 + lane];
#pragma unroll
              for (int i = 0; i < 4; ++i) y[4 * gq + i] += f * x[i];
            }
          }
        } else {
          tot = T;
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
#pragma unroll
            for (int i = 0; i < 4; ++i) y[4 * gq + i] = acc[gq][i];
        }
        const float inv = tot > 0.f ? 1.0f / tot : 0.f;
        write_unit<D, GATE>(p, g * G + uh, udb, rb, L, c, h, y, inv);
      }
      if (k > 1) __syncthreads();
    }
  }

  // second phase: the last workgroup to pass the combine returns the counter to zero
  if (threadIdx.x == 0) {
    const int old = arrive_add(cnt, 1);
    if ((old & (kForeign - 1)) == 2 * S - 1) reset_counter(cnt);
  }
}

}  // namespace dtree

using namespace dtree;

static int attn_max_pchunks(int head_dim, int max_past) {
  const int ck = chunk_keys(head_dim);
  return (max_past + ck - 1) / ck;
}

// Prefix chunks per split and splits per (group, query block): kDefaultCps
// chunks per split, plus the tree split, as many splits as
// fit next to the other pairs in one resident grid (at most one workgroup per
// CU; more chunks per split when the prefix needs it).
// DTREE_ATTN_CHUNKS_PER_SPLIT=n asks for n instead (tuning).
constexpr int kDefaultCps = 2;
static void attn_splits(int head_dim, int max_past, int pairs, int cus, int& S, int& cps) {
  const int npc = attn_max_pchunks(head_dim, max_past);
  cps = kDefaultCps;
  if (const char* e = std::getenv("DTREE_ATTN_CHUNKS_PER_SPLIT")) cps = std::max(1, std::atoi(e));
  const int cap = cus / pairs;  // >= 2, checked by the caller
  if (1 + (npc + cps - 1) / cps > cap) cps = (npc + cap - 2) / (cap - 1);
  S = 1 + (npc + cps - 1) / cps;
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

static size_t group_attention_workspace_bytes(int32_t num_heads, int32_t head_dim, int32_t max_past_length,
                                              int32_t rows_padded) {
  if (num_heads <= 0 || head_dim <= 0 || max_past_length < 0 || rows_padded <= 0 || rows_padded % 32) return 0;
  const int nt = rows_padded / 32;
  const size_t head_floats = (size_t)(head_dim / 32) * 64 * 16 + 64;
  // splits never exceed one per prefix chunk plus the tree split
  const size_t splits = 1 + (size_t)attn_max_pchunks(head_dim, max_past_length);
  return kWsHeader + attn_ll_bytes(num_heads, head_dim, rows_padded) +
         (size_t)num_heads * nt * splits * head_floats * sizeof(float);
}

static int group_tree_attention(const DtreeAttnArgs* a, hipStream_t stream) {
  DTREE_REQUIRE(a, "attention: null args");
  DTREE_REQUIRE(a->qkv && a->rope_cos && a->rope_sin && a->k_pages && a->v_pages && a->page_table && a->desc &&
                    a->out && a->workspace,
                "attention: null pointer");
  const int D = a->head_dim;
  const int R = a->rope_dims == 0 ? D : a->rope_dims;
  const bool gated = a->gated != 0;
  DTREE_REQUIRE((D == 128 && R == 128 && !gated) || (D == 256 && R == 64 && gated),
                "attention: compiled geometries are head_dim 128 (full RoPE) and gated head_dim 256 (rope_dims 64)");
  DTREE_REQUIRE(a->rows_padded == 32 || a->rows_padded == 64 || a->rows_padded == 96 || a->rows_padded == 128,
                "attention: rows_padded must be 32, 64, 96 or 128");
  const int nt = a->rows_padded / 32;
  DTREE_REQUIRE(a->num_kv_heads > 0 && a->num_heads % a->num_kv_heads == 0, "attention: num_heads % num_kv_heads");
  const int G = a->num_heads / a->num_kv_heads;
  DTREE_REQUIRE(G == 2 || G == 4 || (G == 8 && D == 128), "attention: GQA group of 2, 4 or 8 (8: head_dim 128)");
  DTREE_REQUIRE(a->max_past_length >= 0 && a->max_past_length <= kMaxPast, "attention: max_past_length beyond 16384");
  const int q_stride = gated ? 2 * D : D;
  DTREE_REQUIRE(a->ld_qkv >= a->num_heads * q_stride + 2 * a->num_kv_heads * D && a->ld_qkv % 4 == 0,
                "attention: ld_qkv too small");
  DTREE_REQUIRE(a->ld_out >= a->num_heads * D && a->ld_out % 8 == 0,
                "attention: ld_out below num_heads * head_dim or not a multiple of 8");
  DTREE_REQUIRE(((uintptr_t)a->out & 15) == 0 && ((uintptr_t)a->out_lo & 15) == 0 && ((uintptr_t)a->qkv & 15) == 0,
                "attention: qkv, out and out_lo must be 16-byte aligned");
  DTREE_REQUIRE(a->workspace_bytes >= group_attention_workspace_bytes(a->num_heads, D, a->max_past_length,
                                                                      a->rows_padded),
                "attention: workspace too small");
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR ||
                    ((a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16) &&
                     a->ld_out == a->num_heads * D && a->ld_out % 64 == 0),
                "attention: tiled out needs ld_out == num_heads * head_dim");
  const int pairs = a->num_kv_heads * nt;
  const int cus = device_cus();
  DTREE_REQUIRE(pairs <= kMaxPairs && 2 * pairs <= cus,
                "attention: num_kv_heads * rows_padded / 32 must leave two splits per pair within the CU count");
  AttnParams p{};
  p.qkv = a->qkv; p.ld_qkv = a->ld_qkv;
  p.q_stride = q_stride; p.k_off = a->num_heads * q_stride; p.v_off = p.k_off + a->num_kv_heads * D;
  p.q_norm = a->q_norm; p.k_norm = a->k_norm; p.eps = a->eps;
  p.rope_cos = a->rope_cos; p.rope_sin = a->rope_sin;
  p.kp = a->k_pages; p.vp = a->v_pages; p.page_table = a->page_table; p.desc = a->desc;
  p.out_tiled = a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16;
  p.out_h16 = a->out_layout == DTREE_W_TILED_F16;
  p.out = a->out; p.out_lo = p.out_h16 ? nullptr : a->out_lo; p.ld_out = a->ld_out;  // fp16: one plane
  p.Hq = a->num_heads; p.Hkv = a->num_kv_heads; p.NT = nt;
  p.max_pchunks = attn_max_pchunks(D, a->max_past_length);
  p.max_past = a->max_past_length;
  attn_splits(D, a->max_past_length, pairs, cus, p.S, p.cps);
  p.scale_log2 = a->scale * kLog2e; p.write_cache = a->write_cache;
  p.off_xcd = off_xcd_test();
  p.spin_limit = attn_spin_limit();
  p.err = reinterpret_cast<int*>(a->workspace);
  p.counters = reinterpret_cast<int*>(reinterpret_cast<char*>(a->workspace) + 64);
  p.part = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) + kWsHeader +
                                    attn_ll_bytes(a->num_heads, D, a->rows_padded));
  const int grid = pairs * p.S;
  if (D == 128) {
    if (G == 2) gqa_tree_attn_kernel<128, 128, false, 2><<<grid, 64 * 2, 0, stream>>>(p);
    else if (G == 4) gqa_tree_attn_kernel<128, 128, false, 4><<<grid, 64 * 4, 0, stream>>>(p);
    else gqa_tree_attn_kernel<128, 128, false, 8><<<grid, 64 * 8, 0, stream>>>(p);
  } else {
    if (G == 2) gqa_tree_attn_kernel<256, 64, true, 2><<<grid, 64 * 2, 0, stream>>>(p);
    else gqa_tree_attn_kernel<256, 64, true, 4><<<grid, 64 * 4, 0, stream>>>(p);
  }
  DTREE_LAUNCH_CHECK("attention launch");
  return DTREE_OK;
}

// ---- entry points: per-head or per-KV-group kernel ----------------------------
// Two designs cover the prefix range. The per-head kernel (attention_head.hip:
// a workgroup per (query head, four chunks), last-arriver combine) has the
// shorter fixed latency; the per-KV-group kernel above loads every K/V chunk
// once for the group's G heads and wins once the prefix stream dominates.
// Measured on MI355X (Qwen3-4B layer, 25-node tree, us per launch, per-head /
// per-group): P 128: 11.1 / 24.6; 512: 15.8 / 19.1; 1024: 16.3 / 19.7;
// 2048: 24.2 / 21.5; 4096: 36.0 / 25.7. The choice follows the prefix the grid
// is sized for; DTREE_ATTN_KERNEL=head|group forces one (tests).
namespace dtree {
size_t head_attention_workspace_bytes(int32_t num_heads, int32_t head_dim, int32_t max_past_length,
                                      int32_t rows_padded);
int head_tree_attention(const DtreeAttnArgs* a, hipStream_t stream);
}  // namespace dtree

constexpr int kGroupKernelMinPast = 1536;

static bool use_group_kernel(const DtreeAttnArgs* a) {
  if (const char* e = std::getenv("DTREE_ATTN_KERNEL")) {
    if (e[0] == 'g') return true;
    if (e[0] == 'h') return false;
  }
  return a->max_past_length > kGroupKernelMinPast;
}

extern "C" size_t dtree_attention_workspace_bytes(int32_t num_heads, int32_t head_dim, int32_t max_past_length,
                                                  int32_t rows_padded) {
  const size_t a = group_attention_workspace_bytes(num_heads, head_dim, max_past_length, rows_padded);
  const size_t b = dtree::head_attention_workspace_bytes(num_heads, head_dim, max_past_length, rows_padded);
  return a > b ? a : b;
}

extern "C" int dtree_tree_attention(const DtreeAttnArgs* a, hipStream_t stream) {
  DTREE_REQUIRE(a, "attention: null args");
  return use_group_kernel(a) ? group_tree_attention(a, stream) : dtree::head_tree_attention(a, stream);
}

// ---- allocation-free variant ---------------------------------------------------
// For callers that cannot allocate device memory (code under graph capture,
// serving loops, harnesses that forbid hipMalloc): the same kernels with their
// workspace (error word, split counters, partials) in this file-scope device
// array instead of a caller buffer. Each GPU holds its own copy until the
// process ends; every call on a GPU shares it, so calls that overlap on one
// GPU race.
constexpr size_t kScratchBytes = 32u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {nullptr};
long long g_ll_key[64] = {0};  // exchange placement of the last call per GPU (0: region never used)

// Device address of this GPU's scratch array (the host-side name is only a
// stand-in), looked up once per device with that device current.
int scratch_for_current_device(void** out) {
  int dev = 0;
  int rc = hip_check(hipGetDevice(&dev), "attention (no alloc): hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= 64) return fail(DTREE_E_ARG, "attention (no alloc): device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "attention (no alloc): hipGetSymbolAddress");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DTREE_OK;
}

// Moves a workspace's error word into *status (OR) and clears it. After a
// give-up it also moves every epoch of the per-head flag exchange (table
// place and length in header words 2 and 3) far ahead, so no flag written by
// the failed launch, however late, matches a later launch's.
__global__ void attn_status_kernel(int* err, int* status) {
  const int e = *err;
  if (!e) return;
  const int off = err[2], n = err[3];
  if (off >= (int)kAttnWsHeader && n > 0) {
    uint32_t* ep = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(err) + off);
    for (int i = threadIdx.x; i < n; i += blockDim.x) ep[i] += 1u << 16;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    *status |= e;
    *err = 0;
  }
}

// Zeroes the workspace header (error word and split counters of either
// kernel) before each call: a fill kernel, so the call stays capturable.
__global__ void zero_header_kernel(u32x4_t* p, int n16) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) p[i] = u32x4_t{0u, 0u, 0u, 0u};
}
}  // namespace

extern "C" size_t dtree_tree_attention_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int dtree_tree_attention_noalloc(const DtreeAttnArgs* a, hipStream_t stream) {
  DTREE_REQUIRE(a, "attention (no alloc): null args");
  const bool group = use_group_kernel(a);
  const size_t need = group ? group_attention_workspace_bytes(a->num_heads, a->head_dim, a->max_past_length,
                                                              a->rows_padded)
                            : dtree::head_attention_workspace_bytes(a->num_heads, a->head_dim, a->max_past_length,
                                                                    a->rows_padded);
  DTREE_REQUIRE(need > 0, "attention (no alloc): bad num_heads / head_dim / max_past_length / rows_padded");
  if (need > kScratchBytes)
    return fail(DTREE_E_WORKSPACE, "attention (no alloc): this shape needs " + std::to_string(need) +
                                       " bytes of workspace, beyond the 32 MiB device scratch array");
  void* ws = nullptr;
  int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  {
    // The per-head flag exchange keeps epochs and slots across calls, placed
    // by (heads, head dim); a call with another placement than the last one
    // on this GPU starts from a cleared region.
    int dev = 0;
    rc = hip_check(hipGetDevice(&dev), "attention (no alloc): hipGetDevice");
    if (rc) return rc;
    const size_t llb = attn_ll_bytes(a->num_heads, a->head_dim, a->rows_padded);
    const long long key = ((long long)a->num_heads << 32) | ((long long)a->head_dim << 8) | (a->rows_padded == 32);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (llb > 0 && g_ll_key[dev] != key) {
      const int m16 = static_cast<int>(llb / 16);
      zero_header_kernel<<<(m16 + 255) / 256, 256, 0, stream>>>(
          reinterpret_cast<u32x4_t*>(reinterpret_cast<char*>(ws) + kAttnWsHeader), m16);
      DTREE_LAUNCH_CHECK("attention (no alloc): exchange clear");
      g_ll_key[dev] = key;
    }
  }
  // The group kernel keeps its error word and counters in the first 4 KiB; the
  // per-head kernel keeps one counter per (head, row block) at the start.
  const size_t head_counters = (64 + static_cast<size_t>(a->num_heads) * (a->rows_padded / 32) * 4 + 255) / 256 * 256;
  const int n16 = static_cast<int>(std::min(need, std::max<size_t>(4096, head_counters)) / 16);
  zero_header_kernel<<<(n16 + 255) / 256, 256, 0, stream>>>(reinterpret_cast<u32x4_t*>(ws), n16);
  DTREE_LAUNCH_CHECK("attention (no alloc): header clear");
  DtreeAttnArgs b = *a;
  b.workspace = ws;
  b.workspace_bytes = need;
  return group ? group_tree_attention(&b, stream) : dtree::head_tree_attention(&b, stream);
}

extern "C" int dtree_attention_status(void* workspace, int32_t* status, hipStream_t stream) {
  DTREE_REQUIRE(status, "attention status: null status");
  void* ws = workspace;
  if (!ws) {
    int rc = scratch_for_current_device(&ws);
    if (rc) return rc;
  }
  attn_status_kernel<<<1, 64, 0, stream>>>(reinterpret_cast<int*>(ws), status);
  DTREE_LAUNCH_CHECK("attention status launch");
  return DTREE_OK;
}
