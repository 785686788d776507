// Ancestor-masked GQA tree attention over a paged bf16 KV prefix.
//
// Work split: a workgroup serves one 32-row block of tree queries (rows
// 32*rb .. 32*rb+31) of one query head. The keys are cut into chunks: chunks
// 0 .. npre-1 are runs of CK prefix keys (fully visible): a 64-key page for
// head_dim 128, half a page for head_dim 256 (same registers per wave);
// chunks npre .. npre+NT-1 are the tree itself in 32-key blocks (NT =
// rows_padded / 32; tree chunk tc is masked by word tc of each query's
// ancestor-or-self bitset). A workgroup has four waves, one chunk each, so
// workgroup `split` owns chunks 4*split .. 4*split+3. The tree chunks come
// last: the wave that also normalises, stages and appends the tree rows then
// shares its workgroup with the fewest prefix chunks (at a 1024-key prefix
// the tree is the fifth workgroup's only chunk and the other four hold four
// pages each), so that workgroup is not the last to publish its partial.
//
// Two head geometries are compiled: Qwen3 (head_dim 128, full RoPE) and the
// gated attention of Qwen3.5 (head_dim 256, RoPE on the first 64 dims, q_proj
// rows per head = [q | gate], output multiplied by sigmoid(gate)).
// A wave owns exactly one chunk, so its softmax needs no running rescale: it
// issues Q's loads, then all K and V of its page (32 KB in flight per wave),
// scores both 32-key blocks, takes one max and accumulates P V.
// The four waves merge in LDS; when a head needs more than one workgroup,
// each writes a merged partial (row max, row sum, unnormalised output) and the
// last one to arrive (device-scope counter) combines them, all 256 threads
// with independent loads. The heads of one KV group run on one XCD
// (blockIdx % 8), so their shared K/V reads meet in one L2.
//
// MFMA use (v_mfma_f32_32x32x16_bf16), with the tree rows (<= 32) as one
// MFMA dimension:
//   S^T = K Q^T : A = 32 keys x 16 dims, B = 16 dims x 32 queries. A lane owns
//                 query column lane%32, so softmax statistics are lane-local
//                 (16 registers + one exchange with lane^32).
//   O^T = V^T P^T: A = V^T (32 dims x 16 keys), B = P^T taken straight from
//                 the S^T registers. A-row rho of S^T is loaded from key
//                 pi(rho) = rho with bits 2 and 3 swapped; then register r of
//                 a lane in half h holds key 16*(r/8) + 8*h + r%8, i.e. eight
//                 consecutive keys per PV step, which is one 16-byte read of
//                 the transposed V page.
// K pages are [page][kv_head][64][D]; V pages are [page][kv_head][D][64].
#include <cstdlib>

#include "common.h"

namespace dtree {
namespace head_attn {

constexpr int kWaves = 4;          // waves (chunks) per workgroup
constexpr int kMaxPast = 16384;    // longest prefix the grid is sized for
// Prefix keys per chunk.
__host__ __device__ constexpr int chunk_keys(int D) { return D <= 128 ? DTREE_PAGE : DTREE_PAGE / 2; }
// Workgroups (splits) of one (head, query block) for npre prefix chunks and NT
// tree chunks: head_dim 128 gives the tree chunks a split of their own, then
// four prefix chunks per split; head_dim 256 packs tree chunks after the
// prefix chunks, four chunks per split.
__host__ __device__ constexpr int head_nsplit(int D, int npre, int NT) {
  return D == 128 ? 1 + (npre + kWaves - 1) / kWaves : (npre + NT + kWaves - 1) / kWaves;
}
constexpr float kNeg = -1e30f;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
  const float* qkv; int ld_qkv;
  int q_stride, k_off, v_off;  // qkv row: q of head h at h*q_stride (gate at +D), k / v of group g at k_off / v_off + g*D
  const uint16_t* q_norm; const uint16_t* k_norm; float eps;
  const float* rope_cos; const float* rope_sin;
  uint16_t* kp; uint16_t* vp; const int* page_table;
  const DtreeStepDesc* desc;
  uint16_t* out; uint16_t* out_lo; int ld_out; int out_tiled;
  int out_h16;  // DTREE_W_TILED_F16 output: one fp16 plane
  int Hq, Hkv, max_chunks, splits;
  int tree_chunks;  // 32-key tree chunks = 32-row query blocks = rows_padded / 32
  float scale_log2;
  int write_cache;
  float* part; int* counters;
  int sep_combine;  // partials are combined by attn_combine_kernel (long prefixes)
  int off_xcd;      // test hook: treat every workgroup as off its expected XCD
  // Flag exchange (ll_exchange; rows_padded 32, up to kAttnLLSplits splits):
  // per query head an epoch word and kAttnLLSplits slots.
  int ll;
  uint32_t* ll_epoch; unsigned char* ll_slots; unsigned ll_bytes;
  int* err;         // workspace header: error word, then the epoch table's place
  int spin_limit;   // polls before a waiting workgroup gives up
};

__device__ __forceinline__ int swap_bits23(int c) { return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1); }

// Raw operands of one head row for lane (c, h), which owns dims 16j + 8h + i:
// the fp32 values, the bf16 RMSNorm weights and the RoPE cos/sin of the first
// half of the R rotated dims. Issuing all loads before any use lets a wave
// keep them in flight together with the K/V loads that follow.
template <int D, int R>
struct HeadRow {
  f32x4_t x[D / 16][2];
  u32x4_t nw[D / 16];
  f32x4_t cs[R / 32][2], sn[R / 32][2];
};

// AUX: also the norm weights and the RoPE cos/sin (q and k rows; v has
// none). Without norm weights the loads read the row itself instead and
// row_finish ignores them, so the loads never branch: the whole prologue
// stays one basic block and its loads go out in one round trip.
template <int D, int R, bool AUX>
__device__ __forceinline__ void row_issue(HeadRow<D, R>& r, const float* src, const uint16_t* norm_w, const float* cosr,
                                          const float* sinr, int h) {
  const uint16_t* nwp = norm_w ? norm_w : reinterpret_cast<const uint16_t*>(src);
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    r.x[j][0] = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h);
    r.x[j][1] = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h + 4);
    if constexpr (AUX) r.nw[j] = ld_u32x4(nwp + 16 * j + 8 * h);
  }
  if constexpr (AUX) {
#pragma unroll
    for (int j = 0; j < R / 32; ++j)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        r.cs[j][u] = *reinterpret_cast<const f32x4_t*>(cosr + 16 * j + 8 * h + 4 * u);
        r.sn[j][u] = *reinterpret_cast<const f32x4_t*>(sinr + 16 * j + 8 * h + 4 * u);
      }
  }
}

// RMSNorm over D (sum of squares completed with the partner lane^32), then
// RoPE on (dim d, dim d + R/2) pairs for d < R/2, which live in the same lane
// (registers j and j + R/32); dims >= R pass through.
template <int D, int R>
__device__ __forceinline__ void row_finish(const HeadRow<D, R>& r, bool norm, bool rope, float eps,
                                           float (&v)[D / 16][8]) {
  constexpr int NJ = D / 16;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[j][i] = r.x[j][0][i];
      v[j][i + 4] = r.x[j][1][i];
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
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = r.nw[j][i >> 1];
        v[j][i] *= rs * __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
      }
  }
  if (rope) {
    constexpr int RJ = R / 32;
#pragma unroll
    for (int j = 0; j < RJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float cs = r.cs[j][i >> 2][i & 3], sn = r.sn[j][i >> 2][i & 3];
        const float x1 = v[j][i], x2 = v[j + RJ][i];
        v[j][i] = x1 * cs - x2 * sn;
        v[j + RJ][i] = x1 * sn + x2 * cs;
      }
  }
}

template <int D>
__device__ __forceinline__ void pack_frag(const float (&v)[D / 16][8], u32x4_t (&f)[D / 16]) {
#pragma unroll
  for (int j = 0; j < D / 16; ++j)
    f[j] = u32x4_t{pack_bf2(v[j][0], v[j][1]), pack_bf2(v[j][2], v[j][3]), pack_bf2(v[j][4], v[j][5]),
                   pack_bf2(v[j][6], v[j][7])};
}

// v = hi + lo with hi = bf16(v), lo = bf16(v - hi): about 16 significant bits
// through two bf16 MFMAs.
__device__ __forceinline__ void split8(const float* v, u32x4_t& hi, u32x4_t& lo) {
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = v[i] - bf2f(f2bf(v[i]));
  hi = u32x4_t{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7])};
  lo = u32x4_t{pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]), pack_bf2(r[4], r[5]), pack_bf2(r[6], r[7])};
}

// P.V step s2 of a 32-key block: B operand = probabilities of registers
// 8*s2 .. 8*s2+7 (split hi/lo), A operand = V^T fragments.
template <int ND>
__device__ __forceinline__ void pv_step(const f32x16_t& p, int s2, const u32x4_t (&va)[ND], f32x16_t (&o)[ND]) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = p[8 * s2 + i];
  u32x4_t ph, pl;
  split8(v, ph, pl);
#pragma unroll
  for (int db = 0; db < ND; ++db) {
    o[db] = mfma32(va[db], ph, o[db]);
    o[db] = mfma32(va[db], pl, o[db]);
  }
}

// Softmax numerators of NB 32-key blocks that start a chunk: every wave owns
// exactly one chunk, so the running max starts here and no rescale exists.
// s[] is already scaled (log2 units) and masked (kNeg).
template <int NB>
__device__ __forceinline__ void softmax_fresh(f32x16_t (&s)[NB], float& m_run, float& l_run) {
  float bmax = kNeg;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) bmax = fmaxf(bmax, s[b][r]);
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
  float lsum = 0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[b][r] = fast_exp2(s[b][r] - bmax);
      lsum += s[b][r];
    }
  m_run = bmax;
  l_run = lsum;
}

// Zeroes the bf16 elements of a V^T fragment whose key (first + e) is >= end:
// keys past the prefix may hold stale or non-finite data, and 0 * NaN would
// reach the output through the PV MFMA.
__device__ __forceinline__ u32x4_t mask_keys(u32x4_t v, int first, int end) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo_ok = (first + 2 * i) < end ? 0xffffu : 0u;
    const uint32_t hi_ok = (first + 2 * i + 1) < end ? 0xffff0000u : 0u;
    v[i] &= lo_ok | hi_ok;
  }
  return v;
}

template <int D, int R>
__device__ __forceinline__ void q_fragments(const HeadRow<D, R>& qr, bool norm, float eps, u32x4_t (&qf)[D / 16],
                                            u32x4_t (&ql)[D / 16]) {
  float q[D / 16][8];
  row_finish<D, R>(qr, norm, true, eps, q);
#pragma unroll
  for (int j = 0; j < D / 16; ++j) split8(q[j], qf[j], ql[j]);
}

// ---- query rows staged once per workgroup -----------------------------------
// The four waves of a workgroup score the same 32 query rows of one head, so
// the rows are loaded, normalised and rotated once: thread (row r = t / 8,
// part j = t % 8) owns
// * head_dim 128 (RoPE pairs (d, d + 64)): dims 8j .. 8j+7 and 64+8j .. +7;
// * head_dim 256 (RoPE on dims 0..63, pairs (d, d + 32)): dims 4j .. 4j+3,
//   32+4j .. +3 and the unrotated 64+24j .. 64+24j+23;
// so each RoPE pair stays in one thread, and the RMSNorm sum of squares is
// completed over the row's 8 threads with DPP. The rows go to LDS, from which
// each wave reads its MFMA fragments. The row stride (D + 4 floats) keeps
// those 32-byte fragment reads apart in the LDS banks.
template <int D>
__host__ __device__ constexpr int qs_stride() { return D + 4; }
template <int D> struct QStage;
template <> struct QStage<128> {
  f32x4_t x[4];
  u32x4_t nw[2];
  f32x4_t cs[2], sn[2];
};
template <> struct QStage<256> {
  f32x4_t x[8];      // rotated pair halves [4j, +4), [32+4j, +4); then 64+24j .. +24
  u32x2_t nwr[2];    // norm weights of the rotated dims
  u32x4_t nwp[3];    // of the unrotated dims
  f32x4_t cs, sn;    // RoPE entries 4j .. 4j+3
};

template <int D>
__device__ __forceinline__ void q_stage_issue(const AttnParams& p, int hq, int rb, QStage<D>& q) {
  const int t = threadIdx.x, r = t >> 3, j = t & 7;
  const int row = 32 * rb + r;
  const float* src = p.qkv + (size_t)row * p.ld_qkv + hq * p.q_stride;
  // without q_norm the weight loads read the row itself (ignored below)
  const uint16_t* nwb = p.q_norm ? p.q_norm : reinterpret_cast<const uint16_t*>(src);
  if constexpr (D == 128) {
    q.x[0] = *reinterpret_cast<const f32x4_t*>(src + 8 * j);
    q.x[1] = *reinterpret_cast<const f32x4_t*>(src + 8 * j + 4);
    q.x[2] = *reinterpret_cast<const f32x4_t*>(src + 8 * j + 64);
    q.x[3] = *reinterpret_cast<const f32x4_t*>(src + 8 * j + 68);
    q.nw[0] = ld_u32x4(nwb + 8 * j);
    q.nw[1] = ld_u32x4(nwb + 8 * j + 64);
    const float* cr = p.rope_cos + row * 64 + 8 * j;
    const float* sr = p.rope_sin + row * 64 + 8 * j;
    q.cs[0] = *reinterpret_cast<const f32x4_t*>(cr);
    q.cs[1] = *reinterpret_cast<const f32x4_t*>(cr + 4);
    q.sn[0] = *reinterpret_cast<const f32x4_t*>(sr);
    q.sn[1] = *reinterpret_cast<const f32x4_t*>(sr + 4);
  } else {
    q.x[0] = *reinterpret_cast<const f32x4_t*>(src + 4 * j);
    q.x[1] = *reinterpret_cast<const f32x4_t*>(src + 32 + 4 * j);
#pragma unroll
    for (int i = 0; i < 6; ++i) q.x[2 + i] = *reinterpret_cast<const f32x4_t*>(src + 64 + 24 * j + 4 * i);
    q.nwr[0] = *reinterpret_cast<const u32x2_t*>(nwb + 4 * j);
    q.nwr[1] = *reinterpret_cast<const u32x2_t*>(nwb + 32 + 4 * j);
#pragma unroll
    for (int i = 0; i < 3; ++i) q.nwp[i] = ld_u32x4(nwb + 64 + 24 * j + 8 * i);
    q.cs = *reinterpret_cast<const f32x4_t*>(p.rope_cos + row * 32 + 4 * j);
    q.sn = *reinterpret_cast<const f32x4_t*>(p.rope_sin + row * 32 + 4 * j);
  }
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <int D>
__device__ __forceinline__ void q_stage_finish(const QStage<D>& q, bool norm, float eps, float* qs) {
  const int t = threadIdx.x, r = t >> 3, j = t & 7;
  constexpr int NV = D / 8;  // values per thread
  float v[NV];
#pragma unroll
  for (int k = 0; k < NV / 4; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) v[4 * k + i] = q.x[k][i];
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) ss += v[i] * v[i];
    ss += dpp<0xB1>(ss);   // lane ^ 1
    ss += dpp<0x4E>(ss);   // lane ^ 2
    ss += dpp<0x141>(ss);  // the other quad of the row's 8 lanes
    const float rs = rsqrtf(ss * (1.0f / D) + eps);
    if constexpr (D == 128) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t w = q.nw[i >> 3][(i & 7) >> 1];
        v[i] *= rs * ((i & 1) ? bf_hi(w) : bf_lo(w));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = q.nwr[i >> 2][(i & 3) >> 1];
        v[i] *= rs * ((i & 1) ? bf_hi(w) : bf_lo(w));
      }
#pragma unroll
      for (int i = 0; i < 24; ++i) {
        const uint32_t w = q.nwp[i >> 3][(i & 7) >> 1];
        v[8 + i] *= rs * ((i & 1) ? bf_hi(w) : bf_lo(w));
      }
    }
  }
  constexpr int NR = D == 128 ? 8 : 4;  // rotated pairs per thread
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    float cs, sn;
    if constexpr (D == 128) {
      cs = q.cs[i >> 2][i & 3];
      sn = q.sn[i >> 2][i & 3];
    } else {
      cs = q.cs[i];
      sn = q.sn[i];
    }
    const float x1 = v[i], x2 = v[NR + i];
    v[i] = x1 * cs - x2 * sn;
    v[NR + i] = x1 * sn + x2 * cs;
  }
  float* dst = qs + r * qs_stride<D>();
  if constexpr (D == 128) {
    *reinterpret_cast<f32x4_t*>(dst + 8 * j) = f32x4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4_t*>(dst + 8 * j + 4) = f32x4_t{v[4], v[5], v[6], v[7]};
    *reinterpret_cast<f32x4_t*>(dst + 8 * j + 64) = f32x4_t{v[8], v[9], v[10], v[11]};
    *reinterpret_cast<f32x4_t*>(dst + 8 * j + 68) = f32x4_t{v[12], v[13], v[14], v[15]};
  } else {
    *reinterpret_cast<f32x4_t*>(dst + 4 * j) = f32x4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4_t*>(dst + 32 + 4 * j) = f32x4_t{v[4], v[5], v[6], v[7]};
#pragma unroll
    for (int i = 0; i < 6; ++i)
      *reinterpret_cast<f32x4_t*>(dst + 64 + 24 * j + 4 * i) =
          f32x4_t{v[8 + 4 * i], v[9 + 4 * i], v[10 + 4 * i], v[11 + 4 * i]};
  }
}

// Lane (c, h)'s q fragment j (dims 16j + 8h .. +7 of query row c) from the
// staged rows, split hi / lo.
template <int D>
__device__ __forceinline__ void q_frag_one(const float* qs, int c, int h, int j, u32x4_t& qf, u32x4_t& ql) {
  const float* src = qs + c * qs_stride<D>() + 16 * j + 8 * h;
  const f32x4_t a = *reinterpret_cast<const f32x4_t*>(src);
  const f32x4_t b = *reinterpret_cast<const f32x4_t*>(src + 4);
  const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  split8(v, qf, ql);
}
template <int D>
__device__ __forceinline__ void q_frag_lds(const float* qs, int c, int h, u32x4_t (&qf)[D / 16],
                                           u32x4_t (&ql)[D / 16]) {
#pragma unroll
  for (int j = 0; j < D / 16; ++j) q_frag_one<D>(qs, c, h, j, qf[j], ql[j]);
}

// Tree chunk tc: k (norm + RoPE) and v of nodes 32*tc .. 32*tc+31 come from
// the fused qkv rows and are staged in LDS (this wave's private region) for
// the MFMA operand layouts; the block's 32 query rows are scored against them
// with word tc of their ancestor-or-self masks, and k/v are written to the
// cache rows P + node (once: query block 0, first head of the group).
// q, k and v are finished one after the other, so at most one raw head row is
// live in registers (head_dim 256 rows are 128 floats per lane pair).
// STAGED: the workgroup has already staged (and appended) this chunk's rows
// (tree_rows_stage); the wave only scores its queries against them.
template <int D, int R, bool QS, bool STAGED = false>
__device__ __forceinline__ void tree_chunk(const AttnParams& p, HeadRow<D, R>& qr, const float* qs, int hq, int g,
                                           int G, int P, int L, int tc, int qrow, bool write_rows, int c, int h,
                                           uint16_t* ks, uint16_t* vt, float& m_run, float& l_run,
                                           f32x16_t (&o)[D / 32]) {
  constexpr int NJ = D / 16, ND = D / 32;
  constexpr int KS = D + 8, VS = 32 + 8;
  constexpr int half_r = R / 2;
  // Lane (c, h) stages key node 32*tc + c and owns query row qrow.
  const int node = 32 * tc + c;
  const float* row = p.qkv + (size_t)node * p.ld_qkv;
  const float* cosr = p.rope_cos + node * half_r;
  const float* sinr = p.rope_sin + node * half_r;
  const uint32_t anc = p.desc->ancestors[qrow][tc];
  // Staged head_dim-256 rows are read one fragment at a time in the QK^T
  // loop (16 fragments would hold 128 registers).
  constexpr bool PERJ = QS && D > 128;
  u32x4_t qf[PERJ ? 1 : NJ], ql[PERJ ? 1 : NJ];
  if constexpr (!QS) {
    row_issue<D, R, true>(qr, p.qkv + (size_t)qrow * p.ld_qkv + hq * p.q_stride, p.q_norm, p.rope_cos + qrow * half_r,
                          p.rope_sin + qrow * half_r, h);
    q_fragments<D, R>(qr, p.q_norm != nullptr, p.eps, qf, ql);
  } else if constexpr (!PERJ) {
    q_frag_lds<D>(qs, c, h, qf, ql);
  }
  u32x4_t kf8[NJ], vf8[NJ];
  if constexpr (STAGED) {
  } else if constexpr (D <= 128) {
    // Both raw rows in flight together: one round trip instead of two.
    HeadRow<D, R> kr, vr;
    row_issue<D, R, true>(kr, row + p.k_off + g * D, p.k_norm, cosr, sinr, h);
    row_issue<D, R, false>(vr, row + p.v_off + g * D, nullptr, nullptr, nullptr, h);
    float kv[NJ][8], vv[NJ][8];
    row_finish<D, R>(kr, p.k_norm != nullptr, true, p.eps, kv);
    pack_frag<D>(kv, kf8);
    row_finish<D, R>(vr, false, false, 0.f, vv);
    pack_frag<D>(vv, vf8);
  } else {
    {
      HeadRow<D, R> kr;
      row_issue<D, R, true>(kr, row + p.k_off + g * D, p.k_norm, cosr, sinr, h);
      float kv[NJ][8];
      row_finish<D, R>(kr, p.k_norm != nullptr, true, p.eps, kv);
      pack_frag<D>(kv, kf8);
    }
    {
      HeadRow<D, R> vr;
      row_issue<D, R, false>(vr, row + p.v_off + g * D, nullptr, nullptr, nullptr, h);
      float vv[NJ][8];
      row_finish<D, R>(vr, false, false, 0.f, vv);
      pack_frag<D>(vv, vf8);
    }
  }
  if constexpr (!STAGED) {
    if (node >= L) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) vf8[j] = u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      *reinterpret_cast<u32x4_t*>(&ks[c * KS + 16 * j + 8 * h]) = kf8[j];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t word = vf8[j][i >> 1];
        vt[(16 * j + 8 * h + i) * VS + c] = (uint16_t)((i & 1) ? (word >> 16) : (word & 0xffff));
      }
    }
  }
  // Only this wave touches ks/vt, and a wave's LDS operations complete in
  // order: waiting for them (and fencing the compiler) suffices.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int kr_row = swap_bits23(c);
  f32x16_t s[1];
#pragma unroll
  for (int r = 0; r < 16; ++r) s[0][r] = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&ks[kr_row * KS + 16 * j + 8 * h]);
    if constexpr (PERJ) {
      u32x4_t f, l;
      q_frag_one<D>(qs, c, h, j, f, l);
      s[0] = mfma32(a, f, s[0]);
      s[0] = mfma32(a, l, s[0]);
    } else {
      s[0] = mfma32(a, qf[j], s[0]);
      s[0] = mfma32(a, ql[j], s[0]);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = 16 * (r >> 3) + 8 * h + (r & 7);
    const bool ok = qrow < L && 32 * tc + t < L && ((anc >> t) & 1u);
    s[0][r] = ok ? s[0][r] * p.scale_log2 : kNeg;
  }
  softmax_fresh<1>(s, m_run, l_run);
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    u32x4_t va[ND];
#pragma unroll
    for (int db = 0; db < ND; ++db)
      va[db] = *reinterpret_cast<const u32x4_t*>(&vt[(32 * db + c) * VS + 16 * s2 + 8 * h]);
    pv_step<ND>(s[0], s2, va, o);
  }
  if (!STAGED && p.write_cache && (hq % G) == 0 && write_rows && node < L) {
    const int pos = P + node;
    const int page = p.page_table[pos / DTREE_PAGE], off = pos % DTREE_PAGE;
    uint16_t* kblk = p.kp + (size_t)(page * p.Hkv + g) * DTREE_PAGE * D;
    uint16_t* vblk = p.vp + (size_t)(page * p.Hkv + g) * DTREE_PAGE * D;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // dims 16j + 8h .. +7 of this key are one 16-byte run of the K block
      *reinterpret_cast<u32x4_t*>(kblk + kv_k_off(off, 16 * j + 8 * h, D)) = kf8[j];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t word = vf8[j][i >> 1];
        vblk[kv_v_off(off, 16 * j + 8 * h + i, D)] = (uint16_t)((i & 1) ? (word >> 16) : (word & 0xffff));
      }
    }
  }
}

// ---- tree rows prepared by the whole workgroup (head_dim 128) --------------
// Split 0 of a head holds the tree chunks alone. Its 256 threads load,
// normalise, rotate and stage the tree's k and v rows for the scoring waves
// and append them to the cache, instead of one wave doing all of it after the
// query staging: thread t owns node 32 tc + t / 8 and dims 8j .. 8j+7 and
// 64+8j .. +7 (j = t % 8), so each RoPE pair (d, d + 64) stays in one thread
// and the k RMSNorm sum is completed over the row's 8 threads with DPP (the
// query staging's layout). Chunk 0's loads go out at the kernel's start,
// before the step descriptor is read.
struct TreeRows {
  f32x4_t k[4], v[4];
  u32x4_t nw[2];
  f32x4_t cs[2], sn[2];
};

__device__ __forceinline__ void tree_rows_issue(const AttnParams& p, int g, int tc, TreeRows& t) {
  constexpr int D = 128;
  const int n = 32 * tc + (threadIdx.x >> 3), j = threadIdx.x & 7;
  const float* kr = p.qkv + (size_t)n * p.ld_qkv + p.k_off + g * D;
  const float* vr = p.qkv + (size_t)n * p.ld_qkv + p.v_off + g * D;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = (i >> 1) * 64 + 8 * j + 4 * (i & 1);
    t.k[i] = *reinterpret_cast<const f32x4_t*>(kr + d);
    t.v[i] = *reinterpret_cast<const f32x4_t*>(vr + d);
  }
  // without k_norm the weight loads read the row itself (ignored)
  const uint16_t* nwb = p.k_norm ? p.k_norm : reinterpret_cast<const uint16_t*>(kr);
  t.nw[0] = ld_u32x4(nwb + 8 * j);
  t.nw[1] = ld_u32x4(nwb + 64 + 8 * j);
  const float* cr = p.rope_cos + n * 64 + 8 * j;
  const float* sr = p.rope_sin + n * 64 + 8 * j;
  t.cs[0] = *reinterpret_cast<const f32x4_t*>(cr);
  t.cs[1] = *reinterpret_cast<const f32x4_t*>(cr + 4);
  t.sn[0] = *reinterpret_cast<const f32x4_t*>(sr);
  t.sn[1] = *reinterpret_cast<const f32x4_t*>(sr + 4);
}

// k: RMSNorm (k_norm) then RoPE; v: zero past the tree. Both go to the
// chunk's LDS staging as bf16 (K rows [32][D + 8], V^T [D][40]) and, when
// this workgroup appends (query block 0, first head of the KV group), to the
// cache rows P + node.
__device__ __forceinline__ void tree_rows_stage(const AttnParams& p, const TreeRows& t, int g, bool append, int P,
                                                int L, int tc, uint16_t* ks, uint16_t* vt) {
  constexpr int D = 128, KS = D + 8, VS = 32 + 8;
  const int r = threadIdx.x >> 3, j = threadIdx.x & 7, n = 32 * tc + r;
  float k[16], v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      k[4 * i + e] = t.k[i][e];
      v[4 * i + e] = n < L ? t.v[i][e] : 0.f;
    }
  if (p.k_norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss += k[i] * k[i];
    ss += dpp<0xB1>(ss);   // lane ^ 1
    ss += dpp<0x4E>(ss);   // lane ^ 2
    ss += dpp<0x141>(ss);  // the other quad of the row's 8 lanes
    const float rs = rsqrtf(ss * (1.0f / D) + p.eps);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t w = t.nw[i >> 3][(i & 7) >> 1];
      k[i] *= rs * ((i & 1) ? bf_hi(w) : bf_lo(w));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float cs = t.cs[i >> 2][i & 3], sn = t.sn[i >> 2][i & 3];
    const float x1 = k[i], x2 = k[8 + i];
    k[i] = x1 * cs - x2 * sn;
    k[8 + i] = x1 * sn + x2 * cs;
  }
  const u32x4_t k0{pack_bf2(k[0], k[1]), pack_bf2(k[2], k[3]), pack_bf2(k[4], k[5]), pack_bf2(k[6], k[7])};
  const u32x4_t k1{pack_bf2(k[8], k[9]), pack_bf2(k[10], k[11]), pack_bf2(k[12], k[13]), pack_bf2(k[14], k[15])};
  *reinterpret_cast<u32x4_t*>(&ks[r * KS + 8 * j]) = k0;
  *reinterpret_cast<u32x4_t*>(&ks[r * KS + 64 + 8 * j]) = k1;
  uint16_t vb[16];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const uint32_t w = pack_bf2(v[i], v[i + 1]);
    vb[i] = (uint16_t)(w & 0xffffu);
    vb[i + 1] = (uint16_t)(w >> 16);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    vt[(8 * j + i) * VS + r] = vb[i];
    vt[(64 + 8 * j + i) * VS + r] = vb[8 + i];
  }
  if (append && n < L) {
    const int pos = P + n;
    const int page = p.page_table[pos / DTREE_PAGE], off = pos % DTREE_PAGE;
    uint16_t* kblk = p.kp + (size_t)(page * p.Hkv + g) * DTREE_PAGE * D;
    uint16_t* vblk = p.vp + (size_t)(page * p.Hkv + g) * DTREE_PAGE * D;
    // dims 8j .. 8j+7 (and 64 + 8j ..) of a key are one 16-byte run of the K block
    *reinterpret_cast<u32x4_t*>(kblk + kv_k_off(off, 8 * j, D)) = k0;
    *reinterpret_cast<u32x4_t*>(kblk + kv_k_off(off, 64 + 8 * j, D)) = k1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      vblk[kv_v_off(off, 8 * j + i, D)] = vb[i];
      vblk[kv_v_off(off, 64 + 8 * j + i, D)] = vb[8 + i];
    }
  }
}

// One prefix chunk = CK consecutive keys inside one page (the whole page for
// head_dim 128, half of it for 256): its K and V fragments, loaded by
// prefix_issue and consumed by prefix_chunk. Keys past the
// prefix in the last chunk are masked (scores) and zeroed (V), since the page
// may hold stale or non-finite data there.
template <int D>
struct ChunkKV {
  static constexpr int NJ = D / 16, ND = D / 32, NB = chunk_keys(D) / 32;
  u32x4_t kf[NB][NJ];
  u32x4_t vf[NB][2][ND];
};

template <int D>
__device__ __forceinline__ void prefix_issue(const AttnParams& p, ChunkKV<D>& kv, int page, int g, int pc, int c,
                                             int h) {
  constexpr int NJ = D / 16, ND = D / 32;
  constexpr int CK = chunk_keys(D), NB = CK / 32;
  // The page block stores every fragment as one contiguous kilobyte in lane
  // order (kv_k_off / kv_v_off): K fragment (j, key half) and V fragment (key
  // step, dim block) are each one fully coalesced 16-byte load per lane.
  const int po = (pc * CK) % DTREE_PAGE;
  const int lane = 32 * h + c;
  const uint16_t* kbase = p.kp + (size_t)(page * p.Hkv + g) * DTREE_PAGE * D + 8 * lane;
  const uint16_t* vbase = p.vp + (size_t)(page * p.Hkv + g) * DTREE_PAGE * D + 8 * lane;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) kv.kf[b][j] = ld_u32x4_stream(kbase + (size_t)((po / 32 + b) * NJ + j) * 512);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int db = 0; db < ND; ++db)
        kv.vf[b][s2][db] = ld_u32x4_stream(vbase + (size_t)((po / 16 + 2 * b + s2) * ND + db) * 512);
  }
}

template <int D, int R, bool QS>
__device__ __forceinline__ void prefix_chunk(const AttnParams& p, HeadRow<D, R>& qr, const float* qs,
                                             const ChunkKV<D>& kv, int P, int pc, int c, int h, float& m_run,
                                             float& l_run, f32x16_t (&o)[D / 32]) {
  constexpr int NJ = D / 16, ND = D / 32;
  constexpr int CK = chunk_keys(D), NB = CK / 32;
  const int k_begin = pc * CK;  // prefix chunk pc: keys pc*CK ..
  const int k_end = min(k_begin + CK, P);
  constexpr bool PERJ = QS && D > 128;  // staged head_dim 256: one fragment at a time
  u32x4_t qf[PERJ ? 1 : NJ], ql[PERJ ? 1 : NJ];
  if constexpr (!QS) q_fragments<D, R>(qr, p.q_norm != nullptr, p.eps, qf, ql);
  else if constexpr (!PERJ) q_frag_lds<D>(qs, c, h, qf, ql);

  f32x16_t s[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[b][r] = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    u32x4_t f, l;
    if constexpr (PERJ) q_frag_one<D>(qs, c, h, j, f, l);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      s[b] = mfma32(kv.kf[b][j], PERJ ? f : qf[PERJ ? 0 : j], s[b]);
      s[b] = mfma32(kv.kf[b][j], PERJ ? l : ql[PERJ ? 0 : j], s[b]);
    }
  }
  const bool ragged = k_end - k_begin < CK;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k_begin + 32 * b + 16 * (r >> 3) + 8 * h + (r & 7);
      s[b][r] = (!ragged || key < k_end) ? s[b][r] * p.scale_log2 : kNeg;
    }
  softmax_fresh<NB>(s, m_run, l_run);
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      u32x4_t va[ND];
      const int first = k_begin + 32 * b + 16 * s2 + 8 * h;
#pragma unroll
      for (int db = 0; db < ND; ++db)
        va[db] = ragged ? mask_keys(kv.vf[b][s2][db], first, k_end) : kv.vf[b][s2][db];
      pv_step<ND>(s[b], s2, va, o);
    }
}

// ---- flag exchange between a head's splits (rows_padded 32) ----------------
// Each split's merged result (row max M, row sum, unnormalised 32 x D output)
// is published as (value, flag) pairs, flag = the launch's epoch + 1, with
// write-through stores whose acknowledgement nobody waits for: a reader takes
// a pair as valid once its flag matches, and an aligned 8-byte store is seen
// whole or not at all. The output is cut into 4 * D / 32 units (32-dim block
// db, 8-dim group gq: four consecutive dims of each query per lane); unit u is
// combined by split u % S, which reads only its partners' pairs of that unit
// and their row statistics, so no split waits for a counter, an
// acknowledgement or a last arriver, and the combine's reads are spread over
// the S workgroups.
//
// Waves 0 and 1 publish, waves 2 and 3 combine: a wave's memory operations
// complete in issue order, so a wave that had just issued write-through
// stores would wait for their acknowledgement (~2 us) before its poll loads
// return. The merged blocks sit in LDS (xm: the merge's exchange slots,
// block db in owner wave db % 4's slot) for both roles.
//
// Epochs: every split reads its head's epoch word E at its start and flags
// its pairs E + 1. A combiner that has seen all partners' flags knows every
// split of this launch has read E, so it raises the word to E + 1 (atomic
// max) for the next launch; slots are stale only with older flags, since a
// slot's place depends on the head count and head dim alone. The wait is
// bounded: a combiner that gives up sets the error word, raises the epoch past
// E + 1, leaves its units unwritten, and dtree_attention_status moves every
// epoch of the table far ahead before the step is recomputed.
template <int D, bool GATE>
__device__ __forceinline__ void ll_exchange(const AttnParams& p, int hq, int split, int S, int wave, int lane, int c,
                                            int h, float M, float tot, const f32x4_t* xm, uint32_t F, int L) {
  constexpr int ND = D / 32, NU = 4 * ND;
  constexpr unsigned kSlot = attn_ll_slot_bytes(D);
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(p.ll_slots, p.ll_bytes);
  const unsigned base = (unsigned)hq * kAttnLLSplits * kSlot;
  // merged values of unit u for this lane: block u / 4 in its owner's slot
  auto own_unit = [&](int u) -> f32x4_t {
    const int db = u >> 2, gq = u & 3;
    return xm[((db * kWaves + db % kWaves) * 4 + gq) * 64 + lane];
  };
  if (wave < 2) {
    // ---- publish: row statistics, then every unit another split combines ----
    // Workgroups go round-robin over the 8 XCDs (workgroup i of a launch to
    // XCD (i + s) % 8, s the dispatcher's position when the launch starts), so
    // with Hkv % 8 == 0 a head's splits, which share blockIdx % 8, share one
    // XCD: there the pairs go to the shared L2 with plain stores
    // (acknowledged by the L2, which serves the partners' polls). Otherwise
    // (or with the test hook) they are written through (sc1) to memory, where
    // polls from another XCD find them. Were placement ever different, the
    // polls would give up and the launch report the error.
    const bool native = !p.off_xcd && p.Hkv % kXcds == 0;
    const unsigned own = base + (unsigned)split * kSlot;
    if (wave == 0 && h == 0) {
      const u32x4_t st{__float_as_uint(M), F, __float_as_uint(tot), F};
      if (native) __builtin_amdgcn_raw_buffer_store_b128(st, rs, (int)(own + 16u * c), 0, 0);
      else __builtin_amdgcn_raw_buffer_store_b128(st, rs, (int)(own + 16u * c), 0, kSc1);
    }
#pragma unroll
    for (int u = wave; u < NU; u += 2) {
      if (u % S == split) continue;
      const f32x4_t v = own_unit(u);
      const float v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
      // two contiguous kilobytes per unit (every store instruction writes
      // whole cache lines): values 0, 1 of each lane, then values 2, 3
      const unsigned off = own + 512u + (unsigned)u * 2048u + (unsigned)lane * 16u;
      const u32x4_t s0{__float_as_uint(v0), F, __float_as_uint(v1), F}, s1{__float_as_uint(v2), F,
                                                                           __float_as_uint(v3), F};
      if (native) {
        __builtin_amdgcn_raw_buffer_store_b128(s0, rs, (int)off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(s1, rs, (int)(off + 1024u), 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(s0, rs, (int)off, 0, kSc1);
        __builtin_amdgcn_raw_buffer_store_b128(s1, rs, (int)(off + 1024u), 0, kSc1);
      }
    }
    return;
  }
  // ---- combine: units split, split + S, ...; wave 2 takes every other one ----
  const unsigned partners = ((1u << S) - 1u) & ~(1u << split);
  const int orow = c;  // query block 0 (rows_padded 32)
  bool seen = false, gave_up = false;
  // A wave's loads complete after its earlier stores, so the output stores
  // wait until every unit of the wave is combined.
  constexpr int kMaxU = NU / 4;  // units per combining wave at S >= 2
  float yo[kMaxU][4];
  int uo_dim[kMaxU];
#pragma unroll
  for (int i = 0; i < kMaxU; ++i) uo_dim[i] = -1;
#pragma unroll
  for (int i = 0; i < kMaxU; ++i) {
    const int u = split + S * (wave - 2) + 2 * S * i;
    if (u >= NU || gave_up) break;
    float pm[kAttnLLSplits], pt[kAttnLLSplits];
    f32x4_t pv[kAttnLLSplits];
#pragma unroll
    for (int q = 0; q < kAttnLLSplits; ++q) {
      pm[q] = kNeg;
      pt[q] = 0.f;
      pv[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (p.spin_limit < 0) {  // test hook: give up before the first poll
      gave_up = true;
      break;
    }
    unsigned pend = partners;  // partners some lane of the wave still lacks
    int it = 0;
    while (true) {
      u32x4_t a[kAttnLLSplits], b0[kAttnLLSplits], b1[kAttnLLSplits];
#pragma unroll
      for (int q = 0; q < kAttnLLSplits; ++q) {
        const bool want = (pend >> q) & 1u;
        const unsigned qs = base + (unsigned)q * kSlot;
        const unsigned uo = qs + 512u + (unsigned)u * 2048u + (unsigned)lane * 16u;
        a[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(want ? qs + 16u * c : kOob), 0, kSc1);
        b0[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(want ? uo : kOob), 0, kSc1);
        b1[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(want ? uo + 1024u : kOob), 0, kSc1);
      }
      unsigned still = 0;
#pragma unroll
      for (int q = 0; q < kAttnLLSplits; ++q) {
        if (!((pend >> q) & 1u)) continue;
        const bool ok = a[q][1] == F && a[q][3] == F && b0[q][1] == F && b0[q][3] == F && b1[q][1] == F &&
                        b1[q][3] == F;
        if (ok) {
          const uint32_t a0 = a[q][0], a2 = a[q][2], c0 = b0[q][0], c2 = b0[q][2], d0 = b1[q][0], d2 = b1[q][2];
          pm[q] = __uint_as_float(a0);
          pt[q] = __uint_as_float(a2);
          pv[q] = f32x4_t{__uint_as_float(c0), __uint_as_float(c2), __uint_as_float(d0), __uint_as_float(d2)};
        }
        if (__builtin_amdgcn_ballot_w64(!ok)) still |= 1u << q;
      }
      pend = still;
      if (!pend) break;
      if (++it > p.spin_limit) {
        gave_up = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      asm volatile("" ::: "memory");  // the next round's loads are issued again
    }
    if (gave_up) break;
    seen = true;
    // Splits in split order, so every combiner of the head forms the same
    // row max and sum.
    const f32x4_t mv = own_unit(u);
    const float m4[4] = {mv[0], mv[1], mv[2], mv[3]};
    float Mx = M;
#pragma unroll
    for (int q = 0; q < kAttnLLSplits; ++q)
      if ((partners >> q) & 1u) Mx = fmaxf(Mx, pm[q]);
    float T = 0.f, y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < kAttnLLSplits; ++q) {
      if (q >= S) continue;
      const bool me = q == split;
      const float w = fast_exp2((me ? M : pm[q]) - Mx);
      T += w * (me ? tot : pt[q]);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] += w * (me ? m4[i] : pv[q][i]);
    }
    const float inv = (orow < L && T > 0.f) ? 1.0f / T : 0.f;
    const int db = u >> 2, gq = u & 3;
    const int dim = 32 * db + 8 * gq + 4 * h;
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = orow < L ? y[i] * inv : 0.f;
    if (GATE && orow < L) {
      const f32x4_t gt =
          *reinterpret_cast<const f32x4_t*>(p.qkv + (size_t)orow * p.ld_qkv + hq * p.q_stride + D + dim);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] *= 1.0f / (1.0f + __expf(-gt[i]));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) yo[i][e] = y[e];
    uo_dim[i] = dim;
  }
#pragma unroll
  for (int i = 0; i < kMaxU; ++i) {
    if (uo_dim[i] < 0) continue;
    const int col = hq * D + uo_dim[i];
    const size_t oi = p.out_tiled ? tiled_index(orow, col, p.ld_out) : (size_t)orow * p.ld_out + col;
    store_act4(p.out, p.out_lo, oi, yo[i], p.out_h16);
  }
  if (lane == 0 && (seen || gave_up)) {
    __hip_atomic_fetch_max(p.ll_epoch + hq, gave_up ? F + 1u : F, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gave_up) __hip_atomic_fetch_or(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Combine of a head's workgroup partials ([block][lane][16] floats, then m and
// l of the 32 queries, per split) by the last workgroup to arrive: kSb splits
// per round with every load of the round in flight (ranged loads past the
// last split return zero) and a running max; AUX is the cache policy of the
// loads (kSc0: all writers on this XCD, else kSc1).
template <int D, int AUX>
__device__ __forceinline__ void combine_splits(__amdgpu_buffer_rsrc_t prs, unsigned pbase, size_t stride, int nsplit,
                                               int wave, int lane, int c, float& tot,
                                               f32x16_t (&mine)[D / 32 / kWaves]) {
  constexpr int NDW = D / 32 / kWaves;
  constexpr int kSb = 8 / NDW;  // 8 splits per round at head_dim 128, 4 at 256
  float Ms = kNeg;
  tot = 0.f;
#pragma unroll
  for (int k = 0; k < NDW; ++k)
#pragma unroll
    for (int r = 0; r < 16; ++r) mine[k][r] = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kSb) {
    f32x4_t v[kSb][NDW][4];
    float mm[kSb], ll[kSb];
#pragma unroll
    for (int b = 0; b < kSb; ++b) {
      const bool ok = s0 + b < nsplit;
      const unsigned so = ok ? pbase + (unsigned)((size_t)(s0 + b) * stride * sizeof(float)) : kOob;
      const float mv = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(so + (32 * D + c) * 4), 0, AUX));
      ll[b] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (int)(so + (32 * D + 32 + c) * 4),
                                                                            0, AUX));
      mm[b] = ok ? mv : kNeg;
#pragma unroll
      for (int k = 0; k < NDW; ++k)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
          v[b][k][gq] = __builtin_bit_cast(
              f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                           prs, (int)(so + (unsigned)(((wave + kWaves * k) * 64 + lane) * 64 + 16 * gq)), 0, AUX));
    }
    float gm = Ms;
#pragma unroll
    for (int b = 0; b < kSb; ++b) gm = fmaxf(gm, mm[b]);
    const float rsc = fast_exp2(Ms - gm);
    tot *= rsc;
#pragma unroll
    for (int k = 0; k < NDW; ++k)
#pragma unroll
      for (int r = 0; r < 16; ++r) mine[k][r] *= rsc;
#pragma unroll
    for (int b = 0; b < kSb; ++b) {
      const float w = fast_exp2(mm[b] - gm);
      tot += w * ll[b];
#pragma unroll
      for (int k = 0; k < NDW; ++k)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
#pragma unroll
          for (int i = 0; i < 4; ++i) mine[k][4 * gq + i] += w * v[b][k][gq][i];
    }
    Ms = gm;
  }
}

// TB: tree chunks the LDS staging is sized for (1 for 32 rows, 4 up to 128).
template <int D, int R, bool GATE, int TB>
__global__ __launch_bounds__(64 * kWaves) void tree_attn_kernel(AttnParams p) {
  constexpr int ND = D / 32;  // 32-dim blocks of O^T
  constexpr int KS = D + 8;   // padded LDS row of tree K
  constexpr int VS = 32 + 8;  // padded LDS row of tree V^T
  constexpr int kStage = (32 * KS + D * VS) * 2;   // one tree chunk's K / V^T staging
  // Query rows are staged in LDS except for head_dim 256 with four tree
  // chunks (their K/V staging leaves no room).
  constexpr bool QS = D <= 128 || TB == 1;
  constexpr int kQs = QS ? 32 * qs_stride<D>() * 4 : 0;  // staged query rows
  constexpr int kMl = kWaves * 64 * 4;               // merge: per wave, m and l of 32 queries
  constexpr int kMerge = kMl + ND * kWaves * 4 * 64 * 16;  // + [block][wave][4][lane] f32x4
  constexpr int kChunkLds = TB * kStage + kQs;
  constexpr int CK = chunk_keys(D);
  constexpr bool TF = D == 128;  // tree chunks first, in a split of their own, staged by the workgroup
  __shared__ __align__(16) unsigned char lds[kChunkLds > kMerge ? kChunkLds : kMerge];
  __shared__ int s_last;

  // Every argument the prologue needs in scalar registers at once: one batch
  // of argument loads and one wait, instead of a batch per basic block.
  asm volatile("" ::"s"(p.qkv), "s"(p.ld_qkv), "s"(p.q_stride), "s"(p.q_norm), "s"(p.rope_cos), "s"(p.rope_sin),
               "s"(p.kp), "s"(p.vp), "s"(p.page_table), "s"(p.desc), "s"(p.Hq), "s"(p.Hkv), "s"(p.max_chunks),
               "s"(p.splits), "s"(p.tree_chunks), "s"(gridDim.x));
  // blockIdx -> (query block, split, kv group, head in group): the G heads of
  // one (split, group) pair share blockIdx % 8, i.e. one XCD.
  const int G = p.Hq / p.Hkv, NT = p.tree_chunks;
  const int per_block = (int)gridDim.x / NT;  // workgroups per query block (a multiple of 8)
  const int rb = blockIdx.x / per_block, bid = blockIdx.x % per_block;
  const int pair = (bid / (8 * G)) * 8 + (bid & 7);
  // Padding workgroups (pair past splits * Hkv) still name an in-range head
  // and a chunk past max_chunks; they return after the loads below are out,
  // which keeps the argument loads in one round trip.
  const int g = pair % p.Hkv, split = pair / p.Hkv;
  const int hq = g * G + (bid >> 3) % G;
  // The head's exchange epoch (flag exchange), read before anything of this
  // launch can raise it.
  const uint32_t ll_flag =
      p.ll ? __hip_atomic_load(p.ll_epoch + hq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u : 0u;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int qrow = 32 * rb + c;  // this lane's query row
  // Chunk roles. head_dim 128 (TF): split 0 holds the tree chunks alone (wave
  // tc scores tree chunk tc; the whole workgroup stages them) and prefix chunk
  // pc is wave pc % 4 of split 1 + pc / 4. head_dim 256: chunk split * 4 +
  // wave, prefix chunks first, then the tree chunks.
  const int chunk = split * kWaves + wave;
  const int pc_fixed = TF ? (split - 1) * kWaves + wave : chunk;  // prefix chunk, if this wave has one
  // Loads that do not depend on the step descriptor go out first, so their
  // latency overlaps the descriptor read: the workgroup's query rows (values,
  // norm weights, RoPE; 10 loads per thread), the page of this wave's prefix
  // chunk and (TF, split 0) the first tree chunk's k / v rows. The prefix
  // chunk's K/V follow the descriptor check: issued before it, they delay the
  // descriptor's own (scalar) load by microseconds.
  // (head_dim 256 with four tree chunks loads its q row per wave inside the
  // chunk: there is no LDS left to stage it.)
  const bool prefix_wave = (!TF || split > 0) && pc_fixed < p.max_chunks - NT;  // at the longest prefix
  const int page = prefix_wave ? p.page_table[pc_fixed * CK / DTREE_PAGE] : 0;
  HeadRow<D, R> qr;
  QStage<D> qst;
  if constexpr (QS) q_stage_issue<D>(p, hq, rb, qst);
  TreeRows trows;
  if constexpr (TF) {
    if (split == 0) tree_rows_issue(p, g, 0, trows);
  }

  if (pair >= p.splits * p.Hkv) return;
  const int P = p.desc->past_length, L = p.desc->num_nodes;
  const int npre = (P + CK - 1) / CK, nchunks = NT + npre;
  // A descriptor beyond the grid's capacity (P > max_past_length) or with more
  // rows than rows_padded leaves the output untouched instead of indexing past
  // buffers.
  if (nchunks > p.max_chunks || L > 32 * NT || L < 1) return;
  const int nsplit = head_nsplit(D, npre, NT);
  if (split >= nsplit) return;
  if (32 * rb >= L) {
    // Query block past the tree: its output rows are zero (split 0 writes).
    if (split == 0) {
      const int q = threadIdx.x >> 3;
      for (int dd = (threadIdx.x & 7) * 8; dd < D; dd += 64) {
        const int col = hq * D + dd;
        const int row = 32 * rb + q;
        const size_t oi = p.out_tiled ? tiled_index(row, col, p.ld_out) : (size_t)row * p.ld_out + col;
        *reinterpret_cast<u32x4_t*>(p.out + oi) = u32x4_t{0u, 0u, 0u, 0u};
        if (p.out_lo) *reinterpret_cast<u32x4_t*>(p.out_lo + oi) = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    return;
  }

  float* qs = reinterpret_cast<float*>(lds + TB * kStage);
  if constexpr (QS) q_stage_finish<D>(qst, p.q_norm != nullptr, p.eps, qs);
  if constexpr (TF) {
    // Split 0 stages tree chunks 0 .. rb (later chunks hold no ancestor of
    // this query block's rows); query block 0 stages and appends them all.
    if (split == 0) {
      const bool append = p.write_cache && (hq % G) == 0 && rb == 0;
      const int last = rb == 0 ? NT - 1 : rb;
      for (int tc = 0; tc <= last && 32 * tc < L; ++tc) {
        if (tc > 0) tree_rows_issue(p, g, tc, trows);
        uint16_t* ks = reinterpret_cast<uint16_t*>(lds + (size_t)tc * kStage);
        tree_rows_stage(p, trows, g, append, P, L, tc, ks, ks + 32 * KS);
      }
    }
  }
  if constexpr (QS || TF) lds_barrier();

  float m_run = kNeg, l_run = 0.f;
  f32x16_t o[ND];
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

  const int tc = TF ? (split == 0 ? wave : -1) : chunk - npre;  // tree chunk index
  const int pc = TF ? (split == 0 ? npre : pc_fixed) : chunk;   // prefix chunk index (npre: none)
  if (tc >= 0 && tc < NT) {
    // Each tree chunk has its own staging.
    if (32 * tc < L && (!TF || tc <= rb)) {
      uint16_t* ks = reinterpret_cast<uint16_t*>(lds + (size_t)tc * kStage);
      tree_chunk<D, R, QS, TF>(p, qr, qs, hq, g, G, P, L, tc, qrow, rb == 0, c, h, ks, ks + 32 * KS, m_run, l_run,
                               o);
    }
  } else if (pc < npre) {
    if constexpr (!QS)
      row_issue<D, R, true>(qr, p.qkv + (size_t)qrow * p.ld_qkv + hq * p.q_stride, p.q_norm,
                            p.rope_cos + qrow * (R / 2), p.rope_sin + qrow * (R / 2), h);
    ChunkKV<D> kv;
    prefix_issue<D>(p, kv, page, g, pc, c, h);
    prefix_chunk<D, R, QS>(p, qr, qs, kv, P, pc, c, h, m_run, l_run, o);
  }

  // ---- merge the four waves ----
  // o holds this wave's chunk for the 32 queries x D dims in MFMA layout:
  // lane (c, h), register r of block db = dim 32 db + acc_row(r, h) of query
  // c. Wave w completes blocks db = w, w + 4, ...: every wave rescales its o
  // to the common max and hands the blocks it does not complete to their
  // owners through LDS in 16-byte pieces.
  constexpr int NDW = ND / kWaves;  // blocks a wave completes: 1 (head_dim 128), 2 (256)
  float* ml = reinterpret_cast<float*>(lds);             // [wave][m | l][32]
  f32x4_t* xch = reinterpret_cast<f32x4_t*>(lds + kMl);  // [block][wave][4][lane]
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  lds_barrier();  // retires the chunk staging (tree K/V, query rows), which shares this memory
  if (h == 0) {
    ml[wave * 64 + c] = m_run;
    ml[wave * 64 + 32 + c] = l_tot;
  }
  lds_barrier();
  float M = kNeg, tot = 0.f, self = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ml[w * 64 + c]);
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float f = fast_exp2(ml[w * 64 + c] - M);
    tot += f * ml[w * 64 + 32 + c];
    if (w == wave) self = f;
  }
#pragma unroll
  for (int db = 0; db < ND; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] *= self;
    if (db % kWaves != wave) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        xch[((db * kWaves + wave) * 4 + gq) * 64 + lane] =
            f32x4_t{o[db][4 * gq], o[db][4 * gq + 1], o[db][4 * gq + 2], o[db][4 * gq + 3]};
    }
  }
  lds_barrier();
  f32x16_t mine[NDW];  // completed blocks wave + kWaves * k
#pragma unroll
  for (int db = 0; db < ND; ++db) {
    if (db % kWaves != wave) continue;
    f32x16_t a = o[db];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      if (w == wave) continue;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4_t x = xch[((db * kWaves + w) * 4 + gq) * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[4 * gq + i] += x[i];
      }
    }
    mine[db / kWaves] = a;
  }

  if (nsplit > 1 && p.ll && nsplit <= kAttnLLSplits) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      // where dtree_attention_status finds the epoch table after a give-up
      p.err[2] = (int)(reinterpret_cast<const unsigned char*>(p.ll_epoch) - reinterpret_cast<const unsigned char*>(p.err));
      p.err[3] = p.Hq;
    }
    // Owner waves put their merged blocks in their own (unused) exchange
    // slots, where both exchange roles read them.
#pragma unroll
    for (int k = 0; k < NDW; ++k) {
      const int db = wave + kWaves * k;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        xch[((db * kWaves + wave) * 4 + gq) * 64 + lane] =
            f32x4_t{mine[k][4 * gq], mine[k][4 * gq + 1], mine[k][4 * gq + 2], mine[k][4 * gq + 3]};
    }
    lds_barrier();
    ll_exchange<D, GATE>(p, hq, split, nsplit, wave, lane, c, h, M, tot, xch, ll_flag, L);
    return;
  }
  if (nsplit > 1) {
    // Workgroup partial: [block][lane][16] floats (each lane moves its block
    // values in 16-byte agent-coherent stores and loads), then m and l of the
    // 32 queries.
    const size_t stride = (size_t)32 * D + 64;
    const int hb = hq * NT + rb;  // (head, query block)
    const __amdgpu_buffer_rsrc_t prs =
        buf_rsrc(p.part, (unsigned)((size_t)p.Hq * NT * p.splits * stride * sizeof(float)));
    const unsigned pbase = (unsigned)((size_t)hb * p.splits * stride * sizeof(float));
    const unsigned mine_off = pbase + (unsigned)((size_t)split * stride * sizeof(float));
#pragma unroll
    for (int k = 0; k < NDW; ++k) {
      const unsigned off = mine_off + (unsigned)(((wave + kWaves * k) * 64 + lane) * 64);
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4_t, f32x4_t{mine[k][4 * gq], mine[k][4 * gq + 1], mine[k][4 * gq + 2],
                                                mine[k][4 * gq + 3]}),
            prs, (int)(off + 16 * gq), 0, kSc1);
    }
    float* part = p.part + ((size_t)hb * p.splits + split) * stride;
    if (wave == 0 && h == 0) {
      st_coherent(part + 32 * D + c, M);
      st_coherent(part + 32 * D + 32 + c, tot);
    }
    if (p.sep_combine) return;  // attn_combine_kernel (next launch) reads the partials
    wait_stores_done();
    __syncthreads();
    if (threadIdx.x == 0) {
      // arrival count in the low half, workgroups off their XCD in the high
      const bool native = !p.off_xcd && xcc_id() == (int)(blockIdx.x % kXcds);
      const int old = arrive_add(&p.counters[hb], native ? 1 : 1 + kForeign);
      int last = 0;
      if ((old & (kForeign - 1)) == nsplit - 1) {
        last = native && old < kForeign && p.Hkv % kXcds == 0 ? 2 : 1;
        reset_counter(&p.counters[hb]);
      }
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;

    // Every split of this head ran on this XCD when all are confirmed on
    // their expected XCD and the heads of a KV group's splits share one
    // (Hkv % 8 == 0): the partials are then read from the local L2.
    if (s_last == 2) combine_splits<D, kSc0>(prs, pbase, stride, nsplit, wave, lane, c, tot, mine);
    else combine_splits<D, kSc1>(prs, pbase, stride, nsplit, wave, lane, c, tot, mine);
  }

  // Output: lane (c, h) holds, per completed block, 4 runs of 4 consecutive
  // dims (registers 4g .. 4g+3 = dims 32 db + 8g + 4h .. +3) of query c.
  const int orow = 32 * rb + c;
  const float inv = (orow < L && tot > 0.f) ? 1.0f / tot : 0.f;
#pragma unroll
  for (int k = 0; k < NDW; ++k) {
    const int db = wave + kWaves * k;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int dim = 32 * db + 8 * gq + 4 * h;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = orow < L ? mine[k][4 * gq + i] * inv : 0.f;
      if (GATE && orow < L) {
        // o_proj input = attention * sigmoid(gate), gate = q_proj row dims D.. of the head
        const f32x4_t gt = *reinterpret_cast<const f32x4_t*>(p.qkv + (size_t)orow * p.ld_qkv + hq * p.q_stride + D +
                                                             dim);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] *= 1.0f / (1.0f + __expf(-gt[i]));
      }
      const int col = hq * D + dim;
      const size_t oi = p.out_tiled ? tiled_index(orow, col, p.ld_out) : (size_t)orow * p.ld_out + col;
      store_act4(p.out, p.out_lo, oi, y, p.out_h16);
    }
  }
}

// Combine of the workgroup partials for long prefixes, as a launch of its
// own: with S splits the in-kernel last arriver reads S partial tiles of
// 32 x D fp32 alone (544 KB at head_dim 256, P = 2048), which one CU's load
// bandwidth turns into ~18 us. Here one workgroup per (head, query block,
// 32-dim block) reads S x 4 KB: wave w takes splits w, w + 4, ... with a
// running max, the four waves merge in LDS and wave 0 writes the block's
// output (normalised, gated, bf16 pair). Splits and partial layout are the
// main kernel's; with one split or a query block past the tree the main
// kernel has written the output itself.
template <int D, bool GATE>
__global__ __launch_bounds__(64 * kWaves) void attn_combine_kernel(AttnParams p) {
  constexpr int ND = D / 32;
  constexpr int kB = 8;  // splits in flight per wave
  const int NT = p.tree_chunks;
  const int db = blockIdx.x % ND, hb = blockIdx.x / ND;  // hb = head * NT + query block
  const int hq = hb / NT, rb = hb % NT;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  constexpr int CK = chunk_keys(D);
  const int P = p.desc->past_length, L = p.desc->num_nodes;
  const int npre = (P + CK - 1) / CK, nchunks = NT + npre;
  if (nchunks > p.max_chunks || L > 32 * NT || L < 1) return;  // the main kernel's guards
  const int nsplit = head_nsplit(D, npre, NT);
  if (nsplit <= 1 || 32 * rb >= L) return;
  if (p.ll && nsplit <= kAttnLLSplits) return;  // the main kernel combined through the exchange
  const size_t stride = (size_t)32 * D + 64;
  const __amdgpu_buffer_rsrc_t prs =
      buf_rsrc(p.part, (unsigned)((size_t)p.Hq * NT * p.splits * stride * sizeof(float)));
  const unsigned pbase = (unsigned)((size_t)hb * p.splits * stride * sizeof(float));
  float Ms = kNeg, tot = 0.f;
  f32x4_t acc[4];
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) acc[gq] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < nsplit; s0 += kWaves * kB) {
    f32x4_t v[kB][4];
    float mm[kB], ll[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int sp = s0 + kWaves * b;
      const unsigned so = sp < nsplit ? pbase + (unsigned)((size_t)sp * stride * sizeof(float)) : kOob;
      const float mv = buf_ldf(prs, so + (32 * D + c) * 4);
      ll[b] = buf_ldf(prs, so + (32 * D + 32 + c) * 4);
      mm[b] = sp < nsplit ? mv : kNeg;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        v[b][gq] = __builtin_bit_cast(f32x4_t, buf_ld(prs, so + (unsigned)((db * 64 + lane) * 64 + 16 * gq)));
    }
    float gm = Ms;
#pragma unroll
    for (int b = 0; b < kB; ++b) gm = fmaxf(gm, mm[b]);
    const float rsc = fast_exp2(Ms - gm);
    tot *= rsc;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) acc[gq] *= rsc;
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const float w = fast_exp2(mm[b] - gm);  // 0 for splits past nsplit
      tot += w * ll[b];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) acc[gq] += w * v[b][gq];
    }
    Ms = gm;
  }
  // Merge the four waves (in wave order) into wave 0.
  __shared__ float ml[kWaves][2][64];
  __shared__ f32x4_t xa[kWaves - 1][4][64];
  ml[wave][0][lane] = Ms;
  ml[wave][1][lane] = tot;
  if (wave > 0) {
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) xa[wave - 1][gq][lane] = acc[gq];
  }
  __syncthreads();
  if (wave != 0) return;
  float M = kNeg;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ml[w][0][lane]);
  float T = 0.f;
  f32x4_t o[4];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float f = fast_exp2(ml[w][0][lane] - M);
    T += f * ml[w][1][lane];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const f32x4_t x = w == 0 ? acc[gq] : xa[w - 1][gq][lane];
      o[gq] = w == 0 ? f * x : o[gq] + f * x;
    }
  }
  // Output of query c, dims 32 db + 8 gq + 4 h .. +3 (MFMA accumulator layout).
  const int orow = 32 * rb + c;
  const float inv = (orow < L && T > 0.f) ? 1.0f / T : 0.f;
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int dim = 32 * db + 8 * gq + 4 * h;
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = orow < L ? o[gq][i] * inv : 0.f;
    if (GATE && orow < L) {
      const f32x4_t gt =
          *reinterpret_cast<const f32x4_t*>(p.qkv + (size_t)orow * p.ld_qkv + hq * p.q_stride + D + dim);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] *= 1.0f / (1.0f + __expf(-gt[i]));
    }
    const int col = hq * D + dim;
    const size_t oi = p.out_tiled ? tiled_index(orow, col, p.ld_out) : (size_t)orow * p.ld_out + col;
    store_act4(p.out, p.out_lo, oi, y, p.out_h16);
  }
}

}  // namespace head_attn
}  // namespace dtree

using namespace dtree::head_attn;

constexpr size_t kSepCombineBytes = 128 * 1024;

static int attn_max_chunks(int head_dim, int max_past, int nt) {
  const int ck = chunk_keys(head_dim);
  return nt + (max_past + ck - 1) / ck;
}
static int attn_splits(int head_dim, int max_past, int nt) {
  return head_nsplit(head_dim, attn_max_chunks(head_dim, max_past, nt) - nt, nt);
}

namespace dtree {
size_t head_attention_workspace_bytes(int32_t num_heads, int32_t head_dim, int32_t max_past_length,
                                      int32_t rows_padded) {
  if (num_heads <= 0 || head_dim <= 0 || max_past_length < 0 || rows_padded <= 0 || rows_padded % 32) return 0;
  const int nt = rows_padded / 32;
  const size_t stride = (size_t)32 * head_dim + 64;
  const size_t hb = (size_t)num_heads * nt;  // (head, query block) pairs
  if (64 + hb * sizeof(int) > kAttnWsHeader) return 0;
  // header (kAttnWsHeader: error word, epoch table place, counters from byte
  // 64; shared layout with the per-group kernel), the flag exchange region,
  // then the last-arriver / separate-combine partials
  return kAttnWsHeader + attn_ll_bytes(num_heads, head_dim, rows_padded) +
         hb * attn_splits(head_dim, max_past_length, nt) * stride * sizeof(float);
}

int head_tree_attention(const DtreeAttnArgs* a, hipStream_t stream) {
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
  DTREE_REQUIRE(a->max_past_length >= 0 && a->max_past_length <= kMaxPast, "attention: max_past_length beyond 16384");
  const int q_stride = gated ? 2 * D : D;
  DTREE_REQUIRE(a->ld_qkv >= a->num_heads * q_stride + 2 * a->num_kv_heads * D && a->ld_qkv % 4 == 0,
                "attention: ld_qkv too small");
  DTREE_REQUIRE(a->ld_out >= a->num_heads * D && a->ld_out % 8 == 0,
                "attention: ld_out below num_heads * head_dim or not a multiple of 8");
  DTREE_REQUIRE(((uintptr_t)a->out & 15) == 0 && ((uintptr_t)a->out_lo & 15) == 0 && ((uintptr_t)a->qkv & 15) == 0,
                "attention: qkv, out and out_lo must be 16-byte aligned");
  DTREE_REQUIRE(a->workspace_bytes >= head_attention_workspace_bytes(a->num_heads, D, a->max_past_length,
                                                                     a->rows_padded),
                "attention: workspace too small");
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR ||
                    ((a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16) &&
                     a->ld_out == a->num_heads * D && a->ld_out % 64 == 0),
                "attention: tiled out needs ld_out == num_heads * head_dim");
  AttnParams p{};
  p.qkv = a->qkv; p.ld_qkv = a->ld_qkv;
  p.q_stride = q_stride; p.k_off = a->num_heads * q_stride; p.v_off = p.k_off + a->num_kv_heads * D;
  p.q_norm = a->q_norm; p.k_norm = a->k_norm; p.eps = a->eps;
  p.rope_cos = a->rope_cos; p.rope_sin = a->rope_sin;
  p.kp = a->k_pages; p.vp = a->v_pages; p.page_table = a->page_table; p.desc = a->desc;
  p.out_tiled = a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16;
  p.out_h16 = a->out_layout == DTREE_W_TILED_F16;
  p.out = a->out; p.out_lo = p.out_h16 ? nullptr : a->out_lo; p.ld_out = a->ld_out;  // fp16: one plane
  p.Hq = a->num_heads; p.Hkv = a->num_kv_heads; p.tree_chunks = nt;
  p.max_chunks = attn_max_chunks(D, a->max_past_length, nt);
  p.splits = attn_splits(D, a->max_past_length, nt);
  p.scale_log2 = a->scale * kLog2e; p.write_cache = a->write_cache;
  p.off_xcd = off_xcd_test();
  char* ws = reinterpret_cast<char*>(a->workspace);
  const size_t ll_bytes = attn_ll_bytes(a->num_heads, D, a->rows_padded);
  p.err = reinterpret_cast<int*>(ws);
  p.counters = reinterpret_cast<int*>(ws + 64);
  p.part = reinterpret_cast<float*>(ws + kAttnWsHeader + ll_bytes);
  p.spin_limit = attn_spin_limit();
  const int G = p.Hq / p.Hkv;
  const int pairs = p.splits * p.Hkv;
  const int grid = ((pairs + 7) / 8) * 8 * G * nt;  // nt query blocks of ((pairs+7)/8)*8*G workgroups
  const bool one = nt == 1;
  // Long prefixes combine in a launch of their own (attn_combine_kernel):
  // when the last arriver alone would read more than 128 KB of partials.
  p.sep_combine = (size_t)p.splits * 32 * D * sizeof(float) > kSepCombineBytes;
  // Trees of up to 32 nodes whose splits fit the exchange slots combine
  // through the flag exchange. The step's split count decides on the device,
  // so a grid sized for a long prefix (partials combined by the second launch)
  // still takes the exchange at a short one, and the second launch then has
  // nothing to do. DTREE_ATTN_EXCHANGE=counter keeps the last-arriver combine.
  const char* xe = std::getenv("DTREE_ATTN_EXCHANGE");
  p.ll = ll_bytes > 0 && !(xe && xe[0] == 'c');
  p.ll_epoch = reinterpret_cast<uint32_t*>(ws + kAttnWsHeader);
  p.ll_slots = reinterpret_cast<unsigned char*>(ws + kAttnWsHeader + attn_ll_epoch_bytes(a->num_heads));
  p.ll_bytes = (unsigned)(ll_bytes - attn_ll_epoch_bytes(a->num_heads));
  if (D == 128) {
    if (one) tree_attn_kernel<128, 128, false, 1><<<grid, 64 * kWaves, 0, stream>>>(p);
    else tree_attn_kernel<128, 128, false, 4><<<grid, 64 * kWaves, 0, stream>>>(p);
  } else {
    if (one) tree_attn_kernel<256, 64, true, 1><<<grid, 64 * kWaves, 0, stream>>>(p);
    else tree_attn_kernel<256, 64, true, 4><<<grid, 64 * kWaves, 0, stream>>>(p);
  }
  DTREE_LAUNCH_CHECK("attention launch");
  if (p.sep_combine) {
    const int cgrid = p.Hq * nt * (D / 32);
    if (D == 128) attn_combine_kernel<128, false><<<cgrid, 64 * kWaves, 0, stream>>>(p);
    else attn_combine_kernel<256, true><<<cgrid, 64 * kWaves, 0, stream>>>(p);
    DTREE_LAUNCH_CHECK("attention combine launch");
  }
  return DTREE_OK;
}
}  // namespace dtree
