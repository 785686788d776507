// Ancestor-masked GQA tree attention over a paged bf16 KV prefix.
//
// Work split: a workgroup serves one 32-row block of tree queries (rows
// 32*rb .. 32*rb+31) of one query head. The keys are cut into chunks: chunks
// 0 .. NT-1 are the tree itself in 32-key blocks (NT = rows_padded / 32;
// ancestor-or-self mask, word tc of each query's bitset), chunks NT.. are runs
// of CK prefix keys (fully visible): a 64-key page for head_dim 128, half a
// page for head_dim 256 (same registers per wave). A workgroup has four
// waves, one chunk each, so workgroup `split` owns chunks 4*split .. 4*split+3.
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
#include "common.h"

namespace dtree {

constexpr int kWaves = 4;          // waves (chunks) per workgroup
constexpr int kMaxPast = 16384;    // longest prefix the grid is sized for
constexpr int kMergeDims = 128;    // head dims merged per LDS pass
// Prefix keys per chunk.
__host__ __device__ constexpr int chunk_keys(int D) { return D <= 128 ? DTREE_PAGE : DTREE_PAGE / 2; }
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
  int Hq, Hkv, max_chunks, splits;
  int tree_chunks;  // 32-key tree chunks = 32-row query blocks = rows_padded / 32
  float scale_log2;
  int write_cache;
  float* part; int* counters;
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

template <int D, int R>
__device__ __forceinline__ void row_issue(HeadRow<D, R>& r, const float* src, const uint16_t* norm_w, const float* cosr,
                                          const float* sinr, int h) {
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    r.x[j][0] = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h);
    r.x[j][1] = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h + 4);
    if (norm_w) r.nw[j] = ld_u32x4(norm_w + 16 * j + 8 * h);
  }
  if (cosr) {
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

// Tree chunk tc: k (norm + RoPE) and v of nodes 32*tc .. 32*tc+31 come from
// the fused qkv rows and are staged in LDS (this wave's private region) for
// the MFMA operand layouts; the block's 32 query rows are scored against them
// with word tc of their ancestor-or-self masks, and k/v are written to the
// cache rows P + node (once: query block 0, first head of the group).
// q, k and v are finished one after the other, so at most one raw head row is
// live in registers (head_dim 256 rows are 128 floats per lane pair).
template <int D, int R>
__device__ __forceinline__ void tree_chunk(const AttnParams& p, HeadRow<D, R>& qr, int hq, int g, int G, int P,
                                           int L, int tc, int qrow, bool write_rows, int c, int h, uint16_t* ks,
                                           uint16_t* vt, float& m_run, float& l_run, f32x16_t (&o)[D / 32]) {
  constexpr int NJ = D / 16, ND = D / 32;
  constexpr int KS = D + 8, VS = 32 + 8;
  constexpr int half_r = R / 2;
  // Lane (c, h) stages key node 32*tc + c and owns query row qrow.
  const int node = 32 * tc + c;
  const float* row = p.qkv + (size_t)node * p.ld_qkv;
  const float* cosr = p.rope_cos + node * half_r;
  const float* sinr = p.rope_sin + node * half_r;
  const uint32_t anc = p.desc->ancestors[qrow][tc];
  u32x4_t qf[NJ], ql[NJ];
  if constexpr (D > 128)
    row_issue<D, R>(qr, p.qkv + (size_t)qrow * p.ld_qkv + hq * p.q_stride, p.q_norm, p.rope_cos + qrow * half_r,
                    p.rope_sin + qrow * half_r, h);
  q_fragments<D, R>(qr, p.q_norm != nullptr, p.eps, qf, ql);
  u32x4_t kf8[NJ], vf8[NJ];
  {
    HeadRow<D, R> kr;
    row_issue<D, R>(kr, row + p.k_off + g * D, p.k_norm, cosr, sinr, h);
    float kv[NJ][8];
    row_finish<D, R>(kr, p.k_norm != nullptr, true, p.eps, kv);
    pack_frag<D>(kv, kf8);
  }
  {
    HeadRow<D, R> vr;
    row_issue<D, R>(vr, row + p.v_off + g * D, nullptr, nullptr, nullptr, h);
    float vv[NJ][8];
    row_finish<D, R>(vr, false, false, 0.f, vv);
    pack_frag<D>(vv, vf8);
  }
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
    s[0] = mfma32(a, qf[j], s[0]);
    s[0] = mfma32(a, ql[j], s[0]);
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
  if (p.write_cache && (hq % G) == 0 && write_rows && node < L) {
    const int pos = P + node;
    const int page = p.page_table[pos / DTREE_PAGE], off = pos % DTREE_PAGE;
    uint16_t* krow = p.kp + ((size_t)(page * p.Hkv + g) * DTREE_PAGE + off) * D;
    uint16_t* vcol = p.vp + (size_t)(page * p.Hkv + g) * D * DTREE_PAGE + off;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      *reinterpret_cast<u32x4_t*>(krow + 16 * j + 8 * h) = kf8[j];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t word = vf8[j][i >> 1];
        vcol[(size_t)(16 * j + 8 * h + i) * DTREE_PAGE] = (uint16_t)((i & 1) ? (word >> 16) : (word & 0xffff));
      }
    }
  }
}

// One prefix chunk = CK consecutive keys inside one page (the whole page for
// head_dim 128, half of it for 256). Q's loads go out first, then all K and V
// of the chunk, so Q's norm/RoPE overlaps the K/V flight. Keys past the prefix
// in the last chunk are masked (scores) and zeroed (V), since the page may
// hold stale or non-finite data there.
template <int D, int R>
__device__ __forceinline__ void prefix_chunk(const AttnParams& p, HeadRow<D, R>& qr, int page, int hq, int g, int P,
                                             int pc, int qrow, int c, int h, float& m_run, float& l_run,
                                             f32x16_t (&o)[D / 32]) {
  constexpr int NJ = D / 16, ND = D / 32;
  constexpr int CK = chunk_keys(D), NB = CK / 32;
  if constexpr (D > 128)
    row_issue<D, R>(qr, p.qkv + (size_t)qrow * p.ld_qkv + hq * p.q_stride, p.q_norm, p.rope_cos + qrow * (R / 2),
                    p.rope_sin + qrow * (R / 2), h);
  const int k_begin = pc * CK;  // prefix chunk pc: keys pc*CK ..
  const int k_end = min(k_begin + CK, P);
  const int po = k_begin % DTREE_PAGE;
  const uint16_t* kbase = p.kp + ((size_t)(page * p.Hkv + g) * DTREE_PAGE + po + swap_bits23(c)) * D;
  const uint16_t* vbase = p.vp + (size_t)(page * p.Hkv + g) * D * DTREE_PAGE + po;
  u32x4_t kf[NB][NJ];
  u32x4_t vf[NB][2][ND];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) kf[b][j] = ld_u32x4_stream(kbase + (size_t)32 * b * D + 16 * j + 8 * h);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int db = 0; db < ND; ++db)
        vf[b][s2][db] = ld_u32x4_stream(vbase + (size_t)(32 * db + c) * DTREE_PAGE + 32 * b + 16 * s2 + 8 * h);
  }
  u32x4_t qf[NJ], ql[NJ];
  q_fragments<D, R>(qr, p.q_norm != nullptr, p.eps, qf, ql);

  f32x16_t s[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[b][r] = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      s[b] = mfma32(kf[b][j], qf[j], s[b]);
      s[b] = mfma32(kf[b][j], ql[j], s[b]);
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
      for (int db = 0; db < ND; ++db) va[db] = ragged ? mask_keys(vf[b][s2][db], first, k_end) : vf[b][s2][db];
      pv_step<ND>(s[b], s2, va, o);
    }
}

// TB: tree chunks the LDS staging is sized for (1 for 32 rows, 4 up to 128).
template <int D, int R, bool GATE, int TB>
__global__ __launch_bounds__(64 * kWaves) void tree_attn_kernel(AttnParams p) {
  constexpr int ND = D / 32;  // 32-dim blocks of O^T
  constexpr int KS = D + 8;   // padded LDS row of tree K
  constexpr int VS = 32 + 8;  // padded LDS row of tree V^T
  constexpr int MS = 33;      // row stride of a wave's O^T in the LDS merge
  constexpr int NP = D / kMergeDims;               // merge passes
  constexpr int kWaveMerge = kMergeDims * MS + 64;  // floats per wave: O^T slice, m, l
  constexpr int kStage = (32 * KS + D * VS) * 2;
  constexpr int kMerge = kWaves * kWaveMerge * 4;
  constexpr int CK = chunk_keys(D);
  __shared__ __align__(16) unsigned char lds[TB * kStage > kMerge ? TB * kStage : kMerge];
  __shared__ int s_last;

  // blockIdx -> (query block, split, kv group, head in group): the G heads of
  // one (split, group) pair share blockIdx % 8, i.e. one XCD.
  const int G = p.Hq / p.Hkv, NT = p.tree_chunks;
  const int per_block = (int)gridDim.x / NT;  // workgroups per query block (a multiple of 8)
  const int rb = blockIdx.x / per_block, bid = blockIdx.x % per_block;
  const int pair = (bid / (8 * G)) * 8 + (bid & 7);
  if (pair >= p.splits * p.Hkv) return;
  const int g = pair % p.Hkv, split = pair / p.Hkv;
  const int hq = g * G + (bid >> 3) % G;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const int chunk = split * kWaves + wave;
  const int qrow = 32 * rb + c;  // this lane's query row
  // Loads that do not depend on the step descriptor go out first, so their
  // latency overlaps the descriptor read: this lane's q row (values, norm
  // weights, RoPE) and the page of this wave's prefix chunk.
  // (head_dim 256 issues its q row inside the chunk: live across the
  // descriptor read it would spill.)
  HeadRow<D, R> qr;
  if constexpr (D <= 128)
    row_issue<D, R>(qr, p.qkv + (size_t)qrow * p.ld_qkv + hq * p.q_stride, p.q_norm, p.rope_cos + qrow * (R / 2),
                    p.rope_sin + qrow * (R / 2), h);
  const int page = (chunk >= NT && chunk < p.max_chunks) ? p.page_table[(chunk - NT) * CK / DTREE_PAGE] : 0;

  const int P = p.desc->past_length, L = p.desc->num_nodes;
  const int nchunks = NT + (P + CK - 1) / CK;
  // A descriptor beyond the grid's capacity (P > max_past_length) or with more
  // rows than rows_padded leaves the output untouched instead of indexing past
  // buffers.
  if (nchunks > p.max_chunks || L > 32 * NT || L < 1) return;
  const int nsplit = (nchunks + kWaves - 1) / kWaves;
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

  float m_run = kNeg, l_run = 0.f;
  f32x16_t o[ND];
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

  if (chunk < NT) {
    // Tree chunks are waves 0 .. NT-1 of split 0, each with its own staging.
    if (32 * chunk < L) {
      uint16_t* ks = reinterpret_cast<uint16_t*>(lds + (size_t)chunk * kStage);
      tree_chunk<D, R>(p, qr, hq, g, G, P, L, chunk, qrow, rb == 0, c, h, ks, ks + 32 * KS, m_run, l_run, o);
    }
  } else if (chunk < nchunks) {
    prefix_chunk<D, R>(p, qr, page, hq, g, P, chunk - NT, qrow, c, h, m_run, l_run, o);
  }

  // LDS merge of the four waves, 128 head dims per pass. The first barrier
  // retires the tree chunk's staging, which shares this memory.
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  // Thread t combines query q = t/8, dims pass*128 + d0 .. +15, d0 = 16 (t%8).
  constexpr int kDims = 32 * D / (64 * kWaves);  // dims per thread: 16 per pass
  const int t = threadIdx.x;
  const int q = t >> 3, d0 = (t & 7) * 16;
  float* mw = reinterpret_cast<float*>(lds) + wave * kWaveMerge;
  const float* m0 = reinterpret_cast<const float*>(lds);
  float acc[kDims];
  float M = kNeg, tot = 0.f, wk[kWaves];
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    __syncthreads();
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) mw[(32 * db + acc_row(r, h)) * MS + c] = o[4 * pass + db][r];
    if (pass == 0 && h == 0) {
      mw[kMergeDims * MS + c] = m_run;
      mw[kMergeDims * MS + 32 + c] = l_tot;
    }
    __syncthreads();
    if (pass == 0) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, m0[w * kWaveMerge + kMergeDims * MS + q]);
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        wk[w] = fast_exp2(m0[w * kWaveMerge + kMergeDims * MS + q] - M);
        tot += wk[w] * m0[w * kWaveMerge + kMergeDims * MS + 32 + q];
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float a = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) a += wk[w] * m0[w * kWaveMerge + (d0 + i) * MS + q];
      acc[16 * pass + i] = a;
    }
  }

  if (nsplit > 1) {
    // Workgroup partial, laid out [i][thread] so both the stores here and the
    // loads of the combining workgroup are coalesced.
    const size_t stride = (size_t)32 * D + 64;
    const int hb = hq * NT + rb;  // (head, query block)
    float* part = p.part + ((size_t)hb * p.splits + split) * stride;
#pragma unroll
    for (int i = 0; i < kDims; ++i) st_coherent(part + (size_t)i * 64 * kWaves + t, acc[i]);
    if ((t & 7) == 0) {
      st_coherent(part + 32 * D + q, M);
      st_coherent(part + 32 * D + 32 + q, tot);
    }
    wait_stores_done();
    __syncthreads();
    if (t == 0) s_last = arrive(&p.counters[hb]) == nsplit - 1;
    __syncthreads();
    if (!s_last) return;
    if (t == 0) reset_counter(&p.counters[hb]);

    // Partials are read kSb splits at a time (all loads of a batch in flight
    // together) with a running max: one memory round trip per batch instead
    // of two per split.
    constexpr int kSb = 128 / kDims;  // 8 splits per batch at head_dim 128, 4 at 256
    const float* base = p.part + (size_t)hb * p.splits * stride;
    float Ms = kNeg;
#pragma unroll
    for (int i = 0; i < kDims; ++i) acc[i] = 0.f;
    tot = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += kSb) {
      float v[kSb][kDims], mm[kSb], ll[kSb];
#pragma unroll
      for (int b = 0; b < kSb; ++b) {
        const bool ok = s0 + b < nsplit;
        const float* ps = base + (size_t)(ok ? s0 + b : 0) * stride;
        mm[b] = ok ? ld_coherent(ps + 32 * D + q) : kNeg;
        ll[b] = ok ? ld_coherent(ps + 32 * D + 32 + q) : 0.f;
#pragma unroll
        for (int i = 0; i < kDims; ++i) v[b][i] = ok ? ld_coherent(ps + (size_t)i * 64 * kWaves + t) : 0.f;
      }
      float gm = Ms;
#pragma unroll
      for (int b = 0; b < kSb; ++b) gm = fmaxf(gm, mm[b]);
      const float r = fast_exp2(Ms - gm);
      tot *= r;
#pragma unroll
      for (int i = 0; i < kDims; ++i) acc[i] *= r;
#pragma unroll
      for (int b = 0; b < kSb; ++b) {
        const float w = fast_exp2(mm[b] - gm);
        tot += w * ll[b];
#pragma unroll
        for (int i = 0; i < kDims; ++i) acc[i] += w * v[b][i];
      }
      Ms = gm;
    }
  }

  const int orow = 32 * rb + q;  // output row of thread t
  const float inv = (orow < L && tot > 0.f) ? 1.0f / tot : 0.f;
#pragma unroll
  for (int i0 = 0; i0 < kDims; i0 += 8) {
    const int dd = (i0 / 16) * kMergeDims + d0 + (i0 % 16);  // head dim of acc[i0]
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = orow < L ? acc[i0 + i] * inv : 0.f;
    if (GATE && orow < L) {
      // o_proj input = attention * sigmoid(gate), gate = q_proj row dims D.. of the head
      const float* gp = p.qkv + (size_t)orow * p.ld_qkv + hq * p.q_stride + D + dd;
      const f32x4_t g0 = *reinterpret_cast<const f32x4_t*>(gp);
      const f32x4_t g1 = *reinterpret_cast<const f32x4_t*>(gp + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y[i] *= 1.0f / (1.0f + __expf(-g0[i]));
        y[i + 4] *= 1.0f / (1.0f + __expf(-g1[i]));
      }
    }
    u32x4_t hi, lo;
    split8(y, hi, lo);
    const int col = hq * D + dd;
    const size_t oi = p.out_tiled ? tiled_index(orow, col, p.ld_out) : (size_t)orow * p.ld_out + col;
    *reinterpret_cast<u32x4_t*>(p.out + oi) = hi;
    if (p.out_lo) *reinterpret_cast<u32x4_t*>(p.out_lo + oi) = lo;
  }
}

}  // namespace dtree

using namespace dtree;

static int attn_max_chunks(int head_dim, int max_past, int nt) {
  const int ck = chunk_keys(head_dim);
  return nt + (max_past + ck - 1) / ck;
}
static int attn_splits(int head_dim, int max_past, int nt) {
  return (attn_max_chunks(head_dim, max_past, nt) + kWaves - 1) / kWaves;
}

extern "C" size_t dtree_attention_workspace_bytes(int32_t num_heads, int32_t head_dim, int32_t max_past_length,
                                                  int32_t rows_padded) {
  if (num_heads <= 0 || head_dim <= 0 || max_past_length < 0 || rows_padded <= 0 || rows_padded % 32) return 0;
  const int nt = rows_padded / 32;
  const size_t stride = (size_t)32 * head_dim + 64;
  const size_t hb = (size_t)num_heads * nt;  // (head, query block) pairs
  return ((hb * sizeof(int) + 255) & ~(size_t)255) +
         hb * attn_splits(head_dim, max_past_length, nt) * stride * sizeof(float);
}

extern "C" int dtree_tree_attention(const DtreeAttnArgs* a, hipStream_t stream) {
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
  DTREE_REQUIRE(a->workspace_bytes >= dtree_attention_workspace_bytes(a->num_heads, D, a->max_past_length,
                                                                      a->rows_padded),
                "attention: workspace too small");
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR ||
                    (a->out_layout == DTREE_W_TILED && a->ld_out == a->num_heads * D && a->ld_out % 64 == 0),
                "attention: tiled out needs ld_out == num_heads * head_dim");
  AttnParams p{};
  p.qkv = a->qkv; p.ld_qkv = a->ld_qkv;
  p.q_stride = q_stride; p.k_off = a->num_heads * q_stride; p.v_off = p.k_off + a->num_kv_heads * D;
  p.q_norm = a->q_norm; p.k_norm = a->k_norm; p.eps = a->eps;
  p.rope_cos = a->rope_cos; p.rope_sin = a->rope_sin;
  p.kp = a->k_pages; p.vp = a->v_pages; p.page_table = a->page_table; p.desc = a->desc;
  p.out = a->out; p.out_lo = a->out_lo; p.ld_out = a->ld_out;
  p.out_tiled = a->out_layout == DTREE_W_TILED;
  p.Hq = a->num_heads; p.Hkv = a->num_kv_heads; p.tree_chunks = nt;
  p.max_chunks = attn_max_chunks(D, a->max_past_length, nt);
  p.splits = attn_splits(D, a->max_past_length, nt);
  p.scale_log2 = a->scale * kLog2e; p.write_cache = a->write_cache;
  p.counters = reinterpret_cast<int*>(a->workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) +
                                    (((size_t)a->num_heads * nt * sizeof(int) + 255) & ~(size_t)255));
  const int G = p.Hq / p.Hkv;
  const int pairs = p.splits * p.Hkv;
  const int grid = ((pairs + 7) / 8) * 8 * G * nt;  // nt query blocks of ((pairs+7)/8)*8*G workgroups
  const bool one = nt == 1;
  if (D == 128) {
    if (one) tree_attn_kernel<128, 128, false, 1><<<grid, 64 * kWaves, 0, stream>>>(p);
    else tree_attn_kernel<128, 128, false, 4><<<grid, 64 * kWaves, 0, stream>>>(p);
  } else {
    if (one) tree_attn_kernel<256, 64, true, 1><<<grid, 64 * kWaves, 0, stream>>>(p);
    else tree_attn_kernel<256, 64, true, 4><<<grid, 64 * kWaves, 0, stream>>>(p);
  }
  DTREE_LAUNCH_CHECK("attention launch");
  return DTREE_OK;
}
