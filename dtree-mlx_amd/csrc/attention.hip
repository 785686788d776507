// Ancestor-masked GQA tree attention over a paged bf16 KV prefix.
//
// One workgroup is one wavefront and owns (query head, key chunk): chunk 0 is
// the tree itself (the L new keys, ancestor-or-self mask), chunks 1.. are
// 128-key slices of the prefix (fully visible). Each chunk produces a
// flash-decoding partial (row max, row sum, unnormalised output); the last
// chunk of a head to finish (device-scope counter) merges them in chunk order.
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

constexpr int kChunkKeys = 128;  // prefix keys per chunk
constexpr int kMaxChunks = 128;  // merge-weight capacity (prefix <= 16256)
constexpr float kNeg = -1e30f;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
  const float* qkv; int ld_qkv;
  const uint16_t* q_norm; const uint16_t* k_norm; float eps;
  const float* rope_cos; const float* rope_sin;
  uint16_t* kp; uint16_t* vp; const int* page_table;
  const DtreeStepDesc* desc;
  uint16_t* out; uint16_t* out_lo; int ld_out; int out_tiled;
  int Hq, Hkv, max_chunks;
  float scale_log2;
  int write_cache;
  float* part; int* counters;
};

__device__ __forceinline__ int swap_bits23(int c) { return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1); }

// Loads 64 values of row `row` (dims 16j + 8h + i) from an fp32 row, applies
// an optional RMSNorm over D (with the partner lane^32) and RoPE.
template <int D>
__device__ __forceinline__ void load_head_row(const float* src, const uint16_t* norm_w, float eps, bool rope,
                                              const float* cosr, const float* sinr, int h,
                                              float (&v)[D / 16][8]) {
  constexpr int NJ = D / 16;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(src + 16 * j + 8 * h + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[j][i] = a[i];
      v[j][i + 4] = b[i];
    }
  }
  if (norm_w) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
    ss += __shfl_xor(ss, 32);
    const float r = rsqrtf(ss * (1.0f / D) + eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] *= r * bf2f(norm_w[16 * j + 8 * h + i]);
  }
  if (rope) {
#pragma unroll
    for (int j = 0; j < NJ / 2; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = 16 * j + 8 * h + i;
        const float cs = cosr[d], sn = sinr[d];
        const float x1 = v[j][i], x2 = v[j + NJ / 2][i];
        v[j][i] = x1 * cs - x2 * sn;
        v[j + NJ / 2][i] = x1 * sn + x2 * cs;
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

// Online-softmax update for one 32-key block; s[] already scaled (log2 units).
template <int ND>
__device__ __forceinline__ void softmax_block(f32x16_t& s, float& m_run, float& l_run, f32x16_t (&o)[ND]) {
  float bmax = kNeg;
#pragma unroll
  for (int r = 0; r < 16; ++r) bmax = fmaxf(bmax, s[r]);
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
  const float m_new = fmaxf(m_run, bmax);
  const float alpha = exp2f(m_run - m_new);
  float lsum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    s[r] = exp2f(s[r] - m_new);
    lsum += s[r];
  }
  l_run = l_run * alpha + lsum;
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
  m_run = m_new;
}

template <int D>
__global__ __launch_bounds__(64) void tree_attn_kernel(AttnParams p) {
  constexpr int NJ = D / 16;  // 16-dim K steps of S^T
  constexpr int ND = D / 32;  // 32-dim blocks of O^T
  constexpr int KS = D + 8;   // padded LDS row of tree K
  constexpr int VS = 32 + 8;  // padded LDS row of tree V^T
  __shared__ uint16_t ks[32 * KS];
  __shared__ uint16_t vt[D * VS];
  __shared__ float wts[kMaxChunks * 32];  // merge weights [chunk][query]; reused

  const int P = p.desc->past_length, L = p.desc->num_nodes;
  const int nprefix = (P + kChunkKeys - 1) / kChunkKeys;
  const int hq = blockIdx.x % p.Hq, chunk = blockIdx.x / p.Hq;
  // A descriptor beyond the grid's capacity (P > max_past_length) or with more
  // than 32 rows leaves the output untouched instead of indexing past buffers.
  if (chunk > nprefix || nprefix >= p.max_chunks || L > 32 || L < 1) return;
  const int G = p.Hq / p.Hkv, g = hq / G;
  const int lane = threadIdx.x, c = lane & 31, h = lane >> 5;
  const int half_d = D / 2;

  u32x4_t qf[NJ], ql[NJ];
  {
    float q[NJ][8];
    load_head_row<D>(p.qkv + (size_t)c * p.ld_qkv + hq * D, p.q_norm, p.eps, true, p.rope_cos + c * half_d,
                     p.rope_sin + c * half_d, h, q);
#pragma unroll
    for (int j = 0; j < NJ; ++j) split8(q[j], qf[j], ql[j]);
  }

  float m_run = kNeg, l_run = 0.f;
  f32x16_t o[ND];
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

  if (chunk == 0) {
    // The tree's own keys: build k (norm + RoPE) and v rows for node c.
    float kr[NJ][8], vr[NJ][8];
    load_head_row<D>(p.qkv + (size_t)c * p.ld_qkv + (p.Hq + g) * D, p.k_norm, p.eps, true,
                     p.rope_cos + c * half_d, p.rope_sin + c * half_d, h, kr);
    load_head_row<D>(p.qkv + (size_t)c * p.ld_qkv + (p.Hq + p.Hkv + g) * D, nullptr, 0.f, false, nullptr,
                     nullptr, h, vr);
    u32x4_t kf8[NJ], vf8[NJ];
    pack_frag<D>(kr, kf8);
    pack_frag<D>(vr, vf8);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      *reinterpret_cast<u32x4_t*>(&ks[c * KS + 16 * j + 8 * h]) = kf8[j];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t word = vf8[j][i >> 1];
        vt[(16 * j + 8 * h + i) * VS + c] = (uint16_t)((i & 1) ? (word >> 16) : (word & 0xffff));
      }
    }
    if (p.write_cache && (hq % G) == 0 && c < L) {
      const int pos = P + c;
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
    __syncthreads();
    const int kr_row = swap_bits23(c);
    f32x16_t s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&ks[kr_row * KS + 16 * j + 8 * h]);
      s = mfma32(a, qf[j], s);
      s = mfma32(a, ql[j], s);
    }
    const uint32_t anc = p.desc->ancestors[c][0];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = 16 * (r >> 3) + 8 * h + (r & 7);
      const bool ok = c < L && t < L && ((anc >> t) & 1u);
      s[r] = ok ? s[r] * p.scale_log2 : kNeg;
    }
    softmax_block<ND>(s, m_run, l_run, o);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      u32x4_t va[ND];
#pragma unroll
      for (int db = 0; db < ND; ++db)
        va[db] = *reinterpret_cast<const u32x4_t*>(&vt[(32 * db + c) * VS + 16 * s2 + 8 * h]);
      pv_step<ND>(s, s2, va, o);
    }
  } else {
    const int k_begin = (chunk - 1) * kChunkKeys;
    const int k_end = min(k_begin + kChunkKeys, P);
    const int kr_off = swap_bits23(c);
    for (int kb0 = k_begin; kb0 < k_end; kb0 += 32) {
      const int page = p.page_table[kb0 / DTREE_PAGE];
      const int off0 = kb0 % DTREE_PAGE;
      const uint16_t* kbase = p.kp + ((size_t)(page * p.Hkv + g) * DTREE_PAGE + off0 + kr_off) * D;
      u32x4_t kf[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) kf[j] = ld_u32x4(kbase + 16 * j + 8 * h);
      f32x16_t s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        s = mfma32(kf[j], qf[j], s);
        s = mfma32(kf[j], ql[j], s);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb0 + 16 * (r >> 3) + 8 * h + (r & 7);
        s[r] = key < k_end ? s[r] * p.scale_log2 : kNeg;
      }
      softmax_block<ND>(s, m_run, l_run, o);
      const uint16_t* vbase = p.vp + (size_t)(page * p.Hkv + g) * D * DTREE_PAGE + off0;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        u32x4_t va[ND];
#pragma unroll
        for (int db = 0; db < ND; ++db) va[db] = ld_u32x4(vbase + (size_t)(32 * db + c) * DTREE_PAGE + 16 * s2 + 8 * h);
        pv_step<ND>(s, s2, va, o);
      }
    }
  }

  // Partial for (head, chunk): O[q][d] unnormalised, m[q], l[q].
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const size_t stride = (size_t)32 * D + 64;
  float* part = p.part + ((size_t)hq * p.max_chunks + chunk) * stride;
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) st_coherent(part + (size_t)c * D + 32 * db + acc_row(r, h), o[db][r]);
  if (h == 0) {
    st_coherent(part + 32 * D + c, m_run);
    st_coherent(part + 32 * D + 32 + c, l_tot);
  }
  wait_stores_done();
  __syncthreads();
  int last = 0;
  if (lane == 0) last = arrive(&p.counters[hq]) == nprefix;
  last = __shfl(last, 0);
  if (!last) return;
  if (lane == 0) reset_counter(&p.counters[hq]);

  const int nc = nprefix + 1;
  const float* base = p.part + (size_t)hq * p.max_chunks * stride;
  if (lane < 32) {
    float M = kNeg;
    for (int k = 0; k < nc; ++k) M = fmaxf(M, ld_coherent(base + k * stride + 32 * D + lane));
    float tot = 0.f;
    for (int k = 0; k < nc; ++k) {
      const float mk = ld_coherent(base + k * stride + 32 * D + lane);
      const float lk = ld_coherent(base + k * stride + 32 * D + 32 + lane);
      const float wk = exp2f(mk - M);
      wts[k * 32 + lane] = wk;
      tot += lk * wk;
    }
    const float inv = tot > 0.f ? 1.0f / tot : 0.f;
    for (int k = 0; k < nc; ++k) wts[k * 32 + lane] *= inv;
  }
  __syncthreads();
  for (int q = 0; q < 32; ++q) {
    for (int d = lane; d < D; d += 64) {
      float acc = 0.f;
      if (q < L)
        for (int k = 0; k < nc; ++k) acc += wts[k * 32 + q] * ld_coherent(base + k * stride + (size_t)q * D + d);
      const size_t oi = p.out_tiled ? tiled_index(q, hq * D + d, p.ld_out) : (size_t)q * p.ld_out + hq * D + d;
      const uint16_t hi = f2bf(acc);
      p.out[oi] = hi;
      if (p.out_lo) p.out_lo[oi] = f2bf(acc - bf2f(hi));
    }
  }
}

}  // namespace dtree

using namespace dtree;

static int attn_max_chunks(int max_past) { return 1 + (max_past + kChunkKeys - 1) / kChunkKeys; }

extern "C" size_t dtree_attention_workspace_bytes(int32_t num_heads, int32_t head_dim, int32_t max_past_length) {
  if (num_heads <= 0 || head_dim <= 0 || max_past_length < 0) return 0;
  const size_t stride = (size_t)32 * head_dim + 64;
  return 256 + (size_t)num_heads * sizeof(int) + (size_t)num_heads * attn_max_chunks(max_past_length) * stride * sizeof(float);
}

extern "C" int dtree_tree_attention(const DtreeAttnArgs* a, hipStream_t stream) {
  DTREE_REQUIRE(a, "attention: null args");
  DTREE_REQUIRE(a->qkv && a->rope_cos && a->rope_sin && a->k_pages && a->v_pages && a->page_table && a->desc &&
                    a->out && a->workspace,
                "attention: null pointer");
  DTREE_REQUIRE(a->head_dim == 128, "attention: head_dim 128 is the compiled size");
  DTREE_REQUIRE(a->rows_padded == 32, "attention: trees of up to 32 nodes (rows_padded 32)");
  DTREE_REQUIRE(a->num_kv_heads > 0 && a->num_heads % a->num_kv_heads == 0, "attention: num_heads % num_kv_heads");
  DTREE_REQUIRE(a->max_past_length >= 0, "attention: max_past_length");
  DTREE_REQUIRE(a->ld_qkv >= (a->num_heads + 2 * a->num_kv_heads) * a->head_dim && a->ld_qkv % 4 == 0,
                "attention: ld_qkv too small");
  DTREE_REQUIRE(a->ld_out >= a->num_heads * a->head_dim, "attention: ld_out too small");
  const int max_chunks = attn_max_chunks(a->max_past_length);
  DTREE_REQUIRE(max_chunks <= kMaxChunks, "attention: max_past_length beyond 16256");
  DTREE_REQUIRE(a->workspace_bytes >= dtree_attention_workspace_bytes(a->num_heads, a->head_dim, a->max_past_length),
                "attention: workspace too small");
  AttnParams p{};
  p.qkv = a->qkv; p.ld_qkv = a->ld_qkv; p.q_norm = a->q_norm; p.k_norm = a->k_norm; p.eps = a->eps;
  p.rope_cos = a->rope_cos; p.rope_sin = a->rope_sin;
  p.kp = a->k_pages; p.vp = a->v_pages; p.page_table = a->page_table; p.desc = a->desc;
  p.out = a->out; p.out_lo = a->out_lo; p.ld_out = a->ld_out;
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR ||
                    (a->out_layout == DTREE_W_TILED && a->ld_out == a->num_heads * a->head_dim && a->ld_out % 64 == 0),
                "attention: tiled out needs ld_out == num_heads * head_dim");
  p.out_tiled = a->out_layout == DTREE_W_TILED;
  p.Hq = a->num_heads; p.Hkv = a->num_kv_heads; p.max_chunks = max_chunks;
  p.scale_log2 = a->scale * kLog2e; p.write_cache = a->write_cache;
  p.counters = reinterpret_cast<int*>(a->workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) +
                                    (((size_t)a->num_heads * sizeof(int) + 255) & ~(size_t)255));
  const int grid = a->num_heads * max_chunks;
  tree_attn_kernel<128><<<grid, 64, 0, stream>>>(p);
  DTREE_LAUNCH_CHECK("attention launch");
  return DTREE_OK;
}
