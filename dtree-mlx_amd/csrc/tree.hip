// Draft-tree construction on the GPU (build_dtree_tree, dtree_runtime.py:82-163):
// per-depth top-k of the draft logits with log-probs = logit - logsumexp(row),
// then the best-first heap over cumulative log-probs, written straight into the
// verify step's descriptor (tokens, positions = P + depth, parents, ancestor
// bitsets; compile_dtree_tree, dtree_runtime.py:166-192).
//
// Three launches, all graph-capturable:
//   1. topk_chunk_kernel  (row, 8192-logit chunk): chunk max and sum of
//      exp(x - max), and the chunk's top-k by a four-digit radix select;
//   2. topk_merge_kernel  (row): the union of the chunk candidates (which
//      holds the row's top-k) selected the same way and sorted; log-probs
//      from the merged logsumexp;
//   3. heap_kernel        (one wavefront): the reference's heap order.
//
// Order rules that make the tree identical to the reference's given the same
// top-k lists and log-probs:
//   * a row's top-k is sorted by (logit desc, token id asc);
//   * heap entries compare as the Python tuples (-logw, ranks, ...): larger
//     logw first, then the lexicographically smaller rank tuple (a prefix
//     before its extensions). logw is a double built with the reference's
//     operation order (sibling: (logw - lp[d][r]) + lp[d][r + 1]; child:
//     logw + lp[d + 1][0]); rank tuples are packed 7 bits per level (value
//     rank + 1, zero past the end) into a 128-bit big-endian key, so they
//     compare as integers.
#include "common.h"

namespace dtree {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 8192;                // logits per workgroup in pass 1
constexpr int kE1 = kChunk / kThreads;      // contiguous logits per thread
constexpr int kCand = 4096;                 // candidates per row in pass 2
constexpr int kE2 = kCand / kThreads;
constexpr int kMaxK = 127;                  // rank + 1 fits the 7-bit level field
constexpr int kMaxDepth = 18;               // 18 levels x 7 bits in 128 bits
constexpr int kMaxEntries = 256;            // heap entries: 1 + 2 * budget

__device__ __forceinline__ uint32_t ordered_bits(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_ordered(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

struct SelectLds {
  uint32_t hist[256];
  uint32_t wave_sum[kThreads / 64];
  uint32_t prefix, need, take_all, n_out;
  unsigned long long list[128];
};

// Block-wide exclusive prefix sum over threads in thread order.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, SelectLds& s) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_up(inc, o);
    if (lane >= o) inc += u;
  }
  if (lane == 63) s.wave_sum[w] = inc;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < w; ++i) before += s.wave_sum[i];
  __syncthreads();
  return before + inc - v;
}

// The workgroup's top K (K <= 128) elements, sorted descending by the 64-bit
// key (hi << 32 | lo), into s.list[0 .. K). Thread t holds positions
// E*t .. E*t + E - 1; among elements with equal hi the selection keeps the
// smallest positions (the callers make position order agree with lo order).
// Fewer than K valid elements: all of them, the rest of the list is zero.
template <int E>
__device__ void select_topk(const uint32_t (&hi)[E], const uint32_t (&lo)[E], const bool (&valid)[E], int K,
                            SelectLds& s) {
  const int t = threadIdx.x;
  uint32_t prefix = 0, need = (uint32_t)K;
  bool take_all = false;
  for (int shift = 24; shift >= 0; shift -= 8) {
    s.hist[t] = 0;  // kThreads == 256 bins
    __syncthreads();
    const uint32_t hmask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (valid[e] && (hi[e] & hmask) == (prefix & hmask)) atomicAdd(&s.hist[(hi[e] >> shift) & 255u], 1u);
    __syncthreads();
    if (t < 64) {
      // lane l owns bins 255 - 4l .. 252 - 4l (descending digit order)
      uint32_t c[4], sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = s.hist[255 - 4 * t - j];
        sum += c[j];
      }
      uint32_t inc = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(inc, o);
        if (t >= o) inc += u;
      }
      const uint32_t total = __shfl(inc, 63);
      if (shift == 24 && total <= need) {
        if (t == 0) {
          s.take_all = 1u;
          s.prefix = 0u;
          s.need = 0u;
        }
      } else {
        uint32_t before = inc - sum;
        // the digit where the running count first reaches `need`
        for (int j = 0; j < 4; ++j) {
          if (before < need && before + c[j] >= need) {
            s.take_all = 0u;
            s.prefix = prefix | ((uint32_t)(255 - 4 * t - j) << shift);
            s.need = need - before;
          }
          before += c[j];
        }
      }
    }
    __syncthreads();
    take_all = s.take_all != 0u;
    prefix = s.prefix;
    need = s.need;
    if (take_all) break;
  }
  // T = prefix is the K-th largest hi; keep every hi > T and the first `need`
  // elements (position order) with hi == T.
  uint32_t eq = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) eq += (!take_all && valid[e] && hi[e] == prefix) ? 1u : 0u;
  if (t == 0) s.n_out = 0;
  uint32_t rank = block_exclusive_scan(eq, s);  // also orders n_out's reset before the appends
  for (int e = 0; e < E; ++e) {
    if (!valid[e]) continue;
    bool keep = take_all || hi[e] > prefix;
    if (!keep && hi[e] == prefix) {
      keep = rank < need;
      ++rank;
    }
    if (keep) {
      const uint32_t slot = atomicAdd(&s.n_out, 1u);
      s.list[slot] = ((unsigned long long)hi[e] << 32) | lo[e];
    }
  }
  __syncthreads();
  const uint32_t n = s.n_out;
  int kp = 1;
  while (kp < K) kp <<= 1;
  for (int i = t; i < kp; i += kThreads)
    if ((uint32_t)i >= n) s.list[i] = 0ull;
  __syncthreads();
  // bitonic sort of kp entries, descending
  for (int size = 2; size <= kp; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (t < kp / 2) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const unsigned long long a = s.list[i], b = s.list[j];
        if ((a < b) == desc) {
          s.list[i] = b;
          s.list[j] = a;
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ float block_max(float v, float* red) {
  const int t = threadIdx.x;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int t = threadIdx.x;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < kThreads / 64; ++i) r += red[i];
  __syncthreads();
  return r;
}

struct TreeParams {
  const float* logits;
  int ld, depth, vocab, k, budget, chunks, root, past;
  unsigned long long* part_keys;  // [depth][chunks][k]
  float2* part_ms;                // [depth][chunks] (max, sum exp(x - max))
  int* top_tok;                   // [depth][k]
  float* top_lp;                  // [depth][k]
  DtreeStepDesc* desc;
  int* tree_out;                  // optional [1 + 3 * DTREE_MAX_NODES]
  int* topk_ids;                  // optional [depth][k] copies of top_tok / top_lp
  float* topk_lp;
};

__global__ __launch_bounds__(kThreads) void topk_chunk_kernel(TreeParams p) {
  __shared__ SelectLds s;
  __shared__ float red[kThreads / 64];
  const int row = blockIdx.y, chunk = blockIdx.x, t = threadIdx.x;
  const int base = chunk * kChunk + kE1 * t;
  const float* src = p.logits + (size_t)row * p.ld;
  float x[kE1];
  bool valid[kE1];
#pragma unroll
  for (int q = 0; q < kE1 / 4; ++q) {
    const int i = base + 4 * q;
    const bool in = i < p.vocab;  // vocab % 4 == 0: whole float4 groups
    const f32x4_t v = in ? *reinterpret_cast<const f32x4_t*>(src + i) : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[4 * q + j] = v[j];
      valid[4 * q + j] = in;
    }
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < kE1; ++e)
    if (valid[e]) m = fmaxf(m, x[e]);
  m = block_max(m, red);
  float se = 0.f;
#pragma unroll
  for (int e = 0; e < kE1; ++e)
    if (valid[e] && m > -__builtin_inff()) se += expf(x[e] - m);
  se = block_sum(se, red);
  if (t == 0) p.part_ms[row * p.chunks + chunk] = make_float2(m, se);
  uint32_t hi[kE1], lo[kE1];
#pragma unroll
  for (int e = 0; e < kE1; ++e) {
    hi[e] = ordered_bits(x[e]);
    lo[e] = ~(uint32_t)(base + e);  // smaller token id sorts first among equal logits
  }
  select_topk<kE1>(hi, lo, valid, p.k, s);
  unsigned long long* dst = p.part_keys + ((size_t)row * p.chunks + chunk) * p.k;
  for (int i = t; i < p.k; i += kThreads) dst[i] = s.list[i];
}

__global__ __launch_bounds__(kThreads) void topk_merge_kernel(TreeParams p) {
  __shared__ SelectLds s;
  __shared__ float red[kThreads / 64];
  const int row = blockIdx.x, t = threadIdx.x;
  const int n = p.chunks * p.k;
  const unsigned long long* src = p.part_keys + (size_t)row * n;
  uint32_t hi[kE2], lo[kE2];
  bool valid[kE2];
#pragma unroll
  for (int e = 0; e < kE2; ++e) {
    const int i = kE2 * t + e;  // candidates of chunk c precede chunk c + 1's: position order = token id order
    const unsigned long long key = i < n ? src[i] : 0ull;
    hi[e] = (uint32_t)(key >> 32);
    lo[e] = (uint32_t)key;
    valid[e] = key != 0ull;
  }
  // logsumexp of the row from the chunk partials
  float mm = -__builtin_inff();
  for (int c = t; c < p.chunks; c += kThreads) mm = fmaxf(mm, p.part_ms[row * p.chunks + c].x);
  mm = block_max(mm, red);
  float ss = 0.f;
  for (int c = t; c < p.chunks; c += kThreads) {
    const float2 ms = p.part_ms[row * p.chunks + c];
    if (ms.x > -__builtin_inff()) ss += ms.y * expf(ms.x - mm);
  }
  ss = block_sum(ss, red);
  const float lse = mm + logf(ss);
  select_topk<kE2>(hi, lo, valid, p.k, s);
  for (int i = t; i < p.k; i += kThreads) {
    const unsigned long long key = s.list[i];
    const int tok = (int)~(uint32_t)key;
    const float lp = from_ordered((uint32_t)(key >> 32)) - lse;
    p.top_tok[row * p.k + i] = tok;
    p.top_lp[row * p.k + i] = lp;
    if (p.topk_ids) p.topk_ids[row * p.k + i] = tok;
    if (p.topk_lp) p.topk_lp[row * p.k + i] = lp;
  }
}

// Rank tuple field of level j (1-based): r0 holds levels 1..9, r1 levels 10..18.
__device__ __forceinline__ void add_level(unsigned long long& r0, unsigned long long& r1, int level,
                                          unsigned long long v) {
  if (level <= 9)
    r0 += v << (64 - 7 * level);
  else
    r1 += v << (64 - 7 * (level - 9));
}

// (logw, r0, r1) a better heap entry than (lw, q0, q1)?
__device__ __forceinline__ bool better(double logw, unsigned long long r0, unsigned long long r1, double lw,
                                       unsigned long long q0, unsigned long long q1) {
  if (logw != lw) return logw > lw;
  if (r0 != q0) return r0 < q0;
  return r1 < q1;
}

__global__ __launch_bounds__(64) void heap_kernel(TreeParams p) {
  __shared__ double e_logw[kMaxEntries];
  __shared__ unsigned long long e_r0[kMaxEntries], e_r1[kMaxEntries];
  __shared__ int e_meta[kMaxEntries];  // parent | depth << 8 | rank << 16; -1 = popped
  __shared__ int n_tok[DTREE_MAX_NODES], n_par[DTREE_MAX_NODES], n_dep[DTREE_MAX_NODES];
  __shared__ uint32_t n_anc[DTREE_MAX_NODES][DTREE_MASK_WORDS];
  const int lane = threadIdx.x;
  int n_ent = 0, nodes = 0;
  if (p.budget > 0 && p.depth > 0) {
    if (lane == 0) {
      e_logw[0] = (double)p.top_lp[0];
      e_r0[0] = 1ull << 57;  // ranks (0,)
      e_r1[0] = 0ull;
      e_meta[0] = 0 | (1 << 8) | (0 << 16);
    }
    n_ent = 1;
  }
  __syncthreads();
  while (nodes < p.budget && n_ent > 0) {
    double bl = -__builtin_inff();
    unsigned long long b0 = ~0ull, b1 = ~0ull;
    int bi = -1;
    for (int i = lane; i < n_ent; i += 64) {
      if (e_meta[i] < 0) continue;
      if (bi < 0 || better(e_logw[i], e_r0[i], e_r1[i], bl, b0, b1)) {
        bl = e_logw[i];
        b0 = e_r0[i];
        b1 = e_r1[i];
        bi = i;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const double ol = __shfl_xor(bl, o);
      const unsigned long long o0 = __shfl_xor(b0, o), o1 = __shfl_xor(b1, o);
      const int oi = __shfl_xor(bi, o);
      if (oi >= 0 && (bi < 0 || better(ol, o0, o1, bl, b0, b1))) {
        bl = ol;
        b0 = o0;
        b1 = o1;
        bi = oi;
      }
    }
    if (bi < 0) break;  // heap empty (every lane agrees)
    const int meta = e_meta[bi];
    const int parent = meta & 255, d = (meta >> 8) & 255, r = meta >> 16;
    const int idx = nodes + 1;
    if (lane == 0) {
      e_meta[bi] = -1;
      const int tok = p.top_tok[(d - 1) * p.k + r];
      n_tok[idx] = tok;
      n_par[idx] = parent;
      n_dep[idx] = d;
#pragma unroll
      for (int w = 0; w < DTREE_MASK_WORDS; ++w)
        n_anc[idx][w] = (parent == 0 ? (w == 0 ? 1u : 0u) : n_anc[parent][w]) | (w == idx / 32 ? 1u << (idx % 32) : 0u);
      int ne = n_ent;
      if (r + 1 < p.k) {  // sibling: ranks[:-1] + (rank + 1,)
        e_logw[ne] = (bl - (double)p.top_lp[(d - 1) * p.k + r]) + (double)p.top_lp[(d - 1) * p.k + r + 1];
        unsigned long long s0 = b0, s1 = b1;
        add_level(s0, s1, d, 1ull);
        e_r0[ne] = s0;
        e_r1[ne] = s1;
        e_meta[ne] = parent | (d << 8) | ((r + 1) << 16);
        ++ne;
      }
      if (d < p.depth) {  // first child: ranks + (0,)
        e_logw[ne] = bl + (double)p.top_lp[d * p.k];
        unsigned long long c0 = b0, c1 = b1;
        add_level(c0, c1, d + 1, 1ull);
        e_r0[ne] = c0;
        e_r1[ne] = c1;
        e_meta[ne] = idx | ((d + 1) << 8);
      }
    }
    n_ent += (r + 1 < p.k ? 1 : 0) + (d < p.depth ? 1 : 0);
    ++nodes;
    __syncthreads();
  }
  // descriptor: root + nodes in pop order, rows past L cleared
  const int L = nodes + 1;
  DtreeStepDesc* dd = p.desc;
  for (int i = lane; i < DTREE_MAX_NODES; i += 64) {
    const bool live = i < L;
    dd->tokens[i] = !live ? 0 : (i == 0 ? p.root : n_tok[i]);
    dd->positions[i] = !live ? 0 : p.past + (i == 0 ? 0 : n_dep[i]);
    dd->parents[i] = !live ? -1 : (i == 0 ? -1 : n_par[i]);
#pragma unroll
    for (int w = 0; w < DTREE_MASK_WORDS; ++w)
      dd->ancestors[i][w] = !live ? 0u : (i == 0 ? (w == 0 ? 1u : 0u) : n_anc[i][w]);
    dd->accepted[i] = 0;
    dd->posterior[i] = 0;
    if (p.tree_out && i < DTREE_MAX_NODES - 1) {
      p.tree_out[1 + i] = i + 1 < L ? n_tok[i + 1] : 0;
      p.tree_out[1 + DTREE_MAX_NODES + i] = i + 1 < L ? n_dep[i + 1] : 0;
      p.tree_out[1 + 2 * DTREE_MAX_NODES + i] = i + 1 < L ? n_par[i + 1] : -1;
    }
  }
  if (lane == 0) {
    dd->past_length = p.past;
    dd->num_nodes = L;
    dd->n_accepted = 0;
    dd->bonus_token = -1;
    if (p.tree_out) p.tree_out[0] = nodes;
  }
}

size_t tree_ws_layout(int depth, int vocab, int k, size_t* off_ms, size_t* off_tok, size_t* off_lp) {
  const int chunks = (vocab + kChunk - 1) / kChunk;
  size_t o = (size_t)depth * chunks * k * sizeof(unsigned long long);
  *off_ms = o;
  o += (size_t)depth * chunks * sizeof(float2);
  o = (o + 255) / 256 * 256;
  *off_tok = o;
  o += (size_t)depth * k * sizeof(int);
  o = (o + 255) / 256 * 256;
  *off_lp = o;
  o += (size_t)depth * k * sizeof(float);
  return (o + 255) / 256 * 256;
}

}  // namespace
}  // namespace dtree

using namespace dtree;

extern "C" size_t dtree_tree_build_workspace_bytes(int32_t depth, int32_t vocab, int32_t topk) {
  if (depth <= 0 || vocab <= 0 || topk <= 0) return 0;
  size_t a, b, c;
  return tree_ws_layout(depth, vocab, topk, &a, &b, &c);
}

extern "C" int dtree_tree_build(const float* logits, int32_t ld, int32_t depth, int32_t vocab, int32_t topk,
                                int32_t budget, int32_t root_token, int32_t past_length, void* workspace,
                                size_t workspace_bytes, DtreeStepDesc* desc, int32_t* tree_out, int32_t* topk_ids,
                                float* topk_logprobs, hipStream_t stream) {
  DTREE_REQUIRE(desc, "tree_build: null desc");
  DTREE_REQUIRE(budget >= 0 && budget <= DTREE_MAX_NODES - 1, "tree_build: budget must be in [0, 127]");
  DTREE_REQUIRE(depth >= 0 && depth <= kMaxDepth, "tree_build: depth (draft rows) must be in [0, 18]");
  DTREE_REQUIRE(past_length >= 0 && past_length <= (1 << 30) - kMaxDepth, "tree_build: past_length");
  DTREE_REQUIRE(root_token >= 0, "tree_build: root_token");
  TreeParams p{};
  p.depth = depth;
  p.budget = budget;
  p.root = root_token;
  p.past = past_length;
  p.desc = desc;
  p.tree_out = tree_out;
  p.topk_ids = topk_ids;
  p.topk_lp = topk_logprobs;
  if (budget > 0 && depth > 0) {
    DTREE_REQUIRE(logits && workspace, "tree_build: null logits / workspace");
    DTREE_REQUIRE(vocab > 0 && vocab % 4 == 0 && ld >= vocab && ld % 4 == 0 && ((uintptr_t)logits & 15) == 0,
                  "tree_build: vocab and ld multiples of 4, ld >= vocab, 16-byte aligned logits");
    DTREE_REQUIRE(topk >= 1 && topk <= kMaxK && topk <= vocab, "tree_build: topk must be in [1, min(127, vocab)]");
    const int chunks = (vocab + kChunk - 1) / kChunk;
    DTREE_REQUIRE((size_t)chunks * topk <= (size_t)kCand, "tree_build: vocab / 8192 * topk must be <= 4096");
    size_t off_ms, off_tok, off_lp;
    const size_t need = tree_ws_layout(depth, vocab, topk, &off_ms, &off_tok, &off_lp);
    DTREE_REQUIRE(workspace_bytes >= need, "tree_build: workspace too small");
    char* ws = static_cast<char*>(workspace);
    p.logits = logits;
    p.ld = ld;
    p.vocab = vocab;
    p.k = topk;
    p.chunks = chunks;
    p.part_keys = reinterpret_cast<unsigned long long*>(ws);
    p.part_ms = reinterpret_cast<float2*>(ws + off_ms);
    p.top_tok = reinterpret_cast<int*>(ws + off_tok);
    p.top_lp = reinterpret_cast<float*>(ws + off_lp);
    topk_chunk_kernel<<<dim3(chunks, depth), kThreads, 0, stream>>>(p);
    DTREE_LAUNCH_CHECK("tree_build: top-k pass");
    topk_merge_kernel<<<depth, kThreads, 0, stream>>>(p);
    DTREE_LAUNCH_CHECK("tree_build: merge pass");
  }
  heap_kernel<<<1, 64, 0, stream>>>(p);
  DTREE_LAUNCH_CHECK("tree_build: heap");
  return DTREE_OK;
}
