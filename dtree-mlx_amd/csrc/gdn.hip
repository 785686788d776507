// Qwen3.5 GatedDeltaNet tree primitives: tree conv1d + SiLU, the tree
// gated-delta recurrence, and the commit of an accepted path.
//
// Reference semantics (qwen35_tree_kernels.py:8-152): node t derives its conv
// window and its fp32 state [Dv][Dk] (per value head) from its parent's, the
// root from the base. Evaluation is lazy: the tree kernels return per-node
// outputs and keep node windows / states out of HBM (optional debug outputs
// aside); after the accept walk, dtree_gdn_commit replays only the accepted
// path from the base window / state.
//
// Conv: a node's window is the last K rows of (base window ++ inputs along its
// root path), so every (node, channel) is independent: a thread per channel
// walks up to K - 1 ancestors (parents in LDS) and issues all its loads at once.
// Recurrence: a workgroup owns one value head and RPW state rows (dv); lanes
// per row = Dk / 4 (4 fp32 state elements each, dot products by butterflies
// over the row's lanes). Node inputs (q, k, v, g, beta) and the node states of
// the workgroup's rows live in LDS; nodes run in index order (parent < child).
#include "common.h"

namespace dtree {

constexpr int kConvMaxKeep = 7;
constexpr int kGdnMaxNodes = DTREE_MAX_NODES;

__device__ __forceinline__ float silu_acc(float a) { return a / (1.0f + __expf(-a)); }

template <int KEEP>
__global__ __launch_bounds__(256) void gdn_conv_kernel(const float* __restrict__ x, const float* __restrict__ base,
                                                       const float* __restrict__ w, const int* __restrict__ parents,
                                                       int T, int C, float* __restrict__ out,
                                                       float* __restrict__ windows) {
  constexpr int keep = KEEP;
  __shared__ int par[kGdnMaxNodes];
  for (int t = threadIdx.x; t < T; t += blockDim.x) par[t] = parents[t];
  __syncthreads();
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float wk[keep + 1], bk[keep];
#pragma unroll
  for (int r = 0; r <= keep; ++r) wk[r] = w[(size_t)r * C + c];
#pragma unroll
  for (int r = 0; r < keep; ++r) bk[r] = base[(size_t)r * C + c];
  for (int t = 0; t < T; ++t) {
    // window of t = last keep + 1 rows of (base ++ x along the root path):
    // val[i] is row keep - i (val[0] = x[t]).
    float val[keep + 1];
    int anc = t, nb = 0;
#pragma unroll
    for (int i = 0; i <= keep; ++i) {
      if (anc >= 0) {
        val[i] = x[(size_t)anc * C + c];
        anc = par[anc];
      } else {
        val[i] = bk[keep - 1 - nb];
        ++nb;
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i <= keep; ++i) acc += wk[keep - i] * val[i];
    out[(size_t)t * C + c] = silu_acc(acc);
    if (windows)
#pragma unroll
      for (int r = 0; r < keep; ++r) windows[((size_t)t * keep + r) * C + c] = val[keep - 1 - r];
  }
}

struct GdnParams {
  const float* q; const float* k; const float* v; const float* g; const float* beta;
  float* state;        // [Hv][Dv][Dk] base state (commit: updated in place)
  const int* parents;  // tree kernel
  const int* path; const int* path_len;  // commit kernel (device)
  int T, Hk, Hv, Dv, rpw;
  float* y;            // [T][Hv][Dv]
  float* states;       // optional [T][Hv][Dv][Dk]
};

// Sum over the LPR lanes that share a row (lanes are consecutive).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// One recurrence step on a thread's 4 state elements.
template <int LPR>
__device__ __forceinline__ float gdn_step(f32x4_t& s, f32x4_t kk, f32x4_t qq, float vv, float gg, float bb) {
  s *= gg;
  float kv = s[0] * kk[0] + s[1] * kk[1] + s[2] * kk[2] + s[3] * kk[3];
  kv = row_sum<LPR>(kv);
  const float delta = (vv - kv) * bb;
  s += kk * delta;
  float o = s[0] * qq[0] + s[1] * qq[1] + s[2] * qq[2] + s[3] * qq[3];
  return row_sum<LPR>(o);
}

// Tree recurrence. Dynamic LDS (floats): qk [T][2][DK], vgb [T][rpw + 2],
// node states [T][rpw][DK].
template <int DK>
__global__ __launch_bounds__(256) void gdn_tree_kernel(GdnParams p) {
  constexpr int LPR = DK / 4;
  extern __shared__ float lds[];
  __shared__ int par[kGdnMaxNodes];
  const int T = p.T, rpw = p.rpw;
  const int nslices = p.Dv / rpw;
  const int h = blockIdx.x / nslices, row0 = (blockIdx.x % nslices) * rpw;
  const int hk = h / (p.Hv / p.Hk);
  float* qk = lds;
  float* vgb = qk + (size_t)T * 2 * DK;
  float* st = vgb + (size_t)T * (rpw + 2);
  const int nthr = blockDim.x;
  for (int t = threadIdx.x; t < T; t += nthr) par[t] = p.parents[t];
  for (int e = threadIdx.x; e < T * 2 * DK; e += nthr) {
    const int t = e / (2 * DK), r = e % (2 * DK);
    const float* src = r < DK ? p.q : p.k;
    qk[e] = src[((size_t)t * p.Hk + hk) * DK + (r % DK)];
  }
  for (int e = threadIdx.x; e < T * (rpw + 2); e += nthr) {
    const int t = e / (rpw + 2), r = e % (rpw + 2);
    float val;
    if (r < rpw) val = p.v[((size_t)t * p.Hv + h) * p.Dv + row0 + r];
    else if (r == rpw) val = p.g[(size_t)t * p.Hv + h];
    else val = p.beta[(size_t)t * p.Hv + h];
    vgb[e] = val;
  }
  const int rl = threadIdx.x / LPR, lane4 = threadIdx.x % LPR;
  const int dv = row0 + rl;
  const f32x4_t base = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + dv) * DK + 4 * lane4);
  __syncthreads();
  for (int t = 0; t < T; ++t) {
    const int pa = par[t];
    f32x4_t s = pa < 0 ? base : *reinterpret_cast<const f32x4_t*>(st + ((size_t)pa * rpw + rl) * DK + 4 * lane4);
    const f32x4_t kk = *reinterpret_cast<const f32x4_t*>(qk + (size_t)t * 2 * DK + DK + 4 * lane4);
    const f32x4_t qq = *reinterpret_cast<const f32x4_t*>(qk + (size_t)t * 2 * DK + 4 * lane4);
    const float* vt = vgb + (size_t)t * (rpw + 2);
    const float o = gdn_step<LPR>(s, kk, qq, vt[rl], vt[rpw], vt[rpw + 1]);
    *reinterpret_cast<f32x4_t*>(st + ((size_t)t * rpw + rl) * DK + 4 * lane4) = s;
    if (lane4 == 0) p.y[((size_t)t * p.Hv + h) * p.Dv + dv] = o;
    if (p.states)
      *reinterpret_cast<f32x4_t*>(p.states + (((size_t)t * p.Hv + h) * p.Dv + dv) * DK + 4 * lane4) = s;
    // A node's state slot is read back only by the thread that wrote it (a
    // child at a later t), so program order orders the LDS accesses.
  }
}

// Commit: replay the accepted path (path[0 .. *path_len), a root path) from the
// base state, in place; the conv part moves the base window to the last keep
// rows of (window ++ x along the path). Blocks [0, conv_blocks) do the conv
// window, the rest the state rows.
template <int DK>
__global__ __launch_bounds__(256) void gdn_commit_kernel(GdnParams p, const float* x, float* window, int C,
                                                         int keep, int conv_blocks) {
  constexpr int LPR = DK / 4;
  const int n = min(max(*p.path_len, 0), kGdnMaxNodes);
  if ((int)blockIdx.x < conv_blocks) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C || n == 0) return;
    // New window = the last keep rows of (window ++ x[path]). In place: row r
    // takes old row r + from_path (not yet overwritten) or a path input.
    const int from_path = min(n, keep);
    const int from_win = keep - from_path;
    for (int r = 0; r < keep; ++r) {
      const float val = r < from_win ? window[(size_t)(r + from_path) * C + c]
                                     : x[(size_t)p.path[n - from_path + (r - from_win)] * C + c];
      window[(size_t)r * C + c] = val;
    }
    return;
  }
  const int b = blockIdx.x - conv_blocks;
  const int rpw = p.rpw, nslices = p.Dv / rpw;
  const int h = b / nslices, row0 = (b % nslices) * rpw;
  const int hk = h / (p.Hv / p.Hk);
  const int rl = threadIdx.x / LPR, lane4 = threadIdx.x % LPR;
  if (rl >= rpw) return;  // surplus threads of the 256-thread launch
  const int dv = row0 + rl;
  float* sp = p.state + ((size_t)h * p.Dv + dv) * DK + 4 * lane4;
  f32x4_t s = *reinterpret_cast<const f32x4_t*>(sp);
  for (int i = 0; i < n; ++i) {
    const int t = p.path[i];
    const f32x4_t kk = *reinterpret_cast<const f32x4_t*>(p.k + ((size_t)t * p.Hk + hk) * DK + 4 * lane4);
    const f32x4_t qq = *reinterpret_cast<const f32x4_t*>(p.q + ((size_t)t * p.Hk + hk) * DK + 4 * lane4);
    gdn_step<LPR>(s, kk, qq, p.v[((size_t)t * p.Hv + h) * p.Dv + dv], p.g[(size_t)t * p.Hv + h],
                  p.beta[(size_t)t * p.Hv + h]);
  }
  *reinterpret_cast<f32x4_t*>(sp) = s;
}

// Rows per workgroup: the largest power of two <= 256 / (Dk / 4) and <= Dv
// whose LDS footprint fits in 150 KB.
static int gdn_rpw(int T, int Dk, int Dv, size_t* lds_bytes) {
  const int lpr = Dk / 4;
  for (int rpw = 256 / lpr; rpw >= 1; rpw >>= 1) {
    if (rpw > Dv || Dv % rpw) continue;
    const size_t bytes = ((size_t)T * 2 * Dk + (size_t)T * (rpw + 2) + (size_t)T * rpw * Dk) * sizeof(float);
    if (bytes <= 150 * 1024) {
      *lds_bytes = bytes;
      return rpw;
    }
  }
  return 0;
}

}  // namespace dtree

using namespace dtree;

extern "C" int dtree_gdn_tree_conv(const float* x, const float* base_window, const float* weight,
                                   const int32_t* parents, int32_t num_nodes, int32_t channels, int32_t keep,
                                   float* out, float* windows, hipStream_t stream) {
  DTREE_REQUIRE(x && base_window && weight && parents && out, "gdn_tree_conv: null pointer");
  DTREE_REQUIRE(num_nodes >= 1 && num_nodes <= kGdnMaxNodes, "gdn_tree_conv: num_nodes in [1, 128]");
  DTREE_REQUIRE(channels > 0 && keep >= 1 && keep <= kConvMaxKeep, "gdn_tree_conv: channels / keep (<= 7)");
  const int grid = (channels + 255) / 256;
  switch (keep) {
#define DTREE_CONV_CASE(K) \
  case K: gdn_conv_kernel<K><<<grid, 256, 0, stream>>>(x, base_window, weight, parents, num_nodes, channels, out, windows); break;
    DTREE_CONV_CASE(1) DTREE_CONV_CASE(2) DTREE_CONV_CASE(3) DTREE_CONV_CASE(4) DTREE_CONV_CASE(5) DTREE_CONV_CASE(6)
    DTREE_CONV_CASE(7)
#undef DTREE_CONV_CASE
  }
  DTREE_LAUNCH_CHECK("gdn_tree_conv launch");
  return DTREE_OK;
}

extern "C" int dtree_gdn_tree_recurrence(const float* q, const float* k, const float* v, const float* g,
                                         const float* beta, const float* state, const int32_t* parents,
                                         int32_t num_nodes, int32_t num_k_heads, int32_t num_v_heads,
                                         int32_t head_k_dim, int32_t head_v_dim, float* y, float* states,
                                         hipStream_t stream) {
  DTREE_REQUIRE(q && k && v && g && beta && state && parents && y, "gdn_tree_recurrence: null pointer");
  DTREE_REQUIRE(num_nodes >= 1 && num_nodes <= kGdnMaxNodes, "gdn_tree_recurrence: num_nodes in [1, 128]");
  DTREE_REQUIRE(num_k_heads > 0 && num_v_heads > 0 && num_v_heads % num_k_heads == 0,
                "gdn_tree_recurrence: num_v_heads % num_k_heads");
  DTREE_REQUIRE(head_k_dim == 32 || head_k_dim == 64 || head_k_dim == 128, "gdn_tree_recurrence: head_k_dim 32/64/128");
  DTREE_REQUIRE(head_v_dim > 0, "gdn_tree_recurrence: head_v_dim");
  size_t lds = 0;
  const int rpw = gdn_rpw(num_nodes, head_k_dim, head_v_dim, &lds);
  DTREE_REQUIRE(rpw > 0, "gdn_tree_recurrence: tree too large for the LDS-resident node states");
  GdnParams p{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta; p.state = const_cast<float*>(state); p.parents = parents;
  p.T = num_nodes; p.Hk = num_k_heads; p.Hv = num_v_heads; p.Dv = head_v_dim; p.rpw = rpw;
  p.y = y; p.states = states;
  const int grid = num_v_heads * (head_v_dim / rpw);
  const int threads = rpw * (head_k_dim / 4);
  switch (head_k_dim) {
    case 32: gdn_tree_kernel<32><<<grid, threads, lds, stream>>>(p); break;
    case 64: gdn_tree_kernel<64><<<grid, threads, lds, stream>>>(p); break;
    default: gdn_tree_kernel<128><<<grid, threads, lds, stream>>>(p); break;
  }
  DTREE_LAUNCH_CHECK("gdn_tree_recurrence launch");
  return DTREE_OK;
}

extern "C" int dtree_gdn_commit(const float* x, float* window, int32_t channels, int32_t keep, const float* q,
                                const float* k, const float* v, const float* g, const float* beta, float* state,
                                const int32_t* path, const int32_t* path_len, int32_t num_k_heads,
                                int32_t num_v_heads, int32_t head_k_dim, int32_t head_v_dim, hipStream_t stream) {
  DTREE_REQUIRE(path && path_len, "gdn_commit: null path");
  DTREE_REQUIRE(!window || (x && channels > 0 && keep >= 1 && keep <= kConvMaxKeep), "gdn_commit: conv window");
  DTREE_REQUIRE(!state || (q && k && v && g && beta), "gdn_commit: recurrence inputs");
  DTREE_REQUIRE(num_k_heads > 0 && num_v_heads > 0 && num_v_heads % num_k_heads == 0, "gdn_commit: heads");
  DTREE_REQUIRE(head_k_dim == 32 || head_k_dim == 64 || head_k_dim == 128, "gdn_commit: head_k_dim 32/64/128");
  const int lpr = head_k_dim / 4;
  int rpw = 256 / lpr;
  while (rpw > 1 && head_v_dim % rpw) rpw >>= 1;
  GdnParams p{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta; p.state = state; p.path = path; p.path_len = path_len;
  p.Hk = num_k_heads; p.Hv = num_v_heads; p.Dv = head_v_dim; p.rpw = rpw;
  const int conv_blocks = window ? (channels + 255) / 256 : 0;
  const int state_blocks = state ? num_v_heads * (head_v_dim / rpw) : 0;
  if (conv_blocks + state_blocks == 0) return DTREE_OK;
  // Conv blocks use 256 threads; state blocks rpw * Dk / 4 (<= 256): launch
  // with 256 and let surplus state threads idle.
  const int threads = 256;
  switch (head_k_dim) {
    case 32: gdn_commit_kernel<32><<<conv_blocks + state_blocks, threads, 0, stream>>>(p, x, window, channels, keep, conv_blocks); break;
    case 64: gdn_commit_kernel<64><<<conv_blocks + state_blocks, threads, 0, stream>>>(p, x, window, channels, keep, conv_blocks); break;
    default: gdn_commit_kernel<128><<<conv_blocks + state_blocks, threads, 0, stream>>>(p, x, window, channels, keep, conv_blocks); break;
  }
  DTREE_LAUNCH_CHECK("gdn_commit launch");
  return DTREE_OK;
}
