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
#include <cstdlib>
#include <string>

#include "common.h"

namespace dtree {

constexpr int kConvMaxKeep = 7;
constexpr int kGdnMaxNodes = DTREE_MAX_NODES;

__device__ __forceinline__ float silu_acc(float a) { return a / (1.0f + __expf(-a)); }
// SiLU with the hardware reciprocal (within 1 ulp) in place of the IEEE division.
__device__ __forceinline__ float silu_fast(float a) { return a * __builtin_amdgcn_rcpf(1.0f + __expf(-a)); }

template <int KEEP>
__global__ __launch_bounds__(256) void gdn_conv_kernel(const float* __restrict__ x, const float* __restrict__ base,
                                                       const float* __restrict__ w, const int* __restrict__ parents,
                                                       int T, int C, float* __restrict__ out,
                                                       float* __restrict__ windows) {
  constexpr int keep = KEEP;
  __shared__ int par[kGdnMaxNodes];
  for (int t = threadIdx.x; t < T; t += blockDim.x) par[t] = valid_parent(parents[t], t);
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
  const int* T_dev;    // optional device node count (<= T, which sizes LDS)
  int T, Hk, Hv, Dv, rpw;
  float* y;            // [T][Hv][Dv]
  float* states;       // optional [T][Hv][Dv][Dk]
  float* state_out;    // commit: destination of the new state (nullptr: in place)
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
  const int T = p.T_dev ? min(max(*p.T_dev, 0), p.T) : p.T;
  const int rpw = p.rpw;
  const int nslices = p.Dv / rpw;
  const int h = blockIdx.x / nslices, row0 = (blockIdx.x % nslices) * rpw;
  const int hk = h / (p.Hv / p.Hk);
  float* qk = lds;
  float* vgb = qk + (size_t)T * 2 * DK;
  float* st = vgb + (size_t)T * (rpw + 2);
  const int nthr = blockDim.x;
  for (int t = threadIdx.x; t < T; t += nthr) par[t] = valid_parent(p.parents[t], t);
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

// Sum over the 32 consecutive lanes of a row, three values at once (their
// steps interleave, so the latency of one reduction covers all three): DPP
// quad permutes, half-row and row mirrors, then a lane swap across the two
// 16-lane rows (v_permlane16_swap: VALU only, so the recurrence's critical
// path has no LDS round trip). Every lane of the row ends with the sums.
__device__ __forceinline__ void row_sum32x3(float& a, float& b, float& c) {
  a += dpp<0xB1>(a); b += dpp<0xB1>(b); c += dpp<0xB1>(c);     // lane ^ 1
  a += dpp<0x4E>(a); b += dpp<0x4E>(b); c += dpp<0x4E>(c);     // lane ^ 2
  a += dpp<0x141>(a); b += dpp<0x141>(b); c += dpp<0x141>(c);  // half-row mirror: other quad
  a += dpp<0x140>(a); b += dpp<0x140>(b); c += dpp<0x140>(c);  // row mirror: other 8 lanes
  a = row_pair_sum(a); b = row_pair_sum(b); c = row_pair_sum(c);  // other 16-lane row
}

template <int TMAX>
struct RegTree {
  const GdnParams& p;
  const float* qk;   // [TMAX][2][128]
  const float* vgb;  // [TMAX][8 + 2]
  const int* par;
  int T, h, dv, rl, lane;
  f32x4_t base;
};

// Node t of the register-resident recurrence. The recursion unrolls the node
// loop in the source, so every index into s[] is a constant and the node
// states stay in registers.
template <int TMAX, int t>
__device__ __forceinline__ void reg_tree_step(const RegTree<TMAX>& r, f32x4_t (&s)[TMAX]) {
  if constexpr (t < TMAX) {
    if (t >= r.T) return;
    const int pa = __builtin_amdgcn_readfirstlane(r.par[t]);
    f32x4_t sp = r.base;
#pragma unroll
    for (int j = 0; j < t; ++j) sp = pa == j ? s[j] : sp;
    const f32x4_t kk = *reinterpret_cast<const f32x4_t*>(r.qk + (t * 2 + 1) * 128 + 4 * r.lane);
    const f32x4_t qq = *reinterpret_cast<const f32x4_t*>(r.qk + (t * 2) * 128 + 4 * r.lane);
    float sk = sp[0] * kk[0] + sp[1] * kk[1] + sp[2] * kk[2] + sp[3] * kk[3];
    float sq = sp[0] * qq[0] + sp[1] * qq[1] + sp[2] * qq[2] + sp[3] * qq[3];
    float kq = kk[0] * qq[0] + kk[1] * qq[1] + kk[2] * qq[2] + kk[3] * qq[3];
    row_sum32x3(sk, sq, kq);
    const float* vt = r.vgb + t * 10;
    const float g = vt[8], b = vt[9];
    const float delta = (vt[r.rl] - g * sk) * b;
    s[t] = sp * g + kk * delta;
    const GdnParams& p = r.p;
    if (r.lane == 0) p.y[((size_t)t * p.Hv + r.h) * p.Dv + r.dv] = g * sq + delta * kq;
    if (p.states)
      *reinterpret_cast<f32x4_t*>(p.states + (((size_t)t * p.Hv + r.h) * p.Dv + r.dv) * 128 + 4 * r.lane) = s[t];
    reg_tree_step<TMAX, t + 1>(r, s);
  }
}

// Tree recurrence for trees of up to TMAX nodes with Dk = 128: a workgroup
// owns one value head and 8 state rows (32 lanes x 4 elements per row), and
// every node's state of those elements stays in registers (4 x TMAX), so LDS
// holds only the node inputs and all workgroups of a launch are resident at
// once. The parent's state is picked by a select chain on the wave-uniform
// parent index. Per node one reduction yields S_p k, S_p q and k q:
// kv = g (S_p k), delta = (v - kv) beta, y = g (S_p q) + delta (k q), and
// S = g S_p + delta k, which equals the reference order of operations
// (S = g S_p; S += delta k; y = S q) up to rounding.
template <int TMAX>
__global__ __launch_bounds__(256) void gdn_tree_reg_kernel(GdnParams p) {
  constexpr int DK = 128, RPW = 8, NV = TMAX * 2 * DK / 4 / 256;  // staged f32x4 per thread
  __shared__ __align__(16) float qk[TMAX][2][DK];
  __shared__ float vgb[TMAX][RPW + 2];
  __shared__ int par[TMAX];
  const int T = p.T_dev ? min(max(*p.T_dev, 0), min(p.T, TMAX)) : min(p.T, TMAX);
  const int nslices = p.Dv / RPW;
  const int h = blockIdx.x / nslices, row0 = (blockIdx.x % nslices) * RPW;
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x;
  {
    f32x4_t buf[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid + 256 * i, t = e >> 6, r = e & 63;  // r < 32: q, else k
      if (t < T) {
        const float* src = (r < 32 ? p.q : p.k) + ((size_t)t * p.Hk + hk) * DK + 4 * (r & 31);
        buf[i] = *reinterpret_cast<const f32x4_t*>(src);
      }
    }
    for (int e = tid; e < T * (RPW + 2); e += 256) {
      const int t = e / (RPW + 2), r = e % (RPW + 2);
      float val;
      if (r < RPW) val = p.v[((size_t)t * p.Hv + h) * p.Dv + row0 + r];
      else if (r == RPW) val = p.g[(size_t)t * p.Hv + h];
      else val = p.beta[(size_t)t * p.Hv + h];
      vgb[t][r] = val;
    }
    if (tid < T) par[tid] = valid_parent(p.parents[tid], tid);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = tid + 256 * i, t = e >> 6, r = e & 63;
      if (t < T) *reinterpret_cast<f32x4_t*>(&qk[t][r >> 5][4 * (r & 31)]) = buf[i];
    }
  }
  const int rl = tid >> 5, lane = tid & 31;
  const int dv = row0 + rl;
  const f32x4_t base = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + dv) * DK + 4 * lane);
  __syncthreads();
  RegTree<TMAX> rt{p, &qk[0][0][0], &vgb[0][0], par, T, h, dv, rl, lane, base};
  f32x4_t s[TMAX];
  reg_tree_step<TMAX, 0>(rt, s);
}

// Largest tree of the register-resident recurrence (65-node trees of draft
// budget 64 pad to 96 rows); larger trees use gdn_tree_kernel.
constexpr int kRegTreeMax = 96;

// ---- depth-first recurrence for trees of 33-96 nodes ----------------------
//
// Keeping every node's state in registers (gdn_tree_reg_kernel<96>: 4 x 96
// floats per thread) and the nodes' q / k in LDS (96 KB) leaves one
// workgroup per CU, so the 512 workgroups of a Qwen3.5-9B-shaped layer run in
// two rounds, and each node picks its parent's state through a select chain
// over every earlier node. Visiting the nodes in depth-first preorder needs
// far fewer states: a node with one child hands its state straight to that
// child (the next node in preorder), so only nodes with two or more children
// keep theirs, in a stack slot given by their number of branching ancestors
// (slot 0 holds the committed state for the roots). Chains (prompt prefill)
// use no slot at all. The stack is addressed by a wave-uniform index; node
// inputs are staged in LDS by blocks of 8 preorder positions, two blocks
// ahead (about 34 KB, so two workgroups share a CU).
//
// The order is rebuilt from the parent list by every workgroup (a few
// microseconds of LDS work): ancestor bitsets by pointer doubling, depth =
// |ancestors| - 1, subtree sizes, preorder(t) = depth(t) + the subtree sizes
// of the earlier siblings of t and of each of its ancestors (children in
// increasing index order; nodes with no valid parent are roots, ordered the
// same way).
constexpr int kDfsStack = 32;            // slots; at most 31 nested branching ancestors
constexpr int kDfsWords = (kRegTreeMax + 31) / 32;

// The stack as four 32-wide vectors (element e of slot j = vector e, lane j):
// a wave-uniform index into one vector register tuple compiles to indexed
// register moves (s_set_gpr_idx), so the stack stays in VGPRs.
typedef float f32x32_t __attribute__((ext_vector_type(kDfsStack)));
struct DfsStack {
  f32x32_t e[4];
  __device__ __forceinline__ f32x4_t get(int d) const { return f32x4_t{e[0][d], e[1][d], e[2][d], e[3][d]}; }
  __device__ __forceinline__ void put(int d, f32x4_t v) {
    e[0][d] = v[0];
    e[1][d] = v[1];
    e[2][d] = v[2];
    e[3][d] = v[3];
  }
};

// Depth-first preorder of the first T (<= kRegTreeMax) nodes. For position i:
// order[i] = the node and meta[i] = node | (rslot + 1) << 8 | (wslot + 1) << 16
// with rslot the stack slot its parent's state is read from (-1: the state
// just computed) and wslot the slot its own state is kept in (-1: none).
// Returns the largest slot used. Every thread of the workgroup calls it (it
// holds barriers).
__device__ int tree_preorder(const int* parents, int T, int* order, int* meta) {
  __shared__ uint32_t anc[kRegTreeMax][kDfsWords];
  __shared__ int par[kRegTreeMax], up[kRegTreeMax], sz[kRegTreeMax], esz[kRegTreeMax], dep[kRegTreeMax];
  __shared__ int nch[kRegTreeMax], bd[kRegTreeMax];
  __shared__ int s_max;
  const int t = threadIdx.x;
  if (t == 0) s_max = 0;
  if (t < T) {
    const int pa = valid_parent(parents[t], t);
    par[t] = pa;
    up[t] = pa;
#pragma unroll
    for (int w = 0; w < kDfsWords; ++w) anc[t][w] = (t >> 5) == w ? 1u << (t & 31) : 0u;
  }
  __syncthreads();
  // pointer doubling: after round r, anc[t] holds t and its ancestors within
  // distance 2^r - 1 and up[t] the ancestor at distance 2^r
  for (int r = 0; (1 << r) < kRegTreeMax; ++r) {
    uint32_t a[kDfsWords];
    int u = -1;
    if (t < T) {
      u = up[t];
#pragma unroll
      for (int w = 0; w < kDfsWords; ++w) a[w] = anc[t][w];
      if (u >= 0) {
#pragma unroll
        for (int w = 0; w < kDfsWords; ++w) a[w] |= anc[u][w];
        u = up[u];
      }
    }
    __syncthreads();
    if (t < T) {
#pragma unroll
      for (int w = 0; w < kDfsWords; ++w) anc[t][w] = a[w];
      up[t] = u;
    }
    __syncthreads();
  }
  if (t < T) {
    int d = -1, n = 0, c = 0;
#pragma unroll
    for (int w = 0; w < kDfsWords; ++w) d += __popc(anc[t][w]);
    for (int u = 0; u < T; ++u) {
      n += (anc[u][t >> 5] >> (t & 31)) & 1u;
      c += par[u] == t;
    }
    dep[t] = d;
    sz[t] = n;
    nch[t] = c;
  }
  __syncthreads();
  if (t < T) {
    const int pa = par[t];
    int e = 0;
    for (int u = 0; u < t; ++u) e += par[u] == pa ? sz[u] : 0;
    esz[t] = e;
    int b = 0;  // branching proper ancestors
#pragma unroll
    for (int w = 0; w < kDfsWords; ++w) {
      uint32_t m = anc[t][w];
      while (m) {
        const int a = 32 * w + __ffs(m) - 1;
        m &= m - 1;
        b += a != t && nch[a] >= 2;
      }
    }
    bd[t] = b;
  }
  __syncthreads();
  if (t < T) {
    int pre = dep[t];
#pragma unroll
    for (int w = 0; w < kDfsWords; ++w) {
      uint32_t m = anc[t][w];
      while (m) {
        const int a = 32 * w + __ffs(m) - 1;
        m &= m - 1;
        pre += esz[a];
      }
    }
    const int pa = par[t];
    const int ws = nch[t] >= 2 ? bd[t] + 1 : -1;
    const int rs = pa < 0 ? 0 : (nch[pa] >= 2 ? bd[pa] + 1 : -1);
    order[pre] = t;
    meta[pre] = t | (rs + 1) << 8 | (ws + 1) << 16;
    atomicMax(&s_max, ws);
  }
  __syncthreads();
  return s_max;
}

// The recurrence over the preorder: a workgroup owns one value head and 8
// state rows (32 lanes x 4 elements per row) as in gdn_tree_reg_kernel, with
// the same per-node arithmetic and one reduction for S_p k, S_p q and k q.
// A tree with more than kDfsStack - 1 nested branching nodes writes NaN.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_tree_dfs_kernel(GdnParams p) {
  constexpr int DK = 128, RPW = 8;
  __shared__ int order[kRegTreeMax], meta[kRegTreeMax];
  const int T = p.T_dev ? min(max(*p.T_dev, 0), min(p.T, kRegTreeMax)) : min(p.T, kRegTreeMax);
  const int nslices = p.Dv / RPW;
  const int h = blockIdx.x / nslices, row0 = (blockIdx.x % nslices) * RPW;
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, rl = tid >> 5, lane = tid & 31;
  const int dv = row0 + rl;
  DfsStack st;
  f32x4_t cur = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + dv) * DK + 4 * lane);
  st.put(0, cur);
  const int top = tree_preorder(p.parents, T, order, meta);
  if (top > kDfsStack - 1) {
    for (int t = tid; t < T * RPW; t += 256)
      p.y[((size_t)(t / RPW) * p.Hv + h) * p.Dv + row0 + t % RPW] = __builtin_nanf("");
    return;
  }
  // Node inputs staged in LDS by blocks of 8 preorder positions, in a ring of
  // 4 blocks filled two blocks ahead: k and q of the key head (256 floats per
  // node, two 16-byte pieces per thread), v of the 8 rows, g and beta.
  constexpr int NBK = 8, RING = 4;
  __shared__ __align__(16) float kqs[RING * NBK][2][DK];
  __shared__ float vgs[RING * NBK][RPW + 2];
  const int nblocks = (T + NBK - 1) / NBK;
  f32x4_t rk[2];
  float rv = 0.f;
  auto block_issue = [&](int b) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i, n = e >> 6, w = (e >> 5) & 1, c4 = e & 31;  // node, k|q, 16-byte piece
      const int j = b * NBK + n;
      if (b < nblocks && j < T) {
        const int t = order[j];
        const float* src = (w == 0 ? p.k : p.q) + ((size_t)t * p.Hk + hk) * DK + 4 * c4;
        rk[i] = *reinterpret_cast<const f32x4_t*>(src);
      }
    }
    if (tid < NBK * (RPW + 2)) {
      const int n = tid / (RPW + 2), r = tid % (RPW + 2), j = b * NBK + n;
      if (b < nblocks && j < T) {
        const int t = order[j];
        rv = r < RPW ? p.v[((size_t)t * p.Hv + h) * p.Dv + row0 + r]
                     : (r == RPW ? p.g[(size_t)t * p.Hv + h] : p.beta[(size_t)t * p.Hv + h]);
      }
    }
  };
  auto block_store = [&](int b) {
    const int base = (b % RING) * NBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i, n = e >> 6, w = (e >> 5) & 1, c4 = e & 31;
      *reinterpret_cast<f32x4_t*>(&kqs[base + n][w][4 * c4]) = rk[i];
    }
    if (tid < NBK * (RPW + 2)) vgs[base + tid / (RPW + 2)][tid % (RPW + 2)] = rv;
  };
  block_issue(0);
  block_store(0);
  block_issue(1);
  block_store(1);
  block_issue(2);
  __syncthreads();
  // One node's inputs from the ring (positions past T read stale entries that
  // are never used), loaded a node ahead of its arithmetic.
  struct NodeIn {
    f32x4_t kk, qq;
    float v, g, b;
    int meta;
  };
  auto node_in = [&](int slot, int j) {
    NodeIn r;
    r.kk = *reinterpret_cast<const f32x4_t*>(&kqs[slot][0][4 * lane]);
    r.qq = *reinterpret_cast<const f32x4_t*>(&kqs[slot][1][4 * lane]);
    r.v = vgs[slot][rl];
    r.g = vgs[slot][RPW];
    r.b = vgs[slot][RPW + 1];
    r.meta = meta[min(j, kRegTreeMax - 1)];
    return r;
  };
  for (int b = 0; b < nblocks; ++b) {
    const int base = (b % RING) * NBK;
    const int jn = min(NBK, T - b * NBK);
    NodeIn in = node_in(base, b * NBK);
#pragma unroll
    for (int n = 0; n < NBK; ++n) {
      NodeIn nx;
      if (n + 1 < NBK) nx = node_in(base + n + 1, b * NBK + n + 1);
      if (n < jn) {
        const int m = __builtin_amdgcn_readfirstlane(in.meta);
        const int t = m & 255, rs = ((m >> 8) & 255) - 1, ws = ((m >> 16) & 255) - 1;
        const f32x4_t kk = in.kk, qq = in.qq;
        const f32x4_t sp = rs < 0 ? cur : st.get(rs);
        float sk = sp[0] * kk[0] + sp[1] * kk[1] + sp[2] * kk[2] + sp[3] * kk[3];
        float sq = sp[0] * qq[0] + sp[1] * qq[1] + sp[2] * qq[2] + sp[3] * qq[3];
        float kqd = kk[0] * qq[0] + kk[1] * qq[1] + kk[2] * qq[2] + kk[3] * qq[3];
        row_sum32x3(sk, sq, kqd);
        const float delta = (in.v - in.g * sk) * in.b;
        cur = sp * in.g + kk * delta;
        if (ws >= 0) st.put(ws, cur);
        if (lane == 0) p.y[((size_t)t * p.Hv + h) * p.Dv + dv] = in.g * sq + delta * kqd;
        if (p.states)
          *reinterpret_cast<f32x4_t*>(p.states + (((size_t)t * p.Hv + h) * p.Dv + dv) * DK + 4 * lane) = cur;
      }
      if (n + 1 < NBK) in = nx;
    }
    // block b + 2 (issued one block ago) into its ring slot, b + 3 out
    block_store(b + 2);
    block_issue(b + 3);
    __syncthreads();
  }
}

// Path entries index the per-node buffers ([T] rows); an out-of-range entry
// (a descriptor that no walk filled) is clamped so it can never read past them.
__device__ __forceinline__ int clamp_node(int t, int T) { return min(max(t, 0), T - 1); }

// Commit: replay the accepted path (path[0 .. *path_len), a root path) from the
// base state; the conv part moves the base window to the last keep rows of
// (window ++ x along the path). The results go to window_out / p.state_out,
// or back in place when those are null. Blocks [0, conv_blocks) do the conv
// window, the rest the state rows.
template <int DK>
__device__ __forceinline__ void gdn_commit_body(const GdnParams& p, const float* x, int ldx, const float* window,
                                                float* window_out, int C, int keep, int conv_blocks) {
  constexpr int LPR = DK / 4;
  const int n = min(max(*p.path_len, 0), kGdnMaxNodes);
  if ((int)blockIdx.x < conv_blocks) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    float* wout = window_out ? window_out : const_cast<float*>(window);
    if (c >= C || (n == 0 && wout == window)) return;
    // New window = the last keep rows of (window ++ x[path]). In place, row r
    // takes old row r + from_path (not yet overwritten) or a path input.
    const int from_path = min(n, keep);
    const int from_win = keep - from_path;
    for (int r = 0; r < keep; ++r) {
      const float val = r < from_win ? window[(size_t)(r + from_path) * C + c]
                                     : x[(size_t)clamp_node(p.path[n - from_path + (r - from_win)], p.T) * ldx + c];
      wout[(size_t)r * C + c] = val;
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
  const size_t so = ((size_t)h * p.Dv + dv) * DK + 4 * lane4;
  f32x4_t s = *reinterpret_cast<const f32x4_t*>(p.state + so);
  for (int i = 0; i < n; ++i) {
    // The state update needs S k only (y is not replayed).
    const int t = clamp_node(p.path[i], p.T);
    const f32x4_t kk = *reinterpret_cast<const f32x4_t*>(p.k + ((size_t)t * p.Hk + hk) * DK + 4 * lane4);
    const float vv = p.v[((size_t)t * p.Hv + h) * p.Dv + dv];
    const float gg = p.g[(size_t)t * p.Hv + h], bb = p.beta[(size_t)t * p.Hv + h];
    s *= gg;
    float kv = s[0] * kk[0] + s[1] * kk[1] + s[2] * kk[2] + s[3] * kk[3];
    kv = LPR == 32 ? row_sum32(kv) : row_sum<LPR>(kv);
    s += kk * ((vv - kv) * bb);
  }
  *reinterpret_cast<f32x4_t*>((p.state_out ? p.state_out : p.state) + so) = s;
}

template <int DK>
__global__ __launch_bounds__(256) void gdn_commit_kernel(GdnParams p, const float* x, int ldx, const float* window,
                                                         float* window_out, int C, int keep, int conv_blocks) {
  gdn_commit_body<DK>(p, x, ldx, window, window_out, C, keep, conv_blocks);
}

// The commits of several GatedDeltaNet layers of one step in one launch: row
// blockIdx.y of the grid is layer blockIdx.y of the batch (its projection
// rows, window, state and k / v / g / beta); the layers share the accepted
// path and the shapes. Each layer reads and rewrites its whole committed state
// (2 MB at 32 value heads of 128 x 128), so the batch is one stream of those
// bytes instead of one short launch per layer.
constexpr int kCommitMaxLayers = 32;
struct CommitLayer {
  const float* x; float* window; float* state;
  const float* k; const float* v; const float* g; const float* beta;
  float* window_out; float* state_out;  // nullptr: in place
};
struct CommitBatch {
  CommitLayer l[kCommitMaxLayers];
};

template <int DK>
__global__ __launch_bounds__(256) void gdn_commit_layers_kernel(GdnParams p, CommitBatch b, int ldx, int C, int keep,
                                                                int conv_blocks) {
  const CommitLayer& ly = b.l[blockIdx.y];
  GdnParams q = p;
  q.state = ly.state; q.k = ly.k; q.v = ly.v; q.g = ly.g; q.beta = ly.beta; q.state_out = ly.state_out;
  gdn_commit_body<DK>(q, ly.x, ldx, ly.window, ly.window_out, C, keep, conv_blocks);
}

// Layer prep (qwen35_tree.py:199-308 between the projections and the
// recurrence): tree conv1d + SiLU of the projected conv input, split into
// q | k | v, q = Dk^-1 rms_norm(q), k = Dk^-1/2 rms_norm(k) per key head
// (eps 1e-6), and per (node, value head) g = exp(-exp(A_log) softplus(a +
// dt_bias)), beta = sigmoid(b). Workgroup s < C / DK owns channels
// s*DK .. s*DK + DK - 1 (one q or k head, or DK value channels), a thread per
// channel; the conv outputs of all nodes are staged in LDS so that thread t
// can reduce node t's head for the norm. The last workgroup computes g and
// beta. Node count and parents come from the step descriptor.
struct PrepParams {
  const DtreeStepDesc* desc; int rows;  // rows = node capacity (sizes LDS)
  int chain;  // > 0: a causal chain of `chain` rows (parent of t is t - 1), no desc
  const float* x; int ldx;  // conv input = proj columns [0, C)
  const float* base; const float* w;
  int C, key_dim, Hv, ab_col;  // b at proj column ab_col + h, a at ab_col + Hv + h
  const float* A_log; const float* dt_bias;
  float* q; float* k; float* v; float* g; float* beta;
  float q_scale, k_scale;
};

__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// One workgroup per (128-channel slice, block of kPrepNodes nodes), plus one
// column of workgroups for g and beta. A thread owns one channel of the
// block's nodes: it issues every conv input it needs at once (the node's row
// and up to KEEP ancestors' rows of the projection output, or rows of the
// committed window past the root path), runs the tree conv and SiLU, and for
// q / k slices the head's sum of squares per node is a workgroup reduction
// (wave sums through DPP and the lane swap, then LDS across the two waves).
constexpr int kPrepNodes = 8;

template <int KEEP, int DK>
__global__ __launch_bounds__(DK) void gdn_prep_kernel(PrepParams p) {
  constexpr int NB = kPrepNodes, NW = DK / 64;
  __shared__ int par[kGdnMaxNodes];
  __shared__ float wsum[NB][NW];
  const int L = p.chain > 0 ? p.chain : min(max(p.desc->num_nodes, 0), p.rows);
  const int t0 = blockIdx.y * NB;
  if (t0 >= L) return;
  const int tid = threadIdx.x;
  const int nslices = p.C / DK;
  if ((int)blockIdx.x == nslices) {
    for (int e = tid; e < NB * p.Hv; e += DK) {
      const int t = t0 + e / p.Hv, h = e % p.Hv;
      if (t >= L) continue;
      const float* row = p.x + (size_t)t * p.ldx + p.ab_col;
      const float b = row[h], a = row[p.Hv + h];
      p.g[(size_t)t * p.Hv + h] = __expf(-__expf(p.A_log[h]) * softplus_f(a + p.dt_bias[h]));
      p.beta[(size_t)t * p.Hv + h] = 1.0f / (1.0f + __expf(-b));
    }
    return;
  }
  if (p.chain == 0)
    for (int t = tid; t < L; t += DK) par[t] = valid_parent(p.desc->parents[t], t);
  const int c0 = blockIdx.x * DK, c = c0 + tid;
  float wk[KEEP + 1], bk[KEEP];
#pragma unroll
  for (int r = 0; r <= KEEP; ++r) wk[r] = p.w[(size_t)r * p.C + c];
#pragma unroll
  for (int r = 0; r < KEEP; ++r) bk[r] = p.base[(size_t)r * p.C + c];
  __syncthreads();
  // window of node t = the last KEEP + 1 rows of (committed window ++ x along
  // the root path): val[n][i] is row KEEP - i (val[n][0] = x[t])
  float val[NB][KEEP + 1];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const int t = t0 + n;
    int anc = t < L ? t : -1, nb = 0;
#pragma unroll
    for (int i = 0; i <= KEEP; ++i) {
      if (anc >= 0) {
        val[n][i] = p.x[(size_t)anc * p.ldx + c];
        anc = p.chain > 0 ? anc - 1 : par[anc];
      } else {
        val[n][i] = bk[KEEP - 1 - min(nb, KEEP - 1)];
        ++nb;
      }
    }
  }
  float o[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i <= KEEP; ++i) acc += wk[KEEP - i] * val[n][i];
    o[n] = silu_acc(acc);
  }
  const bool is_q = c0 < p.key_dim, is_k = !is_q && c0 < 2 * p.key_dim;
  float scale[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) scale[n] = 1.f;
  if (is_q || is_k) {
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      float ss = o[n] * o[n];
      ss += dpp<0xB1>(ss);
      ss += dpp<0x4E>(ss);
      ss += dpp<0x141>(ss);
      ss += dpp<0x140>(ss);
      ss = row_pair_sum(ss);                 // 32 lanes
      ss += __shfl_xor(ss, 32);              // 64 lanes
      if (lane == 0) wsum[n][wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      float tot = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) tot += wsum[n][w2];
      scale[n] = rsqrtf(tot * (1.0f / DK) + 1e-6f) * (is_q ? p.q_scale : p.k_scale);
    }
  }
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const int t = t0 + n;
    if (t >= L) break;
    const float v = o[n] * scale[n];
    if (is_q) p.q[(size_t)t * p.key_dim + c] = v;
    else if (is_k) p.k[(size_t)t * p.key_dim + (c - p.key_dim)] = v;
    else p.v[(size_t)t * (p.C - 2 * p.key_dim) + (c - 2 * p.key_dim)] = v;
  }
}

// Prep and the register-resident recurrence in one launch, for trees of up to
// 32 nodes with Dk = Dv = 128 (the verify step's 25-node trees): each
// workgroup of gdn_tree_reg_kernel computes the inputs it reads itself
// instead of loading them from a prep launch. Its threads load, in one round,
// the raw conv inputs of its key head's q and k channels and of its 8 value
// rows for every node, the parents, the conv taps and committed window of
// their channels, b / a of its value head and its committed state; then run
// the tree conv + SiLU (the same window and tap order as gdn_prep_kernel), the
// q / k RMS scaling (a thread holds 4 channels of one node; the 32 lanes of a
// half-wave hold the node's head) and g / beta into the LDS rows the node loop
// reads. The 32 workgroups of a key head repeat its q / k conv (256 channels x
// nodes x taps). k, v, g and beta go out as gdn_prep_kernel writes them, for
// the commit after the accept walk: k and q once per key head, g and beta once
// per value head, v by every workgroup for its rows.
template <int KEEP>
__global__ __launch_bounds__(256, 2) void gdn_prep_reg_kernel(GdnParams p, PrepParams pp) {
  constexpr int TMAX = 32, DK = 128, RPW = 8, NI = TMAX / 4;  // nodes per thread (4 waves)
  __shared__ __align__(16) float qk[TMAX][2][DK];
  __shared__ __align__(16) float raw[TMAX][2][DK];
  __shared__ float vraw[TMAX][RPW];
  __shared__ float vgb[TMAX][RPW + 2];
  __shared__ int par[TMAX];
  const int T = p.T_dev ? min(max(*p.T_dev, 0), min(p.T, TMAX)) : min(p.T, TMAX);
  const int nslices = p.Dv / RPW;
  const int h = blockIdx.x / nslices, row0 = (blockIdx.x % nslices) * RPW;
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane64 = tid & 63, wave = tid >> 6;
  // q / k staging: thread (wave, lane) holds channels ch .. ch+3 of plane
  // (0 = q, 1 = k) for nodes wave, wave + 4, ...
  const int plane = lane64 >> 5, ch = 4 * (lane64 & 31);
  const int cq = plane * pp.key_dim + hk * DK + ch;  // conv column of those channels
  // v staging: thread tid < 8 T owns node tid / 8, value row row0 + tid % 8
  const int vt = tid >> 3, vj = tid & 7;
  const int cv = 2 * pp.key_dim + h * DK + row0 + vj;
  const int rl = tid >> 5, lane = tid & 31;
  const int dv = row0 + rl;
  f32x4_t base, wk[KEEP + 1], bk[KEEP];
  float wvk[KEEP + 1], bvk[KEEP];
  {
    f32x4_t xr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = wave + 4 * i;
      if (t < T) xr[i] = *reinterpret_cast<const f32x4_t*>(pp.x + (size_t)t * pp.ldx + cq);
    }
    f32x4_t vr;
    if (tid < 2 * T)
      vr = *reinterpret_cast<const f32x4_t*>(pp.x + (size_t)(tid >> 1) * pp.ldx + 2 * pp.key_dim + h * DK + row0 +
                                             4 * (tid & 1));
    float bb = 0.f, aa = 0.f;
    if (tid < T) {
      const float* row = pp.x + (size_t)tid * pp.ldx + pp.ab_col;
      bb = row[h];
      aa = row[pp.Hv + h];
      par[tid] = valid_parent(p.parents[tid], tid);
    }
#pragma unroll
    for (int r = 0; r <= KEEP; ++r) wk[r] = *reinterpret_cast<const f32x4_t*>(pp.w + (size_t)r * pp.C + cq);
#pragma unroll
    for (int r = 0; r < KEEP; ++r) bk[r] = *reinterpret_cast<const f32x4_t*>(pp.base + (size_t)r * pp.C + cq);
#pragma unroll
    for (int r = 0; r <= KEEP; ++r) wvk[r] = pp.w[(size_t)r * pp.C + cv];
#pragma unroll
    for (int r = 0; r < KEEP; ++r) bvk[r] = pp.base[(size_t)r * pp.C + cv];
    const float alog = pp.A_log[h], dtb = pp.dt_bias[h];
    base = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + dv) * DK + 4 * lane);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = wave + 4 * i;
      if (t < T) *reinterpret_cast<f32x4_t*>(&raw[t][plane][ch]) = xr[i];
    }
    if (tid < 2 * T) *reinterpret_cast<f32x4_t*>(&vraw[tid >> 1][4 * (tid & 1)]) = vr;
    if (tid < T) {
      vgb[tid][RPW] = __expf(-__expf(alog) * softplus_f(aa + dtb));
      vgb[tid][RPW + 1] = 1.0f / (1.0f + __expf(-bb));
    }
  }
  __syncthreads();
  // q / k: window of node t = the last KEEP + 1 rows of (committed window ++
  // conv inputs along the root path), newest tap first, as gdn_prep_kernel.
  const float qks = plane ? pp.k_scale : pp.q_scale;
#pragma unroll 1
  for (int i = 0; i < NI; ++i) {
    const int t = wave + 4 * i;  // wave-uniform
    if (t >= T) break;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    int anc = t, nb = 0;
#pragma unroll
    for (int i2 = 0; i2 <= KEEP; ++i2) {
      f32x4_t val;
      if (anc >= 0) {
        val = *reinterpret_cast<const f32x4_t*>(&raw[anc][plane][ch]);
        anc = par[anc];
      } else {
        // window row KEEP - 1 - min(nb, KEEP - 1), selected over constant
        // indices (a runtime index would put the rows in scratch memory)
        const int wr = KEEP - 1 - min(nb, KEEP - 1);
        val = bk[0];
#pragma unroll
        for (int r = 1; r < KEEP; ++r) val = wr == r ? bk[r] : val;
        ++nb;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += wk[KEEP - i2][e] * val[e];
    }
    f32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = silu_acc(acc[e]);
    const float ss = row_sum32(o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3]);
    const float sc = rsqrtf(ss * (1.0f / DK) + 1e-6f) * qks;
    *reinterpret_cast<f32x4_t*>(&qk[t][plane][ch]) = o * sc;
  }
  // v of (node vt, row row0 + vj)
  if (vt < T) {
    float acc = 0.f;
    int anc = vt, nb = 0;
#pragma unroll
    for (int i2 = 0; i2 <= KEEP; ++i2) {
      float val;
      if (anc >= 0) {
        val = vraw[anc][vj];
        anc = par[anc];
      } else {
        const int wr = KEEP - 1 - min(nb, KEEP - 1);
        val = bvk[0];
#pragma unroll
        for (int r = 1; r < KEEP; ++r) val = wr == r ? bvk[r] : val;
        ++nb;
      }
      acc += wvk[KEEP - i2] * val;
    }
    const float o = silu_acc(acc);
    vgb[vt][vj] = o;
    pp.v[(size_t)vt * (pp.C - 2 * pp.key_dim) + (cv - 2 * pp.key_dim)] = o;
  }
  __syncthreads();
  // the commit's inputs (k, v, g, beta) and q, once each
  if (row0 == 0) {
    if (tid < T) {
      pp.g[(size_t)tid * p.Hv + h] = vgb[tid][RPW];
      pp.beta[(size_t)tid * p.Hv + h] = vgb[tid][RPW + 1];
    }
    if (h % (p.Hv / p.Hk) == 0) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int t = wave + 4 * i;
        if (t >= T) break;
        float* dst = (plane ? pp.k : pp.q) + (size_t)t * pp.key_dim + hk * DK + ch;
        *reinterpret_cast<f32x4_t*>(dst) = *reinterpret_cast<const f32x4_t*>(&qk[t][plane][ch]);
      }
    }
  }
  RegTree<TMAX> rt{p, &qk[0][0][0], &vgb[0][0], par, T, h, dv, rl, lane, base};
  f32x4_t s[TMAX];
  reg_tree_step<TMAX, 0>(rt, s);
}

// ---- matrix form of the tree recurrence (trees of up to 32 nodes) ----------
//
// Unrolling S_t = g_t S_p(t) + delta_t k_t^T from the committed state S_0
// along the root path of t gives, with D[t][a] = the product of g_b over the
// path from a (exclusive) to t (inclusive) and gamma_t = the product over the
// whole path,
//   g_t S_p(t) = gamma_t S_0 + sum_{a strict ancestor of t} D[t][a] delta_a k_a^T.
// The recurrence's per-node values are therefore
//   delta_t = beta_t (v_t - gamma_t (S_0 k_t)) - sum_a L[t][a] delta_a,
//             L[t][a] = beta_t D[t][a] (k_a . k_t)  (a strict ancestor of t),
//   y_t     = gamma_t (S_0 q_t) + sum_a U[t][a] delta_a,
//             U[t][a] = D[t][a] (k_a . q_t)  (a ancestor or t itself, D[t][t] = 1),
// i.e. Delta = (I + L)^-1 R with R_t = beta_t (v_t - gamma_t S_0 k_t), and
// Y = diag(gamma) (S_0 Q^T)^T + U (I + L)^-1 R. In node order (parents before
// children) L is strictly lower triangular and L^(d+1) = 0 for a tree whose
// deepest node has d strict ancestors, so
//   (I + L)^-1 = (I - L)(I + L^2)(I + L^4) ... (I + L^(2^(K-1))),  2^K > d:
// ceil(log2(d + 1)) squarings and products of 32 x 32 matrices instead of a
// substitution over the nodes. Everything is fp32 on v_mfma_f32_16x16x4_f32:
// the Gram matrices k.k and q.k, S_0 k and S_0 q, the powers and products, and
// Y. D is formed by walking each node's parent chain (products of g, so any
// real g is handled as by the node-by-node recurrence).
//
// A workgroup owns one value head and 16 value rows (S_0 rows [16][128]); it
// loads its key head's k and q rows of every node, and computes the shared
// 32 x 32 matrices itself (the 8 workgroups of a value head repeat them). Node
// states are not formed: the commit replays the accepted path from S_0.
constexpr int kChunkRows = 16;
constexpr int kChunkThreads = 512;  // 8 waves: two per SIMD for the serial VALU phases

__device__ __forceinline__ f32x4_t mfma16_f32(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// acc += sum over k < 16 NJ of A[m][k] Bt[n][k] for a 16 x 16 tile (A, Bt row
// pointers at the tile's first row, row stride LS floats, 16-byte aligned
// rows). Lane l supplies row l % 16 of both; step s of dim group j contracts
// k = 16 j + 4 (l / 16) + s, so each operand is one 16-byte LDS read per four
// MFMAs. Output: lane l, register i holds (m, n) = (4 (l / 16) + i, l % 16).
template <int LS, int NJ>
__device__ __forceinline__ f32x4_t tile16_dot(const float* A, const float* Bt, int lane, f32x4_t acc) {
  const float* ar = A + (lane & 15) * LS + 4 * (lane >> 4);
  const float* br = Bt + (lane & 15) * LS + 4 * (lane >> 4);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(ar + 16 * j);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(br + 16 * j);
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma16_f32(a[s], b[s], acc);
  }
  return acc;
}

// N independent tiles of tile16_dot (zero-initialised), their MFMA chains
// interleaved step by step.
template <int LS, int NJ, int N>
__device__ __forceinline__ void tile16_dot_n(const float* const (&A)[N], const float* const (&Bt)[N], int lane,
                                             f32x4_t (&acc)[N]) {
  const float* ar[N];
  const float* br[N];
#pragma unroll
  for (int n = 0; n < N; ++n) {
    acc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    ar[n] = A[n] + (lane & 15) * LS + 4 * (lane >> 4);
    br[n] = Bt[n] + (lane & 15) * LS + 4 * (lane >> 4);
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    f32x4_t a[N], b[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      a[n] = *reinterpret_cast<const f32x4_t*>(ar[n] + 16 * j);
      b[n] = *reinterpret_cast<const f32x4_t*>(br[n] + 16 * j);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int n = 0; n < N; ++n) acc[n] = mfma16_f32(a[n][s], b[n][s], acc[n]);
  }
}

// 32 x 32 matrices in LDS, row-major with stride 36 floats (16-byte aligned
// rows; 16 rows of a tile read 16 bytes each from distinct banks), kept with
// their transposes so both product operands are row reads.
constexpr int kMS = 36;
struct Mat32 {
  float* a;  // [32][kMS] row-major
  float* t;  // [32][kMS] transposed
};

// C = A B (+ C0 when given) for 32 x 32 matrices: wave w computes tile
// (w / 2, w % 2) and stores it in both orientations.
__device__ __forceinline__ void mat32_mul(Mat32 A, Mat32 B, const float* C0, Mat32 C, int wave, int lane) {
  const int bm = wave >> 1, bn = wave & 1;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (C0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = C0[(16 * bm + 4 * (lane >> 4) + i) * kMS + 16 * bn + (lane & 15)];
  }
  acc = tile16_dot<kMS, 2>(A.a + 16 * bm * kMS, B.t + 16 * bn * kMS, lane, acc);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 16 * bm + 4 * (lane >> 4) + i, n = 16 * bn + (lane & 15);
    C.a[m * kMS + n] = acc[i];
    C.t[n * kMS + m] = acc[i];
  }
}

// Input staging of the fused form: one round of loads (the raw conv inputs of
// the key head's q and k channels and of the 16 value rows for every node, the
// parents, the conv taps and committed window rows of those channels, b / a of
// the value head, the committed state rows), then the tree conv + SiLU (window
// of node t = the last KEEP + 1 rows of committed window ++ conv inputs along
// the root path, newest tap first, as gdn_prep_kernel), the q / k RMS scaling
// and g / beta, straight into the LDS rows of the matrix form. k and q are
// written out by row block 0 of the first value head of a key head, g and beta
// by row block 0 of each value head, v by every workgroup for its rows.
template <int KEEP, int LS>
__device__ __forceinline__ void chunk_prep(const GdnParams& p, const PrepParams& pp, int T, int h, int hk, int r0,
                                           int tid, float (*kq)[32][LS], float (*s0)[LS], float (*vv)[kChunkRows],
                                           float* gg, float* bb, int* par) {
  constexpr int TM = 32, DK = 128, R = kChunkRows, NW = kChunkThreads / 64, NI = TM / NW;
  __shared__ __align__(16) float raw[TM][2][DK];
  __shared__ __align__(16) float vraw[TM][R];
  const int lane64 = tid & 63, wave = tid >> 6;
  // q / k: thread (wave, lane) holds channels ch .. ch+3 of plane (0 = q,
  // 1 = k) for nodes wave, wave + 8, ...
  const int plane = lane64 >> 5, ch = 4 * (lane64 & 31);
  const int cq = plane * pp.key_dim + hk * DK + ch;  // conv column of those channels
  // v: thread owns value row r0 + vj of node tid / 16
  const int vj = tid & 15;
  const int cv = 2 * pp.key_dim + h * DK + r0 + vj;
  f32x4_t wk[KEEP + 1], bk[KEEP];
  float wvk[KEEP + 1], bvk[KEEP];
  {
    f32x4_t xr[NI], sb;
#pragma unroll
    for (int i = 0; i < NI; ++i) {  // rows past the tree are zero (their conv stays finite)
      const int t = wave + NW * i;
      xr[i] = t < T ? *reinterpret_cast<const f32x4_t*>(pp.x + (size_t)t * pp.ldx + cq) : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    f32x4_t vr = {0.f, 0.f, 0.f, 0.f};
    if (tid < 4 * T)
      vr = *reinterpret_cast<const f32x4_t*>(pp.x + (size_t)(tid >> 2) * pp.ldx + 2 * pp.key_dim + h * DK + r0 +
                                             4 * (tid & 3));
    float b_ = 0.f, a_ = 0.f;
    if (tid < T) {
      const float* row = pp.x + (size_t)tid * pp.ldx + pp.ab_col;
      b_ = row[h];
      a_ = row[pp.Hv + h];
    }
    if (tid < TM) par[tid] = tid < T ? valid_parent(p.parents[tid], tid) : -1;
#pragma unroll
    for (int r = 0; r <= KEEP; ++r) wk[r] = *reinterpret_cast<const f32x4_t*>(pp.w + (size_t)r * pp.C + cq);
#pragma unroll
    for (int r = 0; r < KEEP; ++r) bk[r] = *reinterpret_cast<const f32x4_t*>(pp.base + (size_t)r * pp.C + cq);
#pragma unroll
    for (int r = 0; r <= KEEP; ++r) wvk[r] = pp.w[(size_t)r * pp.C + cv];
#pragma unroll
    for (int r = 0; r < KEEP; ++r) bvk[r] = pp.base[(size_t)r * pp.C + cv];
    sb = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + r0 + (tid >> 5)) * DK + 4 * (tid & 31));
    const float alog = pp.A_log[h], dtb = pp.dt_bias[h];
#pragma unroll
    for (int i = 0; i < NI; ++i) *reinterpret_cast<f32x4_t*>(&raw[wave + NW * i][plane][ch]) = xr[i];
    if (tid < 4 * TM) *reinterpret_cast<f32x4_t*>(&vraw[tid >> 2][4 * (tid & 3)]) = vr;
    if (tid < TM) {
      const bool live = tid < T;
      gg[tid] = live ? __expf(-__expf(alog) * softplus_f(a_ + dtb)) : 0.f;
      bb[tid] = live ? 1.0f / (1.0f + __expf(-b_)) : 0.f;
    }
    *reinterpret_cast<f32x4_t*>(&s0[tid >> 5][4 * (tid & 31)]) = sb;
  }
  __syncthreads();
  // conv rows of node t: itself and its first KEEP ancestors (-1 past the root)
  __shared__ int anc_tab[TM][KEEP + 1];
  if (tid < TM) {
    int a = tid < T ? tid : -1;
#pragma unroll
    for (int i2 = 0; i2 <= KEEP; ++i2) {
      anc_tab[tid][i2] = a;
      if (a >= 0) a = par[a];
    }
  }
  __syncthreads();
  const float qks = plane ? pp.k_scale : pp.q_scale;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    // every node computed without a branch (so the unrolled nodes interleave);
    // rows past the tree are set to zero after
    const int t = wave + NW * i;  // wave-uniform
    f32x4_t o;
    {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      int nb = 0;
#pragma unroll
      for (int i2 = 0; i2 <= KEEP; ++i2) {
        const int anc = anc_tab[t][i2];
        f32x4_t val;
        if (anc >= 0) {
          val = *reinterpret_cast<const f32x4_t*>(&raw[anc][plane][ch]);
        } else {
          // window row KEEP - 1 - min(nb, KEEP - 1), selected over constant
          // indices (a runtime index would put the rows in scratch memory)
          const int wr = KEEP - 1 - min(nb, KEEP - 1);
          val = bk[0];
#pragma unroll
          for (int r = 1; r < KEEP; ++r) val = wr == r ? bk[r] : val;
          ++nb;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += wk[KEEP - i2][e] * val[e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = silu_fast(acc[e]);
      const float ss = row_sum32(o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3]);
      o *= rsqrtf(ss * (1.0f / DK) + 1e-6f) * qks;
    }
    if (t >= T) o = f32x4_t{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<f32x4_t*>(&kq[plane ^ 1][t][ch]) = o;  // kq[0] = k rows, kq[1] = q rows
  }
  {
    const int t = tid >> 4;
    float o;
    {
      float acc = 0.f;
      int nb = 0;
#pragma unroll
      for (int i2 = 0; i2 <= KEEP; ++i2) {
        const int anc = anc_tab[t][i2];
        float val;
        if (anc >= 0) {
          val = vraw[anc][vj];
        } else {
          const int wr = KEEP - 1 - min(nb, KEEP - 1);
          val = bvk[0];
#pragma unroll
          for (int r = 1; r < KEEP; ++r) val = wr == r ? bvk[r] : val;
          ++nb;
        }
        acc += wvk[KEEP - i2] * val;
      }
      o = silu_acc(acc);  // v, g and beta equal gdn_prep_kernel's bit for bit
    }
    vv[t][vj] = t < T ? o : 0.f;
  }
  __syncthreads();
}

// The fused form's outputs for the commit (k, v, g, beta and q, as
// gdn_prep_kernel writes them), from the staged LDS rows. Issued after the
// staging barrier and before the MFMA tiles, so no barrier waits for these
// stores while they are in flight.
template <int LS>
__device__ __forceinline__ void chunk_prep_store(const GdnParams& p, const PrepParams& pp, int T, int h, int hk,
                                                 int r0, int tid, const float (*kq)[32][LS],
                                                 const float (*vv)[kChunkRows], const float* gg, const float* bb) {
  constexpr int DK = 128, R = kChunkRows;
  if (r0 == 0 && h % (p.Hv / p.Hk) == 0) {  // q and k once per key head
#pragma unroll
    for (int i = 0; i < 2048 / kChunkThreads; ++i) {
      const int e = tid + kChunkThreads * i, m = e >> 10, t = (e >> 5) & 31, c = e & 31;
      if (t < T)
        *reinterpret_cast<f32x4_t*>((m ? pp.q : pp.k) + (size_t)t * pp.key_dim + hk * DK + 4 * c) =
            *reinterpret_cast<const f32x4_t*>(&kq[m][t][4 * c]);
    }
  }
  {  // v of this workgroup's rows
    const int t = tid >> 4, r = tid & 15;
    if (t < T) pp.v[(size_t)t * (pp.C - 2 * pp.key_dim) + h * DK + r0 + r] = vv[t][r];
  }
  if (r0 == 0 && tid < T) {  // g and beta once per value head
    pp.g[(size_t)tid * p.Hv + h] = gg[tid];
    pp.beta[(size_t)tid * p.Hv + h] = bb[tid];
  }
}

// KEEP = 0: q, k, v, g and beta come from memory (gdn_prep_kernel's output).
// KEEP > 0 (the conv window, 1 .. kConvMaxKeep): the workgroup computes them
// from the in_proj rows as gdn_prep_reg_kernel does (tree conv + SiLU, q / k
// RMS scaling, g and beta), and writes k, v, g, beta and q once each for the
// commit.
template <int KEEP>
__global__ __launch_bounds__(kChunkThreads) void gdn_tree_chunk_kernel(GdnParams p, PrepParams pp) {
  constexpr int DK = 128, TM = 32, R = kChunkRows, LS = DK + 4;
  // Phase 1 (loads, Gram and S_0 products) uses kq and s0; phase 2 (the
  // inverse) reuses their space for eight 32 x 32 matrices.
  constexpr int kPhase1 = (2 * TM + R) * LS;  // floats
  constexpr int kPhase2 = 8 * TM * kMS;
  __shared__ __align__(16) float big[kPhase1 > kPhase2 ? kPhase1 : kPhase2];
  __shared__ __align__(16) float um[TM][kMS];      // U
  __shared__ __align__(16) float rt[R][kMS];       // R^T: [value row][node]
  __shared__ float gkk[TM][TM + 1], gqk[TM][TM + 1];  // k_t . k_a, q_t . k_a
  __shared__ float sk[TM][R + 1], sq[TM][R + 1];  // S_0 k_t, S_0 q_t per value row
  __shared__ float dm[TM][TM + 1];                // D[t][a] for strict ancestors a, else 0
  __shared__ float vv[TM][R], gam[TM], gg[TM], bb[TM];
  __shared__ int par[TM], s_depth;
  float(*kq)[TM][LS] = reinterpret_cast<float(*)[TM][LS]>(big);
  float(*s0)[LS] = reinterpret_cast<float(*)[LS]>(big + 2 * TM * LS);
  const int T = p.T_dev ? min(max(*p.T_dev, 0), min(p.T, TM)) : min(p.T, TM);
  const int nblk = p.Dv / R;
  const int h = blockIdx.x / nblk, r0 = (blockIdx.x % nblk) * R;
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) s_depth = 0;  // ordered before the decays by the loads' barrier

  if constexpr (KEEP == 0) {
    // ---- loads: every load of the workgroup in flight together ----
    constexpr int NK = 2048 / kChunkThreads;  // float4 of k and q rows per thread
    f32x4_t kb[NK], sb;
#pragma unroll
    for (int i = 0; i < NK; ++i) {  // 2 x 32 rows x 32 float4
      const int e = tid + kChunkThreads * i, m = e >> 10, t = (e >> 5) & 31, c = e & 31;
      kb[i] = t < T ? *reinterpret_cast<const f32x4_t*>((m ? p.q : p.k) + ((size_t)t * p.Hk + hk) * DK + 4 * c)
                    : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    sb = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + r0 + (tid >> 5)) * DK + 4 * (tid & 31));
    {  // 32 nodes x 16 rows of v
      const int t = tid >> 4, r = tid & 15;
      vv[t][r] = t < T ? p.v[((size_t)t * p.Hv + h) * p.Dv + r0 + r] : 0.f;
    }
    if (tid < TM) {
      const bool live = tid < T;
      gg[tid] = live ? p.g[(size_t)tid * p.Hv + h] : 0.f;
      bb[tid] = live ? p.beta[(size_t)tid * p.Hv + h] : 0.f;
      par[tid] = live ? valid_parent(p.parents[tid], tid) : -1;
    }
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int e = tid + kChunkThreads * i, m = e >> 10, t = (e >> 5) & 31, c = e & 31;
      *reinterpret_cast<f32x4_t*>(&kq[m][t][4 * c]) = kb[i];
    }
    *reinterpret_cast<f32x4_t*>(&s0[tid >> 5][4 * (tid & 31)]) = sb;
    __syncthreads();
  } else {
    chunk_prep<KEEP>(p, pp, T, h, hk, r0, tid, kq, s0, vv, gg, bb, par);
    chunk_prep_store<LS>(p, pp, T, h, hk, r0, tid, kq, vv, gg, bb);
  }

  // ---- path decays D[t][a] along each node's parent chain (wave 3, which
  // has the fewest MFMA tiles below; LDS operations of a wave are ordered) ----
  if (wave == 3) {
    for (int e = lane; e < TM * TM; e += 64) dm[e >> 5][e & 31] = 0.f;
    const int t = lane;
    if (t < T) {
      float cum = gg[t];
      int a = par[t], depth = 0;
      for (; depth < TM && a >= 0; ++depth) {  // a < t strictly decreasing
        dm[t][a] = cum;
        cum *= gg[a];
        a = par[a];
      }
      gam[t] = cum;
      atomicMax(&s_depth, depth);
    } else if (t < TM) {
      gam[t] = 0.f;
    }
  }
  // ---- Gram blocks (t-block >= a-block) and S_0 products on MFMA ----
  {
    // wave w computes tile w (and w + 8 for waves 0, 1, their MFMA chains
    // interleaved)
    auto operands = [&](int job, const float*& A, const float*& B) {
      if (job < 6) {
        const int bt = job % 3 == 0 ? 0 : 1, ba = job % 3 == 2 ? 1 : 0;  // (0,0), (1,0), (1,1)
        A = &kq[job < 3 ? 0 : 1][16 * bt][0];
        B = &kq[0][16 * ba][0];
      } else {
        A = &s0[0][0];
        B = &kq[job < 8 ? 0 : 1][16 * ((job - 6) & 1)][0];
      }
    };
    auto store = [&](int job, const f32x4_t& d) {
      if (job < 6) {
        const int bt = job % 3 == 0 ? 0 : 1, ba = job % 3 == 2 ? 1 : 0;
        float(*dst)[TM + 1] = job < 3 ? gkk : gqk;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[16 * bt + 4 * (lane >> 4) + i][16 * ba + (lane & 15)] = d[i];
      } else {
        const int nb = (job - 6) & 1;
        float(*dst)[R + 1] = job < 8 ? sk : sq;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[16 * nb + (lane & 15)][4 * (lane >> 4) + i] = d[i];
      }
    };
    const float *A0, *B0, *A1, *B1;
    operands(wave, A0, B0);
    if (wave < 2) {
      operands(wave + 8, A1, B1);
      f32x4_t d[2];
      tile16_dot_n<LS, 8, 2>({A0, A1}, {B0, B1}, lane, d);
      store(wave, d[0]);
      store(wave + 8, d[1]);
    } else {
      f32x4_t d[1];
      tile16_dot_n<LS, 8, 1>({A0}, {B0}, lane, d);
      store(wave, d[0]);
    }
  }
  __syncthreads();

  // ---- L, P_0 = I - L, U and R^T ----
  // eight [32][kMS] matrices: X0, X0^T, X1, X1^T (powers of L), P0, P0^T,
  // P1, P1^T (running product); the index is a pointer offset (an array of
  // Mat32 indexed at run time would live in scratch memory)
  auto Xm = [&](int i) { return Mat32{big + (2 * i) * TM * kMS, big + (2 * i + 1) * TM * kMS}; };
  auto Pmat = [&](int i) { return Mat32{big + (4 + 2 * i) * TM * kMS, big + (5 + 2 * i) * TM * kMS}; };
  for (int e = tid; e < TM * TM; e += kChunkThreads) {
    const int t = e >> 5, a = e & 31;
    const float l = a < t ? bb[t] * dm[t][a] * gkk[t][a] : 0.f;
    Xm(0).a[t * kMS + a] = l;
    Xm(0).t[a * kMS + t] = l;
    const float p0 = (t == a ? 1.f : 0.f) - l;
    Pmat(0).a[t * kMS + a] = p0;
    Pmat(0).t[a * kMS + t] = p0;
    um[t][a] = a < t ? dm[t][a] * gqk[t][a] : (a == t && t < T ? gqk[t][t] : 0.f);
  }
  for (int e = tid; e < R * TM; e += kChunkThreads) {
    const int r = e >> 5, t = e & 31;
    rt[r][t] = t < T ? bb[t] * (vv[t][r] - gam[t] * sk[t][r]) : 0.f;
  }
  __syncthreads();

  // ---- (I + L)^-1 = (I - L)(I + L^2)(I + L^4) ... ----
  const int d = s_depth;
  int cur = 0;
  for (int pw = 1; pw < TM && (1 << pw) <= d; ++pw) {  // factors I + L^(2^pw) while 2^pw <= d
    const Mat32 src = Xm((pw - 1) & 1), dst = Xm(pw & 1);
    if (wave < 4) mat32_mul(src, src, nullptr, dst, wave, lane);  // X_pw = X_(pw-1)^2
    __syncthreads();
    if (wave < 4) mat32_mul(Pmat(cur), dst, Pmat(cur).a, Pmat(cur ^ 1), wave, lane);  // P += P X_pw
    cur ^= 1;
    __syncthreads();
  }

  // ---- Y = diag(gamma) S_0 q + U (I + L)^-1 R ----
  const Mat32 M = Xm(0);  // M = U T (the powers are no longer needed)
  if (wave < 4) mat32_mul(Mat32{&um[0][0], nullptr}, Pmat(cur), nullptr, M, wave, lane);
  __syncthreads();
  if (wave < 2) {
    f32x4_t acc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * (lane >> 4) + i;
      acc[i] = gam[t] * sq[t][lane & 15];
    }
    acc = tile16_dot<kMS, 2>(M.a + 16 * wave * kMS, &rt[0][0], lane, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * (lane >> 4) + i, r = lane & 15;
      if (t < T) p.y[((size_t)t * p.Hv + h) * p.Dv + r0 + r] = acc[i];
    }
  }
}


// ---- matrix form in 32-node blocks (trees of 33-96 nodes) -----------------
//
// In node order (parents before children) I + L is block lower triangular
// over 32-node blocks, so block b of Delta follows from the earlier blocks by
// substitution, and Y needs the earlier blocks' Delta rows only:
//   (I + L_bb) Delta_b = R_b - sum_{a < b} L_ba Delta_a,
//   Y_b = diag(gamma_b) (S_0 Q_b^T)^T + U_bb Delta_b + sum_{a < b} U_ba Delta_a,
// with L, U, R, gamma and D as in the 32-node form above. The diagonal block
// is inverted by the same squaring, over the block's own ancestor depth; the
// off-diagonal terms (a node's ancestors in earlier blocks) are VALU sums
// over the finished Delta rows. A workgroup owns one value head and 16 value
// rows, keeps the k rows of every node and the finished Delta rows in LDS and
// stages one block's q rows at a time. Unlike the depth-first walk it has no
// limit on nested branch points.
constexpr int kBlkMax = 3;               // 32-node blocks
constexpr int kBlkNodes = 32 * kBlkMax;  // 96 nodes

__global__ __launch_bounds__(kChunkThreads) void gdn_tree_blocks_kernel(GdnParams p) {
  constexpr int DK = 128, TM = 32, R = kChunkRows, LS = DK + 4, NM = kBlkNodes;
  static_assert(kChunkThreads == TM * R, "one thread per (block node, value row)");
  __shared__ __align__(16) float kall[NM][LS];  // k rows of every node
  __shared__ __align__(16) float s0[R][LS];     // S_0 rows of this workgroup
  // One block's q rows while its Gram products run, then the inverse's eight
  // 32 x 32 matrices (X0, X0^T, X1, X1^T, P0, P0^T, P1, P1^T).
  constexpr int kQb = TM * LS, kInv = 8 * TM * kMS;
  __shared__ __align__(16) float big[kQb > kInv ? kQb : kInv];
  __shared__ __align__(16) float um[TM][kMS];            // U_bb
  __shared__ float gkk[TM][TM + 1], gqk[TM][TM + 1];     // k_t . k_a, q_t . k_a within the block
  __shared__ float gko[TM][2 * TM + 1], gqo[TM][2 * TM + 1];  // the same against earlier blocks
  __shared__ float sk[TM][R + 1], sq[TM][R + 1];         // S_0 k_t, S_0 q_t per value row
  __shared__ float dm[TM][NM + 1];                       // D[t][a] for the block's nodes t
  __shared__ float dl[NM][R + 1];                        // Delta rows of finished blocks
  __shared__ float rhs[TM][R + 1], yb[TM][R + 1];
  __shared__ float gam[NM], gg[NM], bb[NM];
  __shared__ int par[NM], s_depth;
  float(*qb)[LS] = reinterpret_cast<float(*)[LS]>(big);
  const int T = p.T_dev ? min(max(*p.T_dev, 0), min(p.T, NM)) : min(p.T, NM);
  const int nblk = p.Dv / R;
  const int h = blockIdx.x / nblk, r0 = (blockIdx.x % nblk) * R;
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tr = tid >> 4, rr = tid & 15;  // (block node, value row) of this thread

  // ---- k rows of every node, S_0 rows, g / beta / parents ----
  {
    constexpr int NK = NM * (DK / 4) / kChunkThreads;  // float4 per thread
    f32x4_t kv[NK], sv;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int e = tid + kChunkThreads * i, t = e >> 5, c = e & 31;
      kv[i] = t < T ? *reinterpret_cast<const f32x4_t*>(p.k + ((size_t)t * p.Hk + hk) * DK + 4 * c)
                    : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    sv = *reinterpret_cast<const f32x4_t*>(p.state + ((size_t)h * p.Dv + r0 + (tid >> 5)) * DK + 4 * (tid & 31));
    if (tid < NM) {
      const bool live = tid < T;
      gg[tid] = live ? p.g[(size_t)tid * p.Hv + h] : 0.f;
      bb[tid] = live ? p.beta[(size_t)tid * p.Hv + h] : 0.f;
      par[tid] = live ? valid_parent(p.parents[tid], tid) : -1;
    }
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int e = tid + kChunkThreads * i, t = e >> 5, c = e & 31;
      *reinterpret_cast<f32x4_t*>(&kall[t][4 * c]) = kv[i];
    }
    *reinterpret_cast<f32x4_t*>(&s0[tid >> 5][4 * (tid & 31)]) = sv;
  }
  auto Xm = [&](int i) { return Mat32{big + (2 * i) * TM * kMS, big + (2 * i + 1) * TM * kMS}; };
  auto Pmat = [&](int i) { return Mat32{big + (4 + 2 * i) * TM * kMS, big + (5 + 2 * i) * TM * kMS}; };

  const int B = (T + TM - 1) / TM;
  // q rows of block b (in registers a block ahead) and v of this thread's
  // (node, value row)
  f32x4_t qv[2];
  float vt = 0.f;
  auto q_issue = [&](int n0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + kChunkThreads * i, t = e >> 5, c = e & 31;
      qv[i] = n0 + t < T ? *reinterpret_cast<const f32x4_t*>(p.q + ((size_t)(n0 + t) * p.Hk + hk) * DK + 4 * c)
                         : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    vt = n0 + tr < T ? p.v[((size_t)(n0 + tr) * p.Hv + h) * p.Dv + r0 + rr] : 0.f;
  };
  q_issue(0);
  for (int b = 0; b < B; ++b) {
    const int n0 = TM * b;  // first node of the block
    const float vb = vt;
    // ---- this block's q rows; D[t][.] cleared; the next block's q issued ----
    {
      for (int e = tid; e < TM * (NM + 1); e += kChunkThreads) dm[e / (NM + 1)][e % (NM + 1)] = 0.f;
      if (tid == 0) s_depth = 0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + kChunkThreads * i, t = e >> 5, c = e & 31;
        *reinterpret_cast<f32x4_t*>(&qb[t][4 * c]) = qv[i];
      }
      if (b + 1 < B) q_issue(n0 + TM);
    }
    __syncthreads();
    // ---- Gram tiles and S_0 products on MFMA (wave w: jobs w, w + 8, ...);
    // the path decays of the block's nodes by the last wave's lanes ----
    {
      const int njobs = 12 + 8 * b;
      for (int job = wave; job < njobs; job += kChunkThreads / 64) {
        const float *A, *Bt;
        int kind, th, ah;
        if (job < 8) {  // 0-3 k.k, 4-7 q.k within the block
          kind = job >> 2; th = (job >> 1) & 1; ah = job & 1;
          A = kind ? &qb[16 * th][0] : &kall[n0 + 16 * th][0];
          Bt = &kall[n0 + 16 * ah][0];
        } else if (job < 12) {  // 8-9 S_0 k, 10-11 S_0 q
          kind = job < 10 ? 2 : 3; th = job & 1; ah = 0;
          A = &s0[0][0];
          Bt = kind == 2 ? &kall[n0 + 16 * th][0] : &qb[16 * th][0];
        } else {  // k.k and q.k against the earlier blocks' nodes
          const int idx = (job - 12) % (4 * b);
          kind = job - 12 < 4 * b ? 4 : 5; th = idx & 1; ah = idx >> 1;
          A = kind == 5 ? &qb[16 * th][0] : &kall[n0 + 16 * th][0];
          Bt = &kall[16 * ah][0];
        }
        const f32x4_t d = tile16_dot<LS, DK / 16>(A, Bt, lane, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 4 * (lane >> 4) + i, n = lane & 15;
          if (kind == 0) gkk[16 * th + m][16 * ah + n] = d[i];
          else if (kind == 1) gqk[16 * th + m][16 * ah + n] = d[i];
          else if (kind == 2) sk[16 * th + n][m] = d[i];
          else if (kind == 3) sq[16 * th + n][m] = d[i];
          else if (kind == 4) gko[16 * th + m][16 * ah + n] = d[i];
          else gqo[16 * th + m][16 * ah + n] = d[i];
        }
      }
      if (wave == kChunkThreads / 64 - 1 && lane < TM) {
        const int t = n0 + lane;
        if (t < T) {
          float cum = gg[t];
          int a = par[t], inblk = 0;
          for (int steps = 0; steps < NM && a >= 0; ++steps) {  // a < t strictly decreasing
            dm[lane][a] = cum;
            inblk += a >= n0;
            cum *= gg[a];
            a = par[a];
          }
          gam[t] = cum;
          atomicMax(&s_depth, inblk);
        } else {
          gam[t] = 0.f;
        }
      }
    }
    __syncthreads();
    // ---- L_bb, I - L_bb, U_bb; the right-hand side and Y's known terms ----
    for (int e = tid; e < TM * TM; e += kChunkThreads) {
      const int t = e >> 5, a = e & 31;
      const bool live = n0 + t < T;
      const float l = live && a < t ? bb[n0 + t] * dm[t][n0 + a] * gkk[t][a] : 0.f;
      Xm(0).a[t * kMS + a] = l;
      Xm(0).t[a * kMS + t] = l;
      const float p0 = (t == a ? 1.f : 0.f) - l;
      Pmat(0).a[t * kMS + a] = p0;
      Pmat(0).t[a * kMS + t] = p0;
      um[t][a] = !live ? 0.f : a < t ? dm[t][n0 + a] * gqk[t][a] : (a == t ? gqk[t][t] : 0.f);
    }
    {
      const int t = n0 + tr;
      float rv = 0.f, yv = 0.f;
      if (t < T) {
        float off_r = 0.f;
        for (int a = 0; a < n0; ++a) {
          const float w = dm[tr][a];
          if (w != 0.f) {
            off_r += w * gko[tr][a] * dl[a][rr];
            yv += w * gqo[tr][a] * dl[a][rr];
          }
        }
        rv = bb[t] * (vb - gam[t] * sk[tr][rr]) - bb[t] * off_r;
        yv += gam[t] * sq[tr][rr];
      }
      rhs[tr][rr] = rv;
      yb[tr][rr] = yv;
    }
    __syncthreads();
    // ---- (I + L_bb)^-1 = (I - L)(I + L^2)(I + L^4) ... over the block's depth ----
    const int d = s_depth;
    int cur = 0;
    for (int pw = 1; pw < TM && (1 << pw) <= d; ++pw) {
      const Mat32 src = Xm((pw - 1) & 1), dst = Xm(pw & 1);
      if (wave < 4) mat32_mul(src, src, nullptr, dst, wave, lane);
      __syncthreads();
      if (wave < 4) mat32_mul(Pmat(cur), dst, Pmat(cur).a, Pmat(cur ^ 1), wave, lane);
      cur ^= 1;
      __syncthreads();
    }
    // ---- Delta_b, then Y_b ----
    {
      const float* Pa = Pmat(cur).a;
      float dv = 0.f;
#pragma unroll 8
      for (int a = 0; a < TM; ++a) dv += Pa[tr * kMS + a] * rhs[a][rr];
      dl[n0 + tr][rr] = n0 + tr < T ? dv : 0.f;
    }
    __syncthreads();
    {
      const int t = n0 + tr;
      float yv = yb[tr][rr];
#pragma unroll 8
      for (int a = 0; a < TM; ++a) yv += um[tr][a] * dl[n0 + a][rr];
      if (t < T) p.y[((size_t)t * p.Hv + h) * p.Dv + r0 + rr] = yv;
    }
    __syncthreads();  // big, dm and the block's scratch are rewritten next
  }
}


// Gated RMSNorm of the recurrence output per (node, value head)
// (RMSNormGated, qwen35_tree.py:322): o = rms_norm(y) * w * silu(z), written as
// the split bf16 pair [hi, lo] the out_proj GEMM reads. 16 threads per
// (node, head), 8 dims each; rows >= L are written as zero. chain > 0: L is
// chain (a prompt chain, no desc).
template <int DV>
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(const DtreeStepDesc* desc, int chain,
                                                             const float* __restrict__ y,
                                                             const float* __restrict__ z, int ldz,
                                                             const uint16_t* __restrict__ w, float eps, int Hv,
                                                             int rows, uint16_t* out, uint16_t* out_lo, int layout,
                                                             int ld_out) {
  constexpr int TPH = DV / 8;  // threads per (node, head)
  const int L = chain > 0 ? chain : desc->num_nodes;
  const int gid = blockIdx.x * (256 / TPH) + threadIdx.x / TPH;
  const int part = threadIdx.x % TPH;
  if (gid >= rows * Hv) return;
  const int t = gid / Hv, h = gid % Hv;
  const int d0 = part * 8;
  float o[8];
  if (t < L) {
    const float* yr = y + ((size_t)t * Hv + h) * DV + d0;
    const f32x4_t y0 = *reinterpret_cast<const f32x4_t*>(yr), y1 = *reinterpret_cast<const f32x4_t*>(yr + 4);
    const float* zr = z + (size_t)t * ldz + h * DV + d0;
    const f32x4_t z0 = *reinterpret_cast<const f32x4_t*>(zr), z1 = *reinterpret_cast<const f32x4_t*>(zr + 4);
    const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(w + d0);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += y0[i] * y0[i] + y1[i] * y1[i];
#pragma unroll
    for (int m = TPH / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
    const float r = rsqrtf(ss * (1.0f / DV) + eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float yi = i < 4 ? y0[i] : y1[i - 4];
      const float zi = i < 4 ? z0[i] : z1[i - 4];
      const uint32_t wb = wv[i >> 1];
      const float wi = __uint_as_float((i & 1) ? (wb & 0xffff0000u) : (wb << 16));
      o[i] = yi * r * wi * (zi / (1.0f + __expf(-zi)));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.f;
  }
  const int col = h * DV + d0;
  const size_t oi = layout != DTREE_W_ROWMAJOR ? tiled_index(t, col, ld_out) : (size_t)t * ld_out + col;
  store_act8(out, out_lo, oi, o, layout == DTREE_W_TILED_F16);
}

// ---- causal chain (prompt prefill) -------------------------------------------
// The recurrence over T prompt tokens that continue the committed state
// (gated_delta_update over the prompt, custom_qwen35_model.py:868-878): a
// workgroup owns one value head and 8 state rows (32 lanes x 4 elements per
// row, as gdn_tree_reg_kernel), walks the tokens in order with its state in
// registers and the next kChainAhead tokens' inputs in flight, writes y per
// token (the same step as the tree kernels) and leaves the final state in
// `state`. Workgroups past state_blocks advance the committed conv window to
// the last `keep` rows of (window ++ conv inputs) (custom_qwen35_model.py:
// 849-851), one channel per thread; the prep launch before this one has read
// the old window.
constexpr int kChainAhead = 8;

__global__ __launch_bounds__(256) void gdn_chain_scan_kernel(GdnParams p, const float* __restrict__ x, int ldx,
                                                             float* window, int C, int keep, int state_blocks) {
  const int T = p.T;
  if ((int)blockIdx.x >= state_blocks) {
    const int c = ((int)blockIdx.x - state_blocks) * 256 + threadIdx.x;
    if (c >= C) return;
    float old[kConvMaxKeep];
#pragma unroll
    for (int r = 0; r < kConvMaxKeep; ++r) old[r] = r < keep ? window[(size_t)r * C + c] : 0.f;
#pragma unroll
    for (int r = 0; r < kConvMaxKeep; ++r) {
      if (r >= keep) break;
      // row r of the new window = element T + r of (old window ++ x)
      const int e = T + r;
      float val = 0.f;
      if (e < keep) {
#pragma unroll
        for (int j = 0; j < kConvMaxKeep; ++j) val = j == e ? old[j] : val;
      } else {
        val = x[(size_t)(e - keep) * ldx + c];
      }
      window[(size_t)r * C + c] = val;
    }
    return;
  }
  constexpr int DK = 128, RPW = 8, A = kChainAhead;
  const int nslices = p.Dv / RPW;
  const int h = blockIdx.x / nslices, row0 = (blockIdx.x % nslices) * RPW;
  const int hk = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, rl = tid >> 5, lane = tid & 31;
  const int dv = row0 + rl;
  float* sp = p.state + ((size_t)h * p.Dv + dv) * DK + 4 * lane;
  f32x4_t s = *reinterpret_cast<const f32x4_t*>(sp);
  f32x4_t rk[A], rq[A];
  float rv[A], rg[A], rb[A];
  auto load = [&](int a, int t) {
    if (t < T) {
      rk[a] = *reinterpret_cast<const f32x4_t*>(p.k + ((size_t)t * p.Hk + hk) * DK + 4 * lane);
      rq[a] = *reinterpret_cast<const f32x4_t*>(p.q + ((size_t)t * p.Hk + hk) * DK + 4 * lane);
      rv[a] = p.v[((size_t)t * p.Hv + h) * p.Dv + dv];
      rg[a] = p.g[(size_t)t * p.Hv + h];
      rb[a] = p.beta[(size_t)t * p.Hv + h];
    }
  };
#pragma unroll
  for (int a = 0; a < A; ++a) load(a, a);
  for (int t0 = 0; t0 < T; t0 += A) {
#pragma unroll
    for (int a = 0; a < A; ++a) {
      const int t = t0 + a;
      if (t >= T) break;
      const f32x4_t kk = rk[a], qq = rq[a];
      const float v = rv[a], g = rg[a], b = rb[a];
      load(a, t + A);
      float sk = s[0] * kk[0] + s[1] * kk[1] + s[2] * kk[2] + s[3] * kk[3];
      float sq = s[0] * qq[0] + s[1] * qq[1] + s[2] * qq[2] + s[3] * qq[3];
      float kq = kk[0] * qq[0] + kk[1] * qq[1] + kk[2] * qq[2] + kk[3] * qq[3];
      row_sum32x3(sk, sq, kq);
      const float delta = (v - g * sk) * b;
      s = s * g + kk * delta;
      if (lane == 0) p.y[((size_t)t * p.Hv + h) * p.Dv + dv] = g * sq + delta * kq;
    }
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

// Matrix-form recurrence (gdn_tree_chunk_kernel) for trees of up to 32 nodes
// with 128-dim key heads; DTREE_GDN_KERNEL=reg keeps the node-by-node
// register kernel (timing and cross-checks).
static bool use_chunk_recurrence(int rows, int dk, int dv) {
  static const bool reg = [] {
    const char* e = std::getenv("DTREE_GDN_KERNEL");
    return e && std::string(e) == "reg";
  }();
  return !reg && rows <= 32 && dk == 128 && dv % kChunkRows == 0;
}

// Matrix form in 32-node blocks (gdn_tree_blocks_kernel) for 33-96 nodes;
// DTREE_GDN_KERNEL=reg or dfs keeps the depth-first walk (timing and
// cross-checks).
static bool use_block_recurrence(int rows, int dk, int dv) {
  static const bool node_by_node = [] {
    const char* e = std::getenv("DTREE_GDN_KERNEL");
    return e && (std::string(e) == "reg" || std::string(e) == "dfs");
  }();
  return !node_by_node && rows > 32 && rows <= kBlkNodes && dk == 128 && dv % kChunkRows == 0;
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
  if (!states && use_chunk_recurrence(num_nodes, head_k_dim, head_v_dim)) {
    gdn_tree_chunk_kernel<0><<<num_v_heads * (head_v_dim / kChunkRows), kChunkThreads, 0, stream>>>(p, PrepParams{});
    DTREE_LAUNCH_CHECK("gdn_tree_recurrence launch");
    return DTREE_OK;
  }
  if (!states && use_block_recurrence(num_nodes, head_k_dim, head_v_dim)) {
    gdn_tree_blocks_kernel<<<num_v_heads * (head_v_dim / kChunkRows), kChunkThreads, 0, stream>>>(p);
    DTREE_LAUNCH_CHECK("gdn_tree_recurrence launch");
    return DTREE_OK;
  }
  if (head_k_dim == 128 && num_nodes <= kRegTreeMax && head_v_dim % 8 == 0) {
    if (num_nodes <= 32) gdn_tree_reg_kernel<32><<<num_v_heads * (head_v_dim / 8), 256, 0, stream>>>(p);
    else gdn_tree_dfs_kernel<<<num_v_heads * (head_v_dim / 8), 256, 0, stream>>>(p);
    DTREE_LAUNCH_CHECK("gdn_tree_recurrence launch");
    return DTREE_OK;
  }
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
  p.T = kGdnMaxNodes; p.Hk = num_k_heads; p.Hv = num_v_heads; p.Dv = head_v_dim; p.rpw = rpw;
  const int conv_blocks = window ? (channels + 255) / 256 : 0;
  const int state_blocks = state ? num_v_heads * (head_v_dim / rpw) : 0;
  if (conv_blocks + state_blocks == 0) return DTREE_OK;
  // Conv blocks use 256 threads; state blocks rpw * Dk / 4 (<= 256): launch
  // with 256 and let surplus state threads idle.
  const int threads = 256;
  switch (head_k_dim) {
    case 32: gdn_commit_kernel<32><<<conv_blocks + state_blocks, threads, 0, stream>>>(p, x, channels, window, nullptr, channels, keep, conv_blocks); break;
    case 64: gdn_commit_kernel<64><<<conv_blocks + state_blocks, threads, 0, stream>>>(p, x, channels, window, nullptr, channels, keep, conv_blocks); break;
    default: gdn_commit_kernel<128><<<conv_blocks + state_blocks, threads, 0, stream>>>(p, x, channels, window, nullptr, channels, keep, conv_blocks); break;
  }
  DTREE_LAUNCH_CHECK("gdn_commit launch");
  return DTREE_OK;
}

// ---- layer entry points (node count, parents and accepted path from the
// device step descriptor, so one captured graph serves every step) ----------

static int gdn_layer_check(const DtreeGdnArgs* a, const char* what) {
  DTREE_REQUIRE(a && a->desc, std::string(what) + ": null args / desc");
  DTREE_REQUIRE(a->rows_padded >= 1 && a->rows_padded <= kGdnMaxNodes, std::string(what) + ": rows_padded in [1, 128]");
  DTREE_REQUIRE(a->num_k_heads > 0 && a->num_v_heads > 0 && a->num_v_heads % a->num_k_heads == 0,
                std::string(what) + ": num_v_heads % num_k_heads");
  DTREE_REQUIRE(a->head_k_dim == 128 && a->head_v_dim == 128, std::string(what) + ": head dims 128 are compiled");
  DTREE_REQUIRE(a->conv_keep >= 1 && a->conv_keep <= kConvMaxKeep, std::string(what) + ": conv_keep in [1, 7]");
  return DTREE_OK;
}

extern "C" size_t dtree_gdn_args_bytes(void) { return sizeof(DtreeGdnArgs); }

static_assert(DTREE_GDN_MAX_NESTED_BRANCHES == kDfsStack - 1, "the header's limit is the stack's");

extern "C" int dtree_gdn_tree_check(const int32_t* parents, int32_t num_nodes) {
  if (int rc = dtree_validate_parents(parents, num_nodes)) return rc;
  if (num_nodes <= 32) return DTREE_OK;  // the register-resident recurrence holds any such tree
  // nesting of a branching node = its branching ancestors + 1 (parents precede children)
  int nch[DTREE_MAX_NODES] = {0}, nest[DTREE_MAX_NODES] = {0};
  for (int i = 1; i < num_nodes; ++i) ++nch[parents[i]];
  int deepest = 0;
  for (int i = 0; i < num_nodes; ++i) {
    const int above = i == 0 ? 0 : nest[parents[i]];
    nest[i] = above + (nch[i] >= 2 ? 1 : 0);
    if (nch[i] >= 2) deepest = std::max(deepest, nest[i]);
  }
  if (deepest > DTREE_GDN_MAX_NESTED_BRANCHES)
    return fail(DTREE_E_TREE, "GatedDeltaNet tree recurrence: " + std::to_string(deepest) +
                                  " nested branching nodes, beyond the " +
                                  std::to_string(DTREE_GDN_MAX_NESTED_BRANCHES) + " its state stack holds");
  return DTREE_OK;
}

extern "C" int dtree_gdn_layer_prep(const DtreeGdnArgs* a, hipStream_t stream) {
  if (int rc = gdn_layer_check(a, "gdn_layer_prep")) return rc;
  DTREE_REQUIRE(a->proj && a->window && a->conv_w && a->A_log && a->dt_bias && a->q && a->k && a->v && a->g && a->beta,
                "gdn_layer_prep: null pointer");
  const int key_dim = a->num_k_heads * a->head_k_dim, value_dim = a->num_v_heads * a->head_v_dim;
  const int C = 2 * key_dim + value_dim;
  DTREE_REQUIRE(a->ld_proj >= C + value_dim + 2 * a->num_v_heads, "gdn_layer_prep: ld_proj below C + z + b + a");
  PrepParams p{};
  p.desc = a->desc; p.rows = a->rows_padded;
  p.x = a->proj; p.ldx = a->ld_proj; p.base = a->window; p.w = a->conv_w;
  p.C = C; p.key_dim = key_dim; p.Hv = a->num_v_heads; p.ab_col = C + value_dim;
  p.A_log = a->A_log; p.dt_bias = a->dt_bias;
  p.q = a->q; p.k = a->k; p.v = a->v; p.g = a->g; p.beta = a->beta;
  p.q_scale = 1.0f / (float)a->head_k_dim;
  p.k_scale = 1.0f / sqrtf((float)a->head_k_dim);
  const dim3 grid(C / 128 + 1, (a->rows_padded + kPrepNodes - 1) / kPrepNodes);
  switch (a->conv_keep) {
#define DTREE_PREP_CASE(K) \
  case K: gdn_prep_kernel<K, 128><<<grid, 128, 0, stream>>>(p); break;
    DTREE_PREP_CASE(1) DTREE_PREP_CASE(2) DTREE_PREP_CASE(3) DTREE_PREP_CASE(4) DTREE_PREP_CASE(5)
    DTREE_PREP_CASE(6) DTREE_PREP_CASE(7)
#undef DTREE_PREP_CASE
  }
  DTREE_LAUNCH_CHECK("gdn_layer_prep launch");
  return DTREE_OK;
}

extern "C" int dtree_gdn_layer_recurrence(const DtreeGdnArgs* a, hipStream_t stream) {
  if (int rc = gdn_layer_check(a, "gdn_layer_recurrence")) return rc;
  DTREE_REQUIRE(a->q && a->k && a->v && a->g && a->beta && a->state && a->y, "gdn_layer_recurrence: null pointer");
  size_t lds = 0;
  const int rpw = gdn_rpw(a->rows_padded, a->head_k_dim, a->head_v_dim, &lds);
  DTREE_REQUIRE(rpw > 0, "gdn_layer_recurrence: rows_padded too large for the LDS-resident node states");
  GdnParams p{};
  p.q = a->q; p.k = a->k; p.v = a->v; p.g = a->g; p.beta = a->beta; p.state = a->state;
  p.parents = a->desc->parents; p.T_dev = &a->desc->num_nodes;
  p.T = a->rows_padded; p.Hk = a->num_k_heads; p.Hv = a->num_v_heads; p.Dv = a->head_v_dim; p.rpw = rpw;
  p.y = a->y; p.states = nullptr;
  if (use_chunk_recurrence(a->rows_padded, a->head_k_dim, a->head_v_dim)) {
    p.T = min(a->rows_padded, 32);
    gdn_tree_chunk_kernel<0><<<a->num_v_heads * (a->head_v_dim / kChunkRows), kChunkThreads, 0, stream>>>(p, PrepParams{});
  } else if (use_block_recurrence(a->rows_padded, a->head_k_dim, a->head_v_dim)) {
    p.T = min(a->rows_padded, kBlkNodes);
    gdn_tree_blocks_kernel<<<a->num_v_heads * (a->head_v_dim / kChunkRows), kChunkThreads, 0, stream>>>(p);
  } else if (a->rows_padded <= 32 && a->head_v_dim % 8 == 0) {
    p.T = min(a->rows_padded, 32);
    gdn_tree_reg_kernel<32><<<a->num_v_heads * (a->head_v_dim / 8), 256, 0, stream>>>(p);
  } else if (a->rows_padded <= kRegTreeMax && a->head_v_dim % 8 == 0) {
    p.T = a->rows_padded;
    gdn_tree_dfs_kernel<<<a->num_v_heads * (a->head_v_dim / 8), 256, 0, stream>>>(p);
  } else {
    const int grid = a->num_v_heads * (a->head_v_dim / rpw);
    gdn_tree_kernel<128><<<grid, rpw * (128 / 4), lds, stream>>>(p);
  }
  DTREE_LAUNCH_CHECK("gdn_layer_recurrence launch");
  return DTREE_OK;
}

// dtree_gdn_layer_prep then dtree_gdn_layer_recurrence, as one launch
// (gdn_prep_reg_kernel) for trees of up to 32 nodes with 16-byte aligned
// projection rows, taps and window; otherwise the two launches.
extern "C" int dtree_gdn_layer_prep_recurrence(const DtreeGdnArgs* a, hipStream_t stream) {
  if (int rc = gdn_layer_check(a, "gdn_layer_prep_recurrence")) return rc;
  const int key_dim = a->num_k_heads * a->head_k_dim, value_dim = a->num_v_heads * a->head_v_dim;
  const int C = 2 * key_dim + value_dim;
  const bool fits = a->rows_padded <= 32 && a->head_k_dim == 128 && a->head_v_dim == 128 && a->conv_keep >= 1 &&
                    a->conv_keep <= kConvMaxKeep && a->ld_proj % 4 == 0 && C % 4 == 0 &&
                    (((uintptr_t)a->proj | (uintptr_t)a->conv_w | (uintptr_t)a->window | (uintptr_t)a->state |
                      (uintptr_t)a->q | (uintptr_t)a->k) & 15) == 0;
  if (!fits) {
    const int rc = dtree_gdn_layer_prep(a, stream);
    return rc ? rc : dtree_gdn_layer_recurrence(a, stream);
  }
  DTREE_REQUIRE(a->proj && a->window && a->conv_w && a->A_log && a->dt_bias && a->q && a->k && a->v && a->g &&
                    a->beta && a->state && a->y,
                "gdn_layer_prep_recurrence: null pointer");
  DTREE_REQUIRE(a->ld_proj >= C + value_dim + 2 * a->num_v_heads,
                "gdn_layer_prep_recurrence: ld_proj below C + z + b + a");
  PrepParams pp{};
  pp.desc = a->desc; pp.rows = a->rows_padded;
  pp.x = a->proj; pp.ldx = a->ld_proj; pp.base = a->window; pp.w = a->conv_w;
  pp.C = C; pp.key_dim = key_dim; pp.Hv = a->num_v_heads; pp.ab_col = C + value_dim;
  pp.A_log = a->A_log; pp.dt_bias = a->dt_bias;
  pp.q = a->q; pp.k = a->k; pp.v = a->v; pp.g = a->g; pp.beta = a->beta;
  pp.q_scale = 1.0f / (float)a->head_k_dim;
  pp.k_scale = 1.0f / sqrtf((float)a->head_k_dim);
  GdnParams p{};
  p.q = a->q; p.k = a->k; p.v = a->v; p.g = a->g; p.beta = a->beta; p.state = a->state;
  p.parents = a->desc->parents; p.T_dev = &a->desc->num_nodes;
  p.T = a->rows_padded; p.Hk = a->num_k_heads; p.Hv = a->num_v_heads; p.Dv = a->head_v_dim; p.rpw = 8;
  p.y = a->y; p.states = nullptr;
  if (use_chunk_recurrence(a->rows_padded, a->head_k_dim, a->head_v_dim)) {
    const int cgrid = a->num_v_heads * (a->head_v_dim / kChunkRows);
    p.T = min(a->rows_padded, 32);
    switch (a->conv_keep) {
#define DTREE_PREP_CHUNK_CASE(K) \
  case K: gdn_tree_chunk_kernel<K><<<cgrid, kChunkThreads, 0, stream>>>(p, pp); break;
      DTREE_PREP_CHUNK_CASE(1) DTREE_PREP_CHUNK_CASE(2) DTREE_PREP_CHUNK_CASE(3) DTREE_PREP_CHUNK_CASE(4)
      DTREE_PREP_CHUNK_CASE(5) DTREE_PREP_CHUNK_CASE(6) DTREE_PREP_CHUNK_CASE(7)
#undef DTREE_PREP_CHUNK_CASE
    }
    DTREE_LAUNCH_CHECK("gdn_layer_prep_recurrence launch");
    return DTREE_OK;
  }
  const int grid = a->num_v_heads * (a->head_v_dim / 8);
  switch (a->conv_keep) {
#define DTREE_PREP_REG_CASE(K) \
  case K: gdn_prep_reg_kernel<K><<<grid, 256, 0, stream>>>(p, pp); break;
    DTREE_PREP_REG_CASE(1) DTREE_PREP_REG_CASE(2) DTREE_PREP_REG_CASE(3) DTREE_PREP_REG_CASE(4)
    DTREE_PREP_REG_CASE(5) DTREE_PREP_REG_CASE(6) DTREE_PREP_REG_CASE(7)
#undef DTREE_PREP_REG_CASE
  }
  DTREE_LAUNCH_CHECK("gdn_layer_prep_recurrence launch");
  return DTREE_OK;
}

extern "C" int dtree_gdn_layer_gated_norm(const DtreeGdnArgs* a, hipStream_t stream) {
  if (int rc = gdn_layer_check(a, "gdn_layer_gated_norm")) return rc;
  DTREE_REQUIRE(a->y && a->proj && a->norm_w && a->out, "gdn_layer_gated_norm: null pointer");
  const int key_dim = a->num_k_heads * a->head_k_dim, value_dim = a->num_v_heads * a->head_v_dim;
  const int C = 2 * key_dim + value_dim;
  DTREE_REQUIRE(a->ld_proj >= C + value_dim && a->ld_proj % 4 == 0 && ((uintptr_t)a->proj & 15) == 0,
                "gdn_layer_gated_norm: proj must be 16-byte aligned with ld_proj % 4 == 0");
  DTREE_REQUIRE(((uintptr_t)a->out & 15) == 0 && ((uintptr_t)a->out_lo & 15) == 0 && ((uintptr_t)a->y & 15) == 0 &&
                    ((uintptr_t)a->norm_w & 15) == 0,
                "gdn_layer_gated_norm: y, norm_w, out and out_lo must be 16-byte aligned");
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR ? (a->ld_out >= value_dim && a->ld_out % 8 == 0)
                                                  : ((a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16) &&
                                                     a->ld_out == value_dim &&
                                                     value_dim % 64 == 0 && a->rows_padded % 32 == 0),
                "gdn_layer_gated_norm: out layout (tiled needs ld_out == value dim, rows_padded % 32 == 0)");
  const int pairs = a->rows_padded * a->num_v_heads;
  const int per_block = 256 / (128 / 8);
  gdn_gated_norm_kernel<128><<<(pairs + per_block - 1) / per_block, 256, 0, stream>>>(
      a->desc, 0, a->y, a->proj + C, a->ld_proj, a->norm_w, a->eps, a->num_v_heads, a->rows_padded, a->out, a->out_lo,
      a->out_layout, a->ld_out);
  DTREE_LAUNCH_CHECK("gdn_layer_gated_norm launch");
  return DTREE_OK;
}

// A commit's destination: both buffers given (and each either the source
// itself or disjoint from it) or neither (in place).
static int commit_dest_check(const DtreeGdnArgs* a, const char* what) {
  const size_t C = 2 * (size_t)a->num_k_heads * a->head_k_dim + (size_t)a->num_v_heads * a->head_v_dim;
  const size_t wb = (size_t)a->conv_keep * C * sizeof(float);
  const size_t sb = (size_t)a->num_v_heads * a->head_v_dim * a->head_k_dim * sizeof(float);
  auto disjoint = [](const void* x, const void* y, size_t n) {
    const char* p = static_cast<const char*>(x);
    const char* q = static_cast<const char*>(y);
    return p == q || p + n <= q || q + n <= p;
  };
  if ((a->window_out == nullptr) != (a->state_out == nullptr))
    return ::dtree::fail(DTREE_E_ARG, std::string(what) + ": window_out and state_out are given together or not at all");
  if (a->window_out && !(disjoint(a->window, a->window_out, wb) && disjoint(a->state, a->state_out, sb)))
    return ::dtree::fail(DTREE_E_ARG, std::string(what) + ": a commit destination partly overlaps its source");
  return DTREE_OK;
}

extern "C" int dtree_gdn_layer_commit(const DtreeGdnArgs* a, hipStream_t stream) {
  if (int rc = gdn_layer_check(a, "gdn_layer_commit")) return rc;
  DTREE_REQUIRE(a->proj && a->window && a->state && a->q && a->k && a->v && a->g && a->beta,
                "gdn_layer_commit: null pointer");
  if (int rc = commit_dest_check(a, "gdn_layer_commit")) return rc;
  const int C = 2 * a->num_k_heads * a->head_k_dim + a->num_v_heads * a->head_v_dim;
  const int rpw = 256 / (128 / 4);
  GdnParams p{};
  p.q = a->q; p.k = a->k; p.v = a->v; p.g = a->g; p.beta = a->beta; p.state = a->state;
  p.path = a->desc->accepted; p.path_len = &a->desc->n_accepted;
  p.T = a->rows_padded; p.Hk = a->num_k_heads; p.Hv = a->num_v_heads; p.Dv = a->head_v_dim; p.rpw = rpw;
  const int conv_blocks = (C + 255) / 256;
  const int state_blocks = a->num_v_heads * (a->head_v_dim / rpw);
  p.state_out = a->state_out;
  gdn_commit_kernel<128><<<conv_blocks + state_blocks, 256, 0, stream>>>(p, a->proj, a->ld_proj, a->window,
                                                                          a->window_out, C,
                                                                          a->conv_keep, conv_blocks);
  DTREE_LAUNCH_CHECK("gdn_layer_commit launch");
  return DTREE_OK;
}

extern "C" int dtree_gdn_layers_commit(const DtreeGdnArgs* a, int32_t num_layers, hipStream_t stream) {
  DTREE_REQUIRE(a && num_layers >= 1, "gdn_layers_commit: null args or no layers");
  for (int i = 0; i < num_layers; ++i) {
    if (int rc = gdn_layer_check(&a[i], "gdn_layers_commit")) return rc;
    DTREE_REQUIRE(a[i].proj && a[i].window && a[i].state && a[i].k && a[i].v && a[i].g && a[i].beta,
                  "gdn_layers_commit: null pointer");
    if (int rc = commit_dest_check(&a[i], "gdn_layers_commit")) return rc;
    DTREE_REQUIRE(a[i].desc == a[0].desc && a[i].rows_padded == a[0].rows_padded &&
                      a[i].num_k_heads == a[0].num_k_heads && a[i].num_v_heads == a[0].num_v_heads &&
                      a[i].conv_keep == a[0].conv_keep && a[i].ld_proj == a[0].ld_proj,
                  "gdn_layers_commit: layers must share the step descriptor, node capacity, heads, conv and ld_proj");
  }
  const int C = 2 * a[0].num_k_heads * a[0].head_k_dim + a[0].num_v_heads * a[0].head_v_dim;
  const int rpw = 256 / (128 / 4);
  GdnParams p{};
  p.path = a[0].desc->accepted; p.path_len = &a[0].desc->n_accepted;
  p.T = a[0].rows_padded; p.Hk = a[0].num_k_heads; p.Hv = a[0].num_v_heads; p.Dv = a[0].head_v_dim; p.rpw = rpw;
  const int conv_blocks = (C + 255) / 256;
  const int state_blocks = a[0].num_v_heads * (a[0].head_v_dim / rpw);
  for (int l0 = 0; l0 < num_layers; l0 += kCommitMaxLayers) {
    const int nl = min(num_layers - l0, kCommitMaxLayers);
    CommitBatch b{};
    for (int i = 0; i < nl; ++i) {
      const DtreeGdnArgs& x = a[l0 + i];
      b.l[i] = CommitLayer{x.proj, x.window, x.state, x.k, x.v, x.g, x.beta, x.window_out, x.state_out};
    }
    gdn_commit_layers_kernel<128><<<dim3(conv_blocks + state_blocks, nl), 256, 0, stream>>>(p, b, a[0].ld_proj, C,
                                                                                          a[0].conv_keep,
                                                                                          conv_blocks);
    DTREE_LAUNCH_CHECK("gdn_layers_commit launch");
  }
  return DTREE_OK;
}

// A GatedDeltaNet layer's core over a causal chain of num_tokens prompt tokens
// that continue the committed window and state: conv + SiLU and the q / k / v
// / g / beta prep, the recurrence (final state committed, conv window
// advanced), and the gated RMSNorm into the out_proj input. desc is unused;
// rows_padded is the row capacity of the per-row buffers.
extern "C" int dtree_gdn_layer_chain(const DtreeGdnArgs* a, int32_t num_tokens, hipStream_t stream) {
  DTREE_REQUIRE(a, "gdn_layer_chain: null args");
  DTREE_REQUIRE(num_tokens >= 1 && num_tokens <= a->rows_padded, "gdn_layer_chain: num_tokens in [1, rows_padded]");
  DTREE_REQUIRE(a->num_k_heads > 0 && a->num_v_heads > 0 && a->num_v_heads % a->num_k_heads == 0,
                "gdn_layer_chain: num_v_heads % num_k_heads");
  DTREE_REQUIRE(a->head_k_dim == 128 && a->head_v_dim == 128, "gdn_layer_chain: head dims 128 are compiled");
  DTREE_REQUIRE(a->conv_keep >= 1 && a->conv_keep <= kConvMaxKeep, "gdn_layer_chain: conv_keep in [1, 7]");
  DTREE_REQUIRE(a->proj && a->window && a->conv_w && a->A_log && a->dt_bias && a->state && a->q && a->k && a->v &&
                    a->g && a->beta && a->y && a->norm_w && a->out,
                "gdn_layer_chain: null pointer");
  const int key_dim = a->num_k_heads * a->head_k_dim, value_dim = a->num_v_heads * a->head_v_dim;
  const int C = 2 * key_dim + value_dim;
  DTREE_REQUIRE(a->ld_proj >= C + value_dim + 2 * a->num_v_heads && a->ld_proj % 4 == 0 &&
                    ((uintptr_t)a->proj & 15) == 0,
                "gdn_layer_chain: proj must be 16-byte aligned, ld_proj >= C + z + b + a, ld_proj % 4 == 0");
  DTREE_REQUIRE(((uintptr_t)a->q & 15) == 0 && ((uintptr_t)a->k & 15) == 0 && ((uintptr_t)a->state & 15) == 0 &&
                    ((uintptr_t)a->out & 15) == 0 && ((uintptr_t)a->out_lo & 15) == 0 && ((uintptr_t)a->y & 15) == 0 &&
                    ((uintptr_t)a->norm_w & 15) == 0,
                "gdn_layer_chain: q, k, state, y, norm_w, out and out_lo must be 16-byte aligned");
  DTREE_REQUIRE(a->out_layout == DTREE_W_ROWMAJOR ? (a->ld_out >= value_dim && a->ld_out % 8 == 0)
                                                  : ((a->out_layout == DTREE_W_TILED || a->out_layout == DTREE_W_TILED_F16) &&
                                                     a->ld_out == value_dim &&
                                                     value_dim % 64 == 0 && a->rows_padded % 32 == 0),
                "gdn_layer_chain: out layout (tiled needs ld_out == value dim, rows_padded % 32 == 0)");
  PrepParams pp{};
  pp.desc = nullptr; pp.rows = a->rows_padded; pp.chain = num_tokens;
  pp.x = a->proj; pp.ldx = a->ld_proj; pp.base = a->window; pp.w = a->conv_w;
  pp.C = C; pp.key_dim = key_dim; pp.Hv = a->num_v_heads; pp.ab_col = C + value_dim;
  pp.A_log = a->A_log; pp.dt_bias = a->dt_bias;
  pp.q = a->q; pp.k = a->k; pp.v = a->v; pp.g = a->g; pp.beta = a->beta;
  pp.q_scale = 1.0f / (float)a->head_k_dim;
  pp.k_scale = 1.0f / sqrtf((float)a->head_k_dim);
  const dim3 pgrid(C / 128 + 1, (num_tokens + kPrepNodes - 1) / kPrepNodes);
  switch (a->conv_keep) {
#define DTREE_PREP_CASE(K) \
  case K: gdn_prep_kernel<K, 128><<<pgrid, 128, 0, stream>>>(pp); break;
    DTREE_PREP_CASE(1) DTREE_PREP_CASE(2) DTREE_PREP_CASE(3) DTREE_PREP_CASE(4) DTREE_PREP_CASE(5)
    DTREE_PREP_CASE(6) DTREE_PREP_CASE(7)
#undef DTREE_PREP_CASE
  }
  DTREE_LAUNCH_CHECK("gdn_layer_chain prep launch");
  GdnParams p{};
  p.q = a->q; p.k = a->k; p.v = a->v; p.g = a->g; p.beta = a->beta; p.state = a->state;
  p.T = num_tokens; p.Hk = a->num_k_heads; p.Hv = a->num_v_heads; p.Dv = a->head_v_dim; p.y = a->y;
  const int state_blocks = a->num_v_heads * (a->head_v_dim / 8);
  const int conv_blocks = (C + 255) / 256;
  gdn_chain_scan_kernel<<<state_blocks + conv_blocks, 256, 0, stream>>>(p, a->proj, a->ld_proj, a->window, C,
                                                                         a->conv_keep, state_blocks);
  DTREE_LAUNCH_CHECK("gdn_layer_chain scan launch");
  const int pairs = a->rows_padded * a->num_v_heads;
  const int per_block = 256 / (128 / 8);
  gdn_gated_norm_kernel<128><<<(pairs + per_block - 1) / per_block, 256, 0, stream>>>(
      nullptr, num_tokens, a->y, a->proj + C, a->ld_proj, a->norm_w, a->eps, a->num_v_heads, a->rows_padded, a->out,
      a->out_lo, a->out_layout, a->ld_out);
  DTREE_LAUNCH_CHECK("gdn_layer_chain gated norm launch");
  return DTREE_OK;
}
