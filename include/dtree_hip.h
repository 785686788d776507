/*
 * dtree_hip.h -- C ABI of the MI355X (gfx950) DTree tree-verify step.
 *
 * Every entry point takes plain device pointers, sizes and an explicit
 * hipStream_t, launches asynchronously on that stream, and returns 0 on
 * success or a negative DTREE_E* status; dtree_last_error() then holds a
 * message for the calling thread. Nothing here allocates device memory:
 * callers pass workspaces sized by the *_workspace_bytes queries.
 *
 * Reference citations are paths relative to the DrHB/dtree-mlx checkout.
 */
#ifndef DTREE_HIP_H
#define DTREE_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DTREE_ABI_VERSION 8

#define DTREE_OK 0
#define DTREE_E_ARG (-1)      /* bad shape / pointer / enum */
#define DTREE_E_HIP (-2)      /* HIP runtime error */
#define DTREE_E_TREE (-3)     /* non-topological parents, too many nodes */
#define DTREE_E_WORKSPACE (-4) /* workspace too small */

#define DTREE_MAX_NODES 128   /* tree nodes incl. root per verify step */
#define DTREE_MASK_WORDS 4    /* 32-bit words of an ancestor bitset */
#define DTREE_PAGE 64         /* KV positions per cache page */

/*
 * Device-resident description of one verify step. The host fills the input
 * half (past_length .. ancestors) and copies it to device memory before the
 * kernels run; kernels fill the output half. Keeping P and L in device memory
 * lets one captured HIP graph serve every step.
 *
 * Mirrors the per-step values of dtree_runtime.py:166-192 (ids, positions =
 * start + depth, mask = all prefix columns + ancestor-or-self tree columns)
 * and the walk result of dtree_runtime.py:195-208 (accepted indices, bonus).
 */
typedef struct DtreeStepDesc {
  int32_t past_length;                 /* P: cached positions before the tree */
  int32_t num_nodes;                   /* L: root + draft nodes              */
  int32_t n_accepted;                  /* out: len(accepted_indices)          */
  int32_t bonus_token;                 /* out: posterior token after the walk */
  int32_t tokens[DTREE_MAX_NODES];     /* node token ids (root first)         */
  int32_t positions[DTREE_MAX_NODES];  /* RoPE positions                      */
  int32_t parents[DTREE_MAX_NODES];    /* parent index, root = -1, parent < i */
  uint32_t ancestors[DTREE_MAX_NODES][DTREE_MASK_WORDS]; /* ancestor-or-self */
  int32_t accepted[DTREE_MAX_NODES];   /* out: accepted node indices          */
  int32_t posterior[DTREE_MAX_NODES];  /* out: target argmax per node         */
} DtreeStepDesc;

/*
 * Weight layouts of an [n][k] bf16 matrix (nn.Linear layout).
 *  DTREE_W_ROWMAJOR: plain [n][k].
 *  DTREE_W_TILED:    [n/32][k/64][4][64][8]: block (r, b) holds rows 32r..32r+31
 *                    and columns 64b..64b+63; element (i, l, e) of a block is
 *                    row 32r + l%32, column 64b + 32*(l/32) + 8i + e. This is
 *                    the order the GEMM lanes consume, so each 16-byte load
 *                    instruction of a wavefront reads one contiguous kilobyte.
 *                    dtree_tile_weight converts a row-major matrix.
 *  DTREE_W_Q4G64:    4-bit affine groups of 64 (the MLX quantized format of
 *                    nn.QuantizedLinear, adapters.py:63-71, api.py:46-54:
 *                    W[n][k] = scale[n][k/64] * q[n][k] + bias[n][k/64]),
 *                    repacked: w = uint32 [n/32][k/64][64][4]; word (l, i) of
 *                    block (r, b) holds q of row 32r + l%32 at columns
 *                    64b + 32*(l/32) + 8i + e, e = 0..7, with even e in bits
 *                    4*(e/2) and odd e in bits 16 + 4*(e/2); w_scales = bf16
 *                    [n/32][k/64][32][2] (scale, bias) of row 32r + c, group b.
 *                    Activations must be DTREE_W_TILED, 32 rows.
 *  DTREE_W_TILED_F16: DTREE_W_TILED's order with fp16 elements: bf16 weights
 *                    converted once (dtree_tile_weight_f16; exact for every
 *                    bf16 of magnitude 2^-17 .. 65504), and activations as ONE
 *                    fp16 plane (11 significant bits: no low half). The GEMM
 *                    then runs one fp16 MFMA per weight fragment and each CU
 *                    loads half the activation bytes of the bf16 pair. Both
 *                    operands must be TILED_F16. The format holds values up to
 *                    65504: models whose activations stay in that range (the
 *                    bf16 workloads here: |x| < 50); q4 models, whose random
 *                    residual stream reaches 1e12, keep DTREE_W_TILED.
 *
 * Activations between kernels (GEMM inputs and the *_bf16 / out outputs)
 * take the layout code of their consumer: ROWMAJOR and TILED are bf16 with an
 * optional low half (x = hi + lo), TILED_F16 is one fp16 plane (lo ignored).
 */
#define DTREE_W_ROWMAJOR 0
#define DTREE_W_TILED 1
#define DTREE_W_Q4G64 2
#define DTREE_W_TILED_F16 3

/* GEMM epilogues (dtree_gemm_bf16). */
#define DTREE_EPI_STORE_F32 0  /* out_f32[m][n] = rs[m] * acc                 */
#define DTREE_EPI_RESIDUAL 1   /* x[m][n] += acc; xg = bf16(x*g_next); ss tile */
#define DTREE_EPI_SWIGLU 2     /* act = bf16(silu(rs*gate) * rs*up), W rows
                                  interleaved in 16-row gate/up groups         */
#define DTREE_EPI_STORE_BF16 3 /* out_bf16[m][n] = bf16(rs[m] * acc)          */

/*
 * Skinny bf16 GEMM Y = X W^T for up to 128 rows (tree nodes), fp32 accumulate
 * on gfx950 MFMA 32x32x16. rs[m] is the RMSNorm row scale
 * rsqrt(sum_t ss(t, m) / norm_dim + eps) when ss_in != NULL, else 1, where
 * ss(t, m) = sum over columns 32t .. 32t+31 of row m's x^2, stored at
 * ss_in[((m / 32) * ss_tiles + t) * 32 + m % 32] (every 32-row block is one
 * contiguous [ss_tiles][32] array; for 32 rows this is [ss_tiles][32]).
 * Replaces the nn.Linear projections of the tree block
 * (qwen3_tree.py:50-52, 78, 82) with the RMSNorms of qwen3_tree.py:47, 81
 * folded in (norm weight folded into the producer's bf16 X, row scale here).
 */
typedef struct DtreeGemmArgs {
  const uint16_t* x;      /* bf16 [rows_padded][ldx], rows >= L are zero   */
  const uint16_t* x_lo;   /* optional low half: X = x + x_lo (both bf16)   */
  int32_t x_layout;       /* DTREE_W_ROWMAJOR, or DTREE_W_TILED / _F16 with ldx = k */
  int32_t ldx;
  int32_t rows_padded;    /* 32, 64, 96 or 128                             */
  const uint16_t* w;      /* bf16 [n][k] (nn.Linear layout); Q4G64: packed q
                             (tiled x; above 32 rows one pass per 32 rows) */
  int32_t w_layout;       /* DTREE_W_ROWMAJOR, DTREE_W_TILED, DTREE_W_TILED_F16
                             (with x_layout TILED_F16) or DTREE_W_Q4G64     */
  int32_t n, k;           /* k % 64 == 0; n % 64 == 0 (% 32 above 64 rows) */
  int32_t epilogue;       /* DTREE_EPI_*                                   */
  int32_t split_k;        /* >= 1 split-K (bf16); 0 = automatic; tiled 32
                             rows only, bf16 or Q4G64:
                             -1 one workgroup per 32-column tile,
                             -2 stream-K schedule,
                             -3 / -4 two / three workgroups per 32-column
                                tile, one per part of K
                                (n % 256 == 0, k >= 64 * parts)            */
  const float* ss_in;     /* [rows_padded/32][ss_tiles][32] or NULL        */
  int32_t ss_tiles;
  int32_t norm_dim;       /* divisor of the row mean square                */
  float eps;
  float* out_f32; int32_t ld_out_f32;      /* STORE_F32 out / RESIDUAL x   */
  uint16_t* out_bf16;     /* RESIDUAL xg / SWIGLU / BF16 output (hi half)  */
  uint16_t* out_lo;       /* optional low half of out_bf16 (v - hi)        */
  int32_t out_layout;     /* layout of out_bf16 / out_lo (TILED: ld = width) */
  int32_t ld_out_bf16;
  const uint16_t* next_norm;  /* RESIDUAL: weight of the following RMSNorm */
  float* ss_out;              /* RESIDUAL: [rows_padded/32][n/32][32]      */
  uint16_t* hidden_out; int32_t ld_hidden; /* RESIDUAL: optional bf16 copy */
  void* workspace; size_t workspace_bytes; /* split-K partials + counters  */
  const uint16_t* w_scales;   /* Q4G64: (scale, bias) pairs, else NULL     */
} DtreeGemmArgs;

const char* dtree_last_error(void);
int dtree_abi_version(void);
size_t dtree_step_desc_bytes(void);

/*
 * Host-side tree validation (host pointers; no device work). The kernels read
 * trees from device memory and cannot report a malformed one synchronously:
 * they only read a parent outside [0, i) as -1, which keeps every access in
 * bounds, so a binder validates before the upload.
 *
 * dtree_validate_parents: parents[0] == -1 and 0 <= parents[i] < i (node
 * order = heap-pop order, dtree_runtime.py:125-130), 1 <= num_nodes <= 128;
 * else DTREE_E_TREE. Guards the raw-parent entries dtree_gdn_tree_conv and
 * dtree_gdn_tree_recurrence.
 * dtree_step_desc_validate: the input half of a DtreeStepDesc as
 * compile_dtree_tree (dtree_runtime.py:166-192) produces it: 1 <= num_nodes
 * <= max_nodes, 0 <= past_length <= max_past_length, topological parents,
 * every ancestors[i] = ancestors[parents[i]] | bit i (bit 0 for the root),
 * tokens in [0, vocab_size), positions >= 0, accepted[0 .. n_accepted) in
 * [0, num_nodes). DTREE_E_TREE for the tree shape, DTREE_E_ARG otherwise.
 */
int dtree_validate_parents(const int32_t* parents, int32_t num_nodes);
int dtree_step_desc_validate(const DtreeStepDesc* desc, int32_t max_nodes, int32_t max_past_length,
                             int32_t vocab_size);
/* sizeof(DtreeGemmArgs) / sizeof(DtreeAttnArgs): lets bindings check their
 * mirrored struct layouts. */
size_t dtree_gemm_args_bytes(void);
size_t dtree_attn_args_bytes(void);

/* Workspace for dtree_gemm_bf16 (partials + tile counters). Counters must be
 * zero before the first call; every call leaves them zero again. Calls that
 * share a workspace must not overlap (one stream, or ordered by events).
 * With q4 weights over 64-128 rows the K parts of a tile wait for each other
 * at a bounded wait (~2 ms) to combine their partials in a distributed way;
 * a part that gives up leaves its share to the last part to arrive, so the
 * result never depends on it. */
size_t dtree_gemm_workspace_bytes(int rows_padded, int n, int k, int split_k);
int dtree_gemm_bf16(const DtreeGemmArgs* args, hipStream_t stream);

/*
 * Embedding gather + first RMSNorm fold (adapters.py:580, qwen3_tree.py:47):
 * x[m] = E[tokens[m]] (fp32; E in DTREE_W_* layout embed_layout; DTREE_W_Q4G64
 * dequantises the row with embed_scales, as quantize_model quantises the
 * embedding, api.py:46-54), xg = bf16(x * norm_w) (+ optional low half
 * xg_lo = bf16(x * norm_w - xg)), ss[t][m] = sum of x^2
 * over column tile t (32 columns); rows >= L and token ids outside
 * [0, vocab) embed as zero. Also fills the RoPE
 * table cos/sin [rows_padded][head_dim/2] for desc->positions
 * (mlx nn.RoPE, traditional=False, per-token offsets, qwen3_tree.py:22-27).
 */
int dtree_embed(const DtreeStepDesc* desc, const uint16_t* embed, int32_t embed_layout,
                const uint16_t* embed_scales, int32_t vocab, int32_t hidden, const uint16_t* norm_w, int32_t rows_padded, float* x, uint16_t* xg,
                uint16_t* xg_lo, int32_t xg_layout, float* ss, int32_t head_dim, float rope_base, float* rope_cos,
                float* rope_sin, hipStream_t stream);

/* RoPE table only (used when q/k come from outside dtree_embed). */
int dtree_rope_table(const DtreeStepDesc* desc, int32_t rows_padded, int32_t head_dim,
                     float rope_base, float* rope_cos, float* rope_sin, hipStream_t stream);

/*
 * Ancestor-masked GQA tree attention over a paged bf16 KV prefix
 * (qwen3_tree.py:54-76 and the cache append at :146; mask semantics
 * dtree_runtime.py:190-191). Reads raw q/k/v (fp32, row m = tree node m) from
 * qkv[m][...] laid out as [q heads | k heads | v heads] * head_dim, applies
 * q_norm / k_norm (RMSNorm over head_dim, NULL = none), RoPE from the table
 * (cos/sin [rows][rope_dims/2], pairs (d, d + rope_dims/2), dims >= rope_dims
 * unrotated), writes the L new K/V rows into the cache at logical positions
 * P..P+L-1, and writes softmax(scale * q k^T + mask) v as bf16
 * out[m][h*head_dim + d] (rows >= L zero). K and V pages are
 * [page][kv_head][DTREE_PAGE * head_dim] bf16 blocks (head_dim a multiple of
 * 32) in the order the attention's 32x32x16 MFMAs read their operands, so
 * that each operand fragment is one contiguous kilobyte in lane order. With
 * pi(r) = r with bits 2 and 3 swapped, element (slot s, dim d) of a block is
 *   K: ((((s/32)*(head_dim/16) + d/16)*64 + ((d/8)%2)*32 + pi(s%32)) * 8) + d%8
 *   V: ((((s/16)*(head_dim/32) + d/32)*64 + ((s/8)%2)*32 + d%32) * 8) + s%8
 * (8 consecutive dims of one key, resp. 8 consecutive slots of one dim, are
 * one 16-byte run). page_table maps logical page -> physical page.
 *
 * gated = 1 is the Qwen3.5 gated attention (qwen35_tree.py:503-540): each q
 * head occupies 2*head_dim columns of the qkv row, [q | gate], and the output
 * is multiplied by sigmoid(gate). Compiled geometries: head_dim 128 with
 * rope_dims 128 (or 0), gated 0; head_dim 256 with rope_dims 64, gated 1.
 * Trees of up to rows_padded (32, 64, 96 or 128) nodes; the ancestor bitset
 * word w of a node covers nodes 32w .. 32w+31.
 *
 * workspace: dtree_attention_workspace_bytes(num_heads, head_dim,
 * max_past_length, rows_padded) bytes, zeroed once before its first use and
 * then kept as the launches leave it: its counters return to zero by
 * themselves and, for 32-row trees, the per-head kernel's splits exchange
 * their partial results through flagged slots whose epoch words carry over
 * from launch to launch. One workspace serves one (num_heads, head_dim,
 * rows_padded); zero it again before using it with another.
 */
typedef struct DtreeAttnArgs {
  const float* qkv; int32_t ld_qkv;
  const uint16_t* q_norm; const uint16_t* k_norm; float eps;
  const float* rope_cos; const float* rope_sin;
  uint16_t* k_pages; uint16_t* v_pages; const int32_t* page_table;
  const DtreeStepDesc* desc;
  uint16_t* out; uint16_t* out_lo; int32_t ld_out;  /* out_lo optional low half */
  int32_t out_layout;       /* DTREE_W_ROWMAJOR or DTREE_W_TILED (ld_out = width) */
  int32_t num_heads, num_kv_heads, head_dim, rows_padded;  /* rows: 32, 64, 96, 128 */
  float scale;
  int32_t max_past_length;  /* grid is sized for this P; page_table must cover
                               max_past_length positions (entries are read
                               before P is known) */
  int32_t write_cache;      /* 1: append the tree K/V rows to the cache */
  void* workspace; size_t workspace_bytes;
  int32_t rope_dims;        /* rotated dims per head; 0 = head_dim */
  int32_t gated;            /* 1: q heads are [q | gate] and out *= sigmoid(gate) */
} DtreeAttnArgs;

size_t dtree_attention_workspace_bytes(int32_t num_heads, int32_t head_dim,
                                       int32_t max_past_length, int32_t rows_padded);
int dtree_tree_attention(const DtreeAttnArgs* args, hipStream_t stream);

/*
 * dtree_tree_attention without a caller workspace: the same kernels keep their
 * workspace (error word, split counters, partials) in a file-scope device array
 * of dtree_tree_attention_noalloc_max_bytes() (32 MiB) bytes, one per GPU, held
 * until the process ends; args->workspace / workspace_bytes are ignored. A
 * shape whose workspace (dtree_attention_workspace_bytes' formula for the
 * kernel the shape selects) exceeds the array returns DTREE_E_WORKSPACE. Each
 * call clears the array's header with a fill kernel on `stream` (and the
 * flag-exchange region when num_heads, head_dim or rows_padded differ from
 * the previous call on this GPU); calls that overlap on one GPU race (they
 * share the array). No device memory is allocated or freed.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).
 */
size_t dtree_tree_attention_noalloc_max_bytes(void);
int dtree_tree_attention_noalloc(const DtreeAttnArgs* args, hipStream_t stream);
/* Status of the attention launches on a workspace, in stream order: the
 * per-KV-group kernel's splits meet at a bounded wait, and so do the per-head
 * kernel's splits in its flag exchange (32-row trees); a split that gives up
 * (another split was not resident for ~2 s, e.g. when work on another stream
 * holds CUs) sets the workspace's error word and leaves its share of the
 * output unwritten. This ORs that word into *status (device memory; 1 = a
 * wait gave up since the last query) and clears it; after a give-up it also
 * moves the exchange's epoch words far ahead, so no flag the failed launch
 * wrote can match a later one. workspace = NULL reads the allocation-free
 * entry's device scratch of the current GPU, which
 * dtree_tree_attention_noalloc clears before each call: query it after each
 * such call. A step whose status is set must be recomputed; the wait's
 * counters return to zero by themselves, so the next launch is sound. The
 * reference's scaled_dot_product_attention (qwen3_tree.py:69-76) has no such
 * failure mode; this is the error row of the boundary for it. */
int dtree_attention_status(void* workspace, int32_t* status, hipStream_t stream);

/*
 * Fused LM head + argmax (adapters.py:114-118, 489-492, first index on ties
 * as adapters.py:78-81): per row m, argmax_v rs[m] * (x[m] . E[v]).
 * x = x + x_lo (split pair, x_lo optional); E in layout emb_layout
 * (DTREE_W_Q4G64: the quantised tied embedding with its (scale, bias) pairs in
 * emb_scales, tiled rows (one pass per 32 rows), hidden <= 4096;
 * adapters.py:28-85 is the reference's q4 LM-head argmax). Statistics ss_in
 * as for DtreeGemmArgs. Writes per-workgroup (value, index) candidates to
 * `candidates` (pairs of row m, workgroup b at ((m / 32) * blocks + b) * 32 +
 * m % 32, blocks = dtree_lmhead_candidate_blocks); dtree_accept_walk reduces them.
 * logits (optional, [rows_padded][vocab] fp32) receives every logit.
 */
size_t dtree_lmhead_candidates_bytes(int32_t rows_padded);
int dtree_lmhead_candidate_blocks(int32_t vocab, int32_t rows_padded);
int dtree_lmhead_argmax(const uint16_t* x, const uint16_t* x_lo, int32_t x_layout, int32_t ldx, int32_t rows_padded,
                        const uint16_t* emb, int32_t emb_layout, const uint16_t* emb_scales, int32_t vocab,
                        int32_t hidden, const float* ss_in, int32_t ss_tiles, float eps,
                        float* logits, void* candidates, hipStream_t stream);

/*
 * Final argmax reduction + greedy accept walk (dtree_runtime.py:195-208).
 * Writes desc->posterior[0..L), accepted[], n_accepted, bonus_token, and the
 * same values to the device buffer `result` when non-NULL
 * ([3 + 2*DTREE_MAX_NODES] int32: n_accepted, bonus, L, accepted[MAX],
 * posterior[MAX]). num_candidate_blocks = dtree_lmhead_candidate_blocks(vocab).
 */
int dtree_accept_walk(DtreeStepDesc* desc, const void* candidates,
                      int32_t num_candidate_blocks, int32_t rows_padded,
                      int32_t* result, hipStream_t stream);

/*
 * KV compaction (adapters.py:635-668) for `layers` layer caches whose page
 * pools are `layer_stride` elements apart, plus the hidden-state select of
 * dtree_runtime.py:520-521 (hidden_in rows accepted[j] -> hidden_out row j,
 * optional). Reads accepted / n_accepted / P from desc.
 */
int dtree_compact(const DtreeStepDesc* desc, uint16_t* k_pages, uint16_t* v_pages,
                  size_t layer_stride, int32_t layers, int32_t num_kv_heads,
                  int32_t head_dim, const int32_t* page_table,
                  const uint16_t* hidden_in, int32_t hidden_width, uint16_t* hidden_out,
                  hipStream_t stream);

/* Final RMSNorm output (norm_hidden of adapters.py:595): out = bf16(x*rs*w). */
int dtree_rownorm(const float* x, int32_t ldx, int32_t rows_padded, int32_t hidden,
                  const float* ss_in, int32_t ss_tiles, const uint16_t* w, float eps,
                  uint16_t* out, int32_t ld_out, hipStream_t stream);

/*
 * Prompt prefill (forward_with_hidden_states, adapters.py:494-533: the
 * target's causal forward over the prompt). dtree_gemm_long is the
 * compute-bound GEMM for rows_padded = a multiple of 128 (any length):
 * tiled bf16 activations (split pair optional) and tiled bf16 or q4
 * group-64 weights (DTREE_W_Q4G64 with w_scales 16-byte aligned),
 * n a multiple of 128 (of 64 with DTREE_EPI_STORE_F32: the Qwen3.5 in_proj),
 * the four epilogues of dtree_gemm_bf16 with outputs,
 * statistics and hidden rows laid out as there (per 32-row block).
 * dtree_embed_tokens is dtree_embed for a device token array of any length
 * (rows n .. rows_padded - 1 zero), without the RoPE table.
 */
int dtree_gemm_long(const DtreeGemmArgs* args, hipStream_t stream);
int dtree_embed_tokens(const int32_t* tokens, int32_t n, const uint16_t* embed, int32_t embed_layout,
                       const uint16_t* embed_scales, int32_t vocab, int32_t hidden, const uint16_t* norm_w,
                       int32_t rows_padded, float* x, uint16_t* xg, uint16_t* xg_lo, int32_t xg_layout, float* ss,
                       hipStream_t stream);

/*
 * Layer input from caller rows instead of token ids: the DFlash drafter's
 * noise embedding enters its first decoder layer (DFlashDraftModel.__call__,
 * draft.py:349-364, input_layernorm at draft.py:294-295). rows: bf16
 * [n_rows][ld_rows] row-major; rows >= n_rows read as zero. Outputs as
 * dtree_embed: x (fp32 [rows_padded][hidden]), xg (+ optional xg_lo) =
 * split(x * norm_w) in xg_layout, ss statistics.
 */
int dtree_rows_in(const uint16_t* rows, int32_t ld_rows, int32_t n_rows, const uint16_t* norm_w,
                  int32_t rows_padded, int32_t hidden, float* x, uint16_t* xg, uint16_t* xg_lo,
                  int32_t xg_layout, float* ss, hipStream_t stream);

/*
 * Context K/V append of the DFlash drafter (DFlashAttention.
 * precompute_context_kv, draft.py:186-206): kv holds fp32 projections
 * [n_rows][ld_kv] = [k heads | v heads] * head_dim of the prepared target
 * hidden rows; row r becomes position first_position + r:
 * k = RoPE(k_norm(k)) (k_norm NULL = none; head_dim 128, every dim rotated),
 * v as is, both stored bf16 in the paged layout of dtree_tree_attention.
 * window = 0: slot = position (mlx KVCache.update_and_fetch, draft.py:206).
 * window > 0: the sink + window context cache (ContextOnlyDraftKVCache,
 * draft.py:67-110, sink 64 / window 1024 there): positions below `sink` keep
 * their slot, later ones go to ring slot sink + (position - sink) % window, so
 * the slots always hold the sink and the newest `window` positions (a row
 * that a later row of the same call replaces is skipped). The ring changes
 * only the order of the keys, which unmasked attention does not see.
 * capacity = positions covered by page_table; every slot written lies below.
 */
int dtree_kv_append(const float* kv, int32_t ld_kv, int32_t n_rows, int32_t first_position,
                    const uint16_t* k_norm, float eps, int32_t num_kv_heads, int32_t head_dim,
                    float rope_base, int32_t sink, int32_t window, uint16_t* k_pages, uint16_t* v_pages,
                    const int32_t* page_table, int32_t capacity, hipStream_t stream);

/*
 * Draft tree on the GPU (build_dtree_tree, dtree_runtime.py:82-163, and the
 * verify inputs of compile_dtree_tree, dtree_runtime.py:166-192). logits:
 * fp32 [depth][ld] draft logits (row d = depth d + 1); per row the top `topk`
 * tokens by (logit desc, token id asc) with log-probs logit - logsumexp(row)
 * (fp32); then the reference's best-first heap over cumulative log-probs
 * (fp64, its operation order and tuple tie-break) pops `budget` nodes. The
 * tree is written into `desc`: tokens = [root_token, nodes...], positions =
 * past_length + depth, parents, ancestor bitsets, num_nodes = 1 + nodes,
 * past_length, n_accepted = 0; rows past the tree cleared. tree_out
 * (optional, int32 [1 + 3 * DTREE_MAX_NODES]): node count, then node tokens,
 * depths and parents of nodes 1.. at offsets 1, 1 + DTREE_MAX_NODES,
 * 1 + 2 * DTREE_MAX_NODES. topk_ids / topk_logprobs (optional, [depth][topk]
 * int32 / fp32) receive the per-row top-k lists (row-wise argmax = column 0).
 * Limits: depth <= 18, topk <= min(127, vocab),
 * budget <= 127, vocab and ld multiples of 4, ceil(vocab / 8192) * topk <=
 * 4096. budget = 0 or depth = 0 gives the root alone (no logits read).
 */
size_t dtree_tree_build_workspace_bytes(int32_t depth, int32_t vocab, int32_t topk);
int dtree_tree_build(const float* logits, int32_t ld, int32_t depth, int32_t vocab, int32_t topk,
                     int32_t budget, int32_t root_token, int32_t past_length, void* workspace,
                     size_t workspace_bytes, DtreeStepDesc* desc, int32_t* tree_out, int32_t* topk_ids,
                     float* topk_logprobs, hipStream_t stream);

/*
 * Qwen3.5 GatedDeltaNet tree primitives (qwen35_tree_kernels.py:8-152, the
 * tree layer qwen35_tree.py:180-480), fp32, nodes in heap order (parent <
 * child, root parent -1), num_nodes <= DTREE_MAX_NODES.
 *
 * Tree causal conv1d + SiLU (tree_conv1d_kernel): x [T][C] conv inputs,
 * base_window [keep][C], weight [keep + 1][C] (newest tap last). Node t's
 * input rows are its parent's window (the base for the root) followed by
 * x[t]; out[t] = silu(sum_r rows[r] * weight[r]). windows ([T][keep][C],
 * optional) receives each node's window; NULL keeps evaluation lazy.
 */
int dtree_gdn_tree_conv(const float* x, const float* base_window, const float* weight, const int32_t* parents,
                        int32_t num_nodes, int32_t channels, int32_t keep, float* out, float* windows,
                        hipStream_t stream);
/*
 * Tree gated-delta recurrence (tree_gated_delta_kernel): q, k [T][Hk][Dk],
 * v [T][Hv][Dv], g (multiplicative decay) and beta [T][Hv], base state
 * [Hv][Dv][Dk]; value head h reads key head h / (Hv / Hk). Per node:
 * S = S_parent * g; S += ((v - S k) * beta) (outer) k; y[t] = S q.
 * states ([T][Hv][Dv][Dk], optional) receives every node's state; NULL keeps
 * the node states in LDS only (lazy). Dk in {32, 64, 128}.
 */
int dtree_gdn_tree_recurrence(const float* q, const float* k, const float* v, const float* g, const float* beta,
                              const float* state, const int32_t* parents, int32_t num_nodes, int32_t num_k_heads,
                              int32_t num_v_heads, int32_t head_k_dim, int32_t head_v_dim, float* y, float* states,
                              hipStream_t stream);
/*
 * Commit of an accepted root path (commit_qwen35_tree_path,
 * qwen35_tree.py:708-732): window (optional) becomes the last keep rows of
 * (window ++ x[path]) and state (optional) the path's replayed state, both in
 * place. path / path_len are device pointers (DtreeStepDesc.accepted /
 * n_accepted), so a captured graph can run it after dtree_accept_walk.
 */
int dtree_gdn_commit(const float* x, float* window, int32_t channels, int32_t keep, const float* q, const float* k,
                     const float* v, const float* g, const float* beta, float* state, const int32_t* path,
                     const int32_t* path_len, int32_t num_k_heads, int32_t num_v_heads, int32_t head_k_dim,
                     int32_t head_v_dim, hipStream_t stream);

/*
 * Qwen3.5 GatedDeltaNet layer of the verify step (qwen35_tree.py:329-480 with
 * the batched-kernel body :180-327), split into four launches that read the
 * node count, parents and accepted path from the device step descriptor:
 *
 *  proj (fp32 [rows][ld_proj]) is the fused input projection of the
 *  RMS-normalised hidden state: columns [conv input C = 2*Hk*Dk + Hv*Dv |
 *  z (Hv*Dv) | b (Hv) | a (Hv)] (in_proj_qkv, in_proj_z, in_proj_b, in_proj_a).
 *
 *  dtree_gdn_layer_prep: tree conv1d + SiLU from the committed window, split
 *    q | k | v, q = rms_norm(q) / Dk, k = rms_norm(k) / sqrt(Dk) (eps 1e-6,
 *    :304-306), g = exp(-exp(A_log) softplus(a + dt_bias)), beta = sigmoid(b)
 *    (:307-308) -> q, k [rows][Hk][Dk], v [rows][Hv][Dv], g, beta [rows][Hv].
 *  dtree_gdn_layer_recurrence: tree gated-delta recurrence from the committed
 *    state -> y [rows][Hv][Dv]; node states stay in LDS (lazy).
 *  dtree_gdn_layer_gated_norm: out = rms_norm(y) * norm_w * silu(z) per value
 *    head (:322) as bf16 [hi, lo] (out_lo optional) for out_proj; rows >= L zero.
 *  dtree_gdn_layer_commit: commit_qwen35_tree_path (:708-732) for this layer:
 *    replays desc->accepted[0 .. n_accepted) on window and state (in place,
 *    or into window_out / state_out).
 *
 * The per-node buffers (proj, q, k, v, g, beta) must stay untouched between
 * the layer's prep and its commit. Compiled for Dk = Dv = 128.
 */
typedef struct DtreeGdnArgs {
  const DtreeStepDesc* desc;
  int32_t rows_padded;               /* node capacity of the per-node buffers (<= 128) */
  int32_t num_k_heads, num_v_heads, head_k_dim, head_v_dim;
  int32_t conv_keep;                 /* conv kernel size - 1 */
  const float* proj; int32_t ld_proj;
  float* window;                     /* [conv_keep][C] committed conv window */
  const float* conv_w;               /* [conv_keep + 1][C], newest tap last */
  const float* A_log; const float* dt_bias;  /* [Hv] */
  float* state;                      /* [Hv][Dv][Dk] committed state */
  float* q; float* k; float* v; float* g; float* beta;
  float* y;                          /* [rows][Hv][Dv] */
  const uint16_t* norm_w; float eps; /* gated RMSNorm weight [Dv] (bf16) */
  uint16_t* out; uint16_t* out_lo; int32_t out_layout; int32_t ld_out;
  /* Commit destination (dtree_gdn_layer_commit / dtree_gdn_layers_commit):
   * the new window and state go to window_out / state_out, read from window /
   * state. NULL (both) commits in place. A second buffer lets a verify step
   * run its commit without touching the state it started from, so it can be
   * replayed (the host flips the two buffers when it keeps the commit). */
  float* window_out; float* state_out;
} DtreeGdnArgs;

size_t dtree_gdn_args_bytes(void);
/* Host check of a tree for the recurrence (the reference's tree kernel,
 * qwen35_tree_kernels.py:8-83, takes any tree): trees of more than 32 nodes
 * run depth first with a register stack of the states of branching nodes,
 * which holds at most DTREE_GDN_MAX_NESTED_BRANCHES nested ones; DTREE_E_TREE
 * for a tree beyond that (or malformed parents), else DTREE_OK. Trees of up
 * to 32 nodes always pass. The device tree build (depth <= 18) never exceeds
 * it; call this for caller-built trees before the recurrence. */
#define DTREE_GDN_MAX_NESTED_BRANCHES 31
int dtree_gdn_tree_check(const int32_t* parents, int32_t num_nodes);
int dtree_gdn_layer_prep(const DtreeGdnArgs* args, hipStream_t stream);
int dtree_gdn_layer_recurrence(const DtreeGdnArgs* args, hipStream_t stream);
/* dtree_gdn_layer_prep followed by dtree_gdn_layer_recurrence (the same
 * outputs: q, k, v, g, beta and y), as one launch when rows_padded <= 32, the
 * head dims are 128 and proj (ld_proj % 4 == 0), conv_w, window, state, q and
 * k are 16-byte aligned; otherwise the two launches. Replaces
 * qwen35_tree.py:199-320 between the projections and the gated norm. */
int dtree_gdn_layer_prep_recurrence(const DtreeGdnArgs* args, hipStream_t stream);
int dtree_gdn_layer_gated_norm(const DtreeGdnArgs* args, hipStream_t stream);
int dtree_gdn_layer_commit(const DtreeGdnArgs* args, hipStream_t stream);
/* dtree_gdn_layer_commit for num_layers layers (args[0 .. num_layers)) in one
 * launch: the layers of one verify step share desc (the accepted path),
 * rows_padded, heads, conv_keep and ld_proj; each has its own proj, window,
 * state, k, v, g and beta. Replaces the per-layer loop of
 * commit_qwen35_tree_path (qwen35_tree.py:708-732). */
int dtree_gdn_layers_commit(const DtreeGdnArgs* args, int32_t num_layers, hipStream_t stream);
/* One GatedDeltaNet layer over a causal chain of num_tokens prompt tokens that
 * continue the committed window and state (prompt prefill): conv + SiLU and
 * the q / k / v / g / beta prep, the recurrence (y per token; the final state
 * and the last conv_keep conv inputs become the committed state and window),
 * and the gated RMSNorm into out / out_lo. Replaces GatedDeltaNet.__call__
 * over the prompt (custom_qwen35_model.py:823-878, reached from
 * forward_dflash, custom_qwen35_model.py:961-1097, through
 * Qwen35TargetAdapter.forward_with_hidden_states, adapters.py:290-307).
 * desc is unused; rows_padded is the row capacity of q, k, v, g, beta, y,
 * proj and out (num_tokens <= rows_padded). */
int dtree_gdn_layer_chain(const DtreeGdnArgs* args, int32_t num_tokens, hipStream_t stream);

/* Convert a row-major [n][k] bf16 matrix to DTREE_W_TILED (n % 32 == 0,
 * k % 64 == 0; src and dst must not overlap). */
int dtree_tile_weight(const uint16_t* src, uint16_t* dst, int32_t n, int32_t k, hipStream_t stream);
/* The same to DTREE_W_TILED_F16: the elements become fp16 (round to nearest
 * even; exact from 2^-17 to 65504 in magnitude, saturating at +-65504). The
 * weight load of a bf16 checkpoint for the fp16 GEMM path; also the tiling of
 * bf16 caller rows (LM-head inputs, the drafter's target hidden rows) for it. */
int dtree_tile_weight_f16(const uint16_t* src, uint16_t* dst, int32_t n, int32_t k, hipStream_t stream);

/* HIP graph capture of a launch sequence (stands in for the mx.compile region
 * of qwen3_tree.py:38 and the per-step eval of dtree_runtime.py:480). */
int dtree_graph_begin(hipStream_t stream);
int dtree_graph_end(hipStream_t stream, void** graph_exec);
int dtree_graph_launch(void* graph_exec, hipStream_t stream);
int dtree_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif
#endif /* DTREE_HIP_H */
