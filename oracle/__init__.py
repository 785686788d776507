"""CPU oracle for the DTree tree-verify step.

TEST INFRASTRUCTURE ONLY. This package is a plain numpy (fp32 / fp64)
restatement of the reference algorithm of DrHB/dtree-mlx for the verify
path. It exists to check the HIP implementation; it is never the thing
that is measured or shipped. Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it. The product
package (``dtree_hip``) must not import it and fails loudly when its
native library is missing.

Modules and what pins each of them (reference paths are relative to the
DrHB/dtree-mlx checkout):

- ``tree``   : best-first tree build (``dtree_runtime.py:82-163``), verify-input
  compile (``:166-192``), greedy walk (``:195-208``), lineages / depth groups
  (``qwen35_tree.py:41-55, 104-123``). Pinned by the reference tests'
  known-answer vectors (``tests/test_dtree_runtime.py``) and by a brute-force
  enumeration of rank tuples on tiny inputs.
- ``qwen3``  : Qwen3 tree block in fp32 (``qwen3_tree.py:22-163``), masked GQA
  SDPA, RoPE, RMSNorm, LM head + first-index argmax (``adapters.py:28-118,
  489-492``), KV compaction (``adapters.py:635-668``). Pinned by closed forms
  and special cases (chain tree == causal attention, star tree == prefix +
  self, L=1 == decode attention, RoPE vs complex rotation, fp64 re-evaluation,
  and a cross-check of the decoder layer against transformers' Qwen3).
- ``q4``     : MLX group-64 affine 4-bit format (``adapters.py:28-85``,
  ``api.py:46-54``). Pinned by known-answer nibble vectors and the grouped
  identity y = s (q . x) + b sum(x) per group.
- ``gdn``    : GatedDeltaNet tree conv1d / tree recurrence / commit
  (``qwen35_tree_kernels.py:8-152``, ``qwen35_tree.py:708-732``). Pinned by the
  reference kernel tests' seeded vectors, the path-window closed form, the
  chain decomposition and transformers' ``torch_recurrent_gated_delta_rule``.
- ``qwen35`` : Qwen3.5 hybrid tree forward + commit (``qwen35_tree.py:180-732``).
  Pinned end to end against transformers' Qwen3.5 text model: chain trees,
  per-node root-path forwards, and commit + next step.

Parity unpinned (MLX internals that only an MLX import could pin): the exact
rounding / accumulation order of ``mx.fast.scaled_dot_product_attention``,
``mx.fast.rms_norm``, ``nn.RoPE`` frequency arithmetic and
``mx.quantized_matmul``. Those are covered only through the 2e-2 relative
logit tolerance of the verify-step parity tests.
"""
