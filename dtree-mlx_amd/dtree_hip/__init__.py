"""dtree_hip: MI355X (gfx950) DTree tree-verify step behind the dtree_mlx
runtime / target-adapter interface.

Host side is Python on PyTorch-ROCm (device memory, streams); every verify
computation runs in the hand-written HIP kernels of libdtree_hip.so, bound
through the C ABI in include/dtree_hip.h.
"""
from .adapters import (ADAPTERS, LoadedTargetModel, Qwen35TargetAdapter, Qwen35TreeModel, Qwen3TargetAdapter,
                       Qwen3TreeModel, adapter_for_model_type, load_target_model)
from .cache import PagedKVCache, Qwen35Cache
from .config import QWEN3_4B, QWEN35_4B, QWEN35_9B, Qwen35Config, Qwen3Config, tiny_qwen3, tiny_qwen35
from .dtree_runtime import (build_dtree_tree, compile_dtree_tree, dtree_generate, follow_verified_tree,
                            lazy_follow_tree_exact, sample_tokens)
from .engine import Qwen3TreeEngine, StepResult, ancestor_bitsets
from .qwen35_engine import Qwen35TreeEngine
from .weights import Qwen35Weights, Qwen3Weights

__all__ = [
    "ADAPTERS", "LoadedTargetModel", "PagedKVCache", "QWEN3_4B", "Qwen3Config", "Qwen3TargetAdapter",
    "Qwen3TreeEngine", "Qwen3TreeModel", "Qwen3Weights", "StepResult", "adapter_for_model_type",
    "ancestor_bitsets", "build_dtree_tree", "compile_dtree_tree", "dtree_generate", "follow_verified_tree",
    "lazy_follow_tree_exact", "load_target_model", "sample_tokens", "tiny_qwen3",
    "Qwen35TargetAdapter", "Qwen35TreeModel", "QWEN35_4B", "QWEN35_9B", "Qwen35Cache", "Qwen35Config", "Qwen35TreeEngine", "Qwen35Weights", "tiny_qwen35",
]
