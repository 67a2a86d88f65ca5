"""treemoe_spec_amd — MI355X (gfx950) implementation of TreeMoE-Spec's
verification hot path: op1 (tree-aware grouped MoE with op3 budget routing)
and op4 (greedy tree verify + paged KV commit).

Module layout mirrors the reference package:
  treemoe_spec_amd.kernels.op1_tree_moe   tree_moe_forward, route_experts, Routing, ...
  treemoe_spec_amd.kernels.op4_commit     fused_verify_commit, VerifyResult
  treemoe_spec_amd.kv_cache               PagedKVCache (page size configurable)
The GPU work lives in libtreemoe_amd.so (C ABI: include/treemoe_amd.h).
"""

__version__ = "0.1.0"

NUM_LAYERS = 32
NUM_EXPERTS = 8
TOP_K = 2
HIDDEN_DIM = 4096
INTERMEDIATE_DIM = 14336
VOCAB_SIZE = 32000
TREE_SIZE = 64
TREE_MAX_DEPTH = 6
