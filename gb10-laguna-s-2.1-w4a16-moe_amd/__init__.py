"""MI355X (gfx950) W4A16 grouped-expert MoE path.

Drop-in for the reference's ``kernels`` package
(vladimir-voinea/gb10-laguna-s-2.1-w4a16-moe, kernels/__init__.py:3): the same
exported names, backed by hand-written HIP kernels behind a C ABI
(include/w4a16_moe.h).
"""

from .w4a16_moe import (  # noqa: F401
    BLOCK_K,
    BLOCK_M,
    BLOCK_N,
    dropped_pairs,
    fused_experts_w4a16,
    fused_experts_w4a16_profiled,
    is_repacked,
    moe_align_block_size,
    moe_align_block_size_full,
    release_graph_workspaces,
    repack_weights,
    workspace_tensor,
)
from .routing import router_topk_softmax  # noqa: F401
from .checkpoint import (  # noqa: F401
    CheckpointError,
    MoELayerWeights,
    W4A16MoELayer,
    list_moe_layers,
    load_moe_layer,
    save_moe_layer,
)
from . import integration  # noqa: F401
from . import tuning  # noqa: F401
from .tuning import Tuning  # noqa: F401

__all__ = ["fused_experts_w4a16", "repack_weights", "moe_align_block_size", "is_repacked",
           "router_topk_softmax", "load_moe_layer", "save_moe_layer", "list_moe_layers",
           "W4A16MoELayer", "integration", "tuning", "Tuning"]
