"""CPU-resident, HBM-streamed Llama-3.1-8B decode on MI355X (gfx950).

Same public names as the reference package (layer_streaming/__init__.py:
26-45); the device work runs on the hand-written kernels of
libcascade_hip.so (see ``layer_streaming._hip``), which must be built --
nothing here falls back to other device code.
"""

from .graph import DecodeGraph
from .llama31 import (
    LLAMA31_8B_MODEL_ID,
    Llama31Config,
    Llama31DecodeExecutor,
    SimpleKVCache,
)
from .plan import (
    Granularity,
    HostPlacement,
    ModelPlan,
    TensorSpec,
    TransferUnit,
    VocabPlan,
    build_llama31_8b_plan,
)
from .runtime import DoubleBufferRuntime, ResidentDeviceArena, ResidentTransformerRuntime
from .vocab import VocabStreamingRuntime, merge_topk
from .weight_store import (
    FullPinnedWeightStore,
    PinnedStagingWeightStore,
    WeightStoreMode,
    create_weight_store,
)

__all__ = [
    "DecodeGraph",
    "DoubleBufferRuntime",
    "FullPinnedWeightStore",
    "Granularity",
    "HostPlacement",
    "LLAMA31_8B_MODEL_ID",
    "Llama31Config",
    "Llama31DecodeExecutor",
    "ModelPlan",
    "PinnedStagingWeightStore",
    "ResidentDeviceArena",
    "ResidentTransformerRuntime",
    "SimpleKVCache",
    "TensorSpec",
    "TransferUnit",
    "VocabPlan",
    "VocabStreamingRuntime",
    "WeightStoreMode",
    "build_llama31_8b_plan",
    "create_weight_store",
    "merge_topk",
]
