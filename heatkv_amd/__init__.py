"""heatkv_amd -- HeatKV's slab compaction + segmented attention on MI355X (gfx950).

Python operator surface (drop-in names of the reference module
real_pruning_fused_attention.py) over hand-written HIP kernels in
libheatkv.so; the static slab layout (offsets, offset tables, copy
descriptors) is computed on the host like the reference's.
"""

from .real_pruning_fused_attention import (  # noqa: F401
    attention_item_shape,
    attention_queries_per_item,
    fused_real_pruning_flat_segmented_attention,
    pack_flat_segments_kv,
    segmented_attention_plan,
)
from .slab_schedule import (  # noqa: F401
    SIDES_1M,
    SlabSchedule,
    build_slab_schedule,
    build_static_slot_schedule,
    scale_token_ranges,
)
from .policy import (  # noqa: F401
    ScaleSpecificPruningController,
    pruned_heads_for_budget,
    strict_pruning_schedule_for_budget_scale_specific,
    strict_removed_heads_by_scale_specific_for_budget,
)
from .enable import (  # noqa: F401
    METHOD_NAME,
    canonical_method,
    enable_real_pruning_scale_specific_fast,
    enable_real_pruning_scale_specific_fused_segmented,
)
from .phase_profile import (  # noqa: F401
    reset_real_pruning_fast_phase_profile,
    set_real_pruning_fast_phase_profile_enabled,
    snapshot_real_pruning_fast_phase_profile,
)

__version__ = "0.3.0"
