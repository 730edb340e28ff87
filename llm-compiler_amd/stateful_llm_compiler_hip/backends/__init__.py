"""gfx950 kernel wrappers (drop-ins for the reference's backends/triton_*)."""

from .hip_attention import (
    hip_decode_attention,
    hip_decode_attention_noalloc,
    hip_rope_decode_attention,
)
from .hip_fused import (
    hip_linear_residual,
    hip_norm_linear_group,
    hip_norm_linear_swiglu,
    hip_rope_kv_store,
)
from .hip_kv import hip_kv_store
from .hip_paged import hip_paged_decode_attention, hip_paged_kv_store, hip_paged_rope_decode_attention
from .hip_linear import hip_linear
from .hip_ops import (
    hip_add,
    hip_argmax,
    hip_embedding,
    hip_kv_advance,
    hip_rope_table,
    hip_swiglu,
)
from .hip_prefill_attention import hip_prefill_attention, hip_prefill_mask_tiles
from .hip_rmsnorm import hip_rms_norm
from .hip_rope import hip_rope

__all__ = [
    "hip_add",
    "hip_argmax",
    "hip_embedding",
    "hip_kv_advance",
    "hip_rope_table",
    "hip_swiglu",
    "hip_decode_attention",
    "hip_decode_attention_noalloc",
    "hip_rope_decode_attention",
    "hip_linear_residual",
    "hip_norm_linear_group",
    "hip_norm_linear_swiglu",
    "hip_rope_kv_store",
    "hip_kv_store",
    "hip_paged_decode_attention",
    "hip_paged_kv_store",
    "hip_paged_rope_decode_attention",
    "hip_linear",
    "hip_prefill_attention",
    "hip_prefill_mask_tiles",
    "hip_rms_norm",
    "hip_rope",
]
