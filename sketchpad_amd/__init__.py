"""MI355X-native ragged-batch attention for rhi-zone/sketchpad's paged/flash attention path.

The product is the C-ABI library ``lib/libsketchpad_attn.so`` (include/sketchpad_attn.h) built
from the gfx950 HIP kernels under ``csrc/``, plus the C++ mirror of the reference's paged-cache
API under ``host/``. This package only binds the library for Python callers (tests, bench).
"""
from ._lib import (  # noqa: F401
    CacheLayout,
    SketchpadError,
    SP_BF16,
    SP_CAUSAL_BOTTOM_RIGHT,
    SP_CAUSAL_NONE,
    SP_CAUSAL_TOP_LEFT,
    SP_F16,
    SP_F32,
    alloc_decode_workspace,
    flash_attention,
    flash_attention_masked,
    kv_append,
    kv_gather,
    layout,
    load,
    paged_decode,
    paged_decode_workspace_size,
    paged_prefill,
    paged_prefill_workspace_size,
    alloc_paged_prefill_workspace,
    alloc_linear_workspace,
    alloc_polar_pools,
    linear,
    linear_weight_nk,
    linear_workspace_size,
    polar_compress,
    polar_decompress,
    polar_kv_append,
    polar_kv_export,
    polar_kv_gather,
    polar_paged_decode,
    polar_pool_bytes,
    polar_record_bytes,
    rope_kv_append,
    rope_tables,
    varlen_prefill,
)
