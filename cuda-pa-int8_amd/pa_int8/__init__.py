"""pa_int8 -- paged-attention decode for one AMD MI355X (gfx950).

FP16 and per-token INT8 KV decode kernels and an INT8 quantize + paged-cache
write kernel, hand-written in HIP, behind the C ABI of include/pa_mi355x.h
and a thin torch extension with the reference's op names.
"""

from .registry import (  # noqa: F401
    KIND,
    VARIANTS,
    VARIANTS_INT8,
    decode,
    decode_plan,
    paged_decode_attention,
    reshape_and_cache,
    reshape_and_cache_int8,
    reshape_and_cache_int8_static,
)
from .paged_cache import PagedKVCache  # noqa: F401
from ._loader import capi, ext  # noqa: F401
