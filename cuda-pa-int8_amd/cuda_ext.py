"""Drop-in for the reference's loader module name (tests/cuda_ext.py).

With ``cuda-pa-int8_amd/`` on ``sys.path``, ``from cuda_ext import VARIANTS,
VARIANTS_INT8`` resolves to the gfx950 kernels with the same call shapes.
Unlike the reference it compiles nothing at import: the library is built
in-tree beforehand.
"""

from pa_int8.registry import (  # noqa: F401
    VARIANTS,
    VARIANTS_INT8,
    paged_decode_attention,
)
