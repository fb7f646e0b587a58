"""MI355X (gfx950) backend for the Kimi Delta Attention operators.

Mirrors the operator surface of pablo-reyes8/kimi-k3-pytorch ``src/kda``
(src/kda/__init__.py:1-25): ``chunkwise_kda``, ``recurrent_kda``,
``ut_transform``, ``KDAOperatorOutput``, ``UTTransformOutput`` and
``KDAState``, plus the fused stages around the operator in ``kda.fused`` and the
whole-cache reorder and clone in ``kda.cache``, and the layer composed from
them (the caller path of src/kda/kda.py:98-183) in ``kda.layer``.
All arithmetic runs in hand-written HIP kernels in ``libkda_mi355x.so``; see
include/kda_mi355x.h for the C ABI.
"""

from . import cache, fused, layer
from .chunkwise import chunkwise_kda
from .recurrent import KDAOperatorOutput, recurrent_kda
from .state import KDAState, ShortConvState
from .ut_transform import UTTransformOutput, ut_transform

__all__ = [
    "KDAOperatorOutput",
    "KDAState",
    "ShortConvState",
    "UTTransformOutput",
    "cache",
    "chunkwise_kda",
    "fused",
    "layer",
    "recurrent_kda",
    "ut_transform",
]
