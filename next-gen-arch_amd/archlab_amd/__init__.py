"""MI355X-native 2-simplicial (trilinear) sliding-window attention.

Forward-path drop-in for archlab's ``simplicial_attention`` and
``simplicial_paged_attention`` (and the entry points that compute the same
attention: the contiguous / packed decodes, the deterministic form, the determinant
scores and the TileLang signatures); the kernels are hand-written gfx950 HIP behind the C ABI
of ``include/simplicial_mi355x.h``.
"""

from .architectures.simplicial_attention import (  # noqa: F401
    simplicial_attention,
    simplicial_varlen_attention,
    validate_inputs,
)
from .architectures.simplicial_decode import simplicial_decode_attention  # noqa: F401
from .architectures.simplicial_determinant import (  # noqa: F401
    determinant_operands,
    determinant_simplicial_attention,
    oriented_determinant_simplicial_attention,
)
from .architectures.simplicial_deterministic import deterministic_simplicial_attention  # noqa: F401
from .architectures.simplicial_packed import (  # noqa: F401
    packed_simplicial_attention,
    packed_simplicial_decode,
)
from .architectures.simplicial_paged import simplicial_paged_attention  # noqa: F401
from .architectures.tilelang_attention import tilelang_attention, tilelang_decode  # noqa: F401
from .serving import token_layout  # noqa: F401

__all__ = [
    "simplicial_attention",
    "simplicial_varlen_attention",
    "simplicial_paged_attention",
    "validate_inputs",
    "token_layout",
    "simplicial_decode_attention",
    "deterministic_simplicial_attention",
    "packed_simplicial_attention",
    "packed_simplicial_decode",
    "tilelang_attention",
    "tilelang_decode",
    "determinant_operands",
    "determinant_simplicial_attention",
    "oriented_determinant_simplicial_attention",
]
