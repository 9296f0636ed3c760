"""MI355X-native algebraic attention and fused algebraic LM head.

Public entry points keep the reference's signatures:
``algebraic_amd.kernels.flash.flash_attention`` (src/algebraic/kernels/flash.py:763) and
``algebraic_amd.kernels.fused_head.fused_head`` (src/algebraic/kernels/fused_head.py:260).
"""

from .kernels.flash import flash_attention, make_variant  # noqa: F401
from .kernels.fused_head import fused_head  # noqa: F401
