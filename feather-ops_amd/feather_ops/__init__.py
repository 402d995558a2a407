"""feather_ops for MI355X (gfx950): fp16/bf16 x fp8 scaled matmul on hand-written CDNA4 kernels.

Import order mirrors the reference's `feather_ops/__init__.py:1-3`: torch first, then the native
extension, which registers `torch.ops.feather_ops.*`.
"""

import torch  # noqa: F401  torch's libraries must be loaded before the extension

from . import _lib

_lib.load()

from .convert import bf16_to_fp16  # noqa: E402
from .modules import ScaledMMLinear, relabel_modules, relabelled_class, to_scaled_mm_linear  # noqa: E402
from .scaled_mm import (  # noqa: E402
    prepack_b_for_scaled_mm,
    prepack_transpose,
    scaled_mm_hip,
    select_scaled_mm_config,
    select_scaled_mm_splits,
    set_weight_streaming,
    tile_shape,
)

__all__ = [
    "ScaledMMLinear",
    "bf16_to_fp16",
    "prepack_b_for_scaled_mm",
    "prepack_transpose",
    "relabel_modules",
    "relabelled_class",
    "scaled_mm_hip",
    "select_scaled_mm_config",
    "select_scaled_mm_splits",
    "set_weight_streaming",
    "tile_shape",
    "to_scaled_mm_linear",
]
