"""bf16 -> fp16 conversion on the GPU (drop-in for the reference's `feather_ops/convert.py:24-34`).

Same contract as the reference: `x` is a contiguous bfloat16 tensor with an even number of elements,
and the result is a new float16 tensor of the same shape, converted with round-toward-zero (the
reference's `v_cvt_pkrtz_f16_f32`): exact for every bf16 value inside fp16's normal range, finite
overflow saturates to +-65504. The kernel is hand-written HIP (`csrc/convert.hip`), not Triton.
"""

import torch

from . import _lib


def bf16_to_fp16(x: torch.Tensor) -> torch.Tensor:
    assert x.dtype == torch.bfloat16
    assert x.is_contiguous()
    assert x.numel() % 2 == 0
    _lib.require_native()
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    torch.ops.feather_ops.bf16_to_fp16.default(x, out)
    return out
