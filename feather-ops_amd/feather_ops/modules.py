"""Class swaps that route a loaded module's `forward` through the gfx950 kernels.

Drop-in for the reference's `feather_ops/modules.py:21-47`. `relabelled_class(cls, mixin)` builds (once per
pair) a subclass whose MRO is `mixin` then `cls`; `relabel_modules` assigns it as the `__class__` of the
chosen instances of a model that is already built and loaded. Nothing else about an instance changes: its
parameters, buffers, submodule names and `state_dict` keys stay as they were. The caller decides which
instances qualify (`accept`) and what the mixin's `forward` does; `ScaledMMLinear` below is the mixin for
`nn.Linear` on this path.
"""

from collections.abc import Callable

import torch
from torch import nn

# (original class, mixin) -> the relabelled class, so every relabel of the same pair yields one type object.
_CLASS_CACHE: dict[tuple[type, type], type] = {}


def relabelled_class(cls: type, mixin: type) -> type:
    """The cached subclass `Feather<cls>` of `(mixin, cls)`, i.e. with `mixin` ahead of `cls` in the MRO.

    It keeps `cls.__qualname__` and lives in this module, so `type(module)` is stable across calls,
    models and deep copies, and `isinstance(module, cls)` still holds.
    """
    try:
        return _CLASS_CACHE[(cls, mixin)]
    except KeyError:
        pass
    new_cls = type("Feather" + cls.__name__, (mixin, cls), {"__module__": __name__, "__qualname__": cls.__qualname__})
    _CLASS_CACHE[(cls, mixin)] = new_cls
    return new_cls


def relabel_modules(root: nn.Module, mixin: type, accept: Callable[[nn.Module], bool]) -> int:
    """Relabel every module under `root` (itself included) that `accept` approves; return how many changed.

    Modules that already carry `mixin` are skipped, so calling this twice is a no-op the second time.
    """
    changed = 0
    for module in root.modules():
        if isinstance(module, mixin):
            continue
        if accept(module):
            module.__class__ = relabelled_class(type(module), mixin)
            changed += 1
    return changed


_FP8_MAX = {torch.float8_e5m2: 57344.0, torch.float8_e4m3fn: 448.0}


class ScaledMMLinear:
    """Mixin for `nn.Linear` (via `relabel_modules`): `forward` runs the fp8 scaled matmul on a quantized
    copy of the weight. Not in the reference, which leaves the Linear to its consumers; this is the
    consumer-facing drop-in on top of `prepack_transpose`.

    `quantize_weight_` (called by `to_scaled_mm_linear`) fills two non-persistent buffers, so `state_dict`
    keys and values are unchanged: `weight_fp8` `[K_pad/16, N, 16]` and `weight_scale` (one fp32 value per
    tensor, or N per output channel). Inputs are fp16 or bf16 `[..., in_features]`; the output has the
    input's dtype. The weight is frozen; gradients reach the input and the bias (computed in fp32 on the
    dequantized weight), so the layer can sit under trainable adapters.
    """

    def quantize_weight_(self, fp8_dtype: torch.dtype = torch.float8_e5m2, per_channel: bool = False) -> None:
        from .scaled_mm import prepack_transpose

        w = self.weight.detach().float()
        amax = w.abs().amax(dim=1) if per_channel else w.abs().max().reshape(1)
        scale = torch.where(amax > 0, amax / _FP8_MAX[fp8_dtype], torch.ones_like(amax))
        wq = (w / (scale[:, None] if per_channel else scale)).to(fp8_dtype)
        self.register_buffer("weight_fp8", prepack_transpose(wq), persistent=False)
        self.register_buffer("weight_scale", scale.contiguous() if per_channel else scale.reshape(()),
                             persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bias = None if self.bias is None else self.bias.to(x.dtype)
        needs_grad = torch.is_grad_enabled() and (x.requires_grad or (bias is not None and bias.requires_grad))
        if needs_grad or torch.compiler.is_compiling():
            return _scaled_mm_linear(x, self.weight_fp8, self.weight_scale, bias)
        # Eager inference: the same computation without the custom op's Python dispatch (~7 us per call).
        return _linear_forward(x, self.weight_fp8, self.weight_scale, bias)


def _linear_forward(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale: torch.Tensor,
                    bias: torch.Tensor | None) -> torch.Tensor:
    """`[..., K]` -> `[..., N]` in x's dtype through `scaled_mm_hip`."""
    from .scaled_mm import scaled_mm_hip

    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.clone(memory_format=torch.contiguous_format)  # the kernel reads 16-byte-aligned rows
    y = scaled_mm_hip(x2, weight_fp8, weight_scale, bias, x.dtype)
    return y.reshape(*x.shape[:-1], y.shape[-1])


@torch.library.custom_op("feather_ops::scaled_mm_linear", mutates_args=())
def _scaled_mm_linear(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale: torch.Tensor,
                      bias: torch.Tensor | None) -> torch.Tensor:
    """ScaledMMLinear's forward as one opaque op (like `feather_ops::scaled_mm_auto`), so `torch.compile`
    traces neither the flattening nor the alignment check, and autograd has a formula for it."""
    return _linear_forward(x, weight_fp8, weight_scale, bias)


@_scaled_mm_linear.register_fake
def _(x: torch.Tensor, weight_fp8: torch.Tensor, weight_scale: torch.Tensor,
      bias: torch.Tensor | None) -> torch.Tensor:
    return x.new_empty((*x.shape[:-1], weight_fp8.shape[1]))


def _linear_setup_context(ctx, inputs, output) -> None:
    x, weight_fp8, weight_scale, bias = inputs
    ctx.save_for_backward(weight_fp8, weight_scale)
    ctx.x_shape, ctx.x_dtype = x.shape, x.dtype
    ctx.bias_dtype = None if bias is None else bias.dtype


def _linear_backward(ctx, grad: torch.Tensor):
    """Gradients for the activations and the bias (the fp8 weight is frozen): dX = dY @ (Wq * scale)^T in
    fp32 on the dequantized weight, dbias = the column sums of dY."""
    weight_fp8, weight_scale = ctx.saved_tensors
    k = ctx.x_shape[-1]
    chunks, n, _ = weight_fp8.shape
    w = weight_fp8.permute(0, 2, 1).reshape(chunks * 16, n)[:k].float() * weight_scale.float()  # [K, N]
    g = grad.reshape(-1, n).float()
    grad_x = (g @ w.t()).to(ctx.x_dtype).reshape(ctx.x_shape)
    grad_bias = None if ctx.bias_dtype is None else g.sum(0).to(ctx.bias_dtype)
    return grad_x, None, None, grad_bias


_scaled_mm_linear.register_autograd(_linear_backward, setup_context=_linear_setup_context)


def to_scaled_mm_linear(root: nn.Module, fp8_dtype: torch.dtype = torch.float8_e5m2, per_channel: bool = False,
                        accept: Callable[[nn.Module], bool] | None = None) -> int:
    """Relabel the `nn.Linear` modules under `root` (those `accept` approves, by default every Linear whose
    out_features is a multiple of 8 and in_features of 16, the kernel's contract) as `ScaledMMLinear` and
    quantize their weights; return how many changed."""
    def default_accept(module: nn.Module) -> bool:
        return isinstance(module, nn.Linear) and module.out_features % 8 == 0 and module.in_features % 16 == 0

    count = relabel_modules(root, ScaledMMLinear, accept or default_accept)
    for module in root.modules():
        if isinstance(module, ScaledMMLinear) and not hasattr(module, "weight_fp8"):
            module.quantize_weight_(fp8_dtype, per_channel)
    return count
