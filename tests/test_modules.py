"""Relabel semantics (reference tests/test_conv3x3_module.py:210-238), restated on nn.Linear. CPU only."""

import copy

import torch
from torch import nn

from feather_ops.modules import relabel_modules, relabelled_class


class _CountingMixin:
    def forward(self, input):
        self.calls = getattr(self, "calls", 0) + 1
        return super().forward(input)


def test_relabel_modules_is_idempotent_and_transparent():
    torch.manual_seed(0)
    root = nn.Sequential(nn.Linear(8, 16), nn.ReLU(), nn.Linear(16, 4))
    state_before = list(root.state_dict().keys())
    params_before = dict(root.named_parameters())
    x = torch.randn(3, 8)
    expected = root(x)

    patched = relabel_modules(root, _CountingMixin, lambda m: isinstance(m, nn.Linear) and m.out_features == 16)
    assert patched == 1
    assert isinstance(root[0], _CountingMixin) and isinstance(root[0], nn.Linear)
    assert not isinstance(root[2], _CountingMixin)
    assert type(root[0]).__name__ == "FeatherLinear"
    assert type(root[0]).__qualname__ == nn.Linear.__qualname__
    assert list(root.state_dict().keys()) == state_before
    assert dict(root.named_parameters()) == params_before
    assert torch.equal(root(x), expected)
    assert root[0].calls == 1

    assert relabel_modules(root, _CountingMixin, lambda m: isinstance(m, nn.Linear) and m.out_features == 16) == 0
    assert type(root[0]) is relabelled_class(nn.Linear, _CountingMixin)


def test_relabel_modules_leaves_unapproved_subclasses_alone():
    class CustomLinear(nn.Linear):
        def forward(self, input):
            return super().forward(input) * 2

    root = nn.Sequential(CustomLinear(4, 4), nn.Linear(4, 4))
    assert relabel_modules(root, _CountingMixin, lambda m: type(m) is nn.Linear) == 1
    assert type(root[0]) is CustomLinear


def test_relabelled_class_survives_deepcopy():
    root = nn.Sequential(nn.Linear(4, 4))
    relabel_modules(root, _CountingMixin, lambda m: isinstance(m, nn.Linear))
    clone = copy.deepcopy(root)
    assert type(clone[0]) is type(root[0]) is relabelled_class(nn.Linear, _CountingMixin)


# ---- the ScaledMMLinear drop-in (construction and quantization on the CPU; its forward is a GPU test) -------

def test_prepack_transpose_equals_prepack_of_the_transpose():
    """prepack_transpose([N, K]) == prepack_b_for_scaled_mm([K, N]) bit for bit, ragged K included."""
    from feather_ops.scaled_mm import prepack_b_for_scaled_mm, prepack_transpose

    g = torch.Generator().manual_seed(0)
    for n, k in [(8, 16), (24, 200), (136, 384), (40, 1000)]:
        codes = torch.randint(0, 256, (n, k), generator=g, dtype=torch.uint8)
        w = codes.view(torch.float8_e5m2)
        got = prepack_transpose(w).view(torch.uint8)
        want = prepack_b_for_scaled_mm(w.t().contiguous()).view(torch.uint8)
        assert got.shape == (-(-k // 128) * 8, n, 16)
        assert torch.equal(got, want)


def test_to_scaled_mm_linear_relabels_quantizes_and_keeps_the_state_dict():
    from feather_ops.modules import ScaledMMLinear, to_scaled_mm_linear

    torch.manual_seed(1)
    root = nn.Sequential(nn.Linear(64, 32), nn.GELU(), nn.Linear(32, 12), nn.Linear(12, 48, bias=False))
    keys = list(root.state_dict().keys())
    values = {k: v.clone() for k, v in root.state_dict().items()}
    assert to_scaled_mm_linear(root) == 1            # 32 -> 12 has N % 8 != 0 and 12 -> 48 K % 16 != 0
    assert isinstance(root[0], ScaledMMLinear) and not isinstance(root[2], ScaledMMLinear)
    assert list(root.state_dict().keys()) == keys
    assert all(torch.equal(root.state_dict()[k], values[k]) for k in keys)
    assert root[0].weight_fp8.shape == (8, 32, 16) and root[0].weight_fp8.dtype == torch.float8_e5m2
    assert root[0].weight_scale.shape == () and root[0].weight_scale.dtype == torch.float32
    assert to_scaled_mm_linear(root) == 0            # idempotent


def test_scaled_mm_linear_quantization_recipe():
    """Per tensor: scale = max|W| / 57344, Wq = e5m2(W / scale); per channel: one scale per output row; a
    zero row gets scale 1; e4m3fn uses 448. The packed weight decodes back to Wq."""
    from feather_ops.modules import to_scaled_mm_linear
    from feather_ops.scaled_mm import prepack_transpose

    torch.manual_seed(2)
    lin = nn.Linear(128, 16)
    with torch.no_grad():
        lin.weight[3] = 0
    w = lin.weight.detach().clone()
    to_scaled_mm_linear(lin, torch.float8_e5m2, per_channel=False)
    scale = w.abs().max() / 57344
    assert torch.equal(lin.weight_scale, scale)
    assert torch.equal(lin.weight_fp8.view(torch.uint8),
                       prepack_transpose((w / scale).to(torch.float8_e5m2)).view(torch.uint8))

    lin2 = nn.Linear(128, 16)
    with torch.no_grad():
        lin2.weight.copy_(w)
    to_scaled_mm_linear(lin2, torch.float8_e4m3fn, per_channel=True)
    amax = w.abs().amax(dim=1)
    col = torch.where(amax > 0, amax / 448, torch.ones_like(amax))
    assert lin2.weight_scale.shape == (16,) and lin2.weight_scale[3] == 1
    assert torch.equal(lin2.weight_scale, col)
    assert torch.equal(lin2.weight_fp8.view(torch.uint8),
                       prepack_transpose((w / col[:, None]).to(torch.float8_e4m3fn)).view(torch.uint8))
