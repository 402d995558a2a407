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
