"""Relabelling an existing module class so that a kernel can take over its `forward`.

Drop-in for the reference's `feather_ops/modules.py:21-47`. A consumer loads a model with its own
machinery and then gives selected module instances a class that puts a mixin in front of the class they
already have. Parameters, buffers, module names and `state_dict` keys are untouched (only `__class__`
changes), so this can run after a checkpoint is loaded. Which classes may be relabelled and what the
mixin's `forward` does is the consumer's policy, passed in as `accept` and `mixin`.
"""

from collections.abc import Callable

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
