"""Loading of the native code: `_C` (the torch library) and, through it, `libfeather_ops_gfx950.so`.

There is no fallback: if the extension is not built, importing `feather_ops` fails with the build
command, and the ops only have a CUDA (HIP) dispatch key, so CPU tensors are rejected by the dispatcher.
"""

import ctypes
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
LIBRARY = HERE / "libfeather_ops_gfx950.so"
EXTENSION = HERE / "_C.so"
BUILD_HINT = "build it with `make -C feather-ops_amd -j8` or `python -c 'import __graft_entry__ as g; g.build()'`"

_loaded = False


def load() -> None:
    """Import `_C`, which registers `torch.ops.feather_ops.*` and loads the HIP library."""
    global _loaded
    if _loaded:
        return
    if not EXTENSION.exists() or not LIBRARY.exists():
        raise ImportError(f"feather_ops native extension missing ({EXTENSION.name}, {LIBRARY.name}): {BUILD_HINT}")
    from . import _C  # noqa: F401  registers the feather_ops torch library

    _loaded = True


_c_library = None


def c_library() -> ctypes.CDLL:
    """The HIP library's C ABI through ctypes, for the entry points no torch op wraps (the handle is the one
    `_C` already loaded: the same file)."""
    global _c_library
    if _c_library is None:
        load()
        lib = ctypes.CDLL(str(LIBRARY))
        lib.feather_set_weight_streaming.restype = ctypes.c_int
        lib.feather_set_weight_streaming.argtypes = [ctypes.c_int]
        _c_library = lib
    return _c_library


def require_native() -> None:
    """Raise unless the HIP extension is loaded (the product path has no CPU fallback)."""
    if not _loaded:
        load()
