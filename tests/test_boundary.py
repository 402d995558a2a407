"""The C ABI and torch-op boundary, checked without a GPU.

The library must load and export every function include/feather_ops.h declares, refuse out-of-contract
calls before touching the device (it returns false and enqueues nothing), and the torch ops must not
accept CPU tensors (they are registered for the CUDA/HIP key only: no CPU fallback).
"""

import ctypes
import pathlib
import re

import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "feather_ops.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:bool|int64_t|int)\s+(\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    from feather_ops import _lib

    handle = ctypes.CDLL(str(_lib.LIBRARY))
    handle.launch_scaled_mm.restype = ctypes.c_bool
    handle.launch_scaled_mm.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_int] * 2 + \
        [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_void_p]
    for name in ("feather_bf16_to_fp16", "feather_widen_bf16"):
        getattr(handle, name).restype = ctypes.c_bool
        getattr(handle, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    handle.feather_prepack_b.restype = ctypes.c_bool
    handle.feather_prepack_b.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_void_p]
    handle.feather_scaled_mm_splitk.restype = ctypes.c_bool
    handle.feather_scaled_mm_splitk.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + \
        [ctypes.c_int] * 2 + [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_int] + \
        [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    handle.feather_scaled_mm_splitk_noalloc.restype = ctypes.c_bool
    handle.feather_scaled_mm_splitk_noalloc.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + \
        [ctypes.c_int] * 2 + [ctypes.c_bool] * 3 + [ctypes.c_int] * 5 + [ctypes.c_bool, ctypes.c_int, ctypes.c_void_p]
    handle.feather_set_weight_streaming.restype = ctypes.c_int
    handle.feather_set_weight_streaming.argtypes = [ctypes.c_int]
    handle.feather_splitk_workspace_bytes.restype = ctypes.c_int64
    handle.feather_splitk_workspace_bytes.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int] * 5 + \
        [ctypes.c_bool, ctypes.c_int]
    return handle


def test_library_exports_every_declared_symbol(lib):
    names = _declared()
    assert set(names) == {"launch_scaled_mm", "feather_bf16_to_fp16", "feather_widen_bf16", "feather_prepack_b",
                          "feather_scaled_mm_splitk", "feather_splitk_workspace_bytes",
                          "feather_scaled_mm_splitk_noalloc", "feather_set_weight_streaming"}
    for name in names:
        assert hasattr(lib, name), name


def test_weight_streaming_mode_round_trips(lib):
    """The C ABI's process-wide mode: -1 queries, 0/1/2 set and return the previous mode, anything else is
    refused (-1) and changes nothing; the Python wrapper maps the same modes to names."""
    import feather_ops

    first = lib.feather_set_weight_streaming(-1)
    assert first in (0, 1, 2)
    try:
        assert lib.feather_set_weight_streaming(0) == first
        assert lib.feather_set_weight_streaming(1) == 0
        assert lib.feather_set_weight_streaming(-1) == 1
        for bad in (3, -2, 99):
            assert lib.feather_set_weight_streaming(bad) == -1
            assert lib.feather_set_weight_streaming(-1) == 1
        assert lib.feather_set_weight_streaming(2) == 1
        assert feather_ops.set_weight_streaming() == "auto"
        assert feather_ops.set_weight_streaming("off") == "auto"
        assert lib.feather_set_weight_streaming(-1) == 0
        with pytest.raises(ValueError):
            feather_ops.set_weight_streaming("sometimes")
        assert feather_ops.set_weight_streaming("on") == "off"
    finally:
        lib.feather_set_weight_streaming(first)


@pytest.mark.parametrize("env,want", [(None, "auto"), ("0", "off"), ("1", "on"), ("2", "auto"), ("yes", "auto")])
def test_weight_streaming_mode_starts_from_the_environment(env, want):
    import os
    import subprocess
    import sys

    environ = {k: v for k, v in os.environ.items() if k != "FEATHER_OPS_WEIGHT_STREAMING"}
    if env is not None:
        environ["FEATHER_OPS_WEIGHT_STREAMING"] = env
    code = "import feather_ops; print(feather_ops.set_weight_streaming())"
    got = subprocess.run([sys.executable, "-c", code], env=environ, cwd=ROOT / "feather-ops_amd", check=True,
                         capture_output=True, text=True, timeout=300).stdout.split()[-1]
    assert got == want


# Fake, 16-byte aligned device addresses: every call below is refused before anything dereferences them.
A, B, S, BIAS, C = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
GOOD = dict(M=64, N=128, K=256)
TILE = (2, 2, 4, 4, 4, True)


def _call(lib, a=A, b=B, s=S, bias=BIAS, c=C, M=64, N=128, K=256, has_scale=1, has_bias=1, tile=TILE):
    return lib.launch_scaled_mm(a, b, s, bias, c, M, N, K, has_scale, has_bias, True, False, False, *tile, None)


@pytest.mark.parametrize("kwargs", [
    dict(tile=(3, 3, 3, 3, 3, True)),          # not instantiated (the reference's only false case)
    dict(tile=(2, 2, 4, 4, 4, False)),         # right numbers, wrong kernel family
    dict(N=100),                               # N % 8 != 0
    dict(K=40),                                # K % 16 != 0
    dict(K=0),
    dict(M=0),
    dict(a=A + 8),                             # misaligned
    dict(c=C + 2),
    dict(bias=BIAS + 2),
    dict(has_scale=1, s=None),
    dict(has_scale=2, s=S + 4),                # per-column scales must be 16-byte aligned
    dict(has_scale=2, s=None),
    dict(a=None),
    dict(M=1 << 20, K=1 << 11),                # a would be 4 GiB
])
def test_c_abi_refuses_out_of_contract_calls(lib, kwargs):
    assert _call(lib, **kwargs) is False


WS = 0x100000  # fake, 256-byte aligned workspace address


def _split(lib, tile=(2, 2, 4, 4, 4, True), splits=2, ws=WS, ws_bytes=1 << 30, M=64, N=128, K=256, c=C):
    return lib.feather_scaled_mm_splitk(A, B, S, BIAS, c, M, N, K, 1, 1, True, False, False, *tile, splits, ws,
                                        ws_bytes, None)


@pytest.mark.parametrize("kwargs", [
    dict(tile=(4, 1, 4, 1, 4, True)),      # right numbers, wrong kernel family: not instantiated
    dict(tile=(3, 3, 3, 3, 3, True)),      # not instantiated
    dict(splits=0),
    dict(splits=5),                        # K = 256 has 4 stages of 64
    dict(splits=5, tile=(4, 1, 8, 1, 4, False)),  # a streaming tile splits K = 256's 4 groups of 64
    dict(splits=33, K=4096, tile=(8, 1, 4, 1, 4, False)),
    dict(splits=33, K=4096),               # above the 32 maximum
    dict(ws=None),
    dict(ws=WS + 16),                      # workspace not 256-byte aligned
    dict(ws_bytes=1000),                   # workspace too small
    dict(c=C + 2),                         # the launch_scaled_mm contract still applies
])
def test_splitk_c_abi_refuses_out_of_contract_calls(lib, kwargs):
    assert _split(lib, **kwargs) is False


def _header_scratch_bytes() -> int:
    """FEATHER_NOALLOC_SCRATCH_BYTES as the public header defines it (a sum of decimal literals)."""
    m = re.search(r"#define\s+FEATHER_NOALLOC_SCRATCH_BYTES\s+\(([\d\s+]+)\)", HEADER.read_text())
    assert m, "include/feather_ops.h must define FEATHER_NOALLOC_SCRATCH_BYTES"
    return sum(int(term) for term in m.group(1).split("+"))


def test_header_scratch_size_is_the_librarys_refusal_threshold(lib):
    """The static array size the header promises C callers is exactly where the library starts refusing: a
    split launch needing FEATHER_NOALLOC_SCRATCH_BYTES of workspace is accepted, one needing more is not
    (both refused or accepted on the host, before any GPU call). The accepted launch is not made here; its
    size is only checked to sit at the threshold."""
    scratch = _header_scratch_bytes()
    assert scratch == 65536 + (64 << 20)
    tile = (2, 2, 4, 4, 4, True)   # 128 x 128 ring tile: 64 KiB of fp32 partials per tile and split
    # 1024 tiles x 1 x 64 KiB = exactly the partial area; the counters take the first 64 KiB
    assert lib.feather_splitk_workspace_bytes(2048, 4096, 2560, *tile, 2) == scratch
    # 8 more columns make 1056 tiles: past the array, refused before anything is enqueued
    assert lib.feather_splitk_workspace_bytes(2048, 4104, 2560, *tile, 2) > scratch
    assert lib.feather_scaled_mm_splitk_noalloc(A, B, S, BIAS, C, 2048, 4104, 2560, 1, 1, True, False, False,
                                                *tile, 2, None) is False
    # the Python heuristic keeps every split launch within the same array
    from feather_ops.scaled_mm import _SPLIT_MAX_PARTIAL_BYTES

    assert 65536 + _SPLIT_MAX_PARTIAL_BYTES == scratch


def test_noalloc_splitk_refuses_past_its_static_array_and_out_of_contract(lib):
    """feather_scaled_mm_splitk_noalloc refuses, before any GPU call, a launch whose workspace would exceed
    its static array (64 KiB + 64 MiB), and everything feather_scaled_mm_splitk refuses."""
    scratch = _header_scratch_bytes()
    tile = (2, 2, 4, 4, 4, True)

    def call(m, n, k, splits, c=C):
        return lib.feather_scaled_mm_splitk_noalloc(A, B, S, BIAS, c, m, n, k, 1, 1, True, False, False, *tile,
                                                    splits, None)

    assert lib.feather_splitk_workspace_bytes(4096, 4096, 2560, *tile, 8) > scratch
    assert call(4096, 4096, 2560, 8) is False            # 1024 tiles x 8 splits x 64 KiB
    assert lib.feather_splitk_workspace_bytes(2048, 4096, 2560, *tile, 2) == scratch   # 1024 x 64 KiB: fits
    assert lib.feather_splitk_workspace_bytes(2048, 4224, 2560, *tile, 2) > scratch
    assert call(2048, 4224, 2560, 2) is False            # 528 tiles x 2 splits: 32 workgroups over
    assert call(4096, 4096, 2560, 33) is False           # more than 32 splits
    assert call(64, 100, 256, 2) is False                # N % 8
    assert call(64, 128, 256, 2, c=C + 2) is False       # misaligned output


def test_splitk_workspace_bytes_match_the_python_formula(lib):
    from feather_ops.tiles import SCALED_MM_TILES, split_workspace_bytes

    for tile in SCALED_MM_TILES:
        for m, n, k in [(1, 8, 16), (67, 272, 304), (512, 5376, 5120), (4096, 3072, 3072)]:
            for splits in (0, 1, 2, 3, 8, 32, 33):
                want = lib.feather_splitk_workspace_bytes(m, n, k, *tile, splits)
                assert split_workspace_bytes(m, n, k, tile, splits) == want, (tile, m, n, k, splits)
    ws = lib.feather_splitk_workspace_bytes
    # 512 x 5376 with 128 x 128 tiles: the 64 KiB counter area, then 168 tiles x 3 fp32 partial tiles
    assert ws(512, 5376, 5120, 2, 2, 4, 4, 4, True, 3) == 65536 + 168 * 3 * 128 * 128 * 4
    # 16384 (tile, wave) counters at most: 4096 128 x 128 tiles of 4 waves fit, 4097 do not
    assert ws(4096, 16384, 256, 2, 2, 4, 4, 4, True, 2) > 0
    assert ws(4096, 16392, 256, 2, 2, 4, 4, 4, True, 2) == -1
    assert ws(4096, 16392, 256, 2, 2, 4, 4, 4, True, 1) == 0  # unsplit: no workspace
    # a 16 x 64 streaming tile: 84 x 2 tiles of 4 fragments, 16 x 64 fp32 partials per split
    assert ws(32, 5376, 5120, 8, 1, 4, 1, 4, False, 4) == 65536 + 168 * 4 * 16 * 64 * 4
    # streaming splits count 64-deep groups whatever unroll_k is: K = 256 has 4
    assert ws(16, 64, 256, 8, 1, 8, 1, 4, False, 4) > 0 and ws(16, 64, 256, 8, 1, 8, 1, 4, False, 5) == -1
    # 16384 (tile, fragment) counters: 4096 tiles of 4 fragments fit, 4097 do not
    assert ws(16, 4096 * 64, 256, 8, 1, 4, 1, 4, False, 2) > 0
    assert ws(16, 4096 * 64 + 64, 256, 8, 1, 4, 1, 4, False, 2) == -1
    assert ws(512, 5376, 5120, 4, 1, 4, 1, 4, True, 2) == -1  # no such ring tile


@pytest.mark.parametrize("name", ["feather_bf16_to_fp16", "feather_widen_bf16"])
def test_convert_c_abi_refuses_bad_arguments(lib, name):
    convert = getattr(lib, name)
    assert convert(A, C, -1, None) is False
    assert convert(A + 2, C, 16, None) is False
    assert convert(A, C + 8, 16, None) is False
    assert convert(None, C, 16, None) is False
    assert convert(A, C, 1 << 30, None) is False
    assert convert(A, C, 0, None) is True  # nothing to do, nothing enqueued


@pytest.mark.parametrize("args", [
    (B, C, 0, 64),            # K < 1
    (B, C, 128, 12),          # N % 8 != 0
    (B, C, 128, 0),
    (B + 4, C, 128, 64),      # b not 8-byte aligned
    (B, C + 8, 128, 64),      # b_prepacked not 16-byte aligned
    (None, C, 128, 64),
    (B, None, 128, 64),
    (B, C, 1 << 20, 1 << 12),  # prepacked weight 4 GiB
])
def test_prepack_c_abi_refuses_bad_arguments(lib, args):
    assert lib.feather_prepack_b(*args, None) is False


def test_prepack_falls_back_to_torch_permutation_off_gpu():
    """On CPU (and for shapes the kernel does not take) prepack is torch's own permutation of `b`."""
    from feather_ops import prepack_b_for_scaled_mm

    b = torch.arange(200 * 24, dtype=torch.int32).remainder(256).to(torch.uint8).view(200, 24)
    p = prepack_b_for_scaled_mm(b.view(torch.float8_e5m2)).view(torch.uint8)
    assert p.shape == (16, 24, 16)
    k = torch.arange(256).view(-1, 1)
    want = torch.zeros(256, 24, dtype=torch.uint8)
    want[:200] = b
    assert torch.equal(p[k // 16, torch.arange(24).view(1, -1), k % 16], want)


def test_torch_ops_are_registered_for_the_gpu_only():
    import feather_ops  # noqa: F401

    a = torch.zeros(16, 64, dtype=torch.float16)
    b = torch.zeros(8, 32, 16, dtype=torch.float8_e5m2)
    c = torch.empty(16, 32, dtype=torch.float16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.feather_ops.scaled_mm.default(a, b, None, None, c, 2, 2, 4, 4, 4, True)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.feather_ops.bf16_to_fp16.default(torch.zeros(8, dtype=torch.bfloat16), torch.empty(8, dtype=torch.float16))
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.feather_ops.prepack_b.default(torch.zeros(16, 8, dtype=torch.float8_e5m2),
                                                torch.empty(8, 8, 16, dtype=torch.float8_e5m2))
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.feather_ops.scaled_mm_splitk.default(a, b, None, None, c, torch.zeros(1 << 16, dtype=torch.uint8),
                                                       2, 2, 2, 4, 4, 4, True)


def test_scaled_mm_hip_has_no_cpu_fallback():
    from feather_ops import scaled_mm_hip

    a = torch.zeros(16, 64, dtype=torch.float16)
    b = torch.zeros(8, 32, 16, dtype=torch.float8_e5m2)
    with pytest.raises((NotImplementedError, RuntimeError)):
        scaled_mm_hip(a, b, None, None, torch.float16)


def test_heuristic_splits_k_on_underfilled_grids_with_long_k():
    """The split regime (fitted on the tile sweep): fewer 128 x 128 tiles than CUs and K >= 4096."""
    from feather_ops.scaled_mm import select_scaled_mm_config as pick
    from feather_ops.scaled_mm import select_scaled_mm_splits as splits

    def auto(m, n, k):
        tile = pick(m, n, k)
        return tile, splits(m, n, k, tile)

    assert auto(512, 5376, 5120) == ((2, 2, 4, 4, 4, 1), 3)     # 168 tiles -> 504 workgroups
    assert auto(1040, 1536, 6144) == ((1, 4, 4, 4, 2, 1), 2)    # 204 tiles of 64 x 128 (deep ring)
    # more than 256 64 x 128 tiles: the small-grid time model (measured best or within 5% of it)
    assert auto(256, 12288, 4096) == ((1, 4, 4, 4, 2, 1), 2)    # 384 tiles of 64 x 128 -> 768 workgroups
    assert auto(448, 6144, 8192) == ((1, 4, 4, 4, 2, 1), 3)     # 336 tiles -> 1008, the shallow ring
    assert auto(256, 12288, 8192) == ((2, 2, 4, 4, 4, 1), 4)    # 192 tiles of 128 x 128 -> 768, 3 per CU
    assert auto(2320, 1536, 6144) == ((2, 2, 4, 4, 4, 1), 2)    # 444 tiles of 64 x 128: 128 x 128 split
    assert auto(1040, 1024, 5120) == ((1, 4, 4, 4, 2, 1), 3)    # 72 tiles of 128 x 128: 64 x 128, 136 tiles
    assert auto(128, 8192, 5120) == ((1, 4, 4, 4, 2, 1), 4)
    # M > 768, a weight of a few MB: the 64 x 64 ring tile once it fills 3/4 of the CU slots
    assert auto(1000, 1000, 2560) == ((2, 2, 4, 2, 2, 1), 2)    # 256 tiles -> 512 workgroups
    assert auto(1536, 1024, 1536) == ((2, 2, 4, 2, 2, 1), 1)    # 384 tiles, 24 stages: unsplit
    assert auto(1024, 1280, 1280) == ((4, 1, 4, 1, 4, 0), 1)    # 320 tiles fill 5/8: streaming
    assert auto(768, 1024, 2048) == ((4, 1, 4, 1, 4, 0), 1)     # M <= 768: streaming
    assert auto(192, 1536, 6144) == ((2, 2, 4, 2, 2, 0), 1)     # too few tiles to split: the 32-row tile's round
    # 64 < M <= 192: streaming below a 24 MiB weight, the split 64 x 128 ring tile from there on
    assert auto(192, 4096, 4096) == ((4, 1, 4, 1, 4, 0), 1)     # 16 MiB, 64 tiles of 128 x 128
    assert auto(128, 4096, 14336) == ((1, 4, 4, 4, 2, 1), 8)    # 56 MiB, 32 tiles: 64 tiles x 8 = 512
    assert auto(128, 5120, 5120) == ((1, 4, 4, 4, 2, 1), 3)     # 80 tiles: 240 workgroups, not 400
    assert auto(256, 4096, 4096) == ((1, 4, 4, 4, 2, 1), 4)     # 256 MiB of re-reads: the ring
    # bf16 activations: the ring from 288 MiB of re-reads, the 64 x 128 tile split for up to 768 workgroups,
    # and no 64 x 64 ring for M > 768 with a small weight
    bf = torch.bfloat16

    def auto_bf16(m, n, k):
        tile = pick(m, n, k, bf)
        return tile, splits(m, n, k, tile, bf)

    assert auto_bf16(256, 4096, 4096) == ((4, 1, 4, 1, 4, 0), 1)
    assert auto_bf16(128, 8192, 5120) == ((1, 4, 4, 4, 2, 1), 4)   # 320 MiB; 80 stages: at most 5 splits
    assert auto_bf16(1040, 1536, 6144) == ((1, 4, 4, 4, 2, 1), 3)  # 204 tiles x 3 = 612
    assert auto_bf16(1000, 1000, 2560) == ((4, 1, 4, 1, 4, 0), 1)
    assert auto(1040, 1536, 6144)[1] == 2                          # fp16: two per CU at most
    assert auto(4096, 12288, 3072) == ((2, 2, 4, 8, 8, 1), 1)   # full grids never split (C3: the wide tile)
    assert auto(16, 14336, 4096)[1] == 1
    # skinny M, long K, fewer than 171 16 x 64 tiles: a streaming tile split to at most one workgroup per CU
    # (the 16 x 32 tile for M <= 12, the 16 x 64 tile with 4 K slices above), each K range 3072 deep or more
    assert auto(2, 2048, 16384) == ((8, 1, 4, 1, 2, 0), 4)      # 64 tiles of 16 x 32 -> 256 workgroups
    assert auto(6, 4096, 14336) == ((8, 1, 4, 1, 2, 0), 2)      # 128 tiles of 16 x 32 -> 256 workgroups
    assert auto(1, 4096, 28672) == ((8, 1, 4, 1, 2, 0), 2)
    # except M <= 4 with 192-256 blocks of 16 x 16 and K <= 16384: that tile unsplit (three fetches in flight)
    assert auto(2, 4096, 16384) == ((8, 1, 4, 1, 1, 0), 1)
    assert auto(1, 4096, 14336) == ((8, 1, 4, 1, 1, 0), 1)
    assert auto(4, 3072, 12288) == ((8, 1, 4, 1, 1, 0), 1)
    assert auto(4, 3584, 18944) == ((8, 1, 4, 1, 2, 0), 2)
    assert auto(1, 8192, 28672) == ((8, 1, 4, 1, 2, 0), 1)      # 256 tiles of 16 x 32: no split needed
    assert auto(16, 4096, 16384) == ((4, 1, 4, 1, 4, 0), 4)     # 64 tiles of 16 x 64 -> 256 workgroups
    assert auto(16, 5120, 13824) == ((4, 1, 4, 1, 4, 0), 3)     # 80 tiles -> 240
    assert auto(32, 5120, 13824) == ((4, 1, 4, 1, 4, 0), 2)     # two rows of tiles: up to 320 workgroups
    assert auto(16, 10240, 16384) == ((4, 1, 4, 1, 4, 0), 3)    # 160 tiles: 3 from 129 on
    assert auto(1, 10240, 16384) == ((4, 1, 4, 1, 4, 0), 1)     # ... but not for M <= 4
    assert auto(16, 2048, 8192) == ((8, 1, 4, 1, 1, 0), 1)      # 128 workgroups either way: unsplit 16 x 16
    assert auto(1, 512, 65536) == ((8, 1, 4, 1, 2, 0), 8)       # at most 8; more workgroups than unsplit
    assert auto(16, 14336, 16384) == ((4, 1, 4, 1, 4, 0), 1)    # 224 tiles: unsplit
    assert auto(16, 11264, 11264) == ((4, 1, 4, 1, 4, 0), 1)    # 176 tiles: 3 splits would pass 2 per CU
    assert auto(8, 28672, 8192) == ((4, 1, 4, 1, 4, 0), 1)      # 448 tiles: a full grid, 4 slices, unsplit
    assert auto(16, 4096, 6144) == ((8, 1, 4, 1, 1, 0), 1)      # K < 8192: narrower tiles instead
    assert auto(32, 25600, 2048) == ((2, 2, 4, 2, 2, 0), 1)     # the 32-row tile's grid is full
    # 32 < M <= 64 with a weight of 40 MB or more: the 64-row ring tiles (64 x 128 once 64 x 64 would have more
    # tiles than CUs), split by the residency model
    assert auto(64, 16384, 4096) == ((2, 2, 4, 2, 2, 1), 2)     # 256 tiles of 64 x 64 -> 512 workgroups
    assert auto(64, 14336, 4096) == ((2, 2, 4, 2, 2, 1), 2)     # 58.7 MB: 224 tiles -> 448
    assert auto(48, 12288, 4096) == ((2, 2, 4, 2, 2, 1), 4)     # 192 tiles -> 768, 3 per CU
    assert auto(56, 11008, 4096) == ((2, 2, 4, 2, 2, 1), 4)     # 172 tiles -> 688
    assert auto(64, 8192, 4096) == ((4, 1, 4, 1, 4, 0), 1)      # 32 MB: streaming
    assert auto(52, 17408, 11264) == ((1, 4, 4, 4, 2, 1), 3)    # 272 tiles of 64 x 64: 136 of 64 x 128 -> 408
    assert auto(48, 32768, 4096) == ((1, 4, 4, 4, 2, 1), 2)     # 256 tiles of 64 x 128 -> 512
    assert auto(64, 5120, 13824) == ((2, 2, 4, 2, 2, 1), 6)     # 80 tiles, long K
    assert auto(64, 65536, 4096) == ((1, 4, 4, 4, 2, 1), 1)     # 512 tiles of 64 x 128
    assert auto(48, 40960, 5120) == ((1, 4, 4, 4, 2, 1), 2)     # 320 tiles of 64 x 128
    assert auto(64, 65536, 1024) == ((1, 4, 4, 4, 2, 1), 1)
    assert auto(64, 16384, 2048) == ((4, 1, 4, 1, 4, 0), 1)     # 32 MB weight: streaming
    assert auto(32, 65536, 4096) == ((1, 4, 4, 4, 2, 1), 1)     # M <= 32: from a 96 MB weight
    assert auto(32, 32768, 4096) == ((1, 4, 4, 4, 2, 1), 2)     # 256 tiles of 64 x 128
    assert auto(32, 5120, 25600) == ((2, 2, 4, 2, 2, 1), 6)     # 80 tiles, long K
    assert auto(32, 16384, 4096) == ((2, 2, 4, 2, 2, 0), 1)     # 256 32-row tiles: one round of them
    assert auto(24, 18432, 4096) == ((4, 1, 4, 1, 4, 0), 1)     # 288: a small second round, the 16-row tile
    assert auto(40, 8448, 10496) == ((2, 2, 4, 2, 2, 1), 3)     # 132 tiles: 4 splits would leave 16 over
    # a pinned tile the heuristic would not pick is never split by it
    assert splits(512, 5376, 5120, (2, 2, 4, 2, 2, 1)) == 1
    assert splits(16, 14336, 16384, (4, 1, 4, 1, 4, 0)) == 1    # 224 tiles
    assert splits(2, 4096, 16384, (4, 1, 4, 1, 4, 0)) == 1      # the heuristic picks 16 x 32 there
    for m in (65, 128, 200, 512, 1040, 2320):
        for n in (1024, 1536, 4096, 12288):
            for k in (4096, 6144, 16384):
                tile = pick(m, n, k)
                s = splits(m, n, k, tile)
                assert 1 <= s <= 8 and (s == 1 or -(-k // 64) // s >= 16)


def test_bf16_activations_widen_first_only_where_the_fp16_kernel_repays_it():
    """The auto path's widen-first rule (fitted on the tile sweep's grid, bf16 in place against widened + fp16
    pick): wide weights on the 128 x 256 block (C3's shape 0.88 of the in-place time, 8192^3 0.94), long K on
    the 128 x 128 tile, big weights on the 64 x 64 deep ring; not C2, C5 or the streaming regimes; fp16
    activations never."""
    from feather_ops.scaled_mm import _auto_choice, widen_first

    bf = torch.bfloat16
    w64 = (1, 4, 4, 8, 4, 1)
    wide = (2, 2, 4, 8, 8, 1)
    assert _auto_choice(4096, 12288, 3072, bf) == (wide, 1, True)        # the fp16 pick: the wide tile
    assert _auto_choice(8192, 8192, 8192, bf) == (wide, 1, True)
    assert _auto_choice(4096, 12288, 2048, bf) == (w64, 1, True)         # K < 3072: the 128 x 256 block
    assert _auto_choice(4112, 16384, 3072, bf) == (w64, 1, True)         # 0.896 measured
    # 128 x 128: the lead grows with K (1.06-1.09x measured from K = 4608 on, 0.95-1.0x at K <= 3072)
    assert _auto_choice(4096, 4608, 12288, bf) == ((2, 2, 4, 4, 4, 1), 1, True)    # 1.078-1.09x
    assert _auto_choice(4608, 4096, 16384, bf) == ((2, 2, 4, 4, 4, 1), 1, True)    # 1.087-1.089x
    # C2: the fp16 pick is the 256 x 192 wide tile (57.5 us), widened first (8.8 us) against 69.8 us in place
    assert _auto_choice(4096, 3072, 3072, bf) == ((2, 2, 4, 8, 6, 1), 1, True)
    assert _auto_choice(4097, 5120, 2560, bf) == ((2, 2, 4, 4, 4, 1), 1, False)   # C5's largest: 1.025
    assert _auto_choice(6416, 1536, 6144, bf) == ((2, 2, 4, 4, 4, 1), 1, False)   # narrow weight: 1.158
    assert _auto_choice(9232, 1024, 5120, bf)[2] is False
    assert _auto_choice(512, 5120, 5120, bf) == ((2, 2, 4, 4, 4, 1), 3, False)    # split: in place
    assert _auto_choice(16, 14336, 4096, bf)[2] is False
    # M <= 64 on the 64 x 64 tile (the deep ring, which widens per fragment): big weights, split or not
    # (a big weight with more 64 x 64 tiles than CUs takes the 64 x 128 tile split in place instead, for bf16
    # activations with more splits: 28 x 28672 x 25088 on it 1.13x over widened 64 x 64)
    assert _auto_choice(32, 25600, 5120, bf) == ((1, 4, 4, 4, 2, 1), 4, False)
    assert _auto_choice(32, 5120, 25600, bf) == ((2, 2, 4, 2, 2, 1), 6, True)   # 1.16-1.17x
    assert _auto_choice(64, 16384, 4096, bf)[2] is False                         # 64 MB weight: 1.03x, kept
    assert _auto_choice(32, 14336, 4096, bf)[2] is False                         # streaming tile: 0.89x
    assert _auto_choice(4096, 12288, 3072, torch.float16) == (wide, 1, False)
    assert widen_first(4096, 12288, 3072, wide, 1)
    # the rule itself: a lead of 17% of the modelled fp16 time against 1.2x the pass (>= 4 us)
    assert widen_first(4096, 12288, 3072, w64, 1) and not widen_first(4096, 12288, 3072, w64, 2)
    assert not widen_first(4096, 12288, 3072, (2, 2, 4, 2, 2, 1), 1)   # no measured lead for that tile
    assert not widen_first(256, 4096, 1024, w64, 1)                      # under the pass's 4 us


def test_widen_first_only_on_ring_tiles_with_a_measured_lead():
    """Over seeded random shapes: the auto path widens bf16 activations first only onto the ring tiles whose lead
    was measured (the 128 x 64-wave 128 x 256 block, and the wide tile with its lead, 128 x 128 and 64 x 128
    unsplit, and the 64 x 64 deep ring at
    M <= 64, split or not), onto the fp16-activation pick, and never for fp16 activations."""
    import numpy as np

    from feather_ops.scaled_mm import _auto_choice

    rng = np.random.default_rng(3)
    ring_unsplit = {(1, 4, 4, 8, 4, 1), (2, 2, 4, 4, 4, 1), (1, 4, 4, 4, 2, 1), (2, 2, 4, 8, 8, 1), (2, 2, 4, 8, 6, 1)}
    for _ in range(400):
        m = int(rng.integers(1, 20000))
        n = int(rng.integers(1, 4000)) * 8
        k = int(rng.integers(1, 1200)) * 16
        assert _auto_choice(m, n, k, torch.float16)[2] is False
        tile, splits, widen = _auto_choice(m, n, k, torch.bfloat16)
        if widen:
            assert (tile in ring_unsplit and splits == 1) or (tile == (2, 2, 4, 2, 2, 1) and m <= 64), (m, n, k, tile)
            assert tile == _auto_choice(m, n, k, torch.float16)[0]


def test_wide_tile_rule():
    """The 256 x 256 wide tile's regime (fp16 activations): shapes on its grid with K >= 3072 whose last round of
    256 tiles is whole or at least 170 / 256 full, or at least 1700 tiles; a single partial round only from
    K = 4096; not where the 256 x 192 tile makes one round 205 / 256 full or more. One cell each way from the
    tile sweep."""
    from feather_ops.scaled_mm import select_scaled_mm_config as pick

    wide = (2, 2, 4, 8, 8, 1)
    assert pick(4096, 4096, 4096) == wide               # one whole round: 1.067 over the ring
    assert pick(5376, 5376, 7168) == wide               # 441 tiles, last round 185 / 256: 1.044
    assert pick(4096, 3328, 4096) == wide               # one round of 208 (the 256 x 192 tile: 288)
    assert pick(9216, 18432, 3072) == wide              # 2592 tiles: 1.019
    assert pick(4096, 3072, 3072) != wide               # one partial round at K = 3072: 0.988
    assert pick(4096, 4608, 4608) != wide               # 288 tiles: a 32-tile second round, 0.78
    assert pick(9728, 4096, 4096) != wide               # 608 tiles: 0.972
    assert pick(4096, 8192, 2048) != wide               # K < 3072
    assert pick(4112, 4096, 4096) != wide               # off the grid: masked loads
    assert pick(4096, 12288, 3072, torch.bfloat16) != wide   # bf16 in place: the ring tiles


def test_wide192_tile_rule():
    """The 256 x 192 wide tile's regime (fp16 activations): one round of its tiles at least 205 / 256 full, K >= 3072
    and a multiple of 64, any M and N. The cells of the tile sweep it wins, and its losses either side."""
    from feather_ops.scaled_mm import select_scaled_mm_config as pick

    w192 = (2, 2, 4, 8, 6, 1)
    assert pick(4096, 3072, 3072) == w192               # C2: 256 tiles, 1.114 over the best other tile
    assert pick(4096, 3072, 12288) == w192              # 1.097
    assert pick(6416, 1536, 6144) == w192               # 26 x 8 = 208 tiles (ragged M): 1.052
    assert pick(9232, 1024, 5120) == w192               # 37 x 6 = 222 (ragged M and N): 1.051
    assert pick(9216, 1280, 5120) == w192               # 252: 1.023
    assert pick(4112, 2560, 6912) == w192               # 238: 1.022
    assert pick(4112, 3072, 3072) != w192               # 272 tiles, a second round: 0.60
    assert pick(4096, 4608, 4608) != w192               # 384: 0.97
    assert pick(4096, 4096, 4096) != w192               # 352: 0.66
    assert pick(1024, 10240, 1280) != w192              # 216 tiles, K < 3072: 0.96
    assert pick(6144, 1536, 4112) != w192               # K not a multiple of 64
    assert pick(4096, 3072, 3072, torch.bfloat16) != w192   # bf16 in place: the ring tiles


def test_stream32_tile_rule_for_m_over_64():
    """64 < M <= 512 on the streaming tiles with fp16 activations: the 32-row tile when it makes one round of 144-256 blocks
    or two of 392-512 (it reads the weight half as often as the 16-row tiles); never with bf16 activations, which it
    widens per fragment. Cells of the fitting sweep and of the held-out one."""
    from feather_ops.scaled_mm import select_scaled_mm_config as pick

    s32, s16 = (2, 2, 4, 2, 2, 0), (4, 1, 4, 1, 4, 0)
    assert pick(128, 4096, 4096) == s32        # 256 blocks: 1.116 over the 16-row tile
    assert pick(192, 2560, 2560) == s32        # 240: 1.148
    assert pick(96, 3072, 3072) == s32         # 144: 1.010
    assert pick(256, 1536, 6144) == s32        # 192 (held out): 1.212
    assert pick(80, 5120, 1280) == s32         # 240 (held out): 1.025
    assert pick(96, 2560, 2560) == s16         # 120 blocks: 0.828
    assert pick(192, 4096, 4096) == s16        # 384 blocks, a second round: 0.943
    assert pick(64, 4096, 4096) == s16         # M = 64: the 16-row tile (0.777)
    assert pick(128, 4096, 4096, torch.bfloat16) == s16   # bf16 activations: 0.82 on the held-out cells
    assert pick(512, 1024, 1024) == s32        # 256 blocks: 1.16
    assert pick(384, 1280, 4096) == s32        # 240: 1.21
    assert pick(512, 1152, 1152) == s16        # 288 blocks, a second round: 0.91
    assert pick(256, 2560, 2560) == s16        # 320 blocks: 0.96
    assert pick(224, 3584, 3584) == s32        # 392 blocks, two rounds: 1.083
    assert pick(256, 3584, 3584) == s32        # 448: 1.149
    assert pick(512, 2048, 1024) == s32        # 512: 1.12
    assert pick(512, 2048, 1024, torch.bfloat16) == s16
    assert pick(1024, 1024, 1024) != s32       # past the rows the sweeps covered


def test_mid_m_streaming_and_ring_split_rules():
    """M > 64 with a small grid (96-cell fitting grid, M 80-256, N 1024-3072, K 6144-16384, and a 60-cell held-out
    one): long-K streaming splits stay within one workgroup per CU; one round of unsplit 16 x 64 blocks at K >= 6144
    keeps more weight in flight (fp16: 128-deep steps; bf16: 8 K slices, 128-deep steps from K = 12288); the ring
    tiles' split needs 80 64 x 128 tiles, or 36 (bf16: 64) on a weight of 18 MiB or more. Each cell below is the
    best or within 3% of the best measured candidate; the comment gives the previous pick's ratio."""
    from feather_ops.scaled_mm import _auto_choice

    fp, bf = torch.float16, torch.bfloat16
    u8, ks8, ks4 = (4, 1, 8, 1, 4, 0), (8, 1, 4, 1, 4, 0), (4, 1, 4, 1, 4, 0)
    ring, s32 = (1, 4, 4, 4, 2, 1), (2, 2, 4, 2, 2, 0)
    assert _auto_choice(160, 1024, 8192, fp) == (u8, 1, False)      # split 2 into 320 workgroups: 0.83
    assert _auto_choice(128, 2048, 8192, fp) == (u8, 1, False)      # 4 K slices: 0.90
    assert _auto_choice(128, 2048, 8192, bf) == (ks8, 1, False)     # 0.90
    assert _auto_choice(128, 2048, 12288, bf) == (u8, 1, False)     # 0.91
    assert _auto_choice(80, 1024, 16384, fp) == (ks4, 3, False)     # the ring split on 16 tiles: 0.50
    assert _auto_choice(96, 3072, 12288, bf) == (ks4, 1, False)     # the ring split on 48 tiles (bf16): 0.70
    assert _auto_choice(192, 1536, 8192, fp) == (s32, 1, False)     # the ring split on a 12.6 MB weight: 0.88
    assert _auto_choice(192, 1536, 12288, fp) == (ring, 7, False)   # 36 tiles, 18.9 MB: the ring split stays
    assert _auto_choice(256, 3072, 12288, bf) == (ring, 8, False)   # 96 tiles: the ring split stays
    assert _auto_choice(96, 3072, 6144, fp) == (ks4, 1, False)      # K >= 6144, M < 160: not the 32-row tile


def test_heuristic_returns_instantiated_tiles():
    from feather_ops.scaled_mm import select_scaled_mm_config
    from feather_ops.tiles import SCALED_MM_TILES

    for m in (1, 2, 15, 16, 17, 31, 32, 33, 64, 65, 77, 128, 256, 500, 1000, 4096, 4097, 25344):
        for n in (8, 96, 1000, 1024, 3072, 5120, 12288, 14336, 96768):
            for k in (16, 1024, 2560, 4096):
                assert select_scaled_mm_config(m, n, k) in SCALED_MM_TILES


def test_heuristic_picks_on_representative_cells():
    """The fitted rule's regimes, one cell each (the picks the tile sweep measured best or within noise)."""
    from feather_ops.scaled_mm import select_scaled_mm_config as pick

    assert pick(4096, 12288, 3072) == (2, 2, 4, 8, 8, 1)   # C3: 3 full rounds of the wide tile
    assert pick(4112, 12288, 3072) == (1, 4, 4, 8, 4, 1)   # ragged M: 128 x 256 as 128 x 64 waves
    assert pick(4096, 12288, 3072, torch.bfloat16) == (2, 2, 4, 4, 8, 1)   # bf16: 64 x 128 waves
    assert pick(4096, 3072, 3072) == (2, 2, 4, 8, 6, 1)    # C2: one full round of 256 x 192
    assert pick(9216, 2048, 2048) == (2, 2, 4, 4, 4, 1)    # 128 x 256 would need a second, 1/8-full wave
    assert pick(4112, 1024, 5120) == (1, 4, 4, 4, 2, 1)    # one partial wave: 64 x 128 ring tiles
    assert pick(2304, 1280, 1280) == (2, 2, 4, 2, 2, 1)    # small grid, short K: 64 x 64 ring
    assert pick(512, 1024, 1024) == (2, 2, 4, 2, 2, 0)     # tiny grid: one round of 32-row streaming blocks
    assert pick(32, 25600, 2048) == (2, 2, 4, 2, 2, 0)     # 32 rows, wide: 32-row streaming tile
    assert pick(32, 25600, 5120) == (1, 4, 4, 4, 2, 1)     # ... and a 131 MB weight: the 64 x 128 ring tile
    assert pick(32, 11264, 11264) == (2, 2, 4, 2, 2, 1)    # 127 MB, 176 64 x 64 tiles: that ring tile
    assert pick(16, 14336, 4096) == (4, 1, 4, 1, 4, 0)     # C4: 224 blocks of 64 columns, 4 K slices
    assert pick(16, 4096, 4096) == (8, 1, 4, 1, 1, 0)      # narrow N: 16-column blocks for parallelism
    assert pick(16, 6144, 6144) == (8, 1, 4, 1, 2, 0)
    assert pick(1, 96768, 2688) == (1, 4, 4, 4, 2, 1)      # one row, LM-head width: 756 ring tiles
    assert pick(1, 151936, 3584) == (4, 1, 4, 1, 4, 0)     # 1187 ring tiles: a partial second wave
    assert pick(1, 32000, 4096) == (4, 1, 4, 1, 4, 0)      # 250 ring tiles: streaming


def test_every_auto_launch_is_within_the_c_abi_contract(lib):
    """Over seeded random shapes (M 1-20000, N a multiple of 8 up to 60000, K a multiple of 16 up to 40000) and
    both activation dtypes, the auto path's (tile, splits) is a launch the C ABI accepts: an instantiated tile,
    1 <= splits <= the tile's K units, a split workspace the library sizes (not -1) whose partial sums fit the
    allocation-free entry point's static array, and splits only where the heuristic itself splits. The library
    computes the workspace on the host, so no GPU call is made."""
    import numpy as np

    from feather_ops.scaled_mm import _auto_choice
    from feather_ops.tiles import SCALED_MM_TILES, split_units

    scratch = _header_scratch_bytes()
    rng = np.random.default_rng(2026)
    for _ in range(3000):
        m = int(np.exp(rng.uniform(0, np.log(20000))))
        n = int(rng.integers(1, 7501)) * 8
        k = int(rng.integers(1, 2501)) * 16
        for dt in (torch.float16, torch.bfloat16):
            tile, splits, widen = _auto_choice(m, n, k, dt)
            assert tile in SCALED_MM_TILES, (m, n, k, dt, tile)
            assert 1 <= splits <= min(8, split_units(k, tile)), (m, n, k, dt, tile, splits)
            if splits > 1:
                ws = lib.feather_splitk_workspace_bytes(m, n, k, *tile[:5], bool(tile[5]), splits)
                assert 0 < ws <= scratch, (m, n, k, dt, tile, splits, ws)
            assert not widen or dt == torch.bfloat16
