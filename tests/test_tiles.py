"""The tile table (reference tests/test_tiles.py): header current, heuristic aliases instantiated, no
duplicates, every tile fits gfx950's limits, and every compiled kernel allocates exactly its tile's LDS."""

import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_generated_header_is_current():
    result = subprocess.run([sys.executable, str(ROOT / "feather-ops_amd" / "gen_tiles.py"), "--check"],
                            capture_output=True, text=True, check=False)
    assert result.returncode == 0, f"{result.stdout}{result.stderr}"


def test_heuristic_tiles_are_instantiated():
    from feather_ops import scaled_mm
    from feather_ops.tiles import SCALED_MM_TILES

    aliases = [name for name in dir(scaled_mm) if name.startswith("_TILE_")]
    assert aliases
    for name in aliases:
        assert getattr(scaled_mm, name) in SCALED_MM_TILES, name


def test_no_duplicate_tiles():
    from feather_ops.tiles import SCALED_MM_TILES

    assert len(set(SCALED_MM_TILES)) == len(SCALED_MM_TILES)


def test_tiles_fit_gfx950():
    from feather_ops.tiles import SCALED_MM_TILES, gemm_block_sizes, ring_slots, threads_per_block

    for tile in SCALED_MM_TILES:
        wm, wn, u, rm, rn, pf = tile
        assert pf in (0, 1)
        assert threads_per_block(tile) <= 1024, tile
        bm, bn, ck = gemm_block_sizes(tile)
        if pf:
            assert u % 4 == 0, tile  # whole 64-deep MFMA groups
            slots_a, slots_b = ring_slots(tile)
            assert 2 <= slots_a <= slots_b <= slots_a + 1, tile
            lds = slots_a * bm * ck * 2 + slots_b * bn * ck  # rings of A (2-byte) and B (fp8) stages
        else:
            assert u % 4 == 0, tile  # the streaming kernel works in 64-deep groups
            join = (wm if wm > 1 else 0) * wn * rm * rn * 64 * 16  # K-slice join buffer
            lds = wm * wn * 2 * (u // 4) * rm * 2048 + join  # per-wave activation double buffers + join
        assert lds <= 160 * 1024, tile


def test_ring_slots_rule():
    from feather_ops.tiles import ring_slots

    assert ring_slots((2, 2, 4, 4, 8, 1)) == (2, 3)  # 128 x 256: 32 + 48 KiB, two blocks per CU
    assert ring_slots((2, 2, 4, 4, 4, 1)) == (2, 2)  # 128 x 128: keeps three blocks per CU
    assert ring_slots((2, 2, 4, 8, 4, 1)) == (2, 2)  # 256 x 128: 2 x 32 + 3 x 8 KiB exceeds 80 KiB
    assert ring_slots((4, 2, 4, 4, 8, 1)) == (3, 4)  # 256 x 256, 8 waves: 96 + 64 KiB
    assert ring_slots((1, 4, 4, 4, 2, 1)) == (2, 2)  # 64 x 128: 8 KiB stages, up to four blocks per CU
    assert ring_slots((1, 4, 4, 4, 2, 1), deep=True) == (3, 4)  # its deep variant: 56 KiB
    with pytest.raises(ValueError):
        ring_slots((2, 2, 4, 4, 4, 1), deep=True)  # 128 rows: no deep variant


def test_deep_ring_rule():
    """The launcher's choice: a 64-row tile's launch takes the deep ring when all its workgroups are resident
    at once with it (64 x 128: 56 KiB, 2 blocks per CU -> 512; 64 x 64: 40 KiB, 4 per CU -> 1024)."""
    from feather_ops.tiles import ring_is_deep, ring_lds_bytes

    assert ring_lds_bytes((1, 4, 4, 4, 2, 1), deep=True) == 56 * 1024
    assert ring_lds_bytes((2, 2, 4, 2, 2, 1), deep=True) == 40 * 1024
    assert ring_is_deep(64, 65536, (1, 4, 4, 4, 2, 1))           # 512 tiles
    assert not ring_is_deep(64, 65536 + 128, (1, 4, 4, 4, 2, 1))
    assert ring_is_deep(64, 16384, (1, 4, 4, 4, 2, 1), splits=4)  # 128 tiles x 4
    assert not ring_is_deep(64, 16384, (1, 4, 4, 4, 2, 1), splits=5)
    assert ring_is_deep(2304, 1280, (2, 2, 4, 2, 2, 1))          # 720 tiles of 64 x 64
    assert not ring_is_deep(64, 1024, (2, 2, 4, 4, 4, 1))        # 128 rows
    assert not ring_is_deep(16, 1024, (8, 1, 4, 1, 4, 0))        # streaming
    # bf16 activations: only at M <= 64 and with at most two column waves (per-fragment widening)
    assert ring_is_deep(64, 16384, (2, 2, 4, 2, 2, 1), a_bf16=True)
    assert not ring_is_deep(130, 1000, (2, 2, 4, 2, 2, 1), a_bf16=True)
    assert not ring_is_deep(64, 16384, (1, 4, 4, 4, 2, 1), a_bf16=True)


def test_tile_shape_formula():
    from feather_ops.scaled_mm import tile_shape

    assert tile_shape((2, 4, 4, 8, 4, 1)) == (256, 256, 64)
    assert tile_shape((4, 1, 4, 1, 4, 0)) == (16, 64, 64)  # stream tiles split K across warps_m


def _check_lds():
    import importlib.util

    path = pathlib.Path(__file__).resolve().parents[1] / "feather-ops_amd" / "check_lds.py"
    spec = importlib.util.spec_from_file_location("_check_lds", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_every_kernel_allocates_exactly_its_tiles_lds():
    """The LDS audit (check_lds.py, the reference's tools/check_lds.py role): the compiled gfx950 code
    object's group_segment_fixed_size of every ring (unsplit and split, shallow and, for 64-row tiles, deep),
    wide (unsplit and split, whole and ragged shapes) and streaming instantiation (unsplit and split), and of the non-temporal-weight variants of the streaming
    and 64-row ring ones, equals the size the tile asks for. Compiles one dtype combination (hipcc, device
    code only)."""
    from feather_ops.tiles import SCALED_MM_TILES

    check = _check_lds()
    if not pathlib.Path(check.HIPCC).exists():
        pytest.skip("needs hipcc")
    asm = check.compile_asm("100")
    checked, bad = check.audit(asm)
    small_ring = sum(1 for t in SCALED_MM_TILES if t[5] == 1 and 16 * t[0] * t[3] <= 64)
    streaming = sum(1 for t in SCALED_MM_TILES if t[5] == 0)
    assert small_ring == 2
    non_temporal = 2 * streaming + 4 * small_ring
    wide = sum(1 for t in SCALED_MM_TILES if t[:6] in ((2, 2, 4, 8, 8, 1), (2, 2, 4, 8, 6, 1)))
    assert wide == 2
    # a wide tile has 4 instantiations (unsplit / split x whole / ragged shapes) where a ring tile has 2
    assert checked == 2 * len(SCALED_MM_TILES) + 2 * small_ring + non_temporal + 2 * wide
    assert bad == []
    # a planted off-by-one in the expectation is caught for every instantiation
    real = check.expected_bytes
    check.expected_bytes = lambda kernel, ints, bools=(): real(kernel, ints, bools) + 1
    try:
        assert len(check.audit(asm)[1]) == checked
    finally:
        check.expected_bytes = real
