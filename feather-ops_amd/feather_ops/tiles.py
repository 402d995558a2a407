"""The instantiated scaled_mm tiles for gfx950, and the tile vocabulary the heuristic chooses from.

This file is the single source of truth: `feather-ops_amd/gen_tiles.py` renders `SCALED_MM_TILES` into
`csrc/feather_tiles.h`, which the HIP sources use to instantiate and dispatch, so every tile the
heuristic can return is a compiled kernel (same flow as the reference's `feather_ops/tiles.py:1-15` ->
`tools/gen_tiles.py` -> `csrc/feather_tiles.h`). It must not import torch: the build reads it before the
extension exists.

Tile format: the reference's 6-tuple `(warps_m, warps_n, unroll_k, repeat_m, repeat_n, prefetch)`
(`tiles.py:8-12`, op schema `csrc/hip_kernel.cu:827-840`), re-interpreted for CDNA4's wave64 MFMA:

- A wave is 64 lanes and an MFMA fragment is 16 x 16 outputs (`v_mfma_f32_16x16x32_f16`), so
  `block_m = 16 * warps_m * repeat_m`, `block_n = 16 * warps_n * repeat_n` and `chunk_k = 16 * unroll_k`
  keep their meaning; `unroll_k` must be a multiple of 4 (whole 64-deep MFMA groups).
- `prefetch = 1` selects the LDS ring kernel: `warps_m x warps_n` waves each own a
  `16*repeat_m x 16*repeat_n` sub-tile, and K streams through LDS rings of `chunk_k`-deep stages: the
  activation ring has 2 slots for blocks of up to 4 waves (so two or three blocks share a CU) and 3 for
  8-wave blocks, and the weight ring one more when it fits (see `ring_slots`), so the next stages are in
  flight while the current one feeds the MFMAs. 64-row tiles also have a deep-ring variant (3 + 4 slots)
  that the launcher takes for grids small enough to be resident at once (`ring_is_deep`).
- `prefetch = 0` selects the streaming kernel for skinny M: no LDS staging. The block's `warps_m` waves
  split K instead of M (so `block_m = 16 * repeat_m`), its `warps_n` waves split N, and each wave streams
  its operands from HBM into registers `chunk_k` at a time, double-buffered; a short LDS reduction joins
  the K slices in a fixed order.
- Either kernel can also split K across workgroups (`scaled_mm_hip(..., splits=S)`, the C ABI's
  `feather_scaled_mm_splitk`): each output tile's K range (a ring tile's `chunk_k`-deep stages, a
  streaming tile's 64-deep groups) is cut into S contiguous ranges whose fp32 partial sums meet in a
  caller-owned workspace (`split_workspace_bytes`), for grids with fewer tiles than the GPU has compute
  units.
"""

SCALED_MM_TILES = [
    # LDS ring (prefetch = 1)
    (2, 2, 4, 4, 8, 1),  # 128 x 256, 4 waves of 64 x 128, two blocks per CU
    (1, 4, 4, 8, 4, 1),  # 128 x 256, 4 waves of 128 x 64, two blocks per CU
    (2, 2, 4, 8, 4, 1),  # 256 x 128, 4 waves of 128 x 64, two blocks per CU
    (2, 2, 4, 4, 4, 1),  # 128 x 128, 4 waves of 64 x 64
    (4, 2, 4, 4, 8, 1),  # 256 x 256, 8 waves of 64 x 128, 3-stage ring
    (2, 4, 4, 4, 4, 1),  # 128 x 256, 8 waves of 64 x 64
    (4, 2, 4, 4, 4, 1),  # 256 x 128, 8 waves of 64 x 64
    (1, 4, 4, 4, 2, 1),  # 64 x 128
    (2, 2, 4, 2, 2, 1),  # 64 x 64
    (2, 2, 4, 8, 8, 1),  # 256 x 256, 4 waves of 128 x 128, one block per CU: the software-pipelined wide kernel
    (2, 2, 4, 8, 6, 1),  # 256 x 192, 4 waves of 128 x 96, one block per CU: the wide kernel
    # streaming split-K (prefetch = 0)
    (4, 1, 4, 1, 4, 0),  # 16 x 64, 4 K slices
    (4, 1, 8, 1, 4, 0),  # 16 x 64, 4 K slices, 128-deep steps
    (8, 1, 4, 1, 4, 0),  # 16 x 64, 8 K slices
    (8, 1, 8, 1, 4, 0),  # 16 x 64, 8 K slices, 128-deep steps
    (4, 2, 4, 1, 2, 0),  # 16 x 64, 4 K slices x 2 column waves
    (4, 1, 4, 1, 2, 0),  # 16 x 32, 4 K slices
    (8, 1, 4, 1, 2, 0),  # 16 x 32, 8 K slices
    (4, 1, 4, 1, 1, 0),  # 16 x 16, 4 K slices
    (8, 1, 4, 1, 1, 0),  # 16 x 16, 8 K slices
    (8, 2, 4, 1, 1, 0),  # 16 x 32, 8 K slices x 2 column waves
    (2, 2, 4, 2, 2, 0),  # 32 x 64
    (2, 2, 4, 4, 2, 0),  # 64 x 64
]


def gemm_block_sizes(tile: tuple[int, ...]) -> tuple[int, int, int]:
    """`(block_m, block_n, chunk_k)` of a `SCALED_MM_TILES` entry."""
    warps_m, warps_n, unroll_k, repeat_m, repeat_n = tile[:5]
    prefetch = tile[5] if len(tile) > 5 else 1
    block_m = 16 * repeat_m if prefetch == 0 else 16 * warps_m * repeat_m
    return block_m, 16 * warps_n * repeat_n, 16 * unroll_k


WIDE_TILE = (2, 2, 4, 8, 8, 1)
WIDE_TILE_192 = (2, 2, 4, 8, 6, 1)


def is_wide(tile: tuple[int, ...]) -> bool:
    """Whether a `prefetch = 1` tile runs on the wide kernel (4 waves of 128 x 16 repeat_n, one workgroup per CU,
    512 registers per wave) rather than the ring kernel: `(2, 2, 4, 8, 8, 1)` (256 x 256) and `(2, 2, 4, 8, 6, 1)`
    (256 x 192)."""
    return tuple(tile[:6]) in (WIDE_TILE, WIDE_TILE_192)


def ring_slots(tile: tuple[int, ...], deep: bool = False) -> tuple[int, int]:
    """(activation, weight) LDS ring slots of a `prefetch = 1` tile, the rule the kernel applies.

    The wide tiles (`is_wide`) keep 3 of each. Blocks of up to 4 waves keep 2 activation slots within an 80 KiB budget, bigger blocks 3 within
    160 KiB; the weight ring gets one more slot when that fits the budget and the tile already runs at
    most two blocks per CU (8-wave blocks: always when it fits). `deep`: the deep-ring variant of a
    64-row tile (3 and 4 slots), which the launcher takes for grids whose blocks are all resident at once
    with it (`ring_is_deep`).
    """
    if deep:
        if gemm_block_sizes(tile)[0] > 64:
            raise ValueError(f"the deep ring is for 64-row tiles: {tile}")
        return 3, 4
    if is_wide(tile):
        return 3, 3  # the wide kernel: 3 x (32 + 16 or 12) KiB, one workgroup per CU
    warps_m, warps_n, unroll_k, repeat_m, repeat_n = tile[:5]
    waves = warps_m * warps_n
    a_bytes = 16 * warps_m * repeat_m * unroll_k * 32
    b_bytes = 16 * warps_n * repeat_n * unroll_k * 16
    slots_a = 2 if waves <= 4 else 3
    budget = (80 if waves <= 4 else 160) * 1024
    deep_b = slots_a * a_bytes + (slots_a + 1) * b_bytes <= budget and (
        waves > 4 or 2 * (a_bytes + b_bytes) > 160 * 1024 // 3)
    return slots_a, slots_a + (1 if deep_b else 0)


def ring_lds_bytes(tile: tuple[int, ...], deep: bool = False) -> int:
    """LDS bytes of a ring block: its activation (2-byte) and weight (fp8) rings of `chunk_k`-deep stages."""
    block_m, block_n, chunk_k = gemm_block_sizes(tile)
    slots_a, slots_b = ring_slots(tile, deep)
    return slots_a * block_m * chunk_k * 2 + slots_b * block_n * chunk_k


def ring_is_deep(M: int, N: int, tile: tuple[int, ...], splits: int = 1, a_bf16: bool = False) -> bool:
    """Whether a launch of a ring tile runs the deep-ring variant (the launcher's rule): a 64-row tile
    whose launch has no more workgroups than 256 CUs hold at once with the deep ring's LDS; with bf16
    activations (widened per fragment in the deep ring) only while M <= 64 and the tile has at most two
    column waves."""
    block_m, block_n, _ = gemm_block_sizes(tile)
    if tile[5] != 1 or block_m > 64:
        return False
    if a_bf16 and (M > 64 or tile[1] > 2):
        return False
    blocks = -(-M // block_m) * -(-N // block_n) * splits
    return blocks <= 256 * (160 * 1024 // ring_lds_bytes(tile, deep=True))


MAX_SPLITS = 32
SPLIT_COUNTER_BYTES = 64 * 1024  # fixed counter area at the start of every split workspace


def split_units(K: int, tile: tuple[int, ...]) -> int:
    """The units a split launch cuts K into: a ring tile's `chunk_k`-deep stages, a streaming tile's 64-deep
    groups."""
    return -(-K // (16 * tile[2])) if tile[5] else -(-K // 64)


def split_slots(tile: tuple[int, ...]) -> int:
    """Join slots (arrival counters) per output tile of a split launch: a ring tile's waves, a streaming
    tile's 16 x 16 fragments (its column waves when the block has a single K slice)."""
    warps_m, warps_n, _, repeat_m, repeat_n, prefetch = tile[:6]
    if prefetch:
        return warps_m * warps_n
    return warps_n * repeat_m * repeat_n if warps_m > 1 else warps_n


def split_workspace_bytes(M: int, N: int, K: int, tile: tuple[int, ...], splits: int) -> int:
    """Workspace bytes of a split-K launch (the C ABI's `feather_splitk_workspace_bytes`), -1 if the tile is
    not instantiated, `splits` is outside 1 .. min(32, `split_units`) or the grid needs more than 16384
    join counters (output tiles x `split_slots`).

    Layout (none for `splits` = 1): a fixed 64 KiB counter area (one uint32 arrival counter per output tile
    and join slot; it is the same area for every shape, so a workspace reused across shapes keeps it
    zero), then `splits` fp32 partial tiles per output tile.
    """
    tile = tuple(tile)
    if M < 1 or N < 1 or K < 16 or len(tile) < 6 or tile not in SCALED_MM_TILES:
        return -1
    if not 1 <= splits <= min(MAX_SPLITS, split_units(K, tile)):
        return -1
    if splits == 1:
        return 0
    block_m, block_n, _ = gemm_block_sizes(tile)
    tiles = -(-M // block_m) * -(-N // block_n)
    if tiles * split_slots(tile) * 4 > SPLIT_COUNTER_BYTES:
        return -1
    total = SPLIT_COUNTER_BYTES + tiles * splits * block_m * block_n * 4
    return total if total < 2**31 else -1


def threads_per_block(tile: tuple[int, ...]) -> int:
    """Work-items of one block: 64 per wave, `warps_m * warps_n` waves."""
    return 64 * tile[0] * tile[1]
