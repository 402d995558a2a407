"""gfx950 scaled matmul of fp16/bf16 activations by a prepacked fp8 weight, `Y = (X @ W^T) * scale + bias`.

Drop-in for the reference's `feather_ops/scaled_mm.py` (same names, arguments and op boundary):
`X` is fp16 or bf16 `[M, K]`, `W` is fp8e5m2 or fp8e4m3fn stored as `[K_pad/16, N, 16]` (see
`prepack_b_for_scaled_mm`), `scale` is a per-tensor fp32 scalar on the device (or, beyond the
reference kernel, N fp32 values, one per output column, as the reference's naive path accepts with
`bias_dim=1`, `naive.py:29-33`) and `bias` is optional. The output is fp16 or bf16. Any `M >= 1` works,
with `K` a multiple of 16 and `N` a multiple of 8 (the reference needs 16).

Numerics are the naive path's (`feather_ops/naive.py:4-41`) with fp32 accumulation: bf16 activations are
widened to fp16 (RNE), the weight decodes exactly to fp16, the MFMAs accumulate in fp32, the scale is
applied in fp32, the downcast rounds to nearest even, and the bias is added in the output precision.

`scaled_mm_hip` picks the tile with the static heuristic below and hands it to the kernel through an
opaque custom op, so `torch.compile` sees one node whatever the shape (reference `scaled_mm.py:104-114`).
Pass `tile=` to pin it, which is what the benchmark sweeps and the tests do.
"""

import functools

import torch
from torch.library import custom_op

from . import _lib
from .tiles import gemm_block_sizes, ring_is_deep, split_workspace_bytes

# Tiles the heuristic can return, each an entry of `SCALED_MM_TILES` (gfx950 meaning in tiles.py).
_TILE_RING_128x256 = (2, 2, 4, 4, 8, 1)
# The same block as 4 column waves of 128 x 64: each wave decodes half as many weight fragments per stage
# (32 byte moves instead of 64) for 16 activation reads instead of 8; with fp16 activations and the
# reads-first schedule it measured 1.2% faster in geometric mean over the 41 grid cells that pick 128 x 256
# (C3 +1 to +3%, none slower than -0.5%); with bf16 activations (no reads-first schedule for its 128-row wave
# tile) it measured even.
_TILE_RING_128x256_W64 = (1, 4, 4, 8, 4, 1)
_TILE_RING_256x256 = (4, 2, 4, 4, 8, 1)
# The wide kernel's tiles: 256 x 256 and 256 x 192 on one workgroup per CU, 4 waves of 128 x 128 or 128 x 96
# (tiles.py `is_wide`).
_TILE_WIDE = (2, 2, 4, 8, 8, 1)
_TILE_WIDE_192 = (2, 2, 4, 8, 6, 1)
_TILE_RING_128x128 = (2, 2, 4, 4, 4, 1)
_TILE_RING_64x128 = (1, 4, 4, 4, 2, 1)
_TILE_RING_64x64 = (2, 2, 4, 2, 2, 1)
_TILE_STREAM_32x64 = (2, 2, 4, 2, 2, 0)
_TILE_STREAM_16x64 = (8, 1, 4, 1, 4, 0)
# M > 64 on the streaming tiles, fp16 activations: the 32-row tile from this many of its blocks up to one round
# (its per-piece K-slice join made it 2.6% faster; at 120 blocks it loses 17% to the 16-row tile, at 144 it is
# even). With bf16 activations, which it widens per fragment, it is 0.72-0.92x the 16-row tile there.
_STREAM_32_MIN_BLOCKS = 144
_STREAM_32_MAX_M = 512   # the rows its sweeps covered
# ... and for two rounds of 392-512 blocks: 0.998-1.149x the 16-row tile on the 7 such cells of three sweeps
# (M 160-512, N x K 2048 x 1024 to 3584^2; about 1.08x in geometric mean), where 288-360 blocks lose (0.79-0.97x
# on 11 cells: the second round's few blocks)
_STREAM_32_TWO_ROUND_MIN_BLOCKS = 392
# The same 16 x 64 block with 4 K slices (4 waves), and a 16 x 32 block with 8: with two fetches in flight per
# wave (16 KiB of weight per wave at 64 columns), 4 slices keep ~32 KiB per CU in flight where 8 keep ~64 KiB,
# which oversubscribes HBM on weights of 50-100 MB (C4: 11.86 against 12.14 us, graph-timed, cold weights).
_TILE_STREAM_16x64_KS4 = (4, 1, 4, 1, 4, 0)
_TILE_STREAM_16x64_U8 = (4, 1, 8, 1, 4, 0)
_TILE_STREAM_16x32 = (8, 1, 4, 1, 2, 0)

# MI355X: 256 compute units.
_CUS = 256

# Ring tiles for large grids: (tile, blocks resident per CU, steady-state TFLOP/s on a full grid), measured
# with the tile sweep (feather-ops_amd/benchmarks) on the large cells of its grid. With fp16 activations the
# 128 x 256 block runs as 128 x 64 waves and outpaces the 128 x 128 tile by more: refitted on the 76 large-grid
# cells of the sweep, any 128 x 128 rate from 920 to 980 gives 0.9975 of the best candidate in geometric mean
# (1030: 0.9956); with bf16 activations the fit keeps 1030 (0.9945).
_RING_MODEL = (
    (_TILE_RING_128x256, 2, 1100.0),
    (_TILE_RING_256x256, 1, 1040.0),
    (_TILE_RING_128x128, 3, 1030.0),
    (_TILE_RING_64x128, 3, 600.0),
)
_RING_MODEL_FP16 = (
    (_TILE_RING_128x256_W64, 2, 1100.0),
    (_TILE_RING_256x256, 1, 1040.0),
    (_TILE_RING_128x128, 3, 960.0),
    (_TILE_RING_64x128, 3, 600.0),
)

# The wide tile (fp16 activations; bf16 ones are widened first, `widen_first`): on shapes on its grid (M and N
# multiples of 256, K of 64: its unmasked load path) with K >= 3072, when its last round of tiles is whole or
# at least 170 / 256 full, or the grid runs at least 1700 tiles (6.6 rounds); with a single, partial round
# (fewer than 256 tiles) only from K = 4096. Measured with the tile sweep on the 76 large-grid cells of the
# grid: on the 21 cells this takes, 1.032x the previous pick in geometric mean (C3 1.040, 4096^2 x 4096 1.067,
# 5376^2 x 7168 1.044, 9216 x 1280 x 5120 1.073; worst 0.988 at 4096 x 3072 x 3072 before the K rule); it
# loses on the cells it leaves out: ragged shapes (masked loads, a mostly empty last tile row: 4112 x 4096 x
# 4096 0.88), partial last rounds of few rounds (288 tiles: 0.75-0.87; 560 and 608: 0.97-0.98, where the ring
# tiles' two workgroups per CU split the last round more finely) and K <= 2048 (0.87-0.98).
_WIDE_MIN_K = 3072
_WIDE_SINGLE_ROUND_MIN_K = 4096
_WIDE_MIN_LAST_ROUND = 170
_WIDE_MANY_TILES = 1700


def _wide_fits(M: int, N: int, K: int) -> bool:
    """Whether the fp16-activation heuristic takes the wide tile (see _WIDE_MIN_K)."""
    if M % 256 or N % 256 or K % 64 or K < _WIDE_MIN_K:
        return False
    tiles = (M // 256) * (N // 256)
    if tiles < _CUS and K < _WIDE_SINGLE_ROUND_MIN_K:
        return False
    return tiles % _CUS == 0 or tiles % _CUS >= _WIDE_MIN_LAST_ROUND or tiles >= _WIDE_MANY_TILES


# The 256 x 192 wide tile (fp16 activations; bf16 ones widened first): when its tiles make one round at least
# 205 / 256 full, with K >= 3072 (a multiple of 64), any M and N (ragged ones on its masked path). Measured with
# the tile sweep on the 76 large-grid cells: it takes 6 of them, each faster than every other tile there (4096 x
# 3072 x 3072 1.114x, 4096 x 3072 x 12288 1.097x, 6416 x 1536 x 6144 1.052x, 9232 x 1024 x 5120 1.051x, 9216 x
# 1280 x 5120 1.023x, 4112 x 2560 x 6912 1.022x); past one round it loses (272 tiles: 0.60x; 352: 0.66-0.69x),
# as it does below 3072 deep (1024 x 10240 x 1280, 216 tiles: 0.96x). Against the 256 x 256 tile it fills 4/3
# as many CUs where that one's grid is a partial round.
_WIDE_192_MIN_TILES = 205


def _wide192_fits(M: int, N: int, K: int) -> bool:
    """Whether the fp16-activation heuristic takes the 256 x 192 wide tile (see _WIDE_192_MIN_TILES)."""
    if K % 64 or K < _WIDE_MIN_K:
        return False
    return _WIDE_192_MIN_TILES <= -(-M // 256) * -(-N // 192) <= _CUS


# Split-K applies from this K (64 stages of 64) and keeps at least 16 stages per split.
_SPLIT_MIN_K = 4096
_SPLIT_MIN_STAGES = 16
# M > 64 on a small grid: the 16-row streaming tiles read the weight once per 16 rows (from the L2/MALL
# after the first pass), and their time grows with those bytes over the fraction of the CUs their blocks
# keep busy in the last round; from this many bytes by that measure the split ring tiles (which read the
# weight once per 64 or 128 rows) are faster.
_RING_MIN_REREAD = 216 << 20
# With bf16 activations the ring tiles on small grids (M > 64) widen them in registers on the shallow ring
# and need 4/3 of the re-reads to win; their 64 x 128 tile, light on LDS, then splits for up to three
# workgroups per CU.
_BF16_RING_MIN_REREAD = 288 << 20
# M > 768 with a weight too small for the rules above (a few MB, which the streaming tiles re-read from the
# L2 once per 16 rows): the 64 x 64 ring tile, split along K when that fills more CU slots, wins once its
# workgroups fill this fraction of the CU slots in their last round.
_BIG_M_RING_MIN_BUSY = 0.75

# M > 64 on a small grid with more than 256 64 x 128 tiles: the tile and split count come from a time model of
# the candidates (the 64 x 128 tile split 1-3 ways, the 128 x 128 tile split 1-4 ways), fitted with the tile sweep
# on 106 such cells, fp16 and bf16 activations (feather-ops_amd/benchmarks). Per tile: its rate relative to the
# 128 x 128 tile and how much of a CU's rate 1, 2 and 3+ resident blocks reach; blocks per CU from the compiled
# kernels (128 x 128: 3, by registers and its 48 KiB ring; 64 x 128: 5 on the 32 KiB shallow ring, 2 on the 56 KiB
# deep ring); each block also pays a fixed cost worth _SMALL_GRID_BLOCK_K of K (prologue, epilogue, the partial
# sums' round trip).
_SMALL_GRID_RATE = {_TILE_RING_64x128: (0.85, (0.4, 0.9, 1.0)), _TILE_RING_128x128: (1.0, (0.5, 0.9, 1.0))}
_SMALL_GRID_BLOCK_K = 768
_SMALL_GRID_MAX_SPLITS = {_TILE_RING_64x128: 3, _TILE_RING_128x128: 4}
# Partial sums of one split launch stay within the allocation-free entry point's static array.
_SPLIT_MAX_PARTIAL_BYTES = 64 << 20

# 16 < M <= 64: the 64-row ring tiles once the weight has _MID_M_RING_MIN_WEIGHT bytes or more for 32 < M <= 64
# (_MID_M_RING_MIN_WEIGHT_32 for M <= 32): the 64 x 128 tile from _MID_M_WIDE_TILES of its tiles on (where the
# 64 x 64 tile would have more tiles than CUs: 1.03-1.3x over it on 24 such cells, fp16 and bf16), the 64 x 64
# tile below (1.0-1.4x over the 64 x 128 tile on 22 of 28 cells), split by `_mid_m_ring_splits`; the split
# count of the 64 x 128 tile there was about _MID_M_RING_BLOCKS workgroups before (it still is for M <= 32 at
# LM-head widths). For 32 < M <= 64 the 16-row streaming tiles, which
# read the weight once per 16 rows, lose 4-29% to the split ring tiles from 40 MB on (held-out cells at M 40-64
# and weights of 32-58 MB) and win below it (6144 x 6144, 8192 x 4096 at M <= 48).
_MID_M_RING_MIN_WEIGHT = 40 << 20
_MID_M_RING_MIN_WEIGHT_32 = 96 << 20
_MID_M_WIDE_TILES = 129
_MID_M_RING_BLOCKS = 512
# The 64-row ring tiles' split count (`_mid_m_ring_splits`): workgroups per CU it considers (the 64 x 64 tile's
# deep ring holds 4; the 64 x 128 tile measured best at up to 3), the rate of a block alone on its CU, and the
# fixed cost of one split as a fraction of a tile's time.
_MID_M_MAX_PER_CU = {_TILE_RING_64x64: 4, _TILE_RING_64x128: 3}
_MID_M_LONE_RATE = 0.6
# bf16 activations on the 64 x 128 tile (register-staged ring): the rate at 1, 2, 3 and 4 workgroups per CU; it
# wants 3-4 per CU (best measured splits 544-960 workgroups on 12 cells, against 408-480 with fp16)
_MID_M_STAGED_RATES = (0.6, 0.75, 0.9, 1.0)
_MID_M_SPLIT_COST = 0.04

# Skinny M with a long K and a narrow weight (K >= _STREAM_SPLIT_MIN_K, fewer than _STREAM_SPLIT_MAX_TILES tiles of
# 16 x 64): a streaming tile split along K (`_stream_split`). For M <= _STREAM_TINY_M the 16 x 32 tile (few
# activation rows for every block to re-read, and narrower blocks give more of them), else the 16 x 64 tile with 4 K slices
# (its activations, re-read by every block, are amortized over twice the columns); the most splits of
# _STREAM_SPLIT_COUNTS that keep the workgroups within one per CU and each K range at least
# _STREAM_SPLIT_MIN_RANGE deep; and no split when that
# leaves _STREAM_SPLIT_MIN_WORKGROUPS or fewer workgroups (the unsplit rule's narrower tiles then do better).
# With one row of tiles, workgroup counts just past the CU count lose 10-25% (some CUs run two), hence the
# one-per-CU cap; each further row of tiles raises it by _STREAM_SPLIT_CAP_PER_ROW.
_STREAM_SPLIT_MIN_K = 8192
_STREAM_SPLIT_MAX_TILES = 171
_STREAM_TINY_M = 12
_STREAM_SPLIT_COUNTS = (8, 6, 4, 3, 2)
_STREAM_SPLIT_MIN_RANGE = 3072
_STREAM_SPLIT_MIN_WORKGROUPS = 128
_STREAM_SPLIT_CAP_PER_ROW = 64
# M > 64 (five or more rows of 16-row tiles), measured on a 96-cell grid (M 80-256, N 1024-3072, K 6144-16384,
# fp16 and bf16, graph replays, cold weights):
# - the long-K split keeps within one workgroup per CU (the per-row allowance above let 160-tile grids split
#   into 320 workgroups: 0.83-0.85x the unsplit tile);
# - one round of unsplit 16 x 64 blocks with K >= 6144 takes the tile with more weight in flight, the weight's
#   re-reads then coming from the caches: 128-deep steps (fp16 1.03-1.11x over the 4-slice 64-deep tile on every
#   such cell; bf16 from K = 12288) or 8 K slices (bf16 below K = 12288, 1.04-1.12x);
# - the ring tiles' split-K needs enough tiles: with fewer than 36 64 x 128 tiles it lost on every cell
#   (0.50-0.94x at 16-32 tiles, where 8 splits still leave CUs idle and each split is short); with 36-79 it won
#   only on weights of 18 MiB and more (N x K 1536 x 12288 on: 0.99-1.0 of the best; 12.6-16.8 MB 0.83-0.88),
#   and with bf16 activations (widened in registers on that ring) only from 64 tiles (0.70-0.84x at 36-48);
# - the 32-row streaming tile's one-round rule (`_STREAM_32_MIN_BLOCKS`) holds at K >= 6144 only from M = 160
#   (at M 80-128 the deeper 16-row tiles are 1.1-1.3x faster there).
_STREAM_DEEP_MIN_K = 6144
_STREAM_DEEP_KS8_MAX_K_BF16 = 12288
_RING_SPLIT_MIN_TILES = 80
_RING_SPLIT_FEW_TILES = 36
_RING_SPLIT_FEW_TILES_BF16 = 64
_RING_SPLIT_FEW_TILES_MIN_WEIGHT = 18 << 20
_STREAM_32_LONG_K_MIN_M = 160
# Except: M <= _STREAM_UNSPLIT_TINY_M on a weight whose 16-column fragments fill one round of 192-256 blocks
# (N 3072-4096) and K up to _STREAM_UNSPLIT_MAX_K runs unsplit on the 16 x 16 tile, which keeps three fetches
# in flight per wave: 1.02-1.2x over the 16 x 32 tile split 2 ways on 21 of 24 cells (M 1-4, K 8192-16384;
# same-box A/B, cold weights), while at K 18944-28672 splitting stays ahead or even.
_STREAM_UNSPLIT_TINY_M = 4
_STREAM_UNSPLIT_MAX_K = 16384

# bf16 activations: the auto path widens them once up front (feather_ops::widen_bf16, the kernels' own
# round-to-nearest-even conversion, so the result is the same bits) and runs the fp16-activation kernel when
# that kernel's lead over widening in place repays the pass. Its lead, as a fraction of the fp16 kernel's
# time, measured over the tile-sweep grid: 15-23% where the fp16 pick is the 128 x 256 block of 128 x 64 waves
# (the bf16 form of that block runs 2 x 2 waves without the reads-first schedule: its register-staged
# activations leave no room for it), 4-16% on the 128 x 128 and 64 x 128 tiles, where it varies by more than
# the pass costs (taken at the low end, so no grid cell runs slower; it grows with K: on 128 x 128 6-9% from
# K = 4608 on against 0-3% at K <= 2560 on two boxes, modelled as 0.14 (1 - 1024 / K) for both tiles). The pass moves 4 bytes per
# activation element at ~6.2 TB/s and costs at least ~4 us of launch; the fp16 kernel's time is modelled at
# 1.2 PFLOP/s; the lead has to exceed the pass by a fifth. Split launches keep the in-place widening, except
# on the 64 x 64 tile for M <= 64: that regime runs the deep ring, which widens bf16 per fragment after each
# LDS read, and its lead is 17-22% (split or not) on weights of 100 MB and more (the pass costs its ~4 us
# launch there), with the kernel's time set by the weight read (modelled at 4 TB/s).
_WIDEN_LEAD_W64 = 0.17
_WIDEN_LEAD_SMALL = 0.14   # the 128 x 128 and 64 x 128 tiles: times (1 - _WIDEN_LEAD_SMALL_K0 / K)
_WIDEN_LEAD_SMALL_K0 = 1024
_WIDEN_LEAD_DEEP_64x64 = 0.2
_WIDEN_DEEP_MAX_M = 64
_WIDEN_WEIGHT_BYTES_PER_S = 4e12
_WIDEN_FLOPS = 1.2e15
_WIDEN_BYTES_PER_S = 6.2e12
_WIDEN_MIN_S = 4e-6
_WIDEN_MARGIN = 1.2


def _blocks(M: int, N: int, tile: tuple[int, ...]) -> int:
    bm, bn, _ = gemm_block_sizes(tile)
    return -(-M // bm) * -(-N // bn)


def _stream_reread(M: int, N: int, K: int) -> float:
    """Weight bytes the 16 x 64 streaming tile reads (once per 16 rows), over the fraction of the CU
    slots its blocks fill in their last round."""
    blocks = _blocks(M, N, _TILE_STREAM_16x64)
    return -(-M // 16) * N * K * (_CUS * -(-blocks // _CUS)) / blocks


def _stream_split(M: int, N: int, K: int) -> tuple[tuple[int, int, int, int, int, int], int] | None:
    """(tile, splits) for the long-K streaming regime, or None where the unsplit streaming rule applies (see
    _STREAM_SPLIT_MIN_K above). Measured with the tile sweep on 48 decoder-shaped cells (M 1-32, N 2048-28672,
    K 3072-28672) and the grid's skinny cells, fp16 and bf16, graph-timed with cold weights."""
    if M <= _STREAM_UNSPLIT_TINY_M and 3 * _CUS // 4 <= N // 16 <= _CUS and K <= _STREAM_UNSPLIT_MAX_K:
        return None
    tiny = M <= _STREAM_TINY_M
    tile = _TILE_STREAM_16x32 if tiny else _TILE_STREAM_16x64_KS4
    tiles = _blocks(M, N, tile)
    # more row tiles share each weight panel (its second read hits the caches), and tolerate a few more
    # workgroups than CUs: 32 x 5120 x 13824 runs 1.27x faster split 2 ways (320 workgroups) than unsplit
    cap = _CUS if M > 64 else _CUS + _STREAM_SPLIT_CAP_PER_ROW * (-(-M // 16) - 1)
    for splits in _STREAM_SPLIT_COUNTS:
        if tiles * splits <= cap and K // splits >= _STREAM_SPLIT_MIN_RANGE:
            if tiles * splits > _STREAM_SPLIT_MIN_WORKGROUPS or tiles * splits > _stream_unsplit_shape(M, N)[1]:
                return tile, splits
            return None
    # no split within the cap: from 129 tiles of 16 x 64 on, that tile split 3 ways (two workgroups on most CUs)
    # still beats the unsplit tile for M > 4 (12 x 10240 x 16384, 160 tiles: 1.03x; M <= 2: 0.96x); at 176 tiles
    # it no longer does (above the regime's tile limit)
    if M > 4 and _blocks(M, N, _TILE_STREAM_16x64_KS4) > 128 and K // 3 >= _STREAM_SPLIT_MIN_RANGE:
        return _TILE_STREAM_16x64_KS4, 3
    return None


def _stream_unsplit_shape(M: int, N: int) -> tuple[int, int]:
    """(repeat_n, blocks) of the unsplit 16-row streaming tile `select_scaled_mm_config` falls back to: as wide
    as still gives 160 blocks (64, 32 or 16 columns)."""
    rows = -(-M // 16)
    for repeat_n in (4, 2, 1):
        if rows * (N // (16 * repeat_n)) >= 160:
            break
    blocks = {rn: rows * -(-N // (16 * rn)) for rn in (4, 2, 1)}
    if rows == 1 and _CUS < blocks[repeat_n] <= _CUS * 3 // 2:
        # one row of blocks and a small second round (some CUs run two blocks, most one): a width that keeps
        # within one round (at least 128 blocks) or spreads over more than 1.5 rounds does better (1 x 17408 x
        # 18432 on 32 columns: 1.08x; 16 x 21504 x 4096: 1.04x; 1 x 4608 x 12288 on 32 columns, 144 blocks
        # against 288 of 16 columns: 1.45x)
        fits = [rn for rn in (4, 2, 1) if _CUS // 2 <= blocks[rn] <= _CUS]
        spread = [rn for rn in (4, 2, 1) if blocks[rn] > _CUS * 3 // 2]
        repeat_n = (fits or spread or [repeat_n])[0]
    return repeat_n, blocks[repeat_n]


def _small_grid_time(M: int, N: int, K: int, tile: tuple[int, ...], splits: int, a_bf16: bool) -> float:
    """Modelled time of a ring tile split `splits` ways on a small grid (arbitrary units): the busiest CU
    runs ceil(workgroups / CUs) workgroups, as many at once as fit, each round at the rate its resident count
    reaches, plus a fixed cost per workgroup."""
    bm, bn, _ = gemm_block_sizes(tile)
    workgroups = _blocks(M, N, tile) * splits
    if tile == _TILE_RING_128x128:
        per_cu = 3
    else:
        per_cu = 2 if ring_is_deep(M, N, tile, splits, a_bf16) else 5
    rate, efficiency = _SMALL_GRID_RATE[tile]
    work = bm * bn * K / splits
    left = -(-workgroups // _CUS)
    time = left * bm * bn * _SMALL_GRID_BLOCK_K / rate
    while left > 0:
        resident = min(per_cu, left)
        time += resident * work / (rate * efficiency[min(resident, 3) - 1])
        left -= resident
    return time


def _small_grid_choice(M: int, N: int, K: int, a_bf16: bool) -> tuple[tuple[int, int, int, int, int, int], int]:
    """(tile, splits) with the least modelled time among the 64 x 128 and 128 x 128 ring tiles and their
    split counts (each split at least 16 stages of 64, partial sums within _SPLIT_MAX_PARTIAL_BYTES)."""
    best = None
    for tile in (_TILE_RING_64x128, _TILE_RING_128x128):
        bm, bn, _ = gemm_block_sizes(tile)
        for splits in range(1, _SMALL_GRID_MAX_SPLITS[tile] + 1):
            if splits > 1 and (-(-K // 64) // splits < _SPLIT_MIN_STAGES or
                               _blocks(M, N, tile) * splits * bm * bn * 4 > _SPLIT_MAX_PARTIAL_BYTES):
                break
            time = _small_grid_time(M, N, K, tile, splits, a_bf16)
            if best is None or time < best[0]:
                best = (time, tile, splits)
    return best[1], best[2]


def _ring_time(M: int, N: int, tile: tuple[int, ...], per_cu: int, tflops: float) -> float:
    """Relative time of a ring tile: whole waves of `_CUS * per_cu` blocks, each wave as long as a full one."""
    bm, bn, _ = gemm_block_sizes(tile)
    waves = -(-_blocks(M, N, tile) // (_CUS * per_cu))
    return waves * _CUS * per_cu * bm * bn / tflops


def select_scaled_mm_config(
    M: int,
    N: int,
    K: int,
    a_dtype: torch.dtype = torch.float16,
    b_dtype: torch.dtype = torch.float8_e5m2,
    out_dtype: torch.dtype = torch.bfloat16,
) -> tuple[int, int, int, int, int, int]:
    """Static tile choice for one shape (same signature as the reference's `scaled_mm.py:35-42`).

    Fitted on MI355X with the tile sweep over the benchmark grid (112 cells, every tile and split count;
    with `select_scaled_mm_splits` the pick is within 0.7% of the best candidate in geometric mean) and
    extra cells where the grid had few:
    - M > 64 and at least one CU's worth of 128 x 128 tiles, fp16 activations, K >= 3072 (a multiple of 64), and
      one round of 256 x 192 tiles at least 205 / 256 full: the 256 x 192 wide tile, 1.02-1.11x the best other
      tile there (`_wide192_fits`).
    - Else the same, on the wide tile's grid (M and N multiples of 256, K of 64) with K >= 3072 and a last round
      of 256 x 256 tiles whole or at least 170 / 256 full (or at least 1700 tiles): the 256 x 256 wide tile,
      1.01-1.07x the ring tiles there (`_wide_fits`).
    - Otherwise M > 64 and at least one CU's worth of 128 x 128 tiles: the ring tile whose whole waves of resident
      blocks finish first (a wave-quantization model over 128 x 256, 256 x 256, 128 x 128 and 64 x 128
      tiles with their measured full-grid rates); the 128 x 256 block as 4 column waves of 128 x 64 with
      fp16 activations, as 2 x 2 waves of 64 x 128 with bf16 ones.
    - M > 64 with a smaller grid and K >= 4096, once the 16-row streaming tile would read 216 MiB of
      weight or more (N * K bytes once per 16 rows, over the fraction of CU slots its blocks fill in their
      last round), given at least 80 64 x 128 tiles, or 36 (bf16 activations: 64) on a weight of 18 MiB or
      more (with fewer, the split ring lost to the streaming tiles on every cell of a 96-cell grid, 0.50-0.94x):
      the 64 x 128 ring tile (deep ring) up to 256 of its tiles, split along K
      (`select_scaled_mm_splits`); beyond that the 64 x 128 or 128 x 128 ring tile and split count with the
      least modelled time (`_small_grid_choice`: 0.990 of the best candidate in geometric mean on 58 fp16
      cells of that regime, 0.994 on 30 held-out ones and 0.994 / 0.983 with bf16 activations, against
      0.933 / 0.978 / 0.910 / 0.967 for the rule it replaced, which took the 128 x 128 tile split for two
      workgroups per CU: 448 x 6144 x 8192 runs 814 TFLOP/s on the 64 x 128 tile split 3 ways against 679).
      Below that the streaming tiles' re-reads hit the caches and they win: 192 x 4096 x 4096 (768 blocks,
      201 MB) streams at 461 TFLOP/s against 407 for the best split ring; 128 x 3072 x 8192 (384 blocks, 268 MB
      by the measure) runs 363 on the ring against 323 streaming. With bf16 activations from 288 MiB (the
      shallow ring widens them in registers): 128 x 5120 x 5120 streams at 320 TFLOP/s against 295 on the ring.
    - M > 64 otherwise: the 64 x 64 ring tile once it gives 512 blocks; for M > 768 also when it (split
      along K where that fills more CU slots) fills three quarters of the CU slots in its last round
      (1024 x 1024 x 3072 split 2 ways: 453 TFLOP/s against 397 streaming; with fp16 activations only,
      bf16 ones stream faster there); else streaming.
    - 16 < M <= 64 with a big weight: the 64-row ring tiles, which read the weight once where the 16-row
      streaming tiles read it once per 16 rows (on small grids they run their deep-ring variant): from a
      40 MiB weight (N * K bytes; 96 MiB when M <= 32) the 64 x 128 tile from 320 of its tiles on, else
      the 64 x 64 tile, split along K to fill the CUs (`select_scaled_mm_splits`); for 16 < M <= 32 also
      the 64 x 128 tile from 512 of its tiles on.
    - M <= 16 with 512 to 1024 64 x 128 tiles (N from 65536 to 131072, LM-head widths): that ring tile,
      whose direct-to-LDS weight stream runs 5-12% faster than the streaming tiles there; beyond 1024
      tiles the second, partial wave of blocks makes it slower.
    - 16 < M <= 32: the 32-row streaming tile when it gives more than 384 blocks, or 192-256 (one round:
      1.03-1.28x over two rows of the 16 x 64 tile on 24 cells, M 20-32, N 12288-16384, K 4096-5120, with
      three fetches in flight; at 288 blocks the small second round loses 6%).
    - 64 < M <= 512 where the rules above leave a streaming tile, fp16 activations: the 32-row streaming tile when it
      gives one round of 144-256 blocks or two of 392-512 (at K >= 6144 only from M = 160), which reads the weight half as often as the 16-row tiles (M 96-192, N x K
      2560^2-4096^2: 1.01-1.15x on the 6 such cells of a 48-cell sweep, each of the 3 outside that range
      0.83-0.94x; on 18 held-out cells, M 80-256, 1.01-1.21x on 16 and 0.989-0.998x on 2; at M 320-512 the best
      candidate on all 36 cells of a sweep, 1.03-1.26x; two rounds of 392-512 blocks 0.998-1.149x on 7 cells, where
      288-360 blocks lose). Not with bf16 activations (0.72-0.92x on the 18 cells).
    - K >= 8192 with at most 170 16 x 64 streaming tiles: the 16 x 32 tile (8 K slices) for M <= 12, the
      16 x 64 tile (4 K slices) above, split along K to at most one workgroup per CU (for M <= 64 plus 64 per
      further row of tiles) (`select_scaled_mm_splits`), where that gives more workgroups than the unsplit
      rule below.
    - Otherwise the 16-row split-K streaming tile, as wide as still gives 160 blocks (64, 32 or 16
      columns): 16 x 64 with 4 K slices, the narrower ones with 8 up to one block per CU and 4 beyond; for
      M > 64 and K >= 6144, one round of 16 x 64 blocks keeps more weight in flight: 128-deep steps with fp16
      activations (1.03-1.11x), 8 K slices with bf16 ones below K = 12288 and 128-deep steps from it
      (1.04-1.12x). Over the 96-cell grid these M > 64 rules took the picks from 0.923 to 0.988 of the best
      candidate (bf16 0.915 to 0.975), and on 60 held-out cells (M 72-240, N 1280-3584, K 5120-14336) from
      0.952 to 0.968 (bf16 0.927 to 0.966).
    The streaming picks were refitted after the streaming kernel's loop kept two fetches in flight per wave
    (it had been one): on 193 swept cells with M <= 256 the picks are at 0.994 of the best candidate in
    geometric mean, against 0.953 for the rules before.
    """
    del b_dtype, out_dtype
    a_bf16 = a_dtype == torch.bfloat16
    tiles_128 = _blocks(M, N, _TILE_RING_128x128)
    if M > 64 and tiles_128 >= _CUS:
        if not a_bf16 and _wide192_fits(M, N, K):
            return _TILE_WIDE_192
        if not a_bf16 and _wide_fits(M, N, K):
            return _TILE_WIDE
        return min(_RING_MODEL if a_bf16 else _RING_MODEL_FP16, key=lambda entry: _ring_time(M, N, *entry))[0]
    min_reread = _BF16_RING_MIN_REREAD if a_bf16 else _RING_MIN_REREAD
    ring_tiles = _blocks(M, N, _TILE_RING_64x128)
    few_tiles = _RING_SPLIT_FEW_TILES_BF16 if a_bf16 else _RING_SPLIT_FEW_TILES
    ring_split = (M > 64 and K >= _SPLIT_MIN_K and _stream_reread(M, N, K) >= min_reread
                  and (ring_tiles >= _RING_SPLIT_MIN_TILES
                       or (ring_tiles >= few_tiles and N * K >= _RING_SPLIT_FEW_TILES_MIN_WEIGHT)))
    if ring_split and _blocks(M, N, _TILE_RING_64x128) <= _CUS:
        return _TILE_RING_64x128
    if ring_split:
        return _small_grid_choice(M, N, K, a_bf16)[0]
    if M > 64 and _blocks(M, N, _TILE_RING_64x64) >= 2 * _CUS:
        return _TILE_RING_64x64
    if 16 < M <= 64 and N * K >= (_MID_M_RING_MIN_WEIGHT if M > 32 else _MID_M_RING_MIN_WEIGHT_32):
        wide = _blocks(M, N, _TILE_RING_64x128) >= _MID_M_WIDE_TILES
        return _TILE_RING_64x128 if wide else _TILE_RING_64x64
    if M <= 32:
        ring_tiles = _blocks(M, N, _TILE_RING_64x128)
        if ring_tiles >= 2 * _CUS and (M > 16 or ring_tiles <= 4 * _CUS):
            return _TILE_RING_64x128
    blocks_32 = _blocks(M, N, _TILE_STREAM_32x64)
    if 16 < M <= 32 and (blocks_32 > 3 * _CUS // 2 or 3 * _CUS // 4 <= blocks_32 <= _CUS):
        return _TILE_STREAM_32x64
    if K >= _STREAM_SPLIT_MIN_K and _blocks(M, N, _TILE_STREAM_16x64) < _STREAM_SPLIT_MAX_TILES:
        split = _stream_split(M, N, K)
        if split is not None:
            return split[0]
    if M > 768 and not a_bf16 and _ring_splits(M, N, K, _TILE_RING_64x64)[1] >= _BIG_M_RING_MIN_BUSY:
        return _TILE_RING_64x64
    if (64 < M <= _STREAM_32_MAX_M and not a_bf16
            and (_STREAM_32_MIN_BLOCKS <= blocks_32 <= _CUS or _STREAM_32_TWO_ROUND_MIN_BLOCKS <= blocks_32 <= 2 * _CUS)
            and (K < _STREAM_DEEP_MIN_K or M >= _STREAM_32_LONG_K_MIN_M)):
        return _TILE_STREAM_32x64
    repeat_n, blocks = _stream_unsplit_shape(M, N)
    if M > 64 and repeat_n == 4 and blocks <= _CUS and K >= _STREAM_DEEP_MIN_K:
        return _TILE_STREAM_16x64 if a_bf16 and K < _STREAM_DEEP_KS8_MAX_K_BF16 else _TILE_STREAM_16x64_U8
    # 8 K slices while the blocks fit one per CU, 4 beyond; the 64-column tile takes 4 either way (its 8-slice
    # form keeps twice the weight in flight, past what the HBM serves best: C4 2.5% slower with it)
    return (8 if blocks <= _CUS and repeat_n < 4 else 4, 1, 4, 1, repeat_n, 0)


def select_scaled_mm_splits(M: int, N: int, K: int, tile: tuple[int, ...],
                            a_dtype: torch.dtype = torch.float16) -> int:
    """K splits for a tile `select_scaled_mm_config` picked (1: none). Not in the reference, whose kernel
    has no split-K.

    Three split regimes of `select_scaled_mm_config`:
    - M > 64, K >= 4096, fewer 128 x 128 tiles than CUs: with at most 256 64 x 128 tiles, that tile splits
      into 2 to 8 K ranges of at least 16 stages of 64 deep, for at most 512 workgroups (two per CU): the
      count whose workgroups fill the largest fraction of the CUs in their last round, the larger count
      on a tie (80 tiles: 3 splits, 240 workgroups, 371 TFLOP/s at 128 x 5120 x 5120 against 323 for 4
      and 330 for 6). With bf16 activations the 64 x 128 tile takes up to three workgroups per CU (768):
      1040 x 1536 x 6144 584 TFLOP/s split 3 ways against 532 for 2. Measured 5-40% faster than the best
      unsplit tile on the grid's cells in that regime. With more 64 x 128 tiles, the split count of the
      model that chose the tile (`_small_grid_choice`, 1 to 4).
    - M > 768 on the 64 x 64 ring tile with fewer than 512 tiles: the same rule (at least one split).
      1000 x 1000 x 2560 and 1024 x 1024 x 3072 (256 tiles): 2 splits, 394 and 453 TFLOP/s against 329
      and 358 unsplit.
    - K >= 8192 with at most 170 16 x 64 streaming tiles (skinny M, narrow N, long K: a decoder's down
      projection), on the streaming tile `select_scaled_mm_config` picks there (`_stream_split`): the most of
      8, 6, 4, 3, 2 splits that keep the workgroups within one per CU (plus 64 per further row of 16-row
      tiles) and every K range at least 3072 deep, where that gives more than 128 workgroups or more than the
      unsplit rule would; else 3 splits of the 16 x 64 tile from 129 of its tiles on when M > 4. Workgroup
      counts just past the CU count lose 10-25% (1 x 5120 x 13824 on 16 x 32: 160 workgroups 1.0, 320 0.75,
      480 0.90); 2 x 4096 x 16384 runs 1.05x faster split 2 ways on 16 x 32 than split 3 ways on the
      8-slice 16 x 64 tile the rule before took, 16 x 2048 x 8192 1.27x faster on the unsplit 16 x 16 tile.
    - 16 < M <= 64 on the 64 x 64 ring tile: the split count of a residency model (`_mid_m_ring_splits`,
      1 to 8 splits of at least 16 stages), which matches the measured best on every such cell of the
      sweeps: 64 x 16384 x 4096 2 splits (414 TFLOP/s against 360 unsplit), 64 x 5120 x 13824 6 (379 against
      130), 32 x 11264 x 11264 4 (1.18x the 2 of the ~512-workgroup rule before). On the 64 x 128 tile:
      about 512 workgroups, one split less when the last round would fill under a quarter of the CUs.
    Shorter K loses: the per-split fixed costs (pipeline fill, the partial sums' round trip through
    memory, the workspace lookup on the host) dominate.
    """
    tile = tuple(tile)
    big_weight = N * K >= (_MID_M_RING_MIN_WEIGHT if M > 32 else _MID_M_RING_MIN_WEIGHT_32)
    if tile in (_TILE_RING_64x64, _TILE_RING_64x128) and 16 < M <= 64 and big_weight:
        if tile != select_scaled_mm_config(M, N, K, a_dtype):
            return 1
        return _mid_m_ring_splits(M, N, K, tile, a_dtype == torch.bfloat16)
    if tile == _TILE_RING_64x128 and 16 < M <= 64:
        if tile != select_scaled_mm_config(M, N, K, a_dtype):
            return 1
        tiles = _blocks(M, N, tile)
        splits = max(1, min(8, round(_MID_M_RING_BLOCKS / tiles), -(-K // 64) // _SPLIT_MIN_STAGES))
        # A last round of workgroups that fills under a quarter of the CUs costs a whole round: one split less
        # (40 x 8448 x 10496, 132 tiles: 3 splits 270 TFLOP/s, 4 splits = 528 workgroups 228).
        if splits > 1 and 0 < (tiles * splits) % _CUS < _CUS // 4:
            splits -= 1
        return splits
    if tile in (_TILE_STREAM_16x32, _TILE_STREAM_16x64_KS4) and K >= _STREAM_SPLIT_MIN_K:
        if _blocks(M, N, _TILE_STREAM_16x64) >= _STREAM_SPLIT_MAX_TILES:
            return 1
        split = _stream_split(M, N, K)
        if split is None or split[0] != tile or tile != select_scaled_mm_config(M, N, K, a_dtype):
            return 1
        return split[1]
    if tile == _TILE_RING_64x64 and M > 768:
        return _ring_splits(M, N, K, tile)[0] if tile == select_scaled_mm_config(M, N, K, a_dtype) else 1
    if M <= 64 or K < _SPLIT_MIN_K or tile not in (_TILE_RING_128x128, _TILE_RING_64x128):
        return 1
    if tile != select_scaled_mm_config(M, N, K, a_dtype):
        return 1
    tiles_128 = _blocks(M, N, _TILE_RING_128x128)
    if tiles_128 >= _CUS:
        return 1
    if _blocks(M, N, _TILE_RING_64x128) > _CUS:
        return _small_grid_choice(M, N, K, a_dtype == torch.bfloat16)[1]
    wide_bf16 = a_dtype == torch.bfloat16 and tile == _TILE_RING_64x128
    return _ring_splits(M, N, K, tile, least=2, per_cu=3 if wide_bf16 else 2)[0]


def _mid_m_ring_splits(M: int, N: int, K: int, tile: tuple[int, ...] = _TILE_RING_64x64,
                       a_bf16: bool = False) -> int:
    """Splits of a 64-row ring tile for 16 < M <= 64 and a big weight: the count with the least modelled time,
    where the busiest CU runs ceil(workgroups / CUs) workgroups of 1 / splits of a tile each (all resident at
    once, up to _MID_M_MAX_PER_CU per CU), a block alone on its CU at _MID_M_LONE_RATE of the rate,
    and each split costs _MID_M_SPLIT_COST of a tile's time; counts of _STREAM_SPLIT_COUNTS (the measured
    ones), at least 16 stages of 64 per split. It matches the
    best measured count on every mid-M cell of the sweeps (e.g. 176 tiles: 4 splits, 1.18x faster than the 2 of
    the ~512-workgroup rule it replaced; 80 tiles: 6; 224 tiles: 2)."""
    tiles = _blocks(M, N, tile)
    staged = a_bf16 and tile == _TILE_RING_64x128   # bf16 on its 4 column waves: the register-staged ring
    rates = _MID_M_STAGED_RATES if staged else (_MID_M_LONE_RATE,) + (1.0,) * 3
    best = (float("inf"), 1)
    for splits in (1,) + _STREAM_SPLIT_COUNTS[::-1]:
        if splits > 1 and -(-K // 64) // splits < _SPLIT_MIN_STAGES:
            break
        per_cu = -(-tiles * splits // _CUS)
        if per_cu > (4 if staged else _MID_M_MAX_PER_CU[tile]):
            break
        time = per_cu / splits / rates[per_cu - 1] + _MID_M_SPLIT_COST * splits
        best = min(best, (time, splits))
    return best[1]


def _ring_splits(M: int, N: int, K: int, tile: tuple[int, ...], least: int = 1,
                 per_cu: int = 2) -> tuple[int, float]:
    """(splits, fraction of the CU slots its workgroups fill in their last round) for a ring tile on a
    small grid: of `least` to 8 splits of at least 16 stages each and at most `per_cu` workgroups per CU,
    the count that fills the most slots, the larger count on a tie."""
    tiles = _blocks(M, N, tile)
    most = max(least, min(8, (per_cu * _CUS) // tiles, -(-K // 64) // _SPLIT_MIN_STAGES))

    def busy(splits: int) -> float:
        return tiles * splits / (_CUS * -(-tiles * splits // _CUS))

    splits = max(range(least, most + 1), key=lambda s: (busy(s), s))
    return splits, busy(splits)


def widen_first(M: int, N: int, K: int, tile: tuple[int, ...], splits: int) -> bool:
    """Whether bf16 activations of this shape are widened once up front and run on `tile` (the fp16-activation
    pick, unsplit) rather than widened inside the kernel; not in the reference, whose kernel always widens in
    place. On the tile-sweep grid (`benchmark_scaled_mm_hip --a-dtype bf16 --widen-all`, 112 cells) it widens
    52 cells first, none slower than in place (1.01-1.23x, 1.14x in geometric mean; C3's shape 1.10-1.14x):
    1.063x over the whole grid against 1.068x for the better form per cell. That takes the 128 x 256 block
    on wide weights, the 128 x 128 and 64 x 128 tiles at long K (4096x4608x4608 1.08x, 4608x4096x16384 1.09x,
    1072x5120x8192 1.11x) and, with
    M <= 64, the 64 x 64 tile on big weights (32x25600x5120 1.19x, 32x8192x28672 split 4 ways 1.22x)."""
    kernel_s = 2.0 * M * N * K / _WIDEN_FLOPS
    if M <= _WIDEN_DEEP_MAX_M and tuple(tile) == _TILE_RING_64x64:
        lead = _WIDEN_LEAD_DEEP_64x64
        kernel_s = max(kernel_s, N * K / _WIDEN_WEIGHT_BYTES_PER_S)
    elif splits > 1:
        lead = 0.0
    elif tuple(tile) in (_TILE_RING_128x256_W64, _TILE_WIDE, _TILE_WIDE_192):
        lead = _WIDEN_LEAD_W64
    elif tuple(tile) in (_TILE_RING_128x128, _TILE_RING_64x128):
        lead = max(0.0, _WIDEN_LEAD_SMALL * (1.0 - _WIDEN_LEAD_SMALL_K0 / K))
    else:
        lead = 0.0
    widen_s = max(_WIDEN_MIN_S, 4.0 * M * K / _WIDEN_BYTES_PER_S)
    return lead * kernel_s > _WIDEN_MARGIN * widen_s


@functools.lru_cache(maxsize=4096)
def _auto_choice(M: int, N: int, K: int,
                 a_dtype: torch.dtype) -> tuple[tuple[int, int, int, int, int, int], int, bool]:
    """(tile, splits, widen first) the heuristic picks for a shape, memoized: a model runs the same few shapes
    again and again, and the auto path then skips the model arithmetic (1-5 us of Python per call). With
    `widen first` the tile and splits are the fp16-activation pick."""
    if a_dtype == torch.bfloat16:
        tile = select_scaled_mm_config(M, N, K, torch.float16)
        splits = select_scaled_mm_splits(M, N, K, tile, torch.float16)
        if widen_first(M, N, K, tile, splits):
            return tile, splits, True
    tile = select_scaled_mm_config(M, N, K, a_dtype)
    return tile, select_scaled_mm_splits(M, N, K, tile, a_dtype), False


# Split-K workspaces, one per (device, stream): the counter area at their start must be zero before a
# launch, and every completed launch leaves it zero whatever its shape, so a workspace is zeroed once, when
# it is created, and then reused by the launches of its stream, which are ordered. Other streams get their
# own. Keys are stream handles: torch's streams come from per-device pools and are never destroyed, so a
# handle is never reused for an unrelated stream (an external stream destroyed while work on it is pending
# and recreated at the same address would break this; such streams should not share the cache).
_split_workspaces: dict[tuple[int, int], torch.Tensor] = {}


# The workspace size per (M, N, K, tile, splits): the formula costs ~2 us of Python per call, the cache 0.2.
_workspace_bytes = functools.lru_cache(maxsize=4096)(split_workspace_bytes)


def _split_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        # Under graph capture the zero fill is recorded with the launch, so every replay starts clean.
        return torch.zeros(nbytes, dtype=torch.uint8, device=device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    # The raw handle of the current stream (what torch.cuda.current_stream(device).cuda_stream returns,
    # without building a Stream object: a few microseconds less per launch).
    key = (index, torch._C._cuda_getCurrentRawStream(index))
    ws = _split_workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _split_workspaces[key] = ws
    return ws


def clear_split_workspaces() -> None:
    """Release the cached split-K workspaces (they are recreated, zeroed, on the next split launch).

    Call it only when no split launch is still running on the streams whose workspaces are dropped, e.g.
    after `torch.cuda.synchronize()`; the memory returns to torch's caching allocator.
    """
    _split_workspaces.clear()


_STREAMING_MODES = ("off", "on", "auto")


def set_weight_streaming(mode: str | None = None) -> str:
    """Choose non-temporal weight loads for every later launch in this process and return the previous mode
    (with `mode=None`, only return the current one). A launch whose M fits one row of its tile reads every
    weight byte once, and then loads the weight non-temporally:

    - "auto" (the default): when the prepacked weight holds at least 48 MiB;
    - "on": always;
    - "off": never.

    A cache hint only; results are the same in every mode. It pays when the weight streams from HBM on every
    launch (a model far larger than the GPU's 256 MB MALL: 4-9% on weights of 59-235 MB) and costs when the
    working set would stay in the MALL (up to a third slower): "off" suits small models and one weight timed
    in a loop. The environment variable FEATHER_OPS_WEIGHT_STREAMING (0, 1 or 2) sets the first value. C ABI:
    `feather_set_weight_streaming`. No counterpart in the reference."""
    if mode is not None and mode not in _STREAMING_MODES:
        raise ValueError(f"weight streaming mode must be one of {_STREAMING_MODES}, got {mode!r}")
    previous = _lib.c_library().feather_set_weight_streaming(-1 if mode is None else _STREAMING_MODES.index(mode))
    return _STREAMING_MODES[previous]


def _launch(
    a: torch.Tensor,
    b_prepacked: torch.Tensor,
    scale: torch.Tensor | None,
    bias: torch.Tensor | None,
    out: torch.Tensor,
    tile: tuple[int, int, int, int, int, int],
    splits: int = 1,
    widen: bool = False,
) -> None:
    if widen and a.is_cuda and a.dim() == 2 and a.is_contiguous() and a.numel() < (1 << 30):
        # an fp16 copy of the bf16 activations, rounded as the kernels round them; activations the op would
        # refuse are passed on as they are, so that it reports them as it does without the widening
        wide = torch.empty(a.shape, dtype=torch.float16, device=a.device)
        torch.ops.feather_ops.widen_bf16.default(a, wide)
        a = wide
    if splits == 1:
        torch.ops.feather_ops.scaled_mm.default(a, b_prepacked, scale, bias, out, *tile)
        return
    if a.shape[0] == 0:  # an empty batch: the op checks its arguments and launches nothing
        ws = torch.empty(0, dtype=torch.uint8, device=a.device)
    else:
        nbytes = _workspace_bytes(a.shape[0], b_prepacked.shape[1], a.shape[1], tuple(tile), splits)
        if nbytes < 0:
            raise RuntimeError(
                f"split-K needs an instantiated tile and 1 <= splits <= the K units, got {tile}, {splits}")
        ws = _split_workspace(a.device, nbytes)
    torch.ops.feather_ops.scaled_mm_splitk.default(a, b_prepacked, scale, bias, out, ws, splits, *tile)


@custom_op("feather_ops::scaled_mm_auto", mutates_args=("out",))
def _scaled_mm_auto(
    a: torch.Tensor,
    b_prepacked: torch.Tensor,
    scale: torch.Tensor | None,
    bias: torch.Tensor | None,
    out: torch.Tensor,
) -> None:
    """The auto-picked launch inside one custom op: a compiled graph holds a single node for it, whichever
    tile, split count or widening the shape leads to."""
    _launch(a, b_prepacked, scale, bias, out, *_auto_choice(a.shape[0], b_prepacked.shape[1], a.shape[1], a.dtype))


def scaled_mm_hip(
    a: torch.Tensor,
    b_prepacked: torch.Tensor,
    scale: torch.Tensor | None,
    bias: torch.Tensor | None,
    out_dtype: torch.dtype,
    tile: tuple[int, int, int, int, int, int] | None = None,
    splits: int | None = None,
) -> torch.Tensor:
    """Returns `a @ W^T`, times `scale`, plus `bias`, in `out_dtype`, for the fp8 weight W held prepacked
    in `b_prepacked`.

    Without `tile` the heuristic chooses the launch; passing one (as the tile sweeps and tests do) runs
    exactly that tile, unsplit unless `splits` (not in the reference) asks for a split-K count.

    The heuristic's launch goes through the opaque custom op `feather_ops::scaled_mm_auto` while
    `torch.compile` traces (as in the reference, `scaled_mm.py:104-134`), and straight to the launcher in
    eager mode: the same launch without the custom op's Python dispatch, about 7 us of host time per call,
    which is more than a decode-sized kernel takes.
    """
    _lib.require_native()
    out = torch.empty((a.shape[0], b_prepacked.shape[1]), device=a.device, dtype=out_dtype)
    if tile is None and splits is None:
        if torch.compiler.is_compiling():
            _scaled_mm_auto(a, b_prepacked, scale, bias, out)
        else:
            _launch(a, b_prepacked, scale, bias, out, *_auto_choice(a.shape[0], b_prepacked.shape[1], a.shape[1], a.dtype))
    else:
        if tile is None:
            tile = select_scaled_mm_config(a.shape[0], b_prepacked.shape[1], a.shape[1], a.dtype,
                                           b_prepacked.dtype, out_dtype)
        _launch(a, b_prepacked, scale, bias, out, tile, 1 if splits is None else splits)
    return out


def prepack_b_for_scaled_mm(b: torch.Tensor) -> torch.Tensor:
    """Rearranges a `[K, N]` fp8 weight into the `[K_pad/16, N, 16]` order the kernels read (reference
    `scaled_mm.py:137-150`).

    `K` is zero-padded to a multiple of 128, so a ragged K never needs a staging branch; element
    `[k // 16, n, k % 16]` of the result is `b[k, n]`. A contiguous e5m2 / e4m3fn weight on the GPU with
    N a multiple of 8 is permuted by one HIP kernel (`csrc/prepack.hip`, HBM-bound); anything else
    (a CPU weight, another dtype or width) by torch copy kernels on `b`'s device. Run once per weight.
    """
    k, n = b.shape
    k_pad = -(-k // 128) * 128
    if (b.is_cuda and b.dtype in (torch.float8_e5m2, torch.float8_e4m3fn) and b.is_contiguous()
            and n % 8 == 0 and n > 0 and k > 0 and b.data_ptr() % 8 == 0):
        out = torch.empty((k_pad // 16, n, 16), device=b.device, dtype=b.dtype)
        torch.ops.feather_ops.prepack_b.default(b, out)
        return out
    if k_pad != k:
        padded = torch.zeros((k_pad, n), device=b.device, dtype=b.dtype)
        padded[:k] = b
        b = padded
    return b.view(k_pad // 16, 16, n).permute(0, 2, 1).contiguous()


def prepack_transpose(w: torch.Tensor) -> torch.Tensor:
    """`[N, K]` fp8 weight (an `nn.Linear` weight, out x in) -> `[K_pad/16, N, 16]`: the same layout as
    `prepack_b_for_scaled_mm(w.t())` without materializing the transpose (the external consumer's
    `comfy_feather/quant.py::prepack_transpose`, named at the reference's `scaled_mm.py:141-142`).

    For a row of `w` the 16 k values of a chunk are already 16 contiguous bytes, so the prepack is a
    transpose of `[N, K_pad/16]` 16-byte units.
    """
    n, k = w.shape
    k_pad = -(-k // 128) * 128
    if k_pad != k:
        padded = torch.zeros((n, k_pad), device=w.device, dtype=w.dtype)
        padded[:, :k] = w
        w = padded
    return w.view(n, k_pad // 16, 16).transpose(0, 1).contiguous()


def tile_shape(tile: tuple[int, ...]) -> tuple[int, int, int]:
    """Rows, columns and K depth per stage of one workgroup of `tile`, as `(block_m, block_n, chunk_k)`."""
    return gemm_block_sizes(tile)
