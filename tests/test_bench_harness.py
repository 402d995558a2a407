"""The tile-sweep harness (feather-ops_amd/benchmarks): grid integrity and the timing protocol's pure parts,
and bench.py's clock monitor, on the CPU."""

import pytest

from benchmarks import cells as grid
from benchmarks import protocol


def test_grid_has_no_repeated_cell_and_fits_the_kernel_contract():
    selected = grid.cells()
    assert len(selected) > 90
    for _, m, n, k in selected:
        assert m >= 1 and n % 8 == 0 and k % 16 == 0 and k >= 16, (m, n, k)


def test_grid_contains_the_benchmark_configurations():
    shapes = {(m, n, k) for _, m, n, k in grid.cells({"baseline"})}
    assert {(4096, 12288, 3072), (16, 14336, 4096), (4096, 3072, 3072), (256, 1024, 1024)} <= shapes


def test_repeated_cell_is_rejected(monkeypatch):
    monkeypatch.setitem(grid.GROUPS, "dup", [(4096, 12288, 3072)])
    with pytest.raises(ValueError, match="repeats"):
        grid.cells()


def test_percentile_interpolates():
    assert protocol.percentile([3.0, 1.0, 2.0], 0.5) == 2.0
    assert protocol.percentile([1.0, 2.0], 0.25) == pytest.approx(1.25)
    assert protocol.percentile([5.0], 0.8) == 5.0


def test_rotated_orders_put_every_provider_in_every_position():
    orders = protocol.rotated_orders(["a", "b", "c"], 6)
    for pos in range(3):
        assert sorted(o[pos] for o in orders) == ["a", "a", "b", "b", "c", "c"]


def test_rotated_orders_spread_positions_with_few_rounds():
    names = [str(i) for i in range(23)]
    orders = protocol.rotated_orders(names, 5)
    positions = [o.index("1") for o in orders]
    assert max(positions) - min(positions) >= 15  # not bunched at the start of every round


def test_paired_speedup_is_median_of_round_ratios():
    fast = protocol.Measurement.of([1.0, 1.0, 2.0])
    slow = protocol.Measurement.of([2.0, 3.0, 2.0])
    assert protocol.paired_speedup(fast, slow) == pytest.approx(2.0)


def test_weight_copies_exceed_the_mall_when_cold():
    from benchmarks.benchmark_scaled_mm_hip import weight_copies

    assert weight_copies(12288, 3072, cold=False) == 1
    assert weight_copies(14336, 4096, cold=True) * 14336 * 4096 > 256e6
    assert weight_copies(248320, 4096, cold=True) == 1


def test_clock_monitor_keeps_each_table_rewrite_once_and_drops_the_stale_one():
    """The SMU table is rewritten once a second and polled every few ms: each rewrite counts once, and the
    table present at start() (written before the load window) not at all."""
    import bench

    tables = iter([(100, [1400, 1500]), (100, [1400, 1500]), (100, [1400, 1500]),   # start() + stale polls
                   (200, [2000, 1980]), (200, [2000, 1980]),
                   (300, [1990, 1950]),
                   (400, [2010, 2030]), (400, [2010, 2030])])
    mon = bench.ClockMonitor(reader=lambda: next(tables))
    mon._stale = mon._read()[0]
    while mon._poll():
        pass
    assert [counter for _, counter, _ in mon.tables] == [200, 300, 400]
    s = mon.summary()
    assert s["table_rewrites"] == 3
    assert s["clock_mhz"] == 1990.0 and s["min_mhz"] == 1970.0 and s["max_mhz"] == 2020.0
    assert s["per_xcd_mhz"] == [2000.0, 1980.0]


def test_clock_monitor_without_a_rewrite_reports_nothing():
    import bench

    mon = bench.ClockMonitor(reader=lambda: (7, [2000]))
    mon._stale = mon._read()[0]
    for _ in range(5):
        assert mon._poll()
    assert mon.summary() is None
