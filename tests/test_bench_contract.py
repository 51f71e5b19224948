"""CPU checks of bench.py's contract: the c3 workload it builds and its one-GPU guard."""

from __future__ import annotations

import bench


def test_c3_intervals_are_the_committed_fixture():
    """16 intervals of 4 rows at random 8-token suffix slots (random.Random(2)),
    the c3 budget of the headline configuration."""
    assert bench.c3_intervals() == [
        (2336, 2340), (2504, 2508), (2736, 2740), (2792, 2796), (3344, 3348), (3432, 3436), (3784, 3788),
        (4104, 4108), (4568, 4572), (5000, 5004), (5576, 5580), (6808, 6812), (7008, 7012), (7016, 7020),
        (7528, 7532), (7624, 7628)]
    rows = sum(e - s for s, e in bench.c3_intervals())
    assert rows == 64
    assert all(bench.DELETE_AT <= s and e <= bench.TOTAL - bench.DELETE_SPAN for s, e in bench.c3_intervals())


def test_c3_geometry_and_rotate_bytes():
    suffix = bench.TOTAL - bench.DELETE_AT - bench.DELETE_SPAN
    assert (bench.TOTAL - bench.DELETE_SPAN, suffix) == (7680, 5632)
    assert 2 * bench.LAYERS * bench.HKV * suffix * bench.DIM * 2 == 738_197_504  # rotate bytes, bf16


def test_more_than_one_gpu_is_refused_with_a_message(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "single GPU" in capsys.readouterr().err


def test_workloads_match_the_baseline_configurations():
    c2, c4, c5 = bench.WORKLOADS["c2"], bench.WORKLOADS["c4"], bench.WORKLOADS["c5"]
    assert (c2.edited, c2.suffix, c2.intervals()) == (1920, 1408, [(928, 992)])
    assert c2.intervals() == bench.selected_intervals(1920, 64, 1)  # the reference grid's 1-interval support
    assert (c4.family, c4.layers, c4.mlp, c4.edited, c4.suffix) == ("qwen3", 36, 12288, 31744, 27648)
    assert len(c4.positions()) == 1383 == -(-5 * 27648 // 100) and len(c4.intervals()) == 32
    assert all(4096 <= s and e <= 31744 for s, e in c4.intervals())
    assert all(a[1] < b[0] for a, b in zip(c4.intervals(), c4.intervals()[1:]))  # sorted, non-adjacent
    assert (c5.edited, c5.suffix, len(c5.positions())) == (16128, 15104, 15104)


def test_grid_geometry_keeps_rows_and_causal_pairs_fixed():
    """benchmark_refresh.py:35-49 vectors (tests/test_benchmark_refresh.py:17-28):
    64 rows in 1, 4 or 16 intervals; the causal pair count does not depend on
    the interval count."""
    for length in (2048, 8192):
        pairs = []
        for count in (1, 4, 16):
            intervals = bench.selected_intervals(length, 64, count)
            positions = [p for s, e in intervals for p in range(s, e)]
            assert len(intervals) == count and len(positions) == len(set(positions)) == 64
            assert 0 <= min(positions) and max(positions) < length
            pairs.append(sum(p + 1 for p in positions))
        assert pairs == [pairs[0]] * 3


def test_grid_geometry_rejects_empty_overlapping_or_outside_supports():
    import pytest

    for length, budget, count in ((0, 64, 1), (128, 0, 1), (128, 64, 0), (128, 5, 2), (8, 64, 1), (64, 64, 16)):
        with pytest.raises(ValueError):
            bench.selected_intervals(length, budget, count)
