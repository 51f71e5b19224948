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
