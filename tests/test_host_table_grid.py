"""The table builder's cell grid (no GPU): every power-of-two batch of every
power-of-two N = 16 .. 2^20 up to 2^32 elements, the cells above 2^27
elements built after all the others, and there only the three fastest
challengers of the same N at 2^27 elements timed (with the M0 incumbent)."""
import pytest

from kunlunxin_fft_amd import table_builder as tb
from kunlunxin_fft_amd.config import DesignSpace


def test_grid_covers_every_power_of_two_batch_up_to_2_32_elements():
    for cells in (tb.cells(), tb.real_cells()):
        have = set(cells)
        for k in range(4, 21):
            for j in range(0, 33 - k):
                assert (1 << k, 1 << j) in have, (k, j)
        assert max(n * b for n, b in cells) == 1 << 32
        assert len(cells) == len(have)  # no cell twice


def test_large_cells_come_last_and_follow_their_2_27_cell():
    for cells in (tb.cells(), tb.real_cells()):
        big = [n * b > (1 << tb.PRUNE_LOG_ELEMS) for n, b in cells]
        first_big = big.index(True)
        assert all(big[first_big:]) and not any(big[:first_big])
        pos = {c: i for i, c in enumerate(cells)}
        for n, b in cells[first_big:]:
            assert pos[(n, (1 << tb.PRUNE_LOG_ELEMS) // n)] < pos[(n, b)]


def test_quick_grid_leaves_the_large_cells_out():
    assert max(n * b for n, b in tb.cells(quick=True) if b > 1) <= 1 << 22


def test_pruning_keeps_the_fastest_three_of_the_2_27_cell():
    top = {}
    timed = [(3.0, "a"), (1.0, "b"), (2.0, "c"), (4.0, "d")]
    n = 1024
    tb.record_top(timed, n, (1 << 27) // n // 2, (n, "dit"), top)  # below 2^27: nothing recorded
    assert top == {}
    tb.record_top(timed, n, (1 << 27) // n, (n, "dit"), top)
    assert top == {(n, "dit"): ["b", "c", "a"]}
    cands = [("a", 1), ("b", 2), ("c", 3), ("d", 4)]
    # above 2^27: only the recorded labels, in the candidates' own order
    assert tb.pruned(cands, n, (1 << 28) // n, (n, "dit"), top) == cands[:3]
    # at or below 2^27, or with nothing recorded for the key: every candidate
    assert tb.pruned(cands, n, (1 << 27) // n, (n, "dit"), top) == cands
    assert tb.pruned(cands, n, (1 << 28) // n, (n, "dif"), top) == cands


@pytest.mark.parametrize("n", [16, 4096, 1 << 20])
def test_every_large_cell_has_challengers(n):
    """A 2^27 cell times at least PRUNE_KEEP challengers, so a large cell
    always has some to time."""
    space = DesignSpace.load()
    b = (1 << 27) // n
    assert len(tb.candidates(n, b, "dit", space)) >= tb.PRUNE_KEEP
    for tt in ("r2c", "c2r"):
        assert len(tb.real_candidates(n, b, tt, space)) >= tb.PRUNE_KEEP


def test_refused_plans_are_not_candidates():
    """A plan the library refuses at a shape (a launch past one dispatch's
    2^32 work-items: the real M0 at N = 16 from B = 2^24) times as infinite:
    it is never the best challenger or a recorded one, and a refused M0
    incumbent leaves the best challenger a 100% gain and no incumbent time."""
    inf = float("inf")
    assert tb.guard_gain(inf, (1.0, "lds_e16")) == 100.0
    assert tb.guard_gain(2.0, (1.0, "lds_e16")) == 50.0
    assert tb.guard_gain(2.0, None) == -1.0 and tb.guard_gain(2.0, (inf, "x")) == -1.0
    assert tb._ms(inf) is None and tb._ms(0.123456) == 0.12346
    top = {}
    tb.record_top([(inf, "a"), (1.0, "b")], 16, (1 << 27) // 16, (16, "r2c"), top)
    assert top == {(16, "r2c"): ["b"]}


def test_max_log_elems_bounds_the_grid():
    """--max-log-elems 24: the dense grid stops at 2^24 elements (the config
    sweep and roofline rows stay), for both the C2C and the real cells."""
    for cells in (tb.cells(max_log_elems=24), tb.real_cells(max_log_elems=24)):
        dense = {(n, b) for n, b in cells}
        assert all((1 << k, 1 << j) in dense for k in range(4, 21) for j in range(0, 25 - k))
        # past 2^24 only the roofline rows (real: at twice the batch, 2^27 at N = 2^20)
        assert all(n * b <= 1 << 24 or n in tb.ROOF_SIZES for n, b in cells)
        assert max(n * b for n, b in cells) <= 1 << 27
