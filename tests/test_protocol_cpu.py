"""Exhaustive interleaving checks of the whole-step kernels' synchronisation
schedules (tests/protocol_model.py): every read of an exchange slot sees the
step it must see, no schedule deadlocks, the column kernel's counters are
clear for the next launch, the layer-resident kernel's step flags count on
across launches, and each planted mistake (a dropped wait, a counter left
uncleared, one buffer too few next to the top layer, a missing peer, a launch
counting its steps from zero again, first-step partials rewritten too early)
is caught."""
import pytest

from protocol_model import Violation, column_kernel, resident_kernel


@pytest.mark.parametrize("nblocks,ntile,steps", [(3, 3, 3), (2, 3, 2), (1, 2, 3), (3, 2, 2)])
def test_column_kernel_barriers(nblocks, ntile, steps):
    assert column_kernel(nblocks, ntile, steps, launches=2).explore() > 1


def test_column_kernel_without_the_first_wait_reads_stale_eps():
    with pytest.raises(Violation, match="read"):
        column_kernel(2, 2, 2, launches=1, drop_barrier=True).explore()


@pytest.mark.parametrize("clears", [("bar1",), ("bar0",)])
def test_column_kernel_exit_must_clear_both_counters(clears):
    with pytest.raises(Violation):
        column_kernel(2, 2, 2, launches=2, exit_clears=clears).explore()


@pytest.mark.parametrize("hidden,chunks,halves,steps", [
    (1, 2, 1, 4), (2, 2, 1, 3), (3, 1, 1, 4), (2, 1, 2, 3), (1, 1, 2, 4), (1, 3, 1, 3), (2, 2, 2, 3)])
def test_resident_kernel_exchange(hidden, chunks, halves, steps):
    assert resident_kernel(hidden, chunks, halves, steps).explore() > 1


@pytest.mark.parametrize("hidden,chunks,halves,steps", [(1, 2, 1, 2), (2, 1, 1, 3), (2, 1, 2, 2), (1, 1, 2, 3)])
def test_resident_kernel_flags_count_across_launches(hidden, chunks, halves, steps):
    assert resident_kernel(hidden, chunks, halves, steps, launches=2).explore() > 1


def test_resident_kernel_planted_mistake_counting_from_zero_again():
    with pytest.raises(Violation):
        resident_kernel(2, 1, 1, 2, launches=2, reset_base=True).explore()


def test_resident_kernel_planted_mistake_rewriting_the_first_partials_early():
    # one step per launch: a chunk can finish before a sibling has summed xn
    with pytest.raises(Violation):
        resident_kernel(1, 2, 1, 1, launches=3, xn_wait=False).explore()


@pytest.mark.parametrize("steps", [1, 2])
def test_resident_kernel_first_partials_across_three_launches(steps):
    assert resident_kernel(1, 2, 1, steps, launches=3).explore() > 1


@pytest.mark.parametrize("mistake", [
    dict(g_buffers_top=2),            # W^T eps next to the top layer double- instead of triple-buffered
    dict(top_waits_l2=False),         # top chunks do not wait for workgroup L-2
    dict(chunk0_waits_siblings=False),  # chunk 0 sums partials its siblings have not published
])
def test_resident_kernel_planted_mistakes_next_to_the_top(mistake):
    with pytest.raises(Violation):
        resident_kernel(1, 2, 1, 4, **mistake).explore()


def test_resident_kernel_planted_mistake_between_hidden_layers():
    with pytest.raises(Violation):
        resident_kernel(3, 1, 1, 3, hidden_waits_up=False).explore()
