"""Window ownership (host-side): the reference's own split vector and error
text (kept as data), the oracle's restatement of the ragged row-major rule,
and ownership invariants."""
import pytest

from oracle import swin_oracle as so
from terra_amd.window_assignment import get_window_indices, slab_geometry


# Data from the reference's unit test of this split (TERRA
# tests/unit/test_window_assignment.py): a 2 x 5 window grid over 4 ranks gives
# these flat window ids per rank, and a 2 x 2 topology is refused with this text.
REFERENCE_SPLIT_2x5_OVER_4 = [[0, 1], [2, 3, 4], [5, 6], [7, 8, 9]]
REFERENCE_TOPOLOGY_ERROR = r"requires xfmr_wp_topo=\(m, 1\)"


def _row_major_ids(coords, n_cols):
    """(row, col) window coordinates -> flat row-major window ids."""
    return [r * n_cols + c for r, c in coords]


def test_auto_ragged_split_reproduces_reference_vector():
    owners, lookup = get_window_indices(num_windows_h=2, num_windows_w=5, wp_group_h=4, wp_group_w=1,
                                        mode="terra_m1_ragged_auto")
    split = [_row_major_ids(owners[r], 5) for r in range(4)]
    assert split == REFERENCE_SPLIT_2x5_OVER_4
    # every window is owned exactly once, by a contiguous run of ids whose
    # lengths differ by at most one between ranks
    assert sorted(i for ids in split for i in ids) == list(range(10))
    assert set(lookup) == {(r, c) for r in range(2) for c in range(5)}
    sizes = [len(ids) for ids in split]
    assert max(sizes) - min(sizes) <= 1
    for ids in split:
        assert ids == list(range(ids[0], ids[0] + len(ids)))


def test_auto_ragged_split_refuses_2d_topology():
    with pytest.raises(ValueError, match=REFERENCE_TOPOLOGY_ERROR):
        get_window_indices(num_windows_h=4, num_windows_w=4, wp_group_h=2, wp_group_w=2,
                           mode="terra_m1_ragged_auto")


@pytest.mark.parametrize("nwh,nww,m", [(255, 64, 7), (2, 5, 4), (37, 11, 5), (8, 8, 8)])
def test_row_major_matches_oracle_and_partitions_grid(nwh, nww, m):
    r2i, g2l = get_window_indices(nwh, nww, m, 1, mode="terra_m1_ragged_row_major")
    assert [r2i[r] for r in range(m)] == so.ragged_row_major(nwh, nww, m)
    assert len(g2l) == nwh * nww
    for rank, idx in r2i.items():
        for local, coord in enumerate(idx):
            assert g2l[coord] == (rank, local)


def test_regular_and_ragged_row_modes():
    r2i, _ = get_window_indices(4, 3, 2, 1, mode="terra_m1_regular")
    assert r2i[0] == [(0, 0), (0, 1), (0, 2), (1, 0), (1, 1), (1, 2)]
    with pytest.raises(ValueError, match="divisible"):
        get_window_indices(5, 3, 2, 1, mode="terra_m1_regular")
    r2i, _ = get_window_indices(5, 2, 2, 1, mode="terra_m1_ragged_row")
    assert [len(r2i[0]), len(r2i[1])] == [6, 4]
    with pytest.raises(ValueError, match=">= m"):
        get_window_indices(1, 3, 2, 1, mode="terra_m1_ragged_row")


def test_non_m1_modes():
    r2i, _ = get_window_indices(2, 4, 2, 2, mode="regular")
    assert r2i[0] == [(0, 0), (0, 2)] and r2i[3] == [(1, 1), (1, 3)]
    r2i, _ = get_window_indices(2, 3, 2, 2, mode="ragged_round_robin")
    assert r2i[1] == [(0, 1), (1, 2)]  # flat ids 1 and 5 (mod 4)
    r2i, _ = get_window_indices(5, 2, 2, 1, mode="ragged_round_robin")
    assert len(r2i[0]) == 6 and len(r2i[1]) == 4
    with pytest.raises(ValueError, match="Unsupported"):
        get_window_indices(2, 2, 2, 1, mode="bogus")


def test_slab_geometry_of_c5():
    first, rows, vb, ve = slab_geometry(255, 64, 7, 1)
    assert (first, rows, vb, ve) == (36, 37, 27, 2358)
    r2i, _ = get_window_indices(255, 64, 7, 1, mode="terra_m1_ragged_row_major")
    flat = _row_major_ids(r2i[1], 64)
    assert flat[0] - first * 64 == vb and flat[-1] + 1 - first * 64 == ve
