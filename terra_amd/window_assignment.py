"""Window -> rank ownership on an m x n window-parallel topology
(core/parallel/window_assignment.py:1-178), host-side.

On one GPU it defines which windows one rank's slab holds: the TERRA m x 1
"ragged row-major" mode gives rank r the contiguous flat window ids
``[(r*T)//m, ((r+1)*T)//m)`` of the T = nWh*nWw row-major windows
(:64-76), so a slab may start and end part-way through a window row.
:func:`slab_geometry` turns that ownership into the gather geometry of the
rank's windows (window-row range + valid-window range).
"""
from __future__ import annotations

from typing import Dict, List, Tuple

TERRA_M1_ASSIGNMENT_MODES = frozenset({
    "terra_m1_regular",
    "terra_m1_ragged_row",
    "terra_m1_ragged_row_major",
    "terra_m1_ragged_auto",
})


def is_terra_m1_assignment_mode(mode: str) -> bool:
    return mode in TERRA_M1_ASSIGNMENT_MODES


def get_window_owner(ii: int, jj: int, num_windows_w: int, wp_group_h: int, wp_group_w: int,
                     mode: str = "regular") -> int:
    """Owner rank of window (ii, jj) in the non-m x 1 modes (:19-24)."""
    if mode == "regular":
        return (ii % wp_group_h) * wp_group_w + (jj % wp_group_w)
    if mode == "ragged_round_robin":
        return (ii * num_windows_w + jj) % (wp_group_h * wp_group_w)
    raise ValueError(f"Unsupported window_assignment_mode: {mode}")


def _row_blocks(num_rows: int, parts: int) -> List[Tuple[int, int]]:
    """Split rows into `parts` contiguous blocks, the first (num_rows % parts) one row longer."""
    base, extra = divmod(num_rows, parts)
    out, start = [], 0
    for r in range(parts):
        stop = start + base + (1 if r < extra else 0)
        out.append((start, stop))
        start = stop
    return out


def _m1_flat_ranges(mode: str, nwh: int, nww: int, m: int) -> List[Tuple[int, int]]:
    """Flat row-major window-id range [start, stop) owned by each rank of an m x 1 topology."""
    if mode == "terra_m1_regular":
        if nwh % m != 0:
            raise ValueError(f"terra_m1_regular requires num_windows_h={nwh} divisible by m={m}")
        return [(a * nww, b * nww) for a, b in _row_blocks(nwh, m)]
    if mode == "terra_m1_ragged_row":
        if nwh < m:
            raise ValueError(f"terra_m1_ragged_row requires num_windows_h={nwh} >= m={m}")
        return [(a * nww, b * nww) for a, b in _row_blocks(nwh, m)]
    if mode == "terra_m1_ragged_row_major":
        total = nwh * nww
        if total < m:
            raise ValueError(f"terra_m1_ragged_row_major requires total_windows={total} >= m={m}")
        return [((r * total) // m, ((r + 1) * total) // m) for r in range(m)]
    raise ValueError(f"Unsupported window_assignment_mode: {mode}")


def get_window_indices(num_windows_h: int, num_windows_w: int, wp_group_h: int, wp_group_w: int,
                       mode: str = "regular", debug_rank=None, debug_global_rank=None
                       ) -> Tuple[Dict[int, List[Tuple[int, int]]], Dict[Tuple[int, int], Tuple[int, int]]]:
    """(rank -> [(ii, jj), ...] in local order, (ii, jj) -> (rank, local index)),
    with the reference's mode semantics and errors (:117-178)."""
    wp_size = wp_group_h * wp_group_w
    rank_to_indices: Dict[int, List[Tuple[int, int]]] = {r: [] for r in range(wp_size)}
    global_to_local: Dict[Tuple[int, int], Tuple[int, int]] = {}

    def put(rank: int, ii: int, jj: int) -> None:
        global_to_local[(ii, jj)] = (rank, len(rank_to_indices[rank]))
        rank_to_indices[rank].append((ii, jj))

    if is_terra_m1_assignment_mode(mode):
        if wp_group_w != 1:
            raise ValueError(f"{mode} requires xfmr_wp_topo=(m, 1), got ({wp_group_h}, {wp_group_w})")
        resolved = "terra_m1_ragged_row_major" if mode == "terra_m1_ragged_auto" else mode
        for rank, (start, stop) in enumerate(_m1_flat_ranges(resolved, num_windows_h, num_windows_w, wp_group_h)):
            for flat in range(start, stop):
                put(rank, flat // num_windows_w, flat % num_windows_w)
        return rank_to_indices, global_to_local

    if mode == "ragged_round_robin" and wp_group_w == 1:
        for rank, (a, b) in enumerate(_row_blocks(num_windows_h, wp_group_h)):
            for ii in range(a, b):
                for jj in range(num_windows_w):
                    put(rank, ii, jj)
        return rank_to_indices, global_to_local

    for ii in range(num_windows_h):
        for jj in range(num_windows_w):
            put(get_window_owner(ii, jj, num_windows_w, wp_group_h, wp_group_w, mode), ii, jj)
    return rank_to_indices, global_to_local


def slab_geometry(num_windows_h: int, num_windows_w: int, m: int, rank: int,
                  mode: str = "terra_m1_ragged_row_major") -> Tuple[int, int, int, int]:
    """Window rows and valid windows of one rank's slab under an m x 1 mode.

    Returns (first_row, num_rows, valid_begin, valid_end): the slab spans window
    rows [first_row, first_row + num_rows) of the global grid, and within the
    slab (flat, row-major) the rank owns windows [valid_begin, valid_end); the
    rest of its first and last rows are pad windows.
    """
    resolved = "terra_m1_ragged_row_major" if mode == "terra_m1_ragged_auto" else mode
    start, stop = _m1_flat_ranges(resolved, num_windows_h, num_windows_w, m)[rank]
    if stop <= start:
        raise ValueError(f"rank {rank} owns no windows")
    first_row = start // num_windows_w
    last_row = (stop - 1) // num_windows_w
    base = first_row * num_windows_w
    return first_row, last_row - first_row + 1, start - base, stop - base
