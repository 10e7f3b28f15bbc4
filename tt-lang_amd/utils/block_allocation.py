"""Work splitting over a core grid as the reference's
python/utils/block_allocation.py does it (tuples of coordinates rather than
ttnn core ranges): the examples' tile ownership follows from it, so the
assignment is kept identical.

Coordinates are (..., y, x) with x the last grid dimension; a range is a
(start, end) pair of coordinates, both inclusive.
"""

from __future__ import annotations

from typing import List, Tuple

Coord = Tuple[int, ...]
Range = Tuple[Coord, Coord]


def remove_leading_ones(grid: Tuple[int, ...]) -> Tuple[int, ...]:
    """Drops leading size-1 dimensions (block_allocation.py:13-14)."""
    i = 0
    while i < len(grid) and grid[i] == 1:
        i += 1
    return tuple(grid[i:])


def get_number_of_cores(grid: Tuple[int, ...]) -> int:
    """Product of the grid dimensions, each positive (block_allocation.py:17-22)."""
    n = 1
    for d in grid:
        assert d > 0, "grid dimensions must be positive"
        n *= d
    return n


def num_cores_to_grid_ranges(start_coord: Coord, target_num_cores: int, grid_size: Tuple[int, ...],
                             row_wise: bool = True) -> List[Range]:
    """Rectangles covering `target_num_cores` cores taken in order (x fastest
    when row_wise, else y fastest) from `start_coord`: at most a partial first
    row (column), a block of whole rows (columns) and a partial last one
    (block_allocation.py:37-149)."""
    assert len(start_coord) == len(grid_size), "start_coord and grid_size must have same dimensions"
    assert len(remove_leading_ones(grid_size)) <= 2, "Only supports 2D grids"
    nx = grid_size[-1] if len(grid_size) >= 1 else 1
    ny = grid_size[-2] if len(grid_size) >= 2 else 1
    x0 = start_coord[-1] if len(start_coord) >= 1 else 0
    y0 = start_coord[-2] if len(start_coord) >= 2 else 0
    assert x0 < nx and y0 < ny, "Start coord must be within grid"
    if row_wise:
        available = (ny - 1 - y0) * nx + (nx - x0)
    else:
        available = (nx - 1 - x0) * ny + (ny - y0)
    assert target_num_cores <= available, (
        f"Target {target_num_cores} exceeds available {available}")
    pre = (0,) * (len(grid_size) - 2)
    out: List[Range] = []
    left, x, y = target_num_cores, x0, y0
    if row_wise:
        if x != 0 and left > nx - x0:
            out.append((pre + (y, x), pre + (y, nx - 1)))
            left -= nx - x
            x, y = 0, y + 1
        if left >= nx:
            rows = left // nx
            out.append((pre + (y, x), pre + (y + rows - 1, nx - 1)))
            left -= rows * nx
            x, y = 0, y + rows
        if left > 0:
            out.append((pre + (y, x), pre + (y, x + left - 1)))
    else:
        if y != 0 and left > ny - y0:
            out.append((pre + (y, x), pre + (ny - 1, x)))
            left -= ny - y
            x, y = x + 1, 0
        if left >= ny:
            cols = left // ny
            out.append((pre + (y, x), pre + (ny - 1, x + cols - 1)))
            left -= cols * ny
            x, y = x + cols, 0
        if left > 0:
            out.append((pre + (y, x), pre + (y + left - 1, x)))
    return out


def split_work_to_cores(grid_size: Tuple[int, ...], units_to_divide: int, row_wise: bool = True):
    """Splits work units over the grid: returns (number of cores used, group
    1 range, group 2 range, units per group-1 core, units per group-2 core),
    the groups as (start, end) bounding boxes (block_allocation.py:152-289).

    Fewer units than cores: the first `units` cores (in fill order) get one
    each.  Otherwise every core works; the first `units % cores` cores (group
    1) get one unit more than the others (group 2)."""
    if units_to_divide == 0:
        return (0, (), (), 0, 0)
    simple = remove_leading_ones(grid_size)
    assert len(simple) <= 2, "only supports grids with a single device"
    total = get_number_of_cores(grid_size)
    assert total > 0, "grid must have at least one core"
    origin = (0,) * len(grid_size)
    lead = (0,) * (len(grid_size) - 1)
    if total >= units_to_divide:
        if len(simple) == 1:
            end = lead + (units_to_divide - 1,)
        else:
            end = (0,) * (len(grid_size) - 2) + num_cores_to_grid_ranges(
                origin, units_to_divide, grid_size, row_wise)[-1][1]
        return (units_to_divide, (origin, end), (), 1, 0)
    per, extra = divmod(units_to_divide, total)
    if len(simple) == 1:
        return (total, (origin, lead + (extra,)), (lead + (extra + 1,), lead + (total - 1,)),
                per + 1, per)
    nx, ny = grid_size[-1], grid_size[-2]
    pre = (0,) * (len(grid_size) - 2)
    if extra == 0:
        return (total, (origin, pre + (ny - 1, nx - 1)), (), per, 0)
    last1 = num_cores_to_grid_ranges(origin, extra, grid_size, row_wise)[-1][1]
    ly, lx = last1[-2], last1[-1]
    if row_wise:
        sy, sx = (ly, lx + 1) if lx != nx - 1 else (ly + 1, 0)
    else:
        sy, sx = (ly + 1, lx) if ly != ny - 1 else (0, lx + 1)
    start2 = pre + (sy, sx)
    last2 = num_cores_to_grid_ranges(start2, total - extra, grid_size, row_wise)[-1][1]
    return (total, (origin, last1), (start2, last2), per + 1, per)
