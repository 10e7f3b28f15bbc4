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


# ---------------------------------------------------------------------------
# per-core matmul block sizes (python/utils/block_allocation.py:292-487): the
# heuristic a Tensix matmul host program uses to size its per-core output
# blocks under a 400-tile L1 budget.  Kept identical because callers size
# their grids and loops from its answer (the metal multicore_reuse_matmul
# example); the MI355X kernels do not use it.

from collections import namedtuple  # noqa: E402

MatmulParams = namedtuple("MatmulParams", ["block_h", "block_w", "subblock_h", "subblock_w"])

# (subblock_h, subblock_w) in the order they are tried (the reference's table)
SUBBLOCK_HW_CHOICES = [(4, 2), (2, 4), (8, 1), (1, 8), (7, 1), (1, 7), (3, 2), (2, 3), (6, 1),
                       (1, 6), (5, 1), (1, 5), (2, 2), (4, 1), (1, 4), (3, 1), (1, 3), (2, 1),
                       (1, 2), (1, 1)]

_L1_TILE_BUDGET = 400


def filter_factor_pairs_by_2d_grid(factor_pairs, grid):
    """Pairs that fit the 2-D grid as given or transposed (transposed ones
    are returned transposed)."""
    out = []
    for a, b in factor_pairs:
        if a <= grid[0] and b <= grid[1]:
            out.append((a, b))
        elif b <= grid[0] and a <= grid[1]:
            out.append((b, a))
    return out


def get_prime_factors_with_multiplicity(n: int) -> List[int]:
    """Prime factors of n in ascending order, repeated by multiplicity."""
    out, p = [], 2
    while p * p <= n:
        while n % p == 0:
            out.append(p)
            n //= p
        p += 1
    if n > 1:
        out.append(n)
    return out


def get_possible_products(factors: List[int]) -> List[int]:
    """Every distinct product of a sub-multiset of `factors`, ascending (1 included)."""
    prods = {1}
    for f in factors:
        prods |= {q * f for q in prods}
    return sorted(prods)


def get_maximum_block_dim(block_dim: int, in0_block_w: int) -> int:
    """Largest other block dimension o with 2 k b + 2 k o + b o <= 400 tiles
    (double-buffered A and B plus C, k = in0_block_w, b = block_dim); 0 when
    none fits."""
    o = (_L1_TILE_BUDGET - 2 * in0_block_w * block_dim) // (2 * in0_block_w + block_dim)
    return o if o > 0 else 0


def _subblock(mpc: int, npc: int):
    for sh, sw in SUBBLOCK_HW_CHOICES:
        if mpc % sh == 0 and npc % sw == 0:
            return MatmulParams(mpc, npc, sh, sw)
    return None


def get_large_matmul_params(Mt: int, Nt: int, num_cores_y: int, num_cores_x: int,
                            in0_block_w: int) -> MatmulParams:
    """Per-core block (block_h x block_w tiles of the Mt x Nt output) and
    subblock for a num_cores_y x num_cores_x grid, or MatmulParams(0, 0, 0, 0)
    when no block fits.  Prime factors of Mt / Nt larger than the grid side
    must stay inside one core's block; the rest are grown greedily within the
    L1 budget (the larger dimension first when only one side has such
    factors)."""
    none = MatmulParams(0, 0, 0, 0)
    mf = get_prime_factors_with_multiplicity(Mt)
    nf = get_prime_factors_with_multiplicity(Nt)
    mpc_min = 1
    for f in (f for f in mf if f > num_cores_y):
        mpc_min *= f
    npc_min = 1
    for f in (f for f in nf if f > num_cores_x):
        npc_min *= f
    mf = [f for f in mf if f <= num_cores_y]
    nf = [f for f in nf if f <= num_cores_x]
    if npc_min > get_maximum_block_dim(mpc_min, in0_block_w):
        return none

    def fits(mpc, npc):
        return Mt // mpc <= num_cores_y and Nt // npc <= num_cores_x

    def grow(base, choices, limit):
        best = base
        for c in choices:
            if c * base > limit:
                break
            best = c * base
        return best

    if mpc_min > 1:
        mpc = mpc_min
        npc = grow(npc_min, get_possible_products(nf), get_maximum_block_dim(mpc_min, in0_block_w))
        if not fits(mpc, npc):
            return none
        return _subblock(mpc, npc) or none
    if npc_min > 1:
        npc = npc_min
        mpc = grow(mpc_min, get_possible_products(mf), get_maximum_block_dim(npc_min, in0_block_w))
        if not fits(mpc, npc):
            return none
        return _subblock(mpc, npc) or none
    mchoices = get_possible_products(mf)
    mpc = 1
    for npc in get_possible_products(nf):
        lim = get_maximum_block_dim(npc, in0_block_w)
        for c in mchoices:
            if c <= lim:
                mpc = c
        if not fits(mpc, npc):
            continue
        r = _subblock(mpc, npc)
        if r is not None:
            return r
    return none
