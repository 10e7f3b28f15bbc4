"""tt-lang kernels used by the parity tests.

Each factory takes a `ttl` namespace (this build's drop-in, or the CPU oracle's
eager executor) and returns the kernel, so one kernel source runs on both.
They are written in the styles of the reference examples (examples/
eltwise_add.py, broadcast.py, singlecore_matmul.py, multicore_matmul.py):
column-split elementwise with (2, 1) blocks, 4x4-tile broadcast blocks on an
8x8 grid, (1, 1)-tile matmul with store(acc=True) on one core and split over
a 13x10 grid with split_work_to_cores.
"""

import math

TILE = 32


def make_eltwise_add(ttl, granularity=2, grid="auto"):
    @ttl.kernel(grid=grid)
    def eltwise_add(a_in, b_in, out):
        row_tiles = a_in.shape[0] // ttl.TILE_SHAPE[0]
        col_tiles = a_in.shape[1] // ttl.TILE_SHAPE[1]
        gh, gw = ttl.grid_size()
        cols_per_core = math.ceil(col_tiles / (gh * gw))
        a_cb = ttl.make_circular_buffer_like(a_in, shape=(granularity, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b_in, shape=(granularity, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(granularity, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            start = c * cols_per_core
            end = min(start + cols_per_core, col_tiles)
            for ct in range(start, end):
                for rb in range(row_tiles // granularity):
                    a = a_cb.wait()
                    b = b_cb.wait()
                    o = o_cb.reserve()
                    o.store(a + b)
                    o_cb.push()
                    a_cb.pop()
                    b_cb.pop()

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            start = c * cols_per_core
            end = min(start + cols_per_core, col_tiles)
            for ct in range(start, end):
                for rb in range(row_tiles // granularity):
                    rows = slice(rb * granularity, (rb + 1) * granularity)
                    cols = slice(ct, ct + 1)
                    blk = a_cb.reserve()
                    ttl.copy(a_in[rows, cols], blk).wait()
                    a_cb.push()
                    blk = b_cb.reserve()
                    ttl.copy(b_in[rows, cols], blk).wait()
                    b_cb.push()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            start = c * cols_per_core
            end = min(start + cols_per_core, col_tiles)
            for ct in range(start, end):
                for rb in range(row_tiles // granularity):
                    rows = slice(rb * granularity, (rb + 1) * granularity)
                    blk = o_cb.wait()
                    ttl.copy(blk, out[rows, slice(ct, ct + 1)]).wait()
                    o_cb.pop()

    return eltwise_add


def make_bcast_fma(ttl, g=4, grid=(8, 8)):
    """y = a * b + broadcast(c, dims=[1]) with c a column vector (N, 1)."""

    @ttl.kernel(grid=grid)
    def bcast_fma(a, b, c, y):
        gx, gy = ttl.grid_size(dims=2)
        rows_per_core = a.shape[0] // TILE // gx // g
        cols_per_core = a.shape[1] // TILE // gy // g
        a_cb = ttl.make_circular_buffer_like(a, shape=(g, g), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(g, g), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(g, 1), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(rows_per_core):
                for _ in range(cols_per_core):
                    with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cb, \
                            y_cb.reserve() as yb:
                        yb.store(ab * bb + ttl.math.broadcast(cb, dims=[1]))

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            for i in range(rows_per_core):
                r = (cx * rows_per_core + i) * g
                for j in range(cols_per_core):
                    col = (cy * cols_per_core + j) * g
                    with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cb:
                        ta = ttl.copy(a[r:r + g, col:col + g], ab)
                        tb = ttl.copy(b[r:r + g, col:col + g], bb)
                        tc = ttl.copy(c[r:r + g, 0], cb)
                        ta.wait()
                        tb.wait()
                        tc.wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            for i in range(rows_per_core):
                r = (cx * rows_per_core + i) * g
                for j in range(cols_per_core):
                    col = (cy * cols_per_core + j) * g
                    with y_cb.wait() as yb:
                        ttl.copy(yb, y[r:r + g, col:col + g]).wait()

    return bcast_fma


def make_exp_row_pipe(ttl, g=4, grid=(8, 8)):
    """y = exp(a + broadcast(b_row, dims=[0])) * c, b_row of shape (1, W)
    (BASELINE configs[1])."""

    @ttl.kernel(grid=grid)
    def exp_row_pipe(a, b_row, c, y):
        gx, gy = ttl.grid_size(dims=2)
        rows_per_core = a.shape[0] // TILE // gx // g
        cols_per_core = a.shape[1] // TILE // gy // g
        a_cb = ttl.make_circular_buffer_like(a, shape=(g, g), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b_row, shape=(1, g), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(g, g), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(rows_per_core):
                for _ in range(cols_per_core):
                    with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cb, \
                            y_cb.reserve() as yb:
                        yb.store(ttl.math.exp(ab + ttl.math.broadcast(bb, dims=[0])) * cb)

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            for i in range(rows_per_core):
                r = (cx * rows_per_core + i) * g
                for j in range(cols_per_core):
                    col = (cy * cols_per_core + j) * g
                    with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cb:
                        ttl.copy(a[r:r + g, col:col + g], ab).wait()
                        ttl.copy(b_row[0, col:col + g], bb).wait()
                        ttl.copy(c[r:r + g, col:col + g], cb).wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            for i in range(rows_per_core):
                r = (cx * rows_per_core + i) * g
                for j in range(cols_per_core):
                    col = (cy * cols_per_core + j) * g
                    with y_cb.wait() as yb:
                        ttl.copy(yb, y[r:r + g, col:col + g]).wait()

    return exp_row_pipe


def make_matmul_single(ttl):
    @ttl.kernel(grid=(1, 1))
    def mm_single(a, b, out):
        Mt, Kt, Nt = a.shape[0] // TILE, a.shape[1] // TILE, b.shape[1] // TILE
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(Mt):
                for _ in range(Nt):
                    with o_cb.reserve() as ob:
                        for _ in range(Kt):
                            with a_cb.wait() as ab, b_cb.wait() as bb:
                                ob.store(ab @ bb, acc=True)

        @ttl.datamovement()
        def reader():
            for m in range(Mt):
                for n in range(Nt):
                    for k in range(Kt):
                        with a_cb.reserve() as ab, b_cb.reserve() as bb:
                            ttl.copy(a[m, k], ab).wait()
                            ttl.copy(b[k, n], bb).wait()

        @ttl.datamovement()
        def writer():
            for m in range(Mt):
                for n in range(Nt):
                    with o_cb.wait() as ob:
                        ttl.copy(ob, out[m, n]).wait()

    return mm_single


def make_matmul_multi(ttl, ttnn, grid=(13, 10)):
    @ttl.kernel(grid=grid)
    def mm_multi(a, b, out):
        Kt, Nt = a.shape[1] // TILE, b.shape[1] // TILE
        total = (a.shape[0] * b.shape[1]) // (TILE * TILE)
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)
        ys, xs = ttl.grid_size(dims=2)
        _, _, g1, g2, w1, w2 = ttnn.split_work_to_cores(ttnn.CoreCoord(xs, ys), total,
                                                         row_wise=True)
        n1, n2 = g1.num_cores(), g2.num_cores()

        def tiles_of(cid):
            return w1 if cid < n1 else (w2 if cid < n1 + n2 else 0)

        def first_of(cid):
            return cid * w1 if cid < n1 else n1 * w1 + (cid - n1) * w2

        @ttl.compute()
        def comp():
            cid = ttl.core(dims=1)
            for _ in range(tiles_of(cid)):
                with o_cb.reserve() as ob:
                    for _ in range(Kt):
                        with a_cb.wait() as ab, b_cb.wait() as bb:
                            ob.store(ab @ bb, acc=True)

        @ttl.datamovement()
        def reader():
            cid = ttl.core(dims=1)
            for t in range(tiles_of(cid)):
                tid = first_of(cid) + t
                r, c = tid // Nt, tid % Nt
                for k in range(Kt):
                    with a_cb.reserve() as ab, b_cb.reserve() as bb:
                        ttl.copy(a[r, k], ab).wait()
                        ttl.copy(b[k, c], bb).wait()

        @ttl.datamovement()
        def writer():
            cid = ttl.core(dims=1)
            for t in range(tiles_of(cid)):
                tid = first_of(cid) + t
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[tid // Nt, tid % Nt]).wait()

    return mm_multi


def make_tile_reuse(ttl):
    """One (1, 1) block of `t` broadcast over a (2, 2) block of `a` (block
    broadcasting across the tile grid), minus a scalar-free chain."""

    @ttl.kernel(grid=(2, 2))
    def tile_reuse(a, t, out):
        rt, ct = a.shape[0] // TILE, a.shape[1] // TILE
        gy, gx = ttl.grid_size(dims=2)
        rpc, cpc = rt // gy // 2, ct // gx // 2
        a_cb = ttl.make_circular_buffer_like(a, shape=(2, 2), buffer_factor=2)
        t_cb = ttl.make_circular_buffer_like(t, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(2, 2), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(rpc * cpc):
                with a_cb.wait() as ab, t_cb.wait() as tb, o_cb.reserve() as ob:
                    ob.store((ab - tb) * ab)

        @ttl.datamovement()
        def reader():
            y, x = ttl.core(dims=2)
            for i in range(rpc):
                for j in range(cpc):
                    r, c = (y * rpc + i) * 2, (x * cpc + j) * 2
                    with a_cb.reserve() as ab, t_cb.reserve() as tb:
                        ttl.copy(a[r:r + 2, c:c + 2], ab).wait()
                        ttl.copy(t[0, 0], tb).wait()

        @ttl.datamovement()
        def writer():
            y, x = ttl.core(dims=2)
            for i in range(rpc):
                for j in range(cpc):
                    r, c = (y * rpc + i) * 2, (x * cpc + j) * 2
                    with o_cb.wait() as ob:
                        ttl.copy(ob, out[r:r + 2, c:c + 2]).wait()

    return tile_reuse


def make_branchy_add(ttl):
    """Branches on a loop variable, which forces the scalar trace fallback."""

    @ttl.kernel(grid=(1, 2))
    def branchy(a, b, out):
        rt, ct = a.shape[0] // TILE, a.shape[1] // TILE
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            for _ in range(rt * ct // 2):
                with a_cb.wait() as ab, b_cb.wait() as bb, o_cb.reserve() as ob:
                    ob.store(ab + bb)

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            for i in range(rt * ct):
                if i % 2 == c:  # data-dependent branch on the loop variable
                    with a_cb.reserve() as ab, b_cb.reserve() as bb:
                        ttl.copy(a[i // ct, i % ct], ab).wait()
                        ttl.copy(b[i // ct, i % ct], bb).wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for i in range(rt * ct):
                if i % 2 == c:
                    with o_cb.wait() as ob:
                        ttl.copy(ob, out[i // ct, i % ct]).wait()

    return branchy


def make_outer_fma(ttl, g=2, grid=(4, 4)):
    """y = a_col * b_row + c with a (H, 1), b (1, W), c (1, 1): every operand
    broadcast against the output block (three-argument broadcast), the scalar
    block held by compute for the whole kernel, g x g-tile output blocks split
    over a 2-D grid (the broadcast tutorials' pattern, multicore)."""

    @ttl.kernel(grid=grid)
    def outer_fma(a, b, c, y):
        gx, gy = ttl.grid_size(dims=2)
        rpc = y.shape[0] // TILE // g // gx
        cpc = y.shape[1] // TILE // g // gy
        a_cb = ttl.make_circular_buffer_like(a, shape=(g, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, g), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(1, 1), buffer_factor=1)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)

        @ttl.compute()
        def comp():
            with c_cb.wait() as cs:
                for _ in range(rpc):
                    for _ in range(cpc):
                        with a_cb.wait() as ab, b_cb.wait() as bb, y_cb.reserve() as yb:
                            yb.store(ttl.math.broadcast(ab, yb, dims=[1])
                                     * ttl.math.broadcast(bb, yb, dims=[0])
                                     + ttl.math.broadcast(cs, yb, dims=[0, 1]))

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            with c_cb.reserve() as cs:
                ttl.copy(c[0, 0], cs).wait()
            for i in range(rpc):
                r = (cx * rpc + i) * g
                for j in range(cpc):
                    col = (cy * cpc + j) * g
                    with a_cb.reserve() as ab, b_cb.reserve() as bb:
                        ta = ttl.copy(a[r:r + g, 0], ab)
                        tb = ttl.copy(b[0, col:col + g], bb)
                        ta.wait()
                        tb.wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            for i in range(rpc):
                r = (cx * rpc + i) * g
                for j in range(cpc):
                    col = (cy * cpc + j) * g
                    with y_cb.wait() as yb:
                        ttl.copy(yb, y[r:r + g, col:col + g]).wait()

    return outer_fma


def make_shape_dispatch_fma(ttl, g=2):
    """y = a * b + c where b and c may each be full (H, W), a column (H, 1), a
    row (1, W) or a scalar (1, 1): CB shapes, copy slices and broadcast dims
    are chosen from the operand shapes in Python at trace time
    (general_broadcast.py's pattern, auto grid)."""

    def cb_shape(t):
        return (g if t.shape[0] > TILE else 1, g if t.shape[1] > TILE else 1)

    def src(t, r, col):
        rs = slice(r, r + g) if t.shape[0] > TILE else 0
        cs = slice(col, col + g) if t.shape[1] > TILE else 0
        return t[rs, cs]

    def bcast(x, like, shape):
        dims = [d for d in (0, 1) if shape[d] == 1]
        return ttl.math.broadcast(x, like, dims=dims) if dims else x

    @ttl.kernel(grid="auto")
    def shape_dispatch(a, b, c, y):
        gx, gy = ttl.grid_size(dims=2)
        rpc = y.shape[0] // TILE // g // gx
        cpc = y.shape[1] // TILE // g // gy
        a_cb = ttl.make_circular_buffer_like(a, shape=(g, g), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=cb_shape(b), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=cb_shape(c), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(rpc * cpc):
                with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cb, \
                        y_cb.reserve() as yb:
                    yb.store(ab * bcast(bb, yb, cb_shape(b)) + bcast(cb, yb, cb_shape(c)))

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            for i in range(rpc):
                r = (cx * rpc + i) * g
                for j in range(cpc):
                    col = (cy * cpc + j) * g
                    with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cb:
                        xs = [ttl.copy(a[r:r + g, col:col + g], ab), ttl.copy(src(b, r, col), bb),
                              ttl.copy(src(c, r, col), cb)]
                        for x in xs:
                            x.wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            for i in range(rpc):
                r = (cx * rpc + i) * g
                for j in range(cpc):
                    col = (cy * cpc + j) * g
                    with y_cb.wait() as yb:
                        ttl.copy(yb, y[r:r + g, col:col + g]).wait()

    return shape_dispatch


def make_matmul_split_rows(ttl, grid=(13, 10)):
    """C = A @ B with one (1, 1) output tile per step and the output tiles
    divided over the grid by utils.block_allocation.split_work_to_cores
    (group boxes counted as full rectangles, as the metal examples' tt-lang
    versions do); store(acc=True) over K."""
    from utils.block_allocation import split_work_to_cores

    @ttl.kernel(grid=grid)
    def mm_split(a, b, out):
        mt, kt, nt = a.shape[0] // TILE, a.shape[1] // TILE, b.shape[1] // TILE
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)
        _, g1, g2, u1, u2 = split_work_to_cores(ttl.grid_size(dims=2), mt * nt, row_wise=True)

        def box(g):
            return (g[1][0] - g[0][0] + 1) * (g[1][1] - g[0][1] + 1) if g else 0

        n1, n2 = box(g1), box(g2)

        def count(c):
            return u1 if c < n1 else (u2 if c < n1 + n2 else 0)

        def first(c):
            return c * u1 if c < n1 else n1 * u1 + (c - n1) * u2

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            for _ in range(count(c)):
                with o_cb.reserve() as ob:
                    for _ in range(kt):
                        with a_cb.wait() as ab, b_cb.wait() as bb:
                            ob.store(ab @ bb, acc=True)

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            for i in range(count(c)):
                t = first(c) + i
                for k in range(kt):
                    with a_cb.reserve() as ab, b_cb.reserve() as bb:
                        ta = ttl.copy(a[t // nt, k], ab)
                        tb = ttl.copy(b[k, t % nt], bb)
                        ta.wait()
                        tb.wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for i in range(count(c)):
                t = first(c) + i
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[t // nt, t % nt]).wait()

    return mm_split


def make_row_bias_multicast(ttl, g=2, grid=(2, 4)):
    """y = a + broadcast(bias_row): on every grid row, core (r, 0) reads the
    (1, g)-tile bias block for each column block once per output column block and
    multicasts it over a pipe to the other cores of its row, which use it for
    their own row blocks (the eltwise_pipe.py pattern, one pipe per grid row)."""

    @ttl.kernel(grid=grid)
    def row_bias(a, bias, y):
        gy, gx = ttl.grid_size(dims=2)
        rt, ct = a.shape[0] // TILE, a.shape[1] // TILE
        rows_per_core = rt // g // (gy * gx)
        a_cb = ttl.make_circular_buffer_like(a, shape=(g, g), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(bias, shape=(1, g), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)
        pipes = [ttl.Pipe((r, 0), (r, slice(1, gx))) for r in range(gy)]
        net = ttl.PipeNet(pipes)

        @ttl.compute()
        def comp():
            for _ in range(ct // g):
                with b_cb.wait() as bb:
                    for _ in range(rows_per_core):
                        with a_cb.wait() as ab, y_cb.reserve() as yb:
                            yb.store(ab + ttl.math.broadcast(bb, dims=[0]))

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            for j in range(ct // g):
                with b_cb.reserve() as bb:
                    def send(p):
                        ttl.copy(bias[0, j * g:(j + 1) * g], bb).wait()
                        ttl.copy(bb, p).wait()

                    def recv(p):
                        ttl.copy(p, bb).wait()

                    net.if_src(send)
                    net.if_dst(recv)
                for i in range(rows_per_core):
                    r = (c * rows_per_core + i) * g
                    with a_cb.reserve() as ab:
                        ttl.copy(a[r:r + g, j * g:(j + 1) * g], ab).wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for j in range(ct // g):
                for i in range(rows_per_core):
                    r = (c * rows_per_core + i) * g
                    with y_cb.wait() as yb:
                        ttl.copy(yb, y[r:r + g, j * g:(j + 1) * g]).wait()

    return row_bias


def make_scalar_expand_add(ttl, ttnn):
    """y = a + c with c a (1, 1) tensor expanded in the kernel body to one
    32 x 32 tile (ttnn.repeat / squeeze, as eltwise_pipe.py does): the plan
    refers to a tensor the body creates."""

    @ttl.kernel(grid=(1, 2))
    def scalar_add(a, c, y):
        c_tile = ttnn.squeeze(ttnn.repeat(c, (1, 1, *ttl.TILE_SHAPE)))
        rt, ct = a.shape[0] // TILE, a.shape[1] // TILE
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c_tile, shape=(1, 1), buffer_factor=1)
        y_cb = ttl.make_circular_buffer_like(y, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            with c_cb.wait() as cb:
                for _ in range(rt * ct // 2):
                    with a_cb.wait() as ab, y_cb.reserve() as yb:
                        yb.store(ab + cb)

        @ttl.datamovement()
        def reader():
            k = ttl.core(dims=1)
            with c_cb.reserve() as cb:
                ttl.copy(c_tile[0, 0], cb).wait()
            for t in range(rt * ct // 2):
                i = k * (rt * ct // 2) + t
                with a_cb.reserve() as ab:
                    ttl.copy(a[i // ct, i % ct], ab).wait()

        @ttl.datamovement()
        def writer():
            k = ttl.core(dims=1)
            for t in range(rt * ct // 2):
                i = k * (rt * ct // 2) + t
                with y_cb.wait() as yb:
                    ttl.copy(yb, y[i // ct, i % ct]).wait()

    return scalar_add


def make_reduce_rows(ttl, kind="sum", gr=2, gc=4, grid=(2, 2), scaler_const=None):
    """out[r] = reduce_<kind> over the columns of x[r, :] * s (ttl.math.reduce_*,
    dims=[1], spec TTLangSpecification.md:754-755): (gr, gc)-tile blocks, the
    column blocks of a row accumulated with store(acc=True) when there are
    several.  The scaler is the (1, 1) tile s[0, 0], or a number."""

    @ttl.kernel(grid=grid)
    def reduce_rows(x, s, out):
        gx, gy = ttl.grid_size(dims=2)
        rows_per_core = x.shape[0] // TILE // gr // (gx * gy)
        nk = x.shape[1] // TILE // gc
        x_cb = ttl.make_circular_buffer_like(x, shape=(gr, gc), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(s, shape=(1, 1), buffer_factor=1)
        o_cb = ttl.make_circular_buffer_like(out, shape=(gr, 1), buffer_factor=2)
        red = ttl.math.reduce_sum if kind == "sum" else ttl.math.reduce_max

        @ttl.compute()
        def comp():
            with s_cb.wait() as sb:
                scaler = sb if scaler_const is None else scaler_const
                for _ in range(rows_per_core):
                    with o_cb.reserve() as ob:
                        for _ in range(nk):
                            with x_cb.wait() as xb:
                                ob.store(red(xb, scaler, dims=[1]), acc=nk > 1)

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            with s_cb.reserve() as sb:
                ttl.copy(s[0, 0], sb).wait()
            for i in range(rows_per_core):
                r = (c * rows_per_core + i) * gr
                for k in range(nk):
                    with x_cb.reserve() as xb:
                        ttl.copy(x[r:r + gr, k * gc:(k + 1) * gc], xb).wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for i in range(rows_per_core):
                r = (c * rows_per_core + i) * gr
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[r:r + gr, 0]).wait()

    return reduce_rows


def make_reduce_cols(ttl, kind="sum", gr=4, gc=2, grid=(2, 2)):
    """out[:, c] = reduce_<kind> over the rows of x[:, c] * s (dims=[0]):
    (gr, gc)-tile blocks, the row blocks of a column range accumulated with
    store(acc=True) when there are several."""

    @ttl.kernel(grid=grid)
    def reduce_cols(x, s, out):
        gx, gy = ttl.grid_size(dims=2)
        cols_per_core = x.shape[1] // TILE // gc // (gx * gy)
        nk = x.shape[0] // TILE // gr
        x_cb = ttl.make_circular_buffer_like(x, shape=(gr, gc), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(s, shape=(1, 1), buffer_factor=1)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, gc), buffer_factor=2)
        red = ttl.math.reduce_sum if kind == "sum" else ttl.math.reduce_max

        @ttl.compute()
        def comp():
            with s_cb.wait() as sb:
                for _ in range(cols_per_core):
                    with o_cb.reserve() as ob:
                        for _ in range(nk):
                            with x_cb.wait() as xb:
                                ob.store(red(xb, sb, dims=[0]), acc=nk > 1)

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            with s_cb.reserve() as sb:
                ttl.copy(s[0, 0], sb).wait()
            for j in range(cols_per_core):
                col = (c * cols_per_core + j) * gc
                for k in range(nk):
                    with x_cb.reserve() as xb:
                        ttl.copy(x[k * gr:(k + 1) * gr, col:col + gc], xb).wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for j in range(cols_per_core):
                col = (c * cols_per_core + j) * gc
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[0, col:col + gc]).wait()

    return reduce_cols


def make_reduce_all(ttl, kind="max"):
    """out = reduce_<kind> of exp(x) * y over a whole (R, C)-tile block on one
    core (dims=[0, 1]), scaler s[0, 0]."""

    @ttl.kernel(grid=(1, 1))
    def reduce_all(x, y, s, out):
        R, C = x.shape[0] // TILE, x.shape[1] // TILE
        x_cb = ttl.make_circular_buffer_like(x, shape=(R, C), buffer_factor=1)
        y_cb = ttl.make_circular_buffer_like(y, shape=(R, C), buffer_factor=1)
        s_cb = ttl.make_circular_buffer_like(s, shape=(1, 1), buffer_factor=1)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=1)
        red = ttl.math.reduce_sum if kind == "sum" else ttl.math.reduce_max

        @ttl.compute()
        def comp():
            with x_cb.wait() as xb, y_cb.wait() as yb, s_cb.wait() as sb, \
                    o_cb.reserve() as ob:
                ob.store(red(ttl.math.exp(xb) * yb, sb, dims=[0, 1]))

        @ttl.datamovement()
        def reader():
            with x_cb.reserve() as xb, y_cb.reserve() as yb, s_cb.reserve() as sb:
                tx = ttl.copy(x[0:R, 0:C], xb)
                ty = ttl.copy(y[0:R, 0:C], yb)
                ts = ttl.copy(s[0, 0], sb)
                tx.wait()
                ty.wait()
                ts.wait()

        @ttl.datamovement()
        def writer():
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0, 0]).wait()

    return reduce_all


def make_row_dot(ttl, gr=2, gc=4, grid=(2, 2)):
    """out[r] = sum over c of a[r, c] * b[r, c] (reduce_sum of a product, a
    constant scaler of 1), one block per row run of tiles."""

    @ttl.kernel(grid=grid)
    def row_dot(a, b, out):
        gx, gy = ttl.grid_size(dims=2)
        rows_per_core = a.shape[0] // TILE // gr // (gx * gy)
        a_cb = ttl.make_circular_buffer_like(a, shape=(gr, gc), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(gr, gc), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(gr, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(rows_per_core):
                with a_cb.wait() as ab, b_cb.wait() as bb, o_cb.reserve() as ob:
                    ob.store(ttl.math.reduce_sum(ab * bb, 1.0, dims=[1]))

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            for i in range(rows_per_core):
                r = (c * rows_per_core + i) * gr
                with a_cb.reserve() as ab, b_cb.reserve() as bb:
                    ta = ttl.copy(a[r:r + gr, 0:gc], ab)
                    tb = ttl.copy(b[r:r + gr, 0:gc], bb)
                    ta.wait()
                    tb.wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for i in range(rows_per_core):
                r = (c * rows_per_core + i) * gr
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[r:r + gr, 0]).wait()

    return row_dot


def make_unary_map(ttl, name, params=(), g=2, grid=(2, 2)):
    """y = ttl.math.<name>(x, *params) over (g, g)-tile blocks (the spec's
    math functions, TTLangSpecification.md:700-750)."""

    @ttl.kernel(grid=grid)
    def unary_map(x, y):
        gx, gy = ttl.grid_size(dims=2)
        rows_per_core = x.shape[0] // TILE // gx // g
        cols_per_core = x.shape[1] // TILE // gy // g
        x_cb = ttl.make_circular_buffer_like(x, shape=(g, g), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)
        fn = getattr(ttl.math, name)

        @ttl.compute()
        def comp():
            for _ in range(rows_per_core):
                for _ in range(cols_per_core):
                    with x_cb.wait() as xb, y_cb.reserve() as yb:
                        yb.store(fn(xb, *params))

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            for i in range(rows_per_core):
                r = (cx * rows_per_core + i) * g
                for j in range(cols_per_core):
                    col = (cy * cols_per_core + j) * g
                    with x_cb.reserve() as xb:
                        ttl.copy(x[r:r + g, col:col + g], xb).wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            for i in range(rows_per_core):
                r = (cx * rows_per_core + i) * g
                for j in range(cols_per_core):
                    col = (cy * cols_per_core + j) * g
                    with y_cb.wait() as yb:
                        ttl.copy(yb, y[r:r + g, col:col + g]).wait()

    return unary_map


def make_tile_bcast(ttl, dims, ib=(2, 2), ob=(2, 2), grid=(2, 2), expr="plain"):
    """The compiler's in-tile broadcast ttl.math.broadcast(in, out, dims) over a
    grid of blocks: every core owns a run of block rows; block (r, c) reads
    input tiles [r ib0, c ib1] and writes output tiles [r ob0, c ob1].
    expr: "plain" stores the broadcast, "fma" stores a * 2 + broadcast(x),
    "exp" stores exp(broadcast(x)) * a (a: an output-shaped operand)."""
    @ttl.kernel(grid=grid)
    def tile_bcast(x, a, out):
        rows = out.shape[0] // TILE // ob[0]
        cols = out.shape[1] // TILE // ob[1]
        ncores = grid[0] * grid[1]
        per = -(-rows // ncores)
        x_cb = ttl.make_circular_buffer_like(x, shape=ib, buffer_factor=2)
        a_cb = ttl.make_circular_buffer_like(a, shape=ob, buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=ob, buffer_factor=2)

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                for _ in range(cols):
                    with x_cb.wait() as xb, a_cb.wait() as ab, o_cb.reserve() as o:
                        b = ttl.math.broadcast(xb, o, dims=dims)
                        if expr == "plain":
                            o.store(b)
                        elif expr == "fma":
                            o.store(ab * 2.0 + b)
                        else:
                            o.store(ttl.math.exp(b) * ab)

        @ttl.datamovement()
        def rd():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                for k in range(cols):
                    with x_cb.reserve() as xb, a_cb.reserve() as ab:
                        tx = ttl.copy(x[r * ib[0]:(r + 1) * ib[0], k * ib[1]:(k + 1) * ib[1]], xb)
                        ta = ttl.copy(a[r * ob[0]:(r + 1) * ob[0], k * ob[1]:(k + 1) * ob[1]], ab)
                        tx.wait()
                        ta.wait()

        @ttl.datamovement()
        def wr():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                for k in range(cols):
                    with o_cb.wait() as o:
                        ttl.copy(o, out[r * ob[0]:(r + 1) * ob[0], k * ob[1]:(k + 1) * ob[1]]).wait()

    return tile_bcast


def make_two_stage(ttl, g=2, grid=(2, 2)):
    """An intermediate CB on every core: stage 1 stores relu(x) * 0.5 into
    t_cb, stage 2 waits on it and stores exp(t) + y (two launches through a
    scratch tensor)."""
    @ttl.kernel(grid=grid)
    def two_stage(x, y, out):
        rows = out.shape[0] // TILE // g
        cols = out.shape[1] // TILE // g
        ncores = grid[0] * grid[1]
        per = -(-rows // ncores)
        x_cb = ttl.make_circular_buffer_like(x, shape=(g, g), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(g, g), buffer_factor=2)
        t_cb = ttl.make_circular_buffer_like(x, shape=(g, g), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(g, g), buffer_factor=2)

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                for _ in range(cols):
                    with x_cb.wait() as xb, t_cb.reserve() as tb:
                        tb.store(ttl.math.relu(xb) * 0.5)
                    with t_cb.wait() as tb, y_cb.wait() as yb, o_cb.reserve() as o:
                        o.store(ttl.math.exp(tb) + yb)

        @ttl.datamovement()
        def rd():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                for k in range(cols):
                    with x_cb.reserve() as xb, y_cb.reserve() as yb:
                        tx = ttl.copy(x[r * g:(r + 1) * g, k * g:(k + 1) * g], xb)
                        ty = ttl.copy(y[r * g:(r + 1) * g, k * g:(k + 1) * g], yb)
                        tx.wait()
                        ty.wait()

        @ttl.datamovement()
        def wr():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                for k in range(cols):
                    with o_cb.wait() as o:
                        ttl.copy(o, out[r * g:(r + 1) * g, k * g:(k + 1) * g]).wait()

    return two_stage


def make_held_tile(ttl, n=4, grid=(2, 2)):
    """Core (y, x) holds tile c[y, x] in scope while it adds it to the n x n
    tiles of a it owns: the operand tile is the output tile divided by n, so
    the store site is split into one launch per held tile."""
    @ttl.kernel(grid=grid)
    def held_tile(a, c, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            with c_cb.wait() as cv:
                for _ in range(n * n):
                    with a_cb.wait() as av, o_cb.reserve() as o:
                        o.store(av * 1.5 + cv)

        @ttl.datamovement()
        def rd():
            x, y = ttl.core(dims=2)
            with c_cb.reserve() as cb:
                ttl.copy(c[y, x], cb).wait()
            for i in range(n):
                for j in range(n):
                    with a_cb.reserve() as ab:
                        ttl.copy(a[y * n + i, x * n + j], ab).wait()

        @ttl.datamovement()
        def wr():
            x, y = ttl.core(dims=2)
            for i in range(n):
                for j in range(n):
                    with o_cb.wait() as o:
                        ttl.copy(o, out[y * n + i, x * n + j]).wait()

    return held_tile


def make_long_chain(ttl, g=2, grid=(2, 2)):
    """A 22-op fused expression (more steps than one kernel program holds):
    the planner computes part of it into a temporary first."""
    @ttl.kernel(grid=grid)
    def long_chain(a, b, c, out):
        rows = out.shape[0] // TILE // g
        cols = out.shape[1] // TILE // g
        ncores = grid[0] * grid[1]
        per = -(-rows // ncores)
        a_cb = ttl.make_circular_buffer_like(a, shape=(g, g), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(g, g), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(g, g), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(g, g), buffer_factor=2)

        @ttl.compute()
        def comp():
            c_ = ttl.core(dims=1)
            for r in range(c_ * per, min(rows, (c_ + 1) * per)):
                for _ in range(cols):
                    with a_cb.wait() as av, b_cb.wait() as bv, c_cb.wait() as cv, \
                            o_cb.reserve() as o:
                        v = ttl.math.sigmoid(av)
                        v = ttl.math.tanh(v) * 3.0
                        v = ttl.math.abs(v - bv)
                        v = ttl.math.sigmoid(v + cv)
                        v = ttl.math.neg(v) * bv
                        v = ttl.math.relu(v + 0.25)
                        v = ttl.math.tanh(v * cv)
                        v = ttl.math.max(v, bv) - ttl.math.min(av, cv)
                        v = ttl.math.sigmoid(v) * 2.0 + av
                        o.store(ttl.math.tanh(v))

        @ttl.datamovement()
        def rd():
            c_ = ttl.core(dims=1)
            for r in range(c_ * per, min(rows, (c_ + 1) * per)):
                for k in range(cols):
                    with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cb:
                        sl = (slice(r * g, (r + 1) * g), slice(k * g, (k + 1) * g))
                        t1 = ttl.copy(a[sl[0].start:sl[0].stop, sl[1].start:sl[1].stop], ab)
                        t2 = ttl.copy(b[sl[0].start:sl[0].stop, sl[1].start:sl[1].stop], bb)
                        t3 = ttl.copy(c[sl[0].start:sl[0].stop, sl[1].start:sl[1].stop], cb)
                        t1.wait()
                        t2.wait()
                        t3.wait()

        @ttl.datamovement()
        def wr():
            c_ = ttl.core(dims=1)
            for r in range(c_ * per, min(rows, (c_ + 1) * per)):
                for k in range(cols):
                    with o_cb.wait() as o:
                        ttl.copy(o, out[r * g:(r + 1) * g, k * g:(k + 1) * g]).wait()

    return long_chain


def make_softmax_rows(ttl, w=4, grid=(2, 2)):
    """Row softmax the tt-lang way: per block of one tile row x w tiles,
    m = reduce_max(x) -> e = exp(x - broadcast(m)) -> s = reduce_sum(e) ->
    y = e * broadcast(recip(s)), every stage through an intermediate CB
    (reductions fill column 0 of their result tile; the in-tile broadcast
    spreads it)."""
    @ttl.kernel(grid=grid)
    def softmax_rows(x, scaler, out):
        rows = out.shape[0] // TILE
        ncores = grid[0] * grid[1]
        per = -(-rows // ncores)
        x_cb = ttl.make_circular_buffer_like(x, shape=(1, w), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(scaler, shape=(1, 1), buffer_factor=1)
        m_cb = ttl.make_circular_buffer_like(x, shape=(1, 1), buffer_factor=2)
        e_cb = ttl.make_circular_buffer_like(x, shape=(1, w), buffer_factor=2)
        z_cb = ttl.make_circular_buffer_like(x, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, w), buffer_factor=2)

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            with s_cb.wait() as sc:
                for _ in range(c * per, min(rows, (c + 1) * per)):
                    with x_cb.wait() as xb:
                        with m_cb.reserve() as mb:
                            mb.store(ttl.math.reduce_max(xb, sc, dims=[1]))
                        with m_cb.wait() as mb, e_cb.reserve() as eb:
                            eb.store(ttl.math.exp(xb - ttl.math.broadcast(mb, eb, dims=[1])))
                    with e_cb.wait() as eb:
                        with z_cb.reserve() as zb:
                            zb.store(ttl.math.reduce_sum(eb, sc, dims=[1]))
                        with z_cb.wait() as zb, o_cb.reserve() as ob:
                            ob.store(eb * ttl.math.broadcast(ttl.math.recip(zb), ob, dims=[1]))

        @ttl.datamovement()
        def rd():
            c = ttl.core(dims=1)
            with s_cb.reserve() as sb:
                ttl.copy(scaler[0, 0], sb).wait()
            for r in range(c * per, min(rows, (c + 1) * per)):
                with x_cb.reserve() as xb:
                    ttl.copy(x[r, 0:w], xb).wait()

        @ttl.datamovement()
        def wr():
            c = ttl.core(dims=1)
            for r in range(c * per, min(rows, (c + 1) * per)):
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[r, 0:w]).wait()

    return softmax_rows


def make_row_bcast_forms(ttl, with_out: bool, grid=(1, 1)):
    """out = a + broadcast(b, [out,] dims=[0]) with a (2, 2)-tile block and b
    a (1, 2)-tile block of full 32x32 tiles.  With `out` (the compiler's
    form) each b tile is its row 0 repeated; without it (the simulator's
    form) the b tiles are added as they are, re-used over the tile rows."""
    @ttl.kernel(grid=grid)
    def row_bcast_forms(a, b, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(2, 2), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 2), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(2, 2), buffer_factor=2)
        nr = a.shape[0] // TILE // 2
        nc = a.shape[1] // TILE // 2

        @ttl.compute()
        def comp():
            for _ in range(nr):
                for _ in range(nc):
                    with a_cb.wait() as ab, b_cb.wait() as bb, o_cb.reserve() as ob:
                        if with_out:
                            ob.store(ab + ttl.math.broadcast(bb, ob, dims=[0]))
                        else:
                            ob.store(ab + ttl.math.broadcast(bb, dims=[0]))

        @ttl.datamovement()
        def rd():
            for i in range(nr):
                for j in range(nc):
                    with a_cb.reserve() as ab, b_cb.reserve() as bb:
                        ta = ttl.copy(a[2 * i:2 * i + 2, 2 * j:2 * j + 2], ab)
                        tb = ttl.copy(b[0:1, 2 * j:2 * j + 2], bb)
                        ta.wait()
                        tb.wait()

        @ttl.datamovement()
        def wr():
            for i in range(nr):
                for j in range(nc):
                    with o_cb.wait() as ob:
                        ttl.copy(ob, out[2 * i:2 * i + 2, 2 * j:2 * j + 2]).wait()

    return row_bcast_forms


def make_attention(ttl, seq, scale, grid=(8, 8), exp_form="scaled_max", norm="recip",
                   sum_scale=1.0, max_scale=None, own_head=True):
    """O = softmax(Q K^T * scale) V written with the spec's block ops
    (TTLangSpecification.md:693-761: block matmul `@`, reduce_max,
    exp, broadcast, reduce_sum, recip), one query tile row of one (batch,
    head) per work item: q, v, out are [B*H*seq, D] and kt is K^T of every
    head side by side, [D, B*H*seq] (the spec has no transpose: the caller
    passes it, e.g. as a transposed view of K).  Every stage goes through an
    intermediate CB: the score row S (1 x seq/32 tiles), its scaled maximum,
    P = exp(S * scale - max), its row sum, P @ V, and the normalised output.

    Variants: exp_form "scaled_diff" writes P = exp((S - max) * scale) over
    an unscaled maximum; norm "div" writes O / L instead of O * recip(L);
    sum_scale / max_scale are the reductions' scalers (default 1 and
    `scale`, or 1 for "scaled_diff"); own_head=False reads the keys and
    values of the first head for every query (not attention per head)."""
    if max_scale is None:
        max_scale = scale if exp_form == "scaled_max" else 1.0
    @ttl.kernel(grid=grid)
    def attention(q, kt, v, out):
        dt = q.shape[1] // TILE
        st = seq // TILE
        items = q.shape[0] // TILE
        ncores = grid[0] * grid[1]
        per = -(-items // ncores)
        q_cb = ttl.make_circular_buffer_like(q, shape=(1, dt), buffer_factor=2)
        k_cb = ttl.make_circular_buffer_like(kt, shape=(dt, st), buffer_factor=2)
        v_cb = ttl.make_circular_buffer_like(v, shape=(st, dt), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(q, shape=(1, st), buffer_factor=2)
        m_cb = ttl.make_circular_buffer_like(q, shape=(1, 1), buffer_factor=2)
        p_cb = ttl.make_circular_buffer_like(q, shape=(1, st), buffer_factor=2)
        l_cb = ttl.make_circular_buffer_like(q, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(q, shape=(1, dt), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(out, shape=(1, dt), buffer_factor=2)

        @ttl.compute()
        def comp():
            c = ttl.core(dims=1)
            for _ in range(c * per, min(items, (c + 1) * per)):
                with q_cb.wait() as qb, k_cb.wait() as kb, s_cb.reserve() as sb:
                    sb.store(qb @ kb)
                with s_cb.wait() as sb:
                    with m_cb.reserve() as mb:
                        mb.store(ttl.math.reduce_max(sb, max_scale, dims=[1]))
                    with m_cb.wait() as mb, p_cb.reserve() as pb:
                        mx = ttl.math.broadcast(mb, pb, dims=[1])
                        if exp_form == "scaled_max":
                            pb.store(ttl.math.exp(sb * scale - mx))
                        else:
                            pb.store(ttl.math.exp((sb - mx) * scale))
                with p_cb.wait() as pb:
                    with l_cb.reserve() as lb:
                        lb.store(ttl.math.reduce_sum(pb, sum_scale, dims=[1]))
                    with v_cb.wait() as vb, o_cb.reserve() as ob:
                        ob.store(pb @ vb)
                with o_cb.wait() as ob, l_cb.wait() as lb, y_cb.reserve() as yb:
                    if norm == "recip":
                        yb.store(ob * ttl.math.broadcast(ttl.math.recip(lb), yb, dims=[1]))
                    else:
                        yb.store(ob / ttl.math.broadcast(lb, yb, dims=[1]))

        @ttl.datamovement()
        def rd():
            c = ttl.core(dims=1)
            for r in range(c * per, min(items, (c + 1) * per)):
                h0 = (r // st) * st if own_head else 0
                with q_cb.reserve() as qb, k_cb.reserve() as kb:
                    tq = ttl.copy(q[r:r + 1, 0:dt], qb)
                    tk = ttl.copy(kt[0:dt, h0:h0 + st], kb)
                    tq.wait()
                    tk.wait()
                with v_cb.reserve() as vb:
                    ttl.copy(v[h0:h0 + st, 0:dt], vb).wait()

        @ttl.datamovement()
        def wr():
            c = ttl.core(dims=1)
            for r in range(c * per, min(items, (c + 1) * per)):
                with y_cb.wait() as yb:
                    ttl.copy(yb, out[r:r + 1, 0:dt]).wait()

    return attention


def make_block_matmul(ttl, bm, bk, bn):
    """out = a @ b with one (bm, bk) @ (bk, bn) block matmul per output block
    (the spec's block matmul, TTLangSpecification.md:693), the whole K of a
    and b in one block each: a [bm*32*R, bk*32], b [bk*32, bn*32*C]."""
    @ttl.kernel(grid=(1, 1))
    def block_mm(a, b, out):
        R = a.shape[0] // (bm * TILE)
        C = b.shape[1] // (bn * TILE)
        a_cb = ttl.make_circular_buffer_like(a, shape=(bm, bk), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(bk, bn), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(bm, bn), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(R):
                for _ in range(C):
                    with a_cb.wait() as ab, b_cb.wait() as bb, o_cb.reserve() as ob:
                        ob.store(ab @ bb)

        @ttl.datamovement()
        def reader():
            for r in range(R):
                for c in range(C):
                    with a_cb.reserve() as ab, b_cb.reserve() as bb:
                        ta = ttl.copy(a[r * bm:(r + 1) * bm, 0:bk], ab)
                        tb = ttl.copy(b[0:bk, c * bn:(c + 1) * bn], bb)
                        ta.wait()
                        tb.wait()

        @ttl.datamovement()
        def writer():
            for r in range(R):
                for c in range(C):
                    with o_cb.wait() as ob:
                        ttl.copy(ob, out[r * bm:(r + 1) * bm, c * bn:(c + 1) * bn]).wait()

    return block_mm


def make_matmul_epilogue(ttl, bm, bk, bn, epi="relu_bias", grid=(2, 2)):
    """out = f(a @ b, c) in one store per output block: the spec's block
    matmul (bm, bk) @ (bk, bn) over the whole K of a and b (bk = K / 32) or,
    with bk = 1, the simulator's tile-wise product; c is a bias block of
    the output's shape (or a row vector broadcast over the block's rows).
    epi: "relu_bias" relu(a @ b + c), "row_bias" a @ b + broadcast(c_row),
    "scale_exp" exp(a @ b * 0.125) * c.  Output blocks are dealt to the
    cores of the grid row by row."""

    @ttl.kernel(grid=grid)
    def matmul_epilogue(a, b, c, out):
        gx, gy = ttl.grid_size(dims=2)
        rows = a.shape[0] // (bm * TILE)
        cols = b.shape[1] // (bn * TILE)
        per_core = rows * cols // (gx * gy)
        a_cb = ttl.make_circular_buffer_like(a, shape=(bm, bk), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(bk, bn), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(1 if epi == "row_bias" else bm, bn),
                                             buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(bm, bn), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(per_core):
                with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cc, \
                        o_cb.reserve() as ob:
                    if epi == "relu_bias":
                        ob.store(ttl.math.relu(ab @ bb + cc))
                    elif epi == "row_bias":
                        ob.store(ab @ bb + ttl.math.broadcast(cc, dims=[0]))
                    else:
                        ob.store(ttl.math.exp(ab @ bb * 0.125) * cc)

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            first = (cx * gy + cy) * per_core
            for t in range(per_core):
                r, col = (first + t) // cols, (first + t) % cols
                with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cc:
                    ttl.copy(a[r * bm:(r + 1) * bm, 0:bk], ab).wait()
                    ttl.copy(b[0:bk, col * bn:(col + 1) * bn], bb).wait()
                    if epi == "row_bias":
                        ttl.copy(c[0, col * bn:(col + 1) * bn], cc).wait()
                    else:
                        ttl.copy(c[r * bm:(r + 1) * bm, col * bn:(col + 1) * bn], cc).wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            first = (cx * gy + cy) * per_core
            for t in range(per_core):
                r, col = (first + t) // cols, (first + t) % cols
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[r * bm:(r + 1) * bm, col * bn:(col + 1) * bn]).wait()

    return matmul_epilogue


def make_acc_expr(ttl, bm, bk, bn, form="mm_scale_bias", grid=(2, 2)):
    """An output block accumulated with store(expr, acc=True) over the K
    loop, expr not a lone product: the simulator assigns the first store and
    adds the later ones, block = block + expr, rounded to the block's dtype
    (python/sim/block.py:850-864).  form: "mm_scale_bias" a_k @ b_k * 0.5 + c,
    "relu_mm" relu(a_k @ b_k), "eltwise" exp(a_k * 0.25) * 0.5 (a_k the k-th
    (bm, bk) block of a row band; b and c unused).  Output blocks are dealt to
    the cores row by row."""

    @ttl.kernel(grid=grid)
    def acc_expr(a, b, c, out):
        gx, gy = ttl.grid_size(dims=2)
        rows = out.shape[0] // (bm * TILE)
        cols = out.shape[1] // (bn * TILE)
        kt = a.shape[1] // (bk * TILE)
        per_core = rows * cols // (gx * gy)
        a_cb = ttl.make_circular_buffer_like(a, shape=(bm, bk), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(bk, bn), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(bm, bn), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(bm, bn), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(per_core):
                with o_cb.reserve() as ob:
                    for _ in range(kt):
                        with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cc:
                            if form == "mm_scale_bias":
                                ob.store(ab @ bb * 0.5 + cc, acc=True)
                            elif form == "relu_mm":
                                ob.store(ttl.math.relu(ab @ bb), acc=True)
                            else:
                                ob.store(ttl.math.exp(ab * 0.25) * 0.5, acc=True)

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            first = (cx * gy + cy) * per_core
            for t in range(per_core):
                r, col = (first + t) // cols, (first + t) % cols
                for k in range(kt):
                    with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cc:
                        ttl.copy(a[r * bm:(r + 1) * bm, k * bk:(k + 1) * bk], ab).wait()
                        ttl.copy(b[k * bk:(k + 1) * bk, col * bn:(col + 1) * bn], bb).wait()
                        ttl.copy(c[r * bm:(r + 1) * bm, col * bn:(col + 1) * bn], cc).wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            first = (cx * gy + cy) * per_core
            for t in range(per_core):
                r, col = (first + t) // cols, (first + t) % cols
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[r * bm:(r + 1) * bm, col * bn:(col + 1) * bn]).wait()

    return acc_expr


def make_pipe_chain(ttl, n_blocks=2):
    """y[j, c] = x_j + b[j, c] on a 1 x 3 grid, x_j = a[0, j] read by core 0
    only: core 0 sends it to core 1 on one pipe, core 1 forwards the block it
    received to core 2 on a second pipe (python/sim/copyhandlers.py:229: a
    pipe send takes any block), and every core adds its own bias tile."""

    @ttl.kernel(grid=(1, 3))
    def pipe_chain(a, b, y):
        x_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 1), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(1, 1), buffer_factor=2)
        net01 = ttl.PipeNet([ttl.Pipe((0, 0), (0, 1))])
        net12 = ttl.PipeNet([ttl.Pipe((0, 1), (0, 2))])

        @ttl.compute()
        def comp():
            for _ in range(n_blocks):
                with x_cb.wait() as xb, b_cb.wait() as bb, y_cb.reserve() as yb:
                    yb.store(xb + bb)

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            for j in range(n_blocks):
                with x_cb.reserve() as xb:
                    if c == 0:
                        ttl.copy(a[0, j], xb).wait()

                    def recv(p):
                        ttl.copy(p, xb).wait()

                    def send(p):
                        ttl.copy(xb, p).wait()
                    net01.if_dst(recv)
                    net01.if_src(send)
                    net12.if_dst(recv)
                    net12.if_src(send)
                with b_cb.reserve() as bb:
                    ttl.copy(b[j, c], bb).wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for j in range(n_blocks):
                with y_cb.wait() as yb:
                    ttl.copy(yb, y[j, c]).wait()

    return pipe_chain


def make_softmax_one_store(ttl, gc=4, grid=(2, 2), form="softmax"):
    """Row softmax of x (rows of gc tiles, one block per row band) written as
    ONE store whose expression holds the reductions (the spec's reduce_max /
    reduce_sum are BlockExpr -> BlockExpr, TTLangSpecification.md:754-755):
      m = broadcast(reduce_max(x, s, dims=[1]), out, dims=[1])
      e = exp(x - m)
      y = e * broadcast(recip(reduce_sum(e, s, dims=[1])), out, dims=[1])
    form "center": y = x - broadcast(reduce_sum(x, s, dims=[1]), out, dims=[1]) * (1 / W)
    (a row mean subtracted); form "rms": y = x * rsqrt(broadcast(reduce_sum(x * x, s,
    dims=[1]), out, dims=[1]) * (1 / W) + 1e-5) (RMS normalisation)."""

    @ttl.kernel(grid=grid)
    def softmax_one_store(x, s, y):
        gx, gy = ttl.grid_size(dims=2)
        rows_per_core = x.shape[0] // TILE // (gx * gy)
        width = x.shape[1]
        x_cb = ttl.make_circular_buffer_like(x, shape=(1, gc), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(s, shape=(1, 1), buffer_factor=1)
        y_cb = ttl.make_circular_buffer_like(y, shape=(1, gc), buffer_factor=2)

        @ttl.compute()
        def comp():
            with s_cb.wait() as sb:
                for _ in range(rows_per_core):
                    with x_cb.wait() as xb, y_cb.reserve() as yb:
                        if form == "softmax":
                            m = ttl.math.broadcast(ttl.math.reduce_max(xb, sb, dims=[1]), yb,
                                                   dims=[1])
                            e = ttl.math.exp(xb - m)
                            r = ttl.math.recip(ttl.math.reduce_sum(e, sb, dims=[1]))
                            yb.store(e * ttl.math.broadcast(r, yb, dims=[1]))
                        elif form == "rms":
                            ss = ttl.math.broadcast(ttl.math.reduce_sum(xb * xb, sb, dims=[1]),
                                                    yb, dims=[1])
                            yb.store(xb * ttl.math.rsqrt(ss * (1.0 / width) + 1e-5))
                        else:
                            tot = ttl.math.broadcast(ttl.math.reduce_sum(xb, sb, dims=[1]), yb,
                                                     dims=[1])
                            yb.store(xb - tot * (1.0 / width))

        @ttl.datamovement()
        def reader():
            c = ttl.core(dims=1)
            with s_cb.reserve() as sb:
                ttl.copy(s[0, 0], sb).wait()
            for i in range(rows_per_core):
                r = c * rows_per_core + i
                with x_cb.reserve() as xb:
                    ttl.copy(x[r, 0:gc], xb).wait()

        @ttl.datamovement()
        def writer():
            c = ttl.core(dims=1)
            for i in range(rows_per_core):
                r = c * rows_per_core + i
                with y_cb.wait() as yb:
                    ttl.copy(yb, y[r, 0:gc]).wait()

    return softmax_one_store


def make_matmul_computed_operand(ttl, bm=2, bk=2, bn=2, grid=(2, 2), form="scale"):
    """out = f(a) @ g(b) per (bm, bn) output block over the whole K = bk
    tiles (the spec's block matmul of computed BlockExprs,
    TTLangSpecification.md:693): form "scale" (a * 0.25) @ b, "relu_b"
    a @ relu(b) + c... with c = a bias block of the output's shape,
    "both" (a + a) @ (b * 2) (every a block is read by several output
    blocks, so the same operand tile is computed more than once)."""

    @ttl.kernel(grid=grid)
    def matmul_computed(a, b, c, out):
        gx, gy = ttl.grid_size(dims=2)
        rows = a.shape[0] // (bm * TILE)
        cols = b.shape[1] // (bn * TILE)
        per_core = rows * cols // (gx * gy)
        a_cb = ttl.make_circular_buffer_like(a, shape=(bm, bk), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(bk, bn), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(bm, bn), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(bm, bn), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(per_core):
                with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cc, \
                        o_cb.reserve() as ob:
                    if form == "scale":
                        ob.store((ab * 0.25) @ bb)
                    elif form == "relu_b":
                        ob.store(ab @ ttl.math.relu(bb) + cc)
                    else:
                        ob.store((ab + ab) @ (bb * 2.0))

        @ttl.datamovement()
        def reader():
            cx, cy = ttl.core(dims=2)
            first = (cx * gy + cy) * per_core
            for t in range(per_core):
                r, col = (first + t) // cols, (first + t) % cols
                with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cc:
                    ttl.copy(a[r * bm:(r + 1) * bm, 0:bk], ab).wait()
                    ttl.copy(b[0:bk, col * bn:(col + 1) * bn], bb).wait()
                    ttl.copy(c[r * bm:(r + 1) * bm, col * bn:(col + 1) * bn], cc).wait()

        @ttl.datamovement()
        def writer():
            cx, cy = ttl.core(dims=2)
            first = (cx * gy + cy) * per_core
            for t in range(per_core):
                r, col = (first + t) // cols, (first + t) % cols
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[r * bm:(r + 1) * bm, col * bn:(col + 1) * bn]).wait()

    return matmul_computed
