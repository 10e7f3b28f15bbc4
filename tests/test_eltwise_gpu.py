"""GPU parity of the fused elementwise / broadcast kernel (ttlh_eltwise).

Each case builds one expression twice: as the product's Expr IR (run on the
GPU through the C ABI) and as a nested tuple for the CPU oracle
(oracle.tile_ops.eval_expr, the simulator's per-op torch semantics).
Bar: bit-exact for + - * / max min neg abs relu and all broadcasts (one fp32
op, one RNE rounding, same as torch's CPU kernels); transcendental ops within
1 bf16 ULP (device libm vs torch's CPU libm may differ by one fp32 ulp, which
flips a bf16 rounding only near a tie) and fp32 results within 4 fp32 ULP-ish
relative error.
"""

import pytest
import torch

from oracle import tile_ops as O

pytestmark = pytest.mark.gpu


def _expr(e, env):
    from ttlhip import expr as X
    from ttlhip.kernels import OperandMap

    tag = e[0]
    if tag == "leaf":
        t, m = env[e[1]]
        return X.Leaf(m, t.dtype)
    if tag == "const":
        return X.Const(e[1])
    if tag == "powi":
        x = _expr(e[1], env)
        return X.Unary("powi", x, x.dtype, imm=float(e[2]))
    if tag in O.UNARY:
        x = _expr(e[1], env)
        return X.Unary(tag, x, x.dtype)
    a, b = _expr(e[1], env), _expr(e[2], env)
    if isinstance(a, X.Const):
        dt = b.dtype
    elif isinstance(b, X.Const):
        dt = a.dtype
    else:
        dt = X.promote(a.dtype, b.dtype)
    return X.Binary(tag, a, b, dt)


def run_gpu(e, env_cpu, maps, out_shape, out_dtype, region=None):
    from ttlhip import expr as X
    from ttlhip import kernels as K

    dev = {k: (v.cuda(), maps.get(k, {})) for k, v in env_cpu.items()}
    env = {k: (t, K.OperandMap(t, **m)) for k, (t, m) in dev.items()}
    tree = _expr(e, env)
    prog = X.compile_expr(tree)
    ops = [s.leaf.ref if s.leaf is not None else None for s in prog.steps]
    out = torch.full(out_shape, 7.0, dtype=out_dtype, device="cuda")
    K.eltwise(prog, ops, out, region=region)
    torch.cuda.synchronize()
    return out.cpu()


def assert_bitexact(got, ref):
    ref = ref.to(got.dtype)
    same = (got.view(torch.int16 if got.dtype == torch.bfloat16 else torch.int32)
            == ref.view(torch.int16 if ref.dtype == torch.bfloat16 else torch.int32))
    both_nan = torch.isnan(got) & torch.isnan(ref)
    bad = ~(same | both_nan)
    assert not bad.any(), f"{int(bad.sum())} mismatches; first at {bad.nonzero()[0].tolist()}"


def _u(shape, seed, dtype=torch.bfloat16, lo=-2.0, hi=2.0):
    return O.seeded(shape, "uniform", seed, dtype, lo=lo, hi=hi)


def test_add_bf16_bitexact():
    a, b = _u((256, 512), 1), _u((256, 512), 2)
    e = ("add", ("leaf", "a"), ("leaf", "b"))
    got = run_gpu(e, {"a": a, "b": b}, {}, (256, 512), torch.bfloat16)
    assert_bitexact(got, O.eval_expr(e, {"a": a, "b": b}))


def test_add_f32_bitexact():
    a, b = _u((128, 256), 3, torch.float32), _u((128, 256), 4, torch.float32)
    e = ("add", ("leaf", "a"), ("leaf", "b"))
    got = run_gpu(e, {"a": a, "b": b}, {}, (128, 256), torch.float32)
    assert_bitexact(got, O.eval_expr(e, {"a": a, "b": b}))


def test_fused_exp_rowbcast_mul_bf16():
    # config 2 shape class: Y = exp(A + b_row) * C, b_row (1, W) broadcast over rows
    a, c = _u((512, 1024), 5), _u((512, 1024), 6)
    b = _u((1, 1024), 7)
    env = {"a": a, "b": b, "c": c}
    e = ("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "b"))), ("leaf", "c"))
    got = run_gpu(e, env, {}, (512, 1024), torch.bfloat16)
    ref = O.eval_expr(e, env)
    ulp = O.bf16_ulp_diff(got, ref)
    assert int(ulp.max()) <= 1, f"max ulp {int(ulp.max())}"
    assert float((ulp > 0).float().mean()) < 1e-3


def test_col_broadcast_mul_add():
    # examples/broadcast.py: a * b + broadcast(c, dims=[1]) with c (N, 1)
    a, b = _u((256, 256), 8), _u((256, 256), 9)
    c = _u((256, 1), 10)
    env = {"a": a, "b": b, "c": c}
    e = ("add", ("mul", ("leaf", "a"), ("leaf", "b")), ("leaf", "c"))
    got = run_gpu(e, env, {}, (256, 256), torch.bfloat16)
    assert_bitexact(got, O.eval_expr(e, env))


def test_stack_two_subtrees_and_consts():
    a, b, c, d = (_u((64, 128), s) for s in (11, 12, 13, 14))
    env = {"a": a, "b": b, "c": c, "d": d}
    e = ("sub", ("mul", ("leaf", "a"), ("leaf", "b")),
         ("div", ("mul", ("leaf", "c"), ("leaf", "d")), ("add", ("leaf", "a"), ("const", 3.0))))
    got = run_gpu(e, env, {}, (64, 128), torch.bfloat16)
    assert_bitexact(got, O.eval_expr(e, env))


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "max", "min", "floordiv", "mod"])
def test_binary_ops_bitexact(op):
    a = _u((64, 256), 20, lo=-4, hi=4)
    b = _u((64, 256), 21, lo=0.25, hi=3)
    env = {"a": a, "b": b}
    e = (op, ("leaf", "a"), ("leaf", "b"))
    got = run_gpu(e, env, {}, (64, 256), torch.bfloat16)
    assert_bitexact(got, O.eval_expr(e, env))


@pytest.mark.parametrize("op", ["exp", "log", "sqrt", "rsqrt", "tanh", "abs", "neg", "relu",
                                "sigmoid", "recip"])
def test_unary_ops(op):
    lo, hi = (0.05, 4.0) if op in ("log", "sqrt", "rsqrt", "recip") else (-4.0, 4.0)
    a = _u((64, 256), 30, lo=lo, hi=hi)
    env = {"a": a}
    e = (op, ("leaf", "a"))
    got = run_gpu(e, env, {}, (64, 256), torch.bfloat16)
    ref = O.eval_expr(e, env)
    ulp = O.bf16_ulp_diff(got, ref)
    assert int(ulp.max()) <= 1, f"{op}: max ulp {int(ulp.max())}"
    a32 = a.float()
    got32 = run_gpu(e, {"a": a32}, {}, (64, 256), torch.float32)
    ref32 = O.eval_expr(e, {"a": a32})
    torch.testing.assert_close(got32, ref32, rtol=4e-6, atol=1e-7)


def test_pow_and_powi():
    a = _u((32, 128), 40, lo=0.5, hi=2.0)
    b = _u((32, 128), 41, lo=-2.0, hi=2.0)
    env = {"a": a, "b": b}
    for e in (("pow", ("leaf", "a"), ("leaf", "b")), ("powi", ("leaf", "a"), 3)):
        got = run_gpu(e, env, {}, (32, 128), torch.bfloat16)
        assert int(O.bf16_ulp_diff(got, O.eval_expr(e, env)).max()) <= 1


def test_mixed_dtype_promotes_to_f32():
    a = _u((64, 64), 50)
    b = _u((64, 64), 51, torch.float32)
    env = {"a": a, "b": b}
    e = ("mul", ("leaf", "a"), ("leaf", "b"))
    got = run_gpu(e, env, {}, (64, 64), torch.float32)
    assert_bitexact(got, O.eval_expr(e, env))


def test_tile_reuse_mask_and_region():
    # one 32x32 tile re-used over the whole grid (block broadcast of a (1,1)
    # block), written into a sub-region of a larger output
    a = _u((128, 256), 60)
    t = _u((32, 32), 61)
    env = {"a": a, "t": t}
    maps = {"a": {"row_off": -32, "col_off": -64}, "t": {"row_mask": 31, "col_mask": 31}}
    e = ("add", ("leaf", "a"), ("leaf", "t"))
    got = run_gpu(e, env, maps, (192, 320), torch.bfloat16, region=(32, 64, 128, 256))
    ref = O.eval_expr(e, {"a": a, "t": t.repeat(4, 8)})
    assert_bitexact(got[32:160, 64:320], ref)
    assert (got[:32] == 7.0).all() and (got[:, :64] == 7.0).all()


def test_scalar_path_unaligned_and_column_output():
    # width-1 output (column vector) and an odd region force the 1-wide path
    a = _u((96, 1), 70)
    c = _u((96, 1), 71)
    env = {"a": a, "c": c}
    e = ("mul", ("leaf", "a"), ("leaf", "c"))
    got = run_gpu(e, env, {}, (96, 1), torch.bfloat16)
    assert_bitexact(got, O.eval_expr(e, env))
    b = _u((40, 44), 72)
    got = run_gpu(("neg", ("leaf", "b")), {"b": b}, {}, (40, 44), torch.bfloat16)
    assert_bitexact(got, -b)


def test_special_values_and_ties():
    # NaN / inf propagation and exact bf16 rounding ties
    vals = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1.0,
                         1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 65504.0, 3.0e38, 1e-38, -2.5],
                        dtype=torch.float32)
    a = vals.repeat(8, 1).reshape(8, 12)[:, :8].contiguous()
    a = torch.cat([a, a], 1)  # (8, 16)
    b = torch.full_like(a, 2 ** -9)
    env = {"a": a, "b": b}
    e = ("add", ("leaf", "a"), ("leaf", "b"))
    got = run_gpu(e, env, {}, (8, 16), torch.bfloat16)
    ref = O.eval_expr(e, env).to(torch.bfloat16)  # f32 add, one RNE rounding at the store
    assert_bitexact(got, ref)
    e2 = ("max", ("leaf", "a"), ("leaf", "b"))
    got = run_gpu(e2, env, {}, (8, 16), torch.float32)
    assert_bitexact(got, O.eval_expr(e2, env))


@pytest.mark.parametrize("h,w", [(37, 296), (3, 4104), (1, 8), (5, 2048), (130, 520)])
def test_chain_fast_path_shapes(h, w):
    # bf16 linear chains take the 2-D stream kernel: rows narrower than 256
    # chunks share a workgroup, non-power-of-two chunk counts leave dead lanes,
    # rows wider than 2048 elements span several workgroups
    a, c = _u((h, w), 80), _u((h, w), 81)
    b = _u((1, w), 82)
    env = {"a": a, "b": b, "c": c}
    e = ("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "b"))), ("leaf", "c"))
    got = run_gpu(e, env, {}, (h, w), torch.bfloat16)
    ulp = O.bf16_ulp_diff(got, O.eval_expr(e, env))
    assert int(ulp.max()) <= 1
    e2 = ("sub", ("mul", ("add", ("leaf", "a"), ("const", 3.0)), ("leaf", "c")), ("leaf", "b"))
    got = run_gpu(e2, env, {}, (h, w), torch.bfloat16)
    assert_bitexact(got, O.eval_expr(e2, env))
    got = run_gpu(("add", ("leaf", "a"), ("leaf", "c")), env, {}, (h, w), torch.float32)
    assert_bitexact(got, O.eval_expr(("add", ("leaf", "a"), ("leaf", "c")), env).float())


@pytest.mark.parametrize("h,w,region", [
    (257, 3072, None),                # 384 chunks per row: blocks of 128, not 256
    (9, 1000, None),                  # 125 chunks per row, one block of 128
    (70, 3072, (3, 256, 61, 2816)),   # 352 chunks per row at a column offset: blocks of 128
    (70, 1536, (3, 256, 61, 1024)),   # 128 chunks per row, one block
    (33, 2056, (1, 8, 31, 2000)),     # 250 chunks per row, one block of 256
])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_stream_kernel_row_blocks(h, w, region, out_dtype):
    # C2's program and two linear ones with a row vector take the 2-D stream
    # kernel at row lengths that are not a power of two chunks (whole rows)
    # and at column offsets; its row blocks narrow where the last block of a
    # row would be mostly dead lanes; nothing outside the region is written
    a, c = _u((h, w), 90), _u((h, w), 91)
    b = _u((1, w), 92)
    env = {"a": a, "b": b, "c": c}
    for e in [("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "b"))), ("leaf", "c")),
              ("sub", ("mul", ("add", ("leaf", "a"), ("const", 3.0)), ("leaf", "c")),
               ("leaf", "b")),
              ("add", ("leaf", "a"), ("leaf", "b"))]:
        got = run_gpu(e, env, {}, (h, w), out_dtype, region=region)
        ref = O.eval_expr(e, env)
        if out_dtype == torch.float32:
            ref = ref.float()
        if region is not None:
            y0, x0, rh, rw = region
            outside = torch.ones(h, w, dtype=torch.bool)
            outside[y0:y0 + rh, x0:x0 + rw] = False
            assert bool((got[outside] == 7.0).all()), "a write outside the region"
            got = got[y0:y0 + rh, x0:x0 + rw]
            ref = ref[y0:y0 + rh, x0:x0 + rw]
        if e[0] == "mul":  # exp: within 1 bf16 ulp of the oracle (as the flat path)
            assert int(O.bf16_ulp_diff(got.bfloat16(), ref.bfloat16()).max()) <= 1
        else:
            assert_bitexact(got, ref)


@pytest.mark.parametrize("w", [1024, 4096])
def test_row_path_f32_row_scalar_is_not_rounded(w):
    # a program with a row-scalar subtree over rows of 512+ elements runs on
    # the row kernel, which computes the subtree once per row: an f32 value
    # (here rsqrt(c + 1e-5), c an f32 column) must reach the elementwise
    # steps unrounded, as the oracle computes it
    a = _u((64, w), 95)
    c = _u((64, 1), 96, torch.float32, lo=0.5, hi=4.0)
    env = {"a": a, "c": c}
    e = ("mul", ("leaf", "a"), ("rsqrt", ("add", ("leaf", "c"), ("const", 1e-5))))
    got = run_gpu(e, env, {}, (64, w), torch.float32)
    ref = O.eval_expr(e, env)
    assert ref.dtype == torch.float32
    torch.testing.assert_close(got, ref, rtol=4e-6, atol=1e-7)


def test_chain_exp_special_values():
    # a wave whose arguments include inf / NaN / overflow / subnormal results
    # leaves the straight-line exp path; every element still matches torch
    vals = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1.0, 88.0,
                         89.0, -87.0, -100.0, -104.0, 1e-30], dtype=torch.float32)
    a = vals.repeat(64).reshape(24, 32).bfloat16()
    env = {"a": a}
    e = ("exp", ("leaf", "a"))
    got = run_gpu(e, env, {}, (24, 32), torch.bfloat16)
    ref = O.eval_expr(e, env)
    both_nan = torch.isnan(got) & torch.isnan(ref)
    ulp = O.bf16_ulp_diff(got, ref)
    assert bool(((ulp <= 1) | both_nan).all()), got[~((ulp <= 1) | both_nan)]


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_flat_path_region_rows_and_matrix_row_vector(out_dtype):
    # whole-row regions of bf16 operands take the 1-D flat kernel: a region
    # starting below row 0 of the output, an operand addressed with a row
    # offset, a row vector that is one row (row 5) of a matrix, a flat operand
    # read through a larger tensor's leading rows
    a = _u((128, 256), 90)
    m = _u((16, 256), 91)
    c = _u((160, 256), 92)
    env = {"a": a, "m": m, "c": c}
    maps = {"a": {"row_off": -32}, "m": {"row_mask": 0, "row_off": 5}, "c": {"row_off": -32}}
    e = ("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "m"))), ("leaf", "c"))
    got = run_gpu(e, env, maps, (192, 256), out_dtype, region=(32, 0, 128, 256))
    ref = O.eval_expr(e, {"a": a, "m": m[5:6], "c": c[:128]})
    ulp = O.bf16_ulp_diff(got[32:160].bfloat16(), ref.bfloat16())
    assert int(ulp.max()) <= 1
    assert (got[:32] == 7.0).all() and (got[160:] == 7.0).all()
    e2 = ("sub", ("add", ("leaf", "m"), ("leaf", "a")), ("const", 0.5))
    got = run_gpu(e2, env, maps, (192, 256), out_dtype, region=(32, 0, 128, 256))
    assert_bitexact(got[32:160], O.eval_expr(e2, {"a": a, "m": m[5:6]}).to(out_dtype))


@pytest.mark.parametrize("w", [8, 64, 2048, 8192])
def test_flat_path_widths(w):
    # power-of-two row widths (row vectors allowed) and the C1 add shape class
    h = max(1, 65536 // w) + 3
    a, b = _u((h, w), 93), _u((h, w), 94)
    r = _u((1, w), 95)
    env = {"a": a, "b": b, "r": r}
    for e in (("add", ("leaf", "a"), ("leaf", "b")),
              ("add", ("mul", ("leaf", "a"), ("leaf", "r")), ("leaf", "b")),
              ("neg", ("leaf", "a"))):
        got = run_gpu(e, env, {}, (h, w), torch.bfloat16)
        assert_bitexact(got, O.eval_expr(e, env))


@pytest.mark.parametrize("h", [1, 8, 24, 33])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_flat_path_two_chunks_per_lane(h, out_dtype):
    # the flat kernel's lanes take two chunks 256 apart for programs of two or
    # more steps (a workgroup covers 512 chunks): w = 256 gives 32 h chunks, so
    # h = 1 and 8 leave whole halves of the one workgroup dead, h = 24 and 33
    # end mid-workgroup; every op code goes through the shared dispatch, and a
    # program loading four operands runs one chunk per lane
    w = 256
    a, b, c, d = (_u((h, w), 96 + i) for i in range(4))
    r = _u((1, w), 100, lo=0.25, hi=2.0)
    env = {"a": a, "b": b, "c": c, "d": d, "r": r}
    exact = [
        ("sub", ("leaf", "a"), ("leaf", "b")),
        ("relu", ("sub", ("leaf", "a"), ("leaf", "r"))),
        ("abs", ("mul", ("leaf", "a"), ("const", -3.0))),
        ("neg", ("sub", ("const", 1.0), ("leaf", "a"))),
        ("recip", ("mul", ("leaf", "r"), ("leaf", "c"))),
        ("add", ("mul", ("add", ("leaf", "a"), ("leaf", "b")), ("leaf", "c")), ("leaf", "d")),
        # the row vector as the third and as the fourth loaded operand (the
        # kernel numbers loaded operands in step order)
        ("mul", ("add", ("leaf", "a"), ("leaf", "b")), ("leaf", "r")),
        ("add", ("mul", ("add", ("leaf", "a"), ("leaf", "b")), ("leaf", "c")), ("leaf", "r")),
    ]
    for e in exact:
        got = run_gpu(e, env, {}, (h, w), out_dtype)
        assert_bitexact(got, O.eval_expr(e, env).to(out_dtype))
    e = ("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "r"))), ("leaf", "c"))
    got = run_gpu(e, env, {}, (h, w), out_dtype)
    ulp = O.bf16_ulp_diff(got.bfloat16(), O.eval_expr(e, env).bfloat16())
    assert int(ulp.max()) <= 1


@pytest.mark.parametrize("h,w", [(64, 512), (96, 1536), (40, 4096), (17, 8192)])
def test_row_kernel_stack_programs_with_row_constants(h, w):
    # Programs that are not linear chains run on the row kernel when every
    # binary op has at most one operand computed from the row (rows of 512+
    # columns): a softmax-style exp(x - m) * recip(s) and a scale-and-shift
    # (x - m) * rsqrt(v + eps) * g + b, with m, s, v column broadcasts
    # (constant along a row) and g, b row vectors.  Against the oracle (exp
    # within 1 bf16 ulp), and bit for bit against the generic interpreter,
    # which runs the same program over the first 504 columns (narrower than
    # the row kernel takes).
    x = _u((h, w), 40, lo=-4, hi=4)
    m, s = _u((h, 1), 41), _u((h, 1), 42, lo=0.5, hi=4.0)
    var = _u((h, 1), 43, lo=0.1, hi=2.0)
    g, b = _u((1, w), 44), _u((1, w), 45)
    env = {"x": x, "m": m, "s": s, "v": var, "g": g, "b": b}
    e1 = ("mul", ("exp", ("sub", ("leaf", "x"), ("leaf", "m"))), ("recip", ("leaf", "s")))
    e2 = ("add", ("mul", ("mul", ("sub", ("leaf", "x"), ("leaf", "m")),
                          ("rsqrt", ("add", ("leaf", "v"), ("const", 1e-3)))), ("leaf", "g")),
          ("leaf", "b"))
    got1 = run_gpu(e1, env, {}, (h, w), torch.bfloat16)
    assert int(O.bf16_ulp_diff(got1, O.eval_expr(e1, env)).max()) <= 1
    for e in (e1, e2):
        full = run_gpu(e, env, {}, (h, w), torch.bfloat16)
        part = run_gpu(e, env, {}, (h, w), torch.bfloat16, region=(0, 0, h, 504))
        assert torch.equal(full[:, :504].view(torch.int16), part[:, :504].view(torch.int16))
