"""The spec's further ttl.math functions (TTLangSpecification.md:700-750) with
their parameters and an input range inside each function's domain, shared by
the CPU and GPU tests."""

# name -> (params, (lo, hi))
CASES = {
    "exp2": ((), (-8, 8)),
    "expm1": ((), (-4, 4)),
    "logp1": ((), (-0.9, 4)),
    "square": ((), (-4, 4)),
    "rsub": ((3,), (-4, 4)),
    "sin": ((), (-4, 4)),
    "cos": ((), (-4, 4)),
    "tan": ((), (-1.2, 1.2)),
    "asin": ((), (-0.95, 0.95)),
    "acos": ((), (-0.95, 0.95)),
    "atan": ((), (-6, 6)),
    "asinh": ((), (-6, 6)),
    "acosh": ((), (1.05, 6)),
    "atanh": ((), (-0.95, 0.95)),
    "gelu": ((), (-5, 5)),
    "silu": ((), (-6, 6)),
    "softsign": ((), (-6, 6)),
    "hardsigmoid": ((), (-5, 5)),
    "relu_max": ((2,), (-4, 4)),
    "relu_min": ((1,), (-4, 4)),
    "hardtanh": ((-1, 2), (-4, 4)),
    "leaky_relu": ((0.125,), (-4, 4)),
    "prelu": ((0.25,), (-4, 4)),
    "elu": ((1.5,), (-4, 4)),
    "celu": ((2.0, 0.5), (-4, 4)),
    "selu": ((1.0507, 1.6733), (-4, 4)),
    "softplus": ((2.0, 0.5, 5.0), (-4, 4)),
}
