"""Operand tables and brute-force definitions for the integer, cast and
scalar-coercion rules of the reference's arith dialect.

The brute force works on Python integers and exact rationals, from the
definitions the reference states (dialects/arith_ops.py:35-42 and :98-135,
ops/arith_ops.py:30-36 and :365-480) plus what NumPy does with the results on
an x86-64 host:
* int32 tiles wrap (two's complement);
* divsi / ceildivsi go through float64 (trunc / ceil of a / b); a float64
  that int32 cannot hold (+-inf, NaN, 2^31) converts to INT_MIN, as x86's
  cvttsd2si does;
* floor_divide and remainder by zero give 0 (NumPy's integer loops);
* shifts by an amount outside [0, 32) give 0, or the sign fill for an
  arithmetic right shift (NumPy's npy_lshift / npy_rshift);
* float -> int32 truncates toward zero, and NaN or out-of-range converts to
  INT_MIN (cvttss2si).
"""
from fractions import Fraction
import math

import numpy as np

INT_MIN = -(1 << 31)
INT_MAX = (1 << 31) - 1


def wrap32(v: int) -> int:
    return ((int(v) + (1 << 31)) % (1 << 32)) - (1 << 31)


def to_i32_like_x86(q) -> int:
    """float64 (or exact value) -> int32 as cvttsd2si converts it."""
    if isinstance(q, float) and (math.isnan(q) or math.isinf(q)):
        return INT_MIN
    t = int(q) if not isinstance(q, Fraction) else (q.numerator // q.denominator if q >= 0
                                                    else -((-q.numerator) // q.denominator))
    return t if INT_MIN <= t <= INT_MAX else INT_MIN


def _trunc_q(a, b):
    return to_i32_like_x86(Fraction(a, b)) if b else INT_MIN


def _ceil_q(a, b):
    if not b:
        return INT_MIN
    c = -((-a) // b)            # exact ceiling of a / b
    return c if INT_MIN <= c <= INT_MAX else INT_MIN


def brute_int(op: str, a: int, b: int) -> int:
    a, b = int(a), int(b)
    if op == "arith.addi":
        return wrap32(a + b)
    if op == "arith.subi":
        return wrap32(a - b)
    if op == "arith.muli":
        return wrap32(a * b)
    if op == "arith.divsi":
        return _trunc_q(a, b)
    if op == "arith.remsi":
        return wrap32(a - _trunc_q(a, b) * b)
    if op == "arith.ceildivsi":
        return _ceil_q(a, b)
    if op in ("arith.floordivsi", "arith.divui"):
        return wrap32(a // b) if b else 0
    if op == "arith.remui":
        return wrap32(a % b) if b else 0
    if op == "arith.andi":
        return wrap32(a & b)
    if op == "arith.ori":
        return wrap32(a | b)
    if op == "arith.xori":
        return wrap32(a ^ b)
    if op == "arith.shli":
        return wrap32(a << b) if 0 <= b < 32 else 0
    if op == "arith.shrsi":
        return a >> b if 0 <= b < 32 else (-1 if a < 0 else 0)
    if op == "arith.shrui":
        return wrap32((a & 0xFFFFFFFF) >> b) if 0 <= b < 32 else 0
    if op in ("arith.minsi", "arith.minui"):
        return min(a, b)
    if op in ("arith.maxsi", "arith.maxui"):
        return max(a, b)
    raise KeyError(op)


CMPI = {"eq": lambda a, b: a == b, "ne": lambda a, b: a != b,
        "slt": lambda a, b: a < b, "sle": lambda a, b: a <= b, "sgt": lambda a, b: a > b,
        "sge": lambda a, b: a >= b,
        # the reference compares the values, so the unsigned predicates are the
        # signed ones (dialects/arith_ops.py:154-157)
        "ult": lambda a, b: a < b, "ule": lambda a, b: a <= b, "ugt": lambda a, b: a > b,
        "uge": lambda a, b: a >= b}

INT_OPS = ["arith.addi", "arith.subi", "arith.muli", "arith.divsi", "arith.remsi", "arith.ceildivsi",
           "arith.floordivsi", "arith.divui", "arith.remui", "arith.andi", "arith.ori", "arith.xori",
           "arith.shli", "arith.shrsi", "arith.shrui", "arith.minsi", "arith.maxsi", "arith.minui", "arith.maxui"]
SHIFTS = ("arith.shli", "arith.shrsi", "arith.shrui")


def int_cores(op: str, scalar: bool = False) -> int:
    """Cores of the test kernel.  Two of the reference's integer rules give
    an int64 result for an i32 tile: tile-by-tile shrui computes
    uint32 >> int32, which NumPy promotes to int64 (ops/arith_ops.py:455-457),
    and remsi with a scalar multiplies by np.asarray(scalar), a 0-d int64
    array (dialects/arith_ops.py:41-42).  The reference's store then takes
    the element offset from the 8-byte itemsize (memory.py:278-279), so every
    core after core 0 writes at half its offset.  The values are right and
    the placement is a defect of the reference, so those two are pinned on
    one core."""
    return 1 if (op == "arith.shrui" and not scalar) or (op == "arith.remsi" and scalar) else 4


def int_operands(op: str, n: int = 4096, seed: int = 0):
    """(a, b) int32 vectors: every pair of a table of edge values (zero,
    +-1, INT_MIN, INT_MAX, small and large magnitudes of both signs), then
    random values; shift amounts span [-3, 40]."""
    rng = np.random.default_rng(seed)
    edge = np.array([0, 1, -1, 2, -2, 3, -3, 7, -7, 100, -100, 65535, -65536, INT_MAX, INT_MIN, INT_MIN + 1,
                     12345678, -12345678, 1 << 30, -(1 << 30)], np.int64)
    if op in SHIFTS:
        sh = np.arange(-3, 41, dtype=np.int64)
        a0, b0 = (x.reshape(-1) for x in np.meshgrid(edge, sh))
        b_rand = rng.integers(-3, 41, n)
    else:
        a0, b0 = (x.reshape(-1) for x in np.meshgrid(edge, edge))
        b_rand = rng.integers(-(1 << 31), 1 << 31, n) // (1 << rng.integers(0, 31, n))
    a_rand = rng.integers(-(1 << 31), 1 << 31, n) // (1 << rng.integers(0, 31, n))
    a = np.concatenate([a0, a_rand])[:n].astype(np.int32)
    b = np.concatenate([b0, b_rand])[:n].astype(np.int32)
    return a, b


def fptosi_brute(x) -> int:
    """float -> int32: truncate toward zero; NaN, +-inf and out-of-range give INT_MIN."""
    x = float(x)
    if math.isnan(x) or math.isinf(x):
        return INT_MIN
    return to_i32_like_x86(x)


def float_cast_operands(n: int = 4096, seed: int = 1):
    """f32 values across the int32 range and past it, with halves, NaN and infinities."""
    rng = np.random.default_rng(seed)
    special = np.array([0.0, -0.0, 0.5, -0.5, 0.999, -0.999, 1.5, -1.5, 2.5, -2.5, 2147483520.0,
                        -2147483648.0, 2147483648.0, -2147483904.0, 3e9, -3e9, 1e30, -1e30, np.inf, -np.inf,
                        np.nan, 65504.0, -65504.0, 1e-40], np.float32)
    r = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 10, n)).astype(np.float32)
    return np.concatenate([special, r])[:n]


def f16_coerce_brute(x: float) -> float:
    """The reference's `np.float16(scalar)` for a scalar operand of a float
    binop (dialects/_helpers.py:47-54): round to nearest even at f16's 11
    significant bits, with f16's subnormal step 2^-24 and overflow to inf
    (the largest finite value is 65504; 65520 and above round to inf)."""
    x = Fraction(x)
    if x == 0:
        return 0.0
    s = -1 if x < 0 else 1
    m = abs(x)
    e = max(math.floor(math.log2(m)), -14)
    while Fraction(2) ** e > m:
        e -= 1
    while Fraction(2) ** (e + 1) <= m:
        e += 1
    e = max(e, -14)
    q = m / Fraction(2) ** (e - 10)          # units of the last place
    fl = math.floor(q)
    rem = q - fl
    r = fl + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1) else 0)
    v = Fraction(r) * Fraction(2) ** (e - 10)
    if v >= 65520 or v > 65504:
        return s * math.inf
    return s * float(v)
