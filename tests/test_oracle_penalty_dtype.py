"""Pins the oracle's mlx-lm penalties on 16-bit logits to exact arithmetic.

RepetitionContext and PresencePenaltyContext (Evaluate.swift:586-596,
:620-625) compute `x * p`, `x / p` and `x - p` between a bfloat16 / float16
logits array and a Swift `Float` scalar.  MLX gives such a scalar the array's
dtype; the reference states the rule in its own source ("Swift scalars use the
logits' dtype; a float32 tensor would promote low-precision logits",
Libraries/MLXLMCommon/Gemma4Fusions.swift:9) and tests it bit for bit
(Tests/MLXLMTests/Gemma4FusionTests.swift:19-31).  So:

* the penalty is rounded once to the logits' dtype (from its float32 value);
* each product, quotient and difference is the exact real result rounded once,
  round-half-even, to the dtype (8 significand bits for bfloat16, 11 for half),
  with the dtype's subnormals and overflow to infinity;
* FrequencyPenaltyContext (:649-658) subtracts a float32 histogram times the
  Float penalty, so a row it touches is promoted to float32:
  fl32(x - fl32(count * f)) at every token.

The expected values here are computed with Python integers (exact rationals)
and one rounding; nothing is taken from the oracle's own formula.  The oracle
computes in float32 and rounds once to the dtype; that equals a single
rounding because float32 carries at least 2p + 2 significand bits for p = 8
and p = 11 (Figueroa, "When is double rounding innocuous?", SIGNUM 1995).
Every one of the 2^16 patterns of each dtype is checked at repetition
penalties 1.1, 1.3, 0.7 and -1.5 and presence 0.5 / 1.3.  The alternative rules
(the penalty kept in float32; a result not rounded back to the dtype) are
shown to disagree with the exact rule on many patterns, so an oracle that
followed either would fail these tests.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W

BF16, F16, F32 = _ffi.DTYPE_BF16, _ffi.DTYPE_F16, _ffi.DTYPE_F32
REP, PRES = _ffi.PEN_REPETITION, _ffi.PEN_PRESENCE

# (significand bits p, minimum normal exponent, maximum exponent)
FORMATS = {BF16: (8, -126, 127), F16: (11, -14, 15), F32: (24, -126, 127)}


def _ratio(v):
    """An exactly representable float -> (numerator, denominator)."""
    return float(v).as_integer_ratio()


def round_exact(num, den, fmt):
    """num / den (den > 0) rounded once, half to even, to `fmt`; returns a
    Python float (exact: every value of the three formats is a double), with
    +-inf on overflow.  A zero result keeps the sign of num/den; a result that
    is exactly zero is returned as +0.0."""
    p, emin, emax = FORMATS[fmt]
    neg = num < 0
    a = -num if neg else num
    if a == 0:
        return 0.0
    # e = floor(log2(a / den))
    e = a.bit_length() - den.bit_length()
    if (a << max(0, -e)) < (den << max(0, e)):
        e -= 1
    q = max(e, emin) - p + 1                      # the ulp is 2^q
    if q >= 0:
        dd = den << q
        n, rem = divmod(a, dd)
    else:
        dd = den
        n, rem = divmod(a << -q, den)
    if 2 * rem > dd or (2 * rem == dd and n & 1):
        n += 1
    if n > 0 and n * 2.0 ** q > ((1 << p) - 1) * 2.0 ** (emax - p + 1):
        r = float("inf")
    else:
        r = float(n) * 2.0 ** q
    return -r if neg else r


def dtype_values(dt):
    """All 2^16 patterns of `dt` as float32 (NaNs included)."""
    h = np.arange(1 << 16, dtype=np.uint16)
    return W.bf16_bits_to_f32(h) if dt == BF16 else O.f16_to_f32(h)


def oracle_processed(dt, bits, rep=1.0, pres=0.0, freq=0.0, flags=REP | PRES, counts=None):
    """The oracle's mlx-lm processed row: one row of every pattern, every token
    a penalty entry (the ring's distinct ids)."""
    V = bits.size
    ent = np.zeros(V, O.PENALTY_DTYPE)
    ent["token"] = np.arange(V)
    ent["count"] = 1 if counts is None else counts
    ent["flags"] = flags
    p = W.resolve_mlxlm(temperature=0.0)
    p["repetition_penalty"], p["presence_penalty"], p["frequency_penalty"] = rep, pres, freq
    out = O.sample(semantics=_ffi.SEM_MLXLM, logits=bits.reshape(1, -1), dtype=dt,
                   params=W._params([p]), row_ptr=np.array([0, V], np.int32), entries=ent,
                   uniforms=np.zeros(1, np.float32), want_processed=True)
    return out["processed"][0]


def expected(x, op, pen, fmt):
    """x op pen for one finite or infinite x (pen already in the format)."""
    if np.isinf(x):
        if op == "sub":
            return float(x)
        return float(x) if (pen > 0) else -float(x)
    xn, xd = _ratio(x)
    pn, pd = _ratio(pen)
    if op == "mul":
        num, den = xn * pn, xd * pd
    elif op == "div":
        num, den = xn * pd, xd * pn
    else:
        num, den = xn * pd - pn * xd, xd * pd
    if den < 0:
        num, den = -num, -den
    r = round_exact(num, den, fmt)
    if r == 0.0 and op in ("mul", "div"):
        # a product or quotient that is (or underflows to) zero carries the
        # sign of x * pen; an exact difference of zero is +0 (round-to-nearest)
        neg = (np.signbit(x) != (pen < 0))
        return -0.0 if neg else 0.0
    return r


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.view(np.uint32) == b.view(np.uint32)


@pytest.mark.parametrize("dt", [BF16, F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("penalty", [1.1, 1.3, 0.7, -1.5])
def test_repetition_penalty_single_rounded_in_the_logits_dtype(dt, penalty):
    xs = dtype_values(dt)
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = oracle_processed(dt, bits, rep=penalty, flags=REP)
    pen = round_exact(*_ratio(np.float32(penalty)), dt)          # Float scalar -> dtype
    fin = ~np.isnan(xs)
    want = np.array([expected(x, "mul" if x < 0 else "div", pen, dt) for x in xs[fin]],
                    np.float64).astype(np.float32)
    ok = same_bits(got[fin], want)
    assert ok.all(), (f"{ok.size - ok.sum()} patterns differ, first x={xs[fin][~ok][:4]} "
                      f"got={got[fin][~ok][:4]} want={want[~ok][:4]}")
    # a NaN logit defines no token: the processed row holds -inf there
    assert (got[~fin] == -np.inf).all()


@pytest.mark.parametrize("dt", [BF16, F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("penalty", [0.5, 1.3])
def test_presence_penalty_single_rounded_in_the_logits_dtype(dt, penalty):
    xs = dtype_values(dt)
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = oracle_processed(dt, bits, pres=penalty, flags=PRES)
    pen = round_exact(*_ratio(np.float32(penalty)), dt)
    fin = ~np.isnan(xs)
    want = np.array([expected(x, "sub", pen, dt) for x in xs[fin]], np.float64).astype(np.float32)
    ok = same_bits(got[fin], want)
    assert ok.all(), f"{ok.size - ok.sum()} patterns differ, first x={xs[fin][~ok][:4]}"


@pytest.mark.parametrize("dt", [BF16, F16], ids=["bf16", "f16"])
def test_frequency_penalty_promotes_the_row_to_float32(dt):
    """Repetition 1.3 and presence 0.5 in the dtype, then the float32
    frequency term fl32(x - fl32(count * 0.3)) at every entry (counts 1..7),
    and x itself (exactly) at tokens outside the history."""
    xs = dtype_values(dt)
    bits = np.arange(1 << 16, dtype=np.uint16)
    counts = (np.arange(1 << 16) % 7 + 1).astype(np.int32)
    got = oracle_processed(dt, bits, rep=1.3, pres=0.5, freq=0.3, counts=counts)
    rp = round_exact(*_ratio(np.float32(1.3)), dt)
    pp = round_exact(*_ratio(np.float32(0.5)), dt)
    f = np.float32(0.3)
    fin = np.isfinite(xs)
    want = []
    for x, c in zip(xs[fin], counts[fin]):
        x1 = expected(x, "mul" if x < 0 else "div", rp, dt)
        x2 = expected(np.float32(x1), "sub", pp, dt) if np.isfinite(x1) else x1
        h = round_exact(*_ratio(np.float32(c) * np.float64(f)), F32)   # c * f exact in f64
        want.append(expected(np.float32(x2), "sub", h, F32) if np.isfinite(x2) else x2)
    want = np.array(want, np.float64).astype(np.float32)
    ok = same_bits(got[fin], want)
    assert ok.all(), f"{ok.size - ok.sum()} patterns differ, first x={xs[fin][~ok][:4]}"
    # the float32 results are not all representable in the dtype: promoted
    back = (O.f32_to_bf16(got[fin]) if dt == BF16 else O.f32_to_f16(got[fin]))
    wide = (W.bf16_bits_to_f32(back) if dt == BF16 else O.f16_to_f32(back))
    assert (wide != got[fin]).mean() > 0.5
    # tokens outside the history: x - 0 * f = x, float32 exactly
    other = np.arange(1 << 16, dtype=np.uint16)
    g2 = oracle_processed(dt, other, freq=0.3, counts=np.zeros(1 << 16, np.int32), flags=0)
    assert same_bits(g2[fin], xs[fin]).all()


@pytest.mark.parametrize("dt", [BF16, F16], ids=["bf16", "f16"])
def test_the_exact_rule_rejects_the_alternatives(dt):
    """The checks above discriminate: computing with the float32 penalty, or
    leaving the float32 result unrounded, disagrees with the exact rule (so an
    oracle that did either would fail them), while a float32 computation
    followed by one rounding agrees with it everywhere."""
    xs = dtype_values(dt)
    fin = np.isfinite(xs) & (xs != 0)
    xs = xs[fin]
    p32 = np.float32(1.1)
    pen = round_exact(*_ratio(p32), dt)
    assert pen != float(p32)
    exact = np.array([expected(x, "mul" if x < 0 else "div", pen, dt) for x in xs],
                     np.float64).astype(np.float32)
    # the float32 penalty, each result rounded once to the dtype
    f32_pen = np.array([expected(x, "mul" if x < 0 else "div", float(p32), dt) for x in xs],
                       np.float64).astype(np.float32)
    # the dtype penalty, the result left in float32
    with np.errstate(over="ignore"):
        unrounded = np.where(xs < 0, xs * np.float32(pen), xs / np.float32(pen)).astype(np.float32)
    # float32 arithmetic then one rounding to the dtype (what the oracle does)
    to16 = (lambda v: W.bf16_bits_to_f32(O.f32_to_bf16(v))) if dt == BF16 else \
        (lambda v: O.f16_to_f32(O.f32_to_f16(v)))
    twice = to16(unrounded)
    assert (~same_bits(f32_pen, exact)).sum() > 1000
    assert (~same_bits(unrounded, exact)).sum() > 10000
    assert same_bits(twice, exact).all()
