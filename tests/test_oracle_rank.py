"""CPU tests that pin the oracle's ranking of raw logits (exact top-2 and
log-probabilities) to the reference's own test vectors and to closed forms.

Top-2: Tests/MLXLMTests/CBv2TopTwoTests.swift restated with the same inputs;
the expected ids and values below are derived by hand from the ordering rule
(value descending, id ascending on exact ties, NaN last), and the random
cases are checked against a brute-force full sort.
Log-probabilities: the scripted table model of
Tests/MLXLMTests/CBv2LogprobsTests.swift:40-52 (chosen logprob within 2e-4
of a scalar log-softmax, top-3 in ranking order), scipy's logsumexp, and
closed forms (constant rows, two-token rows, non-finite rows).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
from scipy.special import logsumexp

import oracle as O
from lsamp import _ffi
from rank_common import BF16, DTYPES, F16, F32, bits_to_f32, brute_topk, same_f32, to_bits

NAN, INF = float("nan"), float("inf")

# CBv2TopTwoTests.swift:43-50
REF_ROWS = [
    [7, 7, 7, -1, 0, 2],
    [NAN, -INF, INF, NAN, INF, 0],
    [NAN] * 6,
    [-0.0, 0.0, -1, -2, -3, -4],
    [1.0001, 1.0002, 1.0003, 1, 0, -1],
]


def top2(x, dtype, **kw):
    b = to_bits(x, dtype)
    return O.rank(b, dtype=dtype, k=2, raw_values=True, **kw)


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_rows_exact_order(dtype):
    r = top2(np.array(REF_ROWS, np.float32), dtype)
    ids = r["ids"].tolist()
    vals = r["values"]
    assert ids[0] == [0, 1] and vals[0].tolist() == [7.0, 7.0]
    assert ids[1] == [2, 4] and vals[1].tolist() == [INF, INF]
    assert ids[2] == [0, 1] and np.isnan(vals[2]).all()
    # -0 and +0 tie: the lower id first, each value kept bit for bit
    assert ids[3] == [0, 1]
    assert vals[3].view(np.uint32).tolist() == [0x80000000, 0x00000000]
    if dtype == F32:
        assert ids[4] == [2, 1]
        assert vals[4].tolist() == [np.float32(1.0003), np.float32(1.0002)]
    else:
        # 1.0001 .. 1.0003 round to 1.0 in bf16 and f16: four tied ones
        assert ids[4] == [0, 1] and vals[4].tolist() == [1.0, 1.0]


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_rows_keep_vocabulary_and_row_axes(dtype):
    # CBv2TopTwoTests.swift:52-62: [1, 19, 3] transposed to [1, 3, 19]
    src = np.array([((i * 13) % 23) - 11 for i in range(57)], np.float32)
    b = to_bits(src, dtype)
    r = O.rank(b, dtype=dtype, k=2, raw_values=True, rows=3, vocab=19, row_stride=1, col_stride=3)
    for row in range(3):
        x = [float(src[j * 3 + row]) for j in range(19)]
        exp_ids = brute_topk(x, 2)
        assert r["ids"][row].tolist() == exp_ids
        assert r["values"][row].tolist() == [x[i] for i in exp_ids]


def test_production_and_minimum_vocabulary():
    # CBv2TopTwoTests.swift:64-70
    r = top2(np.array([[NAN, -INF], [4, 4]], np.float32), F32)
    assert r["ids"].tolist() == [[1, 0], [0, 1]]
    assert r["values"][0, 0] == -INF and math.isnan(r["values"][0, 1])
    assert r["values"][1].tolist() == [4.0, 4.0]
    v = np.full(248_320, -1000.0, np.float32)
    v[8_193] = 100
    v[248_319] = 100
    r = top2(v[None, :], F32)
    assert r["ids"].tolist() == [[8_193, 248_319]] and r["values"].tolist() == [[100.0, 100.0]]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k", [1, 2, 5, 32])
def test_topk_matches_brute_force_sort(dtype, k):
    rng = np.random.default_rng(1000 + 10 * dtype + k)
    rows, V = 12, 61
    x = rng.integers(-4, 5, (rows, V)).astype(np.float32)   # many exact ties
    specials = np.array([NAN, INF, -INF, 0.0, -0.0], np.float32)
    for r in range(rows):
        n = rng.integers(0, 12)
        x[r, rng.choice(V, n, replace=False)] = rng.choice(specials, n)
    x[3] = NAN
    x[4] = -INF
    b = to_bits(x, dtype)
    xf = bits_to_f32(b, dtype)
    r = O.rank(b, dtype=dtype, k=k, raw_values=True)
    for i in range(rows):
        exp_ids = brute_topk(xf[i].tolist(), k)
        assert r["ids"][i].tolist() == exp_ids, i
        assert same_f32(r["values"][i], xf[i][exp_ids])


# ------------------------------------------------------------ log-probabilities
def table_row(r, vocab=24):
    """CBv2LogprobsTests.swift:40-52: distinct values on a 1/11 grid, row[r] = 6."""
    row = np.array([np.float32((r * 31 + j * 17) % 89) / np.float32(11.0) - np.float32(4.0)
                    for j in range(vocab)], np.float32)
    row[r] = 6.0
    return row


def scalar_log_softmax(row):
    """The reference test's own scalar reference (CBv2LogprobsTests.swift:62-67), fp32."""
    m = np.float32(row.max())
    s = np.float32(0.0)
    for v in row:
        s = np.float32(s + np.float32(np.exp(np.float32(v - m))))
    lse = np.float32(m + np.float32(np.log(s)))
    return (row - lse).astype(np.float32)


def test_table_model_chosen_and_top3():
    x = np.stack([table_row(r) for r in range(24)])
    tokens = np.arange(24, dtype=np.int32)          # greedy picks the row's 6.0
    r = O.rank(x, dtype=F32, k=3, raw_values=False, tokens=tokens)
    for i in range(24):
        ref = scalar_log_softmax(x[i])
        assert abs(r["chosen"][i] - ref[i]) <= 2e-4
        ranked = sorted(range(24), key=lambda j: -ref[j])[:3]
        assert r["ids"][i].tolist() == ranked and ranked[0] == i
        assert np.all(np.abs(r["values"][i] - ref[ranked]) <= 2e-4)
        # and to double precision against scipy's logsumexp of the same inputs
        exact = x[i].astype(np.float64) - logsumexp(x[i].astype(np.float64))
        assert abs(r["chosen"][i] - exact[i]) <= 1e-6
    assert not r["row_flags"].any()


def test_closed_forms():
    V = 1000
    x = np.full((1, V), 2.5, np.float32)
    r = O.rank(x, dtype=F32, k=4, raw_values=False, tokens=[7])
    assert r["ids"].tolist() == [[0, 1, 2, 3]]       # all tied: lowest ids
    assert np.allclose(r["values"], -math.log(V), atol=1e-6)
    assert abs(r["lse"][0] - (2.5 + math.log(V))) < 1e-12
    a, b = 1.25, -3.5
    r = O.rank(np.array([[a, b]], np.float32), dtype=F32, k=2, raw_values=False, tokens=[1])
    assert abs(r["values"][0, 0] - (-math.log1p(math.exp(b - a)))) < 1e-7
    assert abs(r["chosen"][0] - (b - a - math.log1p(math.exp(b - a)))) < 1e-6


def test_nonfinite_rows_and_token_range():
    x = np.array([[0.0, NAN, 1.0, 2.0],
                  [0.0, INF, 1.0, -INF],
                  [-INF, -INF, -INF, -INF],
                  [0.5, 0.25, -1.0, 3.0]], np.float32)
    r = O.rank(x, dtype=F32, k=2, raw_values=False, tokens=[2, 1, 0, 4])
    assert math.isnan(r["lse"][0])
    assert r["lse"][1] == INF
    assert r["lse"][2] == -INF
    # rows whose log-sum-exp is not finite fail closed (CBv2NonFiniteLogits.swift:8-34):
    # no ids, NaN values and chosen log-probability, the NONFINITE flag
    for i in range(3):
        assert r["ids"][i].tolist() == [-1, -1], i
        assert np.isnan(r["values"][i]).all() and math.isnan(r["chosen"][i]), i
    assert r["ids"][3].tolist() == [3, 0]
    assert math.isnan(r["chosen"][3])                           # token 4 is out of range
    F = _ffi
    assert r["row_flags"].tolist() == [F.ROW_NONFINITE, F.ROW_NONFINITE, F.ROW_NONFINITE,
                                       F.ROW_TOKEN_RANGE]


def test_nonfinite_row_with_finite_lse_keeps_its_logprobs():
    """A row holding -inf beside finite logits has a finite log-sum-exp: it is
    flagged NONFINITE (CBv2NonFiniteLogits.swift:30-34 flags any +-inf) but its
    log-probabilities are defined and written (-inf for the -inf token)."""
    x = np.array([[1.0, -INF, 0.0, -2.0]], np.float32)
    r = O.rank(x, dtype=F32, k=4, raw_values=False, tokens=[1])
    lse = math.log(math.exp(1.0) + 1.0 + math.exp(-2.0))
    assert r["ids"][0].tolist() == [0, 2, 3, 1]
    assert np.allclose(r["values"][0, :3], np.array([1.0, 0.0, -2.0]) - lse, atol=1e-7)
    assert r["values"][0, 3] == -INF and r["chosen"][0] == -INF
    assert r["row_flags"].tolist() == [_ffi.ROW_NONFINITE]


def test_top2_still_ranks_nonfinite_rows():
    """The exact top-2 (raw values) is not a log-probability: it ranks NaN and
    infinite rows by the reference order (CBv2TopTwo.swift:29-47)."""
    x = np.array([[0.0, NAN, 1.0, 2.0], [0.0, INF, 1.0, -INF], [-INF, -INF, -INF, -INF]],
                 np.float32)
    r = O.rank(x, dtype=F32, k=2, raw_values=True)
    assert r["ids"].tolist() == [[3, 2], [1, 2], [0, 1]]


@pytest.mark.parametrize("dtype", [BF16, F16])
def test_logprobs_of_16bit_logits_use_their_exact_values(dtype):
    rng = np.random.default_rng(5 + dtype)
    x = rng.normal(0, 3, (3, 500)).astype(np.float32)
    b = to_bits(x, dtype)
    xf = bits_to_f32(b, dtype).astype(np.float64)
    r = O.rank(b, dtype=dtype, k=5, raw_values=False, tokens=[0, 10, 499])
    for i in range(3):
        lse = logsumexp(xf[i])
        ids = np.argsort(-xf[i], kind="stable")[:5]
        assert r["ids"][i].tolist() == ids.tolist()
        assert np.allclose(r["values"][i], xf[i][ids] - lse, atol=1e-6)
