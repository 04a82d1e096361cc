"""GPU parity of the ranking entry points (lsamp_top2, lsamp_logprobs) through
the C ABI against the oracle: the reference's top-2 test vectors, strided and
misaligned views, slice tails, ties across slices, non-finite rows, the
candidate-heavy worst case, and the 64 x 151,936 bf16 batch.
"""
from __future__ import annotations

import numpy as np
import pytest

from rank_common import (BF16, DTYPES, F16, F32, check_logprobs, check_top2, to_bits)

pytestmark = pytest.mark.gpu

NAN, INF = float("nan"), float("inf")
V = 151936


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=262144)
    yield c
    c.close()


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_rows(ctx, dtype):
    rows = np.array([[7, 7, 7, -1, 0, 2], [NAN, -INF, INF, NAN, INF, 0], [NAN] * 6,
                     [-0.0, 0.0, -1, -2, -3, -4], [1.0001, 1.0002, 1.0003, 1, 0, -1]], np.float32)
    b = to_bits(rows, dtype)
    ids, vals = check_top2(ctx, b, dtype, 5, 6, 6, 1, label="reference rows")
    assert ids[3].tolist() == [0, 1] and vals[3].view(np.uint32).tolist() == [0x80000000, 0]


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_rows(ctx, dtype):
    src = np.array([((i * 13) % 23) - 11 for i in range(57)], np.float32)
    check_top2(ctx, to_bits(src, dtype), dtype, 3, 19, 1, 3, label="strided")


def test_production_and_minimum_vocabulary(ctx):
    check_top2(ctx, np.array([NAN, -INF, 4, 4], np.float32), F32, 2, 2, 2, 1, label="vocab 2")
    v = np.full(248_320, -1000.0, np.float32)
    v[8_193] = 100
    v[248_319] = 100
    ids, _ = check_top2(ctx, v, F32, 1, v.size, v.size, 1, label="vocab 248320")
    assert ids.tolist() == [[8_193, 248_319]]


def special_row(r, i, rng):
    """Row i (1..7) of a batch gets one kind of special value."""
    vocab = r.size
    if i == 1:
        r[rng.choice(vocab, 5, replace=False)] = NAN
    elif i == 2:
        r[rng.choice(vocab, 3, replace=False)] = INF
    elif i == 3:                                   # all -inf but two tokens
        r.fill(-INF)
        r[rng.choice(vocab, 2, replace=False)] = -3.0
    elif i == 4:                                   # every token tied
        r.fill(1.5)
    elif i == 5:                                   # ties across slices
        r[[7, vocab // 2, vocab - 1]] = 50.0
    elif i == 6:
        r.fill(NAN)
    elif i == 7:                                   # non-positive, signed zeros
        np.minimum(r, 0.0, out=r)
        r[rng.choice(vocab, 40, replace=False)] = -0.0


def batch(rng, rows, vocab, dtype, specials=True):
    x = rng.normal(0.0, 2.0, (rows, vocab)).astype(np.float32)
    if specials:
        for i in range(1, min(rows, 8)):
            special_row(x[i], i, rng)
    return to_bits(x, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_batch_top2(ctx, dtype):
    rng = np.random.default_rng(11 + dtype)
    rows = 64 if dtype == BF16 else 12
    b = batch(rng, rows, V, dtype)
    check_top2(ctx, b, dtype, rows, V, V, 1, label="batch")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k", [0, 1, 20, 32])
def test_batch_logprobs(ctx, dtype, k):
    rng = np.random.default_rng(31 + dtype * 7 + k)
    rows = 64 if dtype == BF16 else 12
    b = batch(rng, rows, V, dtype)
    tokens = rng.integers(0, V, rows).astype(np.int32)
    tokens[0] = -1
    tokens[9] = V
    check_logprobs(ctx, b, dtype, rows, V, V, 1, k, tokens=tokens, label=f"k={k}")


@pytest.mark.parametrize("vocab", [7, 1000, 4097, 16385, 151937])
@pytest.mark.parametrize("dtype", [BF16, F32])
def test_tails_and_unaligned_views(ctx, vocab, dtype):
    """Vocab sizes that end inside a 16-byte vector or a slice, rows that are
    not 16-byte aligned (element offset 1: the element-by-element loads)."""
    rng = np.random.default_rng(vocab + dtype)
    rows = 6
    b = batch(rng, rows + 1, vocab, dtype, specials=vocab > 8)
    k = min(20, vocab)
    check_top2(ctx, b, dtype, rows, vocab, vocab, 1, label="aligned")
    check_top2(ctx, b, dtype, rows, vocab, vocab, 1, offset=1, label="offset 1")
    tok = rng.integers(0, vocab, rows).astype(np.int32)
    check_logprobs(ctx, b, dtype, rows, vocab, vocab, 1, k, tokens=tok, label="aligned")
    check_logprobs(ctx, b, dtype, rows, vocab, vocab, 1, k, tokens=tok, offset=1, label="offset 1")


def test_candidate_heavy_slice(ctx):
    """The best tokens of the first two slices all sit in 32 threads (every
    token of threads 0..31 of each slice): each of those threads lists all of
    its tokens, 1,024 candidates per slice."""
    rng = np.random.default_rng(5)
    rows = 4
    x = rng.normal(0.0, 1.0, (rows, V)).astype(np.float32)
    # 4 rows of 151,936 tokens: slices of 16,384 tokens, thread t of a slice
    # holds its 16-byte vectors t, t + 512, t + 1024, t + 1536 (8 bf16 each)
    for q in range(8):
        for t in range(32):
            i0 = (q * 512 + t) * 8
            x[:, i0:i0 + 8] = 10.0 + rng.random((rows, 8))
    b = to_bits(x, BF16)
    check_top2(ctx, b, BF16, rows, V, V, 1, label="heavy top2")
    check_logprobs(ctx, b, BF16, rows, V, V, 1, 32, tokens=np.arange(rows, dtype=np.int32),
                   label="heavy logprobs")


def test_repeated_calls_and_row_stride_zero(ctx):
    """The arrival counters return to zero: calls back to back agree, and a
    view whose rows all alias one row gives that row's answer everywhere."""
    import torch
    rng = np.random.default_rng(9)
    b = batch(rng, 8, V, BF16)
    for _ in range(3):
        check_top2(ctx, b, BF16, 8, V, V, 1, label="repeat")
    ids, _ = check_top2(ctx, b, BF16, 8, V, 0, 1, label="row stride 0")
    assert (ids == ids[0]).all()
    torch.cuda.synchronize()


def test_argument_errors(ctx):
    import torch
    from lsamp import _ffi
    x = torch.zeros((2, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_ffi.LsampError):
        ctx.logprobs(x, top_k=33)
    with pytest.raises(_ffi.LsampError):
        ctx.top2(x[:, :1])
    with pytest.raises(_ffi.LsampError):
        ctx.top2(torch.zeros((65, 100), dtype=torch.bfloat16, device="cuda"))
