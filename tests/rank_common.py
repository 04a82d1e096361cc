"""Helpers of the ranking tests (exact top-2 and raw log-probabilities): logit
bit conversions, a brute-force ordering, and the GPU-vs-oracle comparison.

Parity rules:
* ids: identical;
* top-2 values: the logits converted to float32, bit for bit (NaN: both NaN);
* log-probabilities: within LOGPROB_TOL of the oracle's (the oracle sums in
  double; the kernel sums exp in fp32 per thread and combines in double),
  equal when non-finite.
"""
from __future__ import annotations

import functools
import math

import numpy as np

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W

F32, BF16, F16 = _ffi.DTYPE_F32, _ffi.DTYPE_BF16, _ffi.DTYPE_F16
DTYPES = (F32, BF16, F16)
LOGPROB_TOL = 2e-5


def to_bits(x, dtype):
    """float32 values -> storage of `dtype` (float32, or uint16 bit patterns)."""
    x = np.asarray(x, np.float32)
    if dtype == F32:
        return x.copy()
    if dtype == BF16:
        return W.f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


def bits_to_f32(b, dtype):
    b = np.asarray(b)
    if dtype == F32:
        return b.astype(np.float32)
    if dtype == BF16:
        return W.bf16_bits_to_f32(b)
    return b.view(np.float16).astype(np.float32)


def better(a, ia, b, ib):
    """CBv2TopTwo.swift:29-47 as a comparison of (value, id) pairs."""
    an, bn = math.isnan(a), math.isnan(b)
    if an != bn:
        return not an
    if a > b:
        return True
    if a < b:
        return False
    return ia < ib


def brute_topk(row, k):
    """Full sort of one row by the reference ordering (tiny rows only)."""
    def cmp(i, j):
        if better(row[i], i, row[j], j):
            return -1
        if better(row[j], j, row[i], i):
            return 1
        return 0
    order = sorted(range(len(row)), key=functools.cmp_to_key(cmp))
    return order[:k]


def same_f32(a, b):
    """Bit-equal float32 arrays, NaN matching NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


def close_logprobs(a, b, tol=LOGPROB_TOL):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    fin = np.isfinite(a) & np.isfinite(b)
    same_nonfinite = (~np.isfinite(a)) & (~np.isfinite(b)) & (
        (np.isnan(a) & np.isnan(b)) | (a == b))
    with np.errstate(invalid="ignore"):  # (inf - inf where both are non-finite)
        near = fin & (np.abs(a - b) <= tol)
    return bool(np.all(same_nonfinite | near))


def torch_view(storage, dtype, rows, vocab, row_stride, col_stride, offset=0, device="cuda"):
    """A [rows, vocab] strided torch view of host storage (bits) on the GPU."""
    import torch
    if dtype == F32:
        t = torch.from_numpy(np.ascontiguousarray(storage, np.float32))
    else:
        tdt = torch.bfloat16 if dtype == BF16 else torch.float16
        t = torch.from_numpy(np.ascontiguousarray(storage, np.uint16).view(np.int16)).view(tdt)
    t = t.reshape(-1).to(device)
    return t.as_strided((rows, vocab), (row_stride, col_stride), offset)


def check_top2(ctx, storage, dtype, rows, vocab, row_stride, col_stride, offset=0, label=""):
    """lsamp_top2 on the GPU against the oracle on the same view."""
    import torch
    v = torch_view(storage, dtype, rows, vocab, row_stride, col_stride, offset)
    got = ctx.top2(v)
    torch.cuda.synchronize()
    flat = np.ascontiguousarray(storage).reshape(-1)[offset:]
    ref = O.rank(flat, dtype=dtype, k=2, raw_values=True, rows=rows, vocab=vocab,
                 row_stride=row_stride, col_stride=col_stride)
    ids = got["ids"].cpu().numpy()
    vals = got["values"].cpu().numpy()
    bad = np.nonzero((ids != ref["ids"]).any(axis=1))[0]
    assert bad.size == 0, f"{label}: ids differ in rows {bad[:8]}: {ids[bad[:4]]} vs {ref['ids'][bad[:4]]}"
    assert same_f32(vals, ref["values"]), f"{label}: values differ"
    return ids, vals


def check_logprobs(ctx, storage, dtype, rows, vocab, row_stride, col_stride, top_k, tokens=None,
                   offset=0, label=""):
    import torch
    v = torch_view(storage, dtype, rows, vocab, row_stride, col_stride, offset)
    got = ctx.logprobs(v, tokens=tokens, top_k=top_k)
    torch.cuda.synchronize()
    flat = np.ascontiguousarray(storage).reshape(-1)[offset:]
    ref = O.rank(flat, dtype=dtype, k=top_k, raw_values=False, rows=rows, vocab=vocab,
                 row_stride=row_stride, col_stride=col_stride, tokens=tokens)
    ids = got["top_ids"].cpu().numpy()
    bad = np.nonzero((ids != ref["ids"]).any(axis=1))[0] if top_k else np.zeros(0, int)
    assert bad.size == 0, f"{label}: ids differ in rows {bad[:8]}: {ids[bad[:2]]} vs {ref['ids'][bad[:2]]}"
    assert close_logprobs(got["top_values"].cpu().numpy(), ref["values"]), f"{label}: top values"
    flags = got["row_flags"].cpu().numpy().astype(np.uint32)
    assert np.array_equal(flags, ref["row_flags"]), f"{label}: flags {flags} vs {ref['row_flags']}"
    if tokens is not None:
        assert close_logprobs(got["chosen"].cpu().numpy(), ref["chosen"]), f"{label}: chosen"
    return got, ref
