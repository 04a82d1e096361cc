"""GPU parity of penalty-aware MTP verification (lsamp_verify with penalty
entries; CBv2DefaultSampler.applyWindowPenalties, DefaultSamplerV2.swift:
503-580) against the oracle: per-position counts from the confirmed output
and the drafts before each position, EXACT and TYPICAL modes, a column offset
into a longer draft chain, entries that carry repetition flags and biases
(which the verify window ignores), and the scratch-capacity status.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, csr
from test_gpu_verify import check, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=512, max_vocab=262144)
    yield c
    c.close()


def case(seed, S, Wn, V, dtype, offset=0, hot=12, pkw=None):
    """Windows whose target rows favour a small set of hot tokens, confirmed
    outputs and draft chains drawn from the same set, so the penalties decide
    many positions."""
    rng = np.random.default_rng(seed)
    t = rng.normal(0, 2, (S, Wn, V)).astype(np.float32)
    t[:, :, :hot] += 4.0
    outs = [rng.integers(0, hot, rng.integers(0, 30)).tolist() for _ in range(S)]
    chain = rng.integers(0, hot, (S, offset + Wn - 1)).astype(np.int32)
    drafts = np.ascontiguousarray(chain[:, offset:offset + Wn - 1])
    u = rng.random((S, Wn), dtype=np.float32)
    pkw = pkw or dict(temperature=0.9, top_k=40, top_p=0.95, presence_penalty=0.6,
                      frequency_penalty=0.35)
    ps = []
    for s in range(S):
        if s % 4 == 3:      # a row without presence / frequency: untouched
            ps.append(W.resolve_cbv2(temperature=0.9, top_k=40, vocab=V))
        else:
            ps.append(W.resolve_cbv2(vocab=V, **pkw))
    if dtype == _ffi.DTYPE_BF16:
        tb = W.f32_to_bf16_bits(t)
    else:
        tb = t
    # the sequences' entries as a sampler would keep them: output counts plus
    # repetition flags and biases, which the verify window must ignore
    ents = [Cbv2RowState(prompt=rng.integers(0, hot, 8).tolist(), output=o, repetition_window=8,
                         repetition_on=True, counts_on=True,
                         bias={int(rng.integers(0, V)): 1.5}, vocab=V).entries() for o in outs]
    rp, en = csr(ents)
    return tb, outs, chain, drafts, u, W._params(ps), rp, en


def run(ctx, mode, tb, outs, chain, drafts, u, params, rp, en, dtype, offset, delta=0.0,
        use_chain=False, cap=0):
    import torch
    kw = dict(penalty_row_ptr=rp, penalty_entries=en, scratch_cap=cap)
    if use_chain:
        kw.update(penalty_drafts=chain, column_offset=offset)
    g = ctx.verify(to_dev(tb, dtype), None, drafts, params, u, mode=mode, typical_delta=delta, **kw)
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in g.items()}
    o = O.verify(mode=mode, target=tb, draft=None, draft_tokens=drafts, dtype=dtype, params=params,
                 uniforms=u, typical_delta=delta, threads=8, output_tokens=outs,
                 pen_drafts=chain if use_chain else None, column_offset=offset if use_chain else 0)
    return g, o


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_F32, _ffi.DTYPE_BF16])
def test_exact_mode_with_window_penalties(ctx, dtype):
    tb, outs, chain, drafts, u, params, rp, en = case(5 + dtype, 16, 4, 2000, dtype)
    g, o = run(ctx, _ffi.VERIFY_EXACT, tb, outs, chain, drafts, u, params, rp, en, dtype, 0)
    check(g, o, "exact")
    # the penalties change the outcome somewhere (the test is not vacuous)
    plain = O.verify(mode=_ffi.VERIFY_EXACT, target=tb, draft=None, draft_tokens=drafts,
                     dtype=dtype, params=params, uniforms=u, threads=8)
    assert not np.array_equal(plain["tokens"], o["tokens"])


def test_typical_mode_with_window_penalties(ctx):
    dtype = _ffi.DTYPE_BF16
    tb, outs, chain, drafts, u, params, rp, en = case(9, 16, 5, 151936, dtype)
    g, o = run(ctx, _ffi.VERIFY_TYPICAL, tb, outs, chain, drafts, u, params, rp, en, dtype, 0,
               delta=0.3)
    check(g, o, "typical", typical=True)


def test_column_offset_into_the_draft_chain(ctx):
    dtype = _ffi.DTYPE_F32
    tb, outs, chain, drafts, u, params, rp, en = case(13, 8, 4, 3000, dtype, offset=3)
    g, o = run(ctx, _ffi.VERIFY_EXACT, tb, outs, chain, drafts, u, params, rp, en, dtype, 3,
               use_chain=True)
    check(g, o, "column offset 3")


def test_full_size_window(ctx):
    """32 sequences x 4 positions of 151,936 bf16 logits (the MTP verify
    configuration) with presence / frequency penalties."""
    dtype = _ffi.DTYPE_BF16
    tb, outs, chain, drafts, u, params, rp, en = case(17, 32, 4, 151936, dtype, hot=64)
    g, o = run(ctx, _ffi.VERIFY_EXACT, tb, outs, chain, drafts, u, params, rp, en, dtype, 0)
    check(g, o, "32 x 4")


def test_scratch_capacity_is_reported(ctx):
    import torch
    dtype = _ffi.DTYPE_F32
    tb, outs, chain, drafts, u, params, rp, en = case(21, 4, 3, 500, dtype)
    ctx.read_status()  # clear
    g = ctx.verify(to_dev(tb, dtype), None, drafts, params, u, mode=_ffi.VERIFY_EXACT,
                   penalty_row_ptr=rp, penalty_entries=en, scratch_cap=2)
    torch.cuda.synchronize()
    assert ctx.read_status() & _ffi.STATUS_PENALTY_CAPACITY


def test_residual_mode_rejects_penalties(ctx):
    dtype = _ffi.DTYPE_F32
    tb, outs, chain, drafts, u, params, rp, en = case(23, 2, 3, 100, dtype)
    draft = np.zeros((2, 2, 100), np.float32)
    with pytest.raises(_ffi.LsampError):
        ctx.verify(to_dev(tb, dtype), to_dev(draft, dtype), drafts, params, u,
                   mode=_ffi.VERIFY_RESIDUAL, penalty_row_ptr=rp, penalty_entries=en)
