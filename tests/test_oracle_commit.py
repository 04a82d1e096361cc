"""CPU tests of the oracle's incremental penalty state (LogitsPipelineV2
setRows / commit, LogitsPipelineV2.swift:238-256, 357-384), pinned to the
reference's two commit tests (Tests/MLXLMTests/CBv2SamplingTests.swift:203-266)
and to the rule those tests state: committing tokens one by one lands in the
state a rebuild from the longer history gives.  The host builder of the
sparse entries (lsamp.history.Cbv2RowState) is checked against it too.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp.history import Cbv2RowState

BOTH = _ffi.STATE_COUNTS | _ffi.STATE_REPETITION
V = 16


def nz(a):
    return {int(i): float(a[i]) for i in np.nonzero(a)[0]}


def test_commit_with_window_eviction():
    # CBv2SamplingTests.swift:203-238: window 2, prompt [0, 1], tokens 5, 6, 5, 7
    st = O.DenseRowState(V, [0, 1], [], 2, BOTH)
    for t in [5, 6, 5, 7]:
        st.commit(t)
    assert nz(st.counts) == {5: 2.0, 6: 1.0, 7: 1.0}
    # "only {5, 7} may carry the repetition penalty"
    assert nz(st.window_counts) == {5: 1.0, 7: 1.0}
    assert st.window.tolist() == [5, 7] and st.ring_pos == 0


def test_commit_matches_rebuild():
    # CBv2SamplingTests.swift:240-266: window 3, prompt [1, 2, 3, 4], tokens 8, 9, 8
    inc = O.DenseRowState(V, [1, 2, 3, 4], [], 3, BOTH)
    for t in [8, 9, 8]:
        inc.commit(t)
    rebuilt = O.DenseRowState(V, [1, 2, 3, 4], [8, 9, 8], 3, BOTH)
    assert nz(inc.counts) == nz(rebuilt.counts) == {8: 2.0, 9: 1.0}
    assert nz(inc.window_counts) == nz(rebuilt.window_counts) == {8: 2.0, 9: 1.0}


@pytest.mark.parametrize("W", [1, 2, 5, 40])
@pytest.mark.parametrize("mode", [_ffi.STATE_COUNTS, _ffi.STATE_REPETITION, BOTH])
def test_random_commits_match_rebuild_and_host_entries(W, mode):
    rng = np.random.default_rng(W * 10 + mode)
    prompt = rng.integers(0, V, rng.integers(0, 30)).tolist()
    output = rng.integers(0, V, rng.integers(0, 10)).tolist()
    inc = O.DenseRowState(V, prompt, output, W, mode)
    host = Cbv2RowState(prompt, output, W, repetition_on=bool(mode & 2), counts_on=bool(mode & 1),
                        vocab=V)
    out = list(output)
    for step in range(60):
        t = int(rng.integers(0, V))
        inc.commit(t)
        host.commit(t)
        out.append(t)
        ref = O.DenseRowState(V, prompt, out, W, mode)
        if mode & _ffi.STATE_COUNTS:
            assert nz(inc.counts) == nz(ref.counts)
        if mode & _ffi.STATE_REPETITION:
            assert nz(inc.window_counts) == nz(ref.window_counts)
            # the same tokens, rotated by the write position
            rot = np.concatenate([inc.window[inc.ring_pos:], inc.window[:inc.ring_pos]])
            hist = (prompt + out)[-W:]
            assert rot[-len(hist):].tolist() == hist
        e = host.entries()
        exp = {}
        for tok in set(nz(inc.counts)) | set(nz(inc.window_counts)):
            cnt = int(inc.counts[tok]) if mode & _ffi.STATE_COUNTS else 0
            fl = _ffi.PEN_REPETITION if (mode & 2) and inc.window_counts[tok] > 0 else 0
            if cnt or fl:
                exp[tok] = (cnt, fl)
        assert {int(r["token"]): (int(r["count"]), int(r["flags"])) for r in e} == exp


def test_tokens_outside_the_vocabulary_commit_nothing():
    st = O.DenseRowState(V, [3], [3], 4, BOTH)
    before = (st.counts.copy(), st.window_counts.copy(), st.window.copy(), st.ring_pos)
    st.commit(-1)
    st.commit(V)
    assert np.array_equal(st.counts, before[0]) and np.array_equal(st.window_counts, before[1])
    assert np.array_equal(st.window, before[2]) and st.ring_pos == before[3]
    # the host mirror follows the same rule: its ring does not advance either
    host = Cbv2RowState([3], [3], 4, repetition_on=True, counts_on=True, vocab=V)
    win, pos, ent = list(host.window), host.ring_pos, host.entries().tolist()
    host.commit(-1)
    host.commit(V)
    assert list(host.window) == win and host.ring_pos == pos and host.entries().tolist() == ent
    for t in (5, -1, 6):
        host.commit(t)
        st.commit(t)
    rot = np.concatenate([st.window[st.ring_pos:], st.window[:st.ring_pos]])
    assert host.ring_pos == st.ring_pos and list(host.window) == st.window.tolist(), rot


# ------------------------------------------------- penalty-aware verify windows
@pytest.mark.parametrize("offset", [0, 2])
def test_verify_window_counts_follow_the_drafts_before_each_position(offset):
    """CBv2MTPPenaltyLongRunTests.swift:185-196: at window position j the
    applied counts are a recount of the confirmed output plus a recount of the
    draft chain's first column_offset + j tokens.  The oracle's penalty-aware
    verify must equal an unpenalized verify of logits penalized with exactly
    those counts (recounted here with Counter)."""
    from collections import Counter
    from lsamp import workloads as W
    rng = np.random.default_rng(40 + offset)
    S, Wn, V = 3, 4, 40
    x = rng.normal(0, 2, (S, Wn, V)).astype(np.float32)
    outs = [rng.integers(0, 12, rng.integers(0, 20)).tolist() for _ in range(S)]
    chain = rng.integers(0, 12, (S, offset + Wn - 1)).astype(np.int32)
    drafts = chain[:, offset:offset + Wn - 1]
    u = rng.random((S, Wn), dtype=np.float32)
    p = W.resolve_cbv2(temperature=0.9, top_k=20, presence_penalty=0.7, frequency_penalty=0.4,
                       vocab=V)
    params = W._params([p] * S)
    got = O.verify(mode=_ffi.VERIFY_EXACT, target=x, draft=None, draft_tokens=drafts,
                   dtype=_ffi.DTYPE_F32, params=params, uniforms=u, output_tokens=outs,
                   pen_drafts=chain, column_offset=offset)
    xp = x.copy()
    f, pr = np.float32(0.4), np.float32(0.7)
    for s in range(S):
        for j in range(Wn):
            c = Counter(outs[s]) + Counter(chain[s, :offset + j].tolist())
            cnt = np.zeros(V, np.float32)
            for t, n in c.items():
                cnt[t] = n
            xp[s, j] = (xp[s, j] - f * cnt) - pr * (cnt > 0).astype(np.float32)
    ref = O.verify(mode=_ffi.VERIFY_EXACT, target=xp, draft=None, draft_tokens=drafts,
                   dtype=_ffi.DTYPE_F32, params=params, uniforms=u)
    assert np.array_equal(got["tokens"], ref["tokens"])
    assert np.array_equal(got["accepted"], ref["accepted"])
