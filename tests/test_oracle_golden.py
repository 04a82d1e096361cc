"""CPU tests that pin the oracle (oracle/liblsamp_oracle.so) to the
reference's own known answers, and to properties the mathematics fixes.

The reference (Swift + MLX) cannot run here, so each check below restates one
of its tests with the same inputs and expected values (file:line cited), or a
closed form / brute-force enumeration where no reference vector exists.  The
GPU tests compare the HIP kernels with this oracle, so these tests are what
ties the kernels to the reference.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, TokenRing, csr, mlxlm_entries

F32 = _ffi.DTYPE_F32


# ----------------------------------------------------------------- helpers
def run(semantics, logits, params, entries=None, uniforms=None, dtype=F32, bitmask=None,
        mask_bits=0, mask_tail=0, suppress_ids=None):
    logits = np.atleast_2d(np.asarray(logits))
    if dtype == F32:
        logits = logits.astype(np.float32)
    rows = logits.shape[0]
    if not isinstance(params, (list, tuple)):
        params = [params] * rows
    kw = {}
    if entries is not None:
        kw["row_ptr"], kw["entries"] = csr(entries)
    if uniforms is None:
        uniforms = np.full(rows, 0.5, np.float32)
    return O.sample(semantics=semantics, logits=logits, dtype=dtype, params=W._params(params),
                    uniforms=np.asarray(uniforms, np.float32), want_processed=True,
                    want_keep=True, want_stats=True, bitmask=bitmask, mask_bits=mask_bits,
                    mask_tail=mask_tail, suppress_ids=suppress_ids, **kw)


def mlx_processed(logits, rep=None, rep_ctx=20, pres=None, pres_ctx=20, freq=None,
                  freq_ctx=20, prompt=(), sampled=()):
    """Penalized logits of the mlx-lm PenaltyProcessor (T=1, no filters)."""
    rings = {}
    for name, on, ctx in (("r", rep, rep_ctx), ("p", pres, pres_ctx), ("f", freq, freq_ctx)):
        if on is None:
            rings[name] = None
            continue
        ring = TokenRing(ctx)
        if len(prompt):
            ring.load_prompt(prompt)
        for t in sampled:
            ring.append(t)
        rings[name] = ring
    ents = mlxlm_entries(rings["r"], rings["p"], rings["f"])
    p = W.resolve_mlxlm(temperature=1.0, repetition_penalty=rep, repetition_context_size=rep_ctx,
                        presence_penalty=pres, presence_context_size=pres_ctx,
                        frequency_penalty=freq, frequency_context_size=freq_ctx)
    return run(_ffi.SEM_MLXLM, logits, p, entries=[ents])["processed"][0]


def fixture16():
    """SamplerPenaltyTests.swift:25-31: 0.35 * ((5j + 3) mod 16)."""
    return np.array([np.float32(0.35) * np.float32((j * 5 + 3) % 16) for j in range(16)],
                    np.float32)


def keep_set(out, r=0):
    return set(np.nonzero(out["keep"][r])[0].tolist())


GRID = (np.arange(4096, dtype=np.float64) + 0.5) / 4096.0


def draw_frequencies(semantics, logits, params, n=4096):
    """Token frequencies of the draw over an even grid of uniforms."""
    logits = np.asarray(logits, np.float32)
    u = ((np.arange(n) + 0.5) / n).astype(np.float32)
    out = run(semantics, np.tile(logits, (n, 1)), [params] * n, uniforms=u)
    return np.bincount(out["tokens"], minlength=logits.shape[-1]) / n, out


# ------------------------------------------------- mlx-lm penalties (exact)
def test_presence_penalty_seen_tokens():
    # SampleTests.swift:119-131
    v = mlx_processed([1, 2, 3, 4], pres=0.5, prompt=[1, 1, 3])
    np.testing.assert_allclose(v, [1, 1.5, 3, 3.5], atol=1e-6)


def test_frequency_penalty_counts():
    # SampleTests.swift:133-145
    v = mlx_processed([1, 2, 3, 4], freq=0.5, prompt=[1, 1, 3])
    np.testing.assert_allclose(v, [1, 1, 3, 3.5], atol=1e-6)


def test_presence_penalty_unique_ids():
    # SampleTests.swift:158-170
    v = mlx_processed([0, 0, 0, 0], pres=0.5, pres_ctx=5, prompt=[0, 0, 0, 1, 1])
    np.testing.assert_allclose(v, [-0.5, -0.5, 0, 0], atol=1e-6)


def test_presence_penalty_on_a_view():
    # SampleTests.swift:172-193 (the second row of a [1, 2, 4] source)
    v = mlx_processed([10, 11, 12, 13], pres=0.5, prompt=[1, 3])
    np.testing.assert_allclose(v, [10, 10.5, 12, 12.5], atol=1e-6)


def test_frequency_penalty_by_token_count():
    # SampleTests.swift:195-207
    v = mlx_processed([0, 0, 0, 0], freq=0.5, freq_ctx=5, prompt=[0, 0, 0, 1, 1])
    np.testing.assert_allclose(v, [-1.5, -1, 0, 0], atol=1e-6)


def test_penalty_processor_composes_in_order():
    # SampleTests.swift:209-230: repetition -> presence -> frequency
    v = mlx_processed([1.0, 0.5, 0.0, -0.5], rep=1.5, rep_ctx=5, pres=0.5, pres_ctx=5,
                      freq=0.25, freq_ctx=5, prompt=[0, 0, 0, 1, 1])
    np.testing.assert_allclose(v, [-0.5833, -0.6667, 0.0, -0.5], atol=1e-4)


def test_repetition_penalty_seen_tokens():
    # SampleTests.swift:234-246
    v = mlx_processed([1, 2, 3, 4], rep=2.0, prompt=[1, 1, 3])
    np.testing.assert_allclose(v, [1, 1, 3, 2], atol=1e-6)


@pytest.mark.parametrize("kind,expected_after", [("rep", 1.5), ("pres", 2.5), ("freq", 2.5)])
def test_two_d_prompt_then_append(kind, expected_after):
    # SampleTests.swift:250-308: a [1, S] prompt is flattened; appending token 2
    kw = {"rep": dict(rep=2.0), "pres": dict(pres=0.5), "freq": dict(freq=0.5)}[kind]
    prompt = np.array([[1, 1, 3]])
    before = mlx_processed([1, 2, 3, 4], prompt=prompt, **kw)
    after = mlx_processed([1, 2, 3, 4], prompt=prompt, sampled=[2], **kw)
    np.testing.assert_allclose(before[[0, 2]], [1, 3], atol=1e-6)
    assert after[2] == pytest.approx(expected_after, abs=1e-6)


def test_sampled_tokens_without_prompt():
    # SamplerPenaltyTests.swift:212-229 on logits [3, -1, 2, 5]
    x = [3, -1, 2, 5]
    assert mlx_processed(x, rep=2, rep_ctx=4, sampled=[1, 2]).tolist() == [3, -2, 1, 5]
    assert mlx_processed(x, pres=0.5, pres_ctx=4, sampled=[1, 1]).tolist() == [3, -1.5, 2, 5]
    assert mlx_processed(x, freq=0.5, freq_ctx=4, sampled=[1, 1]).tolist() == [3, -2, 2, 5]


def test_contexts_without_tokens_are_identity():
    # SamplerPenaltyTests.swift:200-210
    x = [3, -1, 2, 5]
    for kw in (dict(rep=2, rep_ctx=4), dict(pres=0.5, pres_ctx=4), dict(freq=0.5, freq_ctx=4)):
        assert mlx_processed(x, **kw).tolist() == x


def test_old_tokens_leave_the_window():
    # SamplerPenaltyTests.swift:231-240
    v = mlx_processed([4, 4, 4, 4], rep=2, rep_ctx=2, prompt=[0, 1], sampled=[2])
    assert v.tolist() == [4, 2, 2, 4]


def test_penalty_processor_forwards_sampled_tokens():
    # SamplerPenaltyTests.swift:242-258: 3/2-0.5-0.25 = 0.75, 5/2-0.5-0.25 = 1.75
    v = mlx_processed([3, -1, 2, 5], rep=2, rep_ctx=4, pres=0.5, pres_ctx=4, freq=0.25,
                      freq_ctx=4, prompt=[3], sampled=[0])
    assert v.tolist() == [0.75, -1, 2, 1.75]


# ------------------------------------------------------------- token ring
def test_token_ring_loads_appends_and_wraps():
    # SamplerPenaltyTests.swift:171-190
    ring = TokenRing(4)
    assert ring.valid_tokens is None and ring.count == 0 and ring.capacity == 4
    ring.load_prompt([7, 8])
    assert ring.valid_tokens == [7, 8] and ring.buffer == [7, 8, 0, 0]
    ring.append(9)
    ring.append(10)
    assert ring.count == 4 and ring.valid_tokens == [7, 8, 9, 10]
    ring.append(11)
    assert ring.count == 4 and ring.buffer == [11, 8, 9, 10]


def test_token_ring_prompt_of_exact_capacity():
    # SamplerPenaltyTests.swift:192-199
    ring = TokenRing(3)
    ring.load_prompt([1, 2, 3])
    assert ring.count == 3 and ring.buffer == [1, 2, 3]
    ring.append(4)
    assert ring.buffer == [4, 2, 3]


def test_token_ring_long_prompt_keeps_the_tail():
    ring = TokenRing(20)
    ring.load_prompt(np.arange(512))
    assert ring.valid_tokens == list(range(492, 512))


# ----------------------------------------------- mlx-lm filters (fixture16)
MLX_FILTERS = [
    # (top_p, min_p, top_k, allowed) from SamplerPenaltyTests.swift:123-150
    (0.9, 0.0, 6, {2, 5, 8, 11, 12, 15}),
    (0.9, 0.2, 6, {2, 5, 8, 12, 15}),
    (1.0, 0.05, 3, {2, 12, 15}),
    (0.9, 0.05, 0, {2, 5, 8, 11, 12, 14, 15}),
    # the single filters of the same comment
    (0.9, 0.0, 0, {2, 5, 8, 11, 12, 14, 15}),
    (1.0, 0.2, 0, {2, 5, 8, 12, 15}),
    (1.0, 0.05, 0, {1, 2, 4, 5, 8, 11, 12, 14, 15}),
    (1.0, 0.0, 6, {2, 5, 8, 11, 12, 15}),
    (1.0, 0.0, 3, {2, 12, 15}),
]


@pytest.mark.parametrize("top_p,min_p,top_k,allowed", MLX_FILTERS)
def test_mlxlm_fixture16_keep_sets(top_p, min_p, top_k, allowed):
    p = W.resolve_mlxlm(temperature=1.0, top_p=top_p, top_k=top_k, min_p=min_p)
    out = run(_ffi.SEM_MLXLM, fixture16(), p)
    assert keep_set(out) == allowed


def test_mlxlm_bfloat16_path():
    # SamplerPenaltyTests.swift:112-122
    x = W.f32_to_bf16_bits(fixture16()[None, :])
    top1 = run(_ffi.SEM_MLXLM, x, W.resolve_mlxlm(temperature=1, top_k=1), dtype=_ffi.DTYPE_BF16,
               uniforms=[0.37])
    assert top1["tokens"][0] == 12
    nucleus = run(_ffi.SEM_MLXLM, np.tile(x, (40, 1)), W.resolve_mlxlm(temperature=1, top_p=0.9),
                  dtype=_ffi.DTYPE_BF16, uniforms=np.linspace(0.01, 0.99, 40))
    assert set(nucleus["tokens"].tolist()) <= {2, 5, 8, 11, 12, 14, 15}


def test_mlxlm_low_temperature_gives_the_argmax():
    # SamplerPenaltyTests.swift:86-98
    u = np.linspace(0.0, 0.999, 20)
    for p in (W.resolve_mlxlm(temperature=0.01), W.resolve_mlxlm(temperature=0.01, top_k=6)):
        out = run(_ffi.SEM_MLXLM, np.tile(fixture16(), (20, 1)), p, uniforms=u)
        assert (out["tokens"] == 12).all()


def test_mlxlm_top_k_at_or_above_vocab_keeps_everything():
    # SamplerPenaltyTests.swift:100-110: same draws as without the filter
    u = np.linspace(0.0, 0.999, 40)
    ref = run(_ffi.SEM_MLXLM, np.tile(fixture16(), (40, 1)), W.resolve_mlxlm(temperature=1),
              uniforms=u)
    for k in (16, 100):
        out = run(_ffi.SEM_MLXLM, np.tile(fixture16(), (40, 1)),
                  W.resolve_mlxlm(temperature=1, top_k=k), uniforms=u)
        assert (out["keep"] == 1).all()
        assert np.array_equal(out["tokens"], ref["tokens"])
    assert len(set(ref["tokens"].tolist())) > 3


# ----------------------------- mlx-lm filtered distributions (SampleTests)
def log_probs(p):
    with np.errstate(divide="ignore"):
        return np.log(np.asarray(p, np.float32))


@pytest.mark.parametrize("probs,kw,expected", [
    # SampleTests.swift:44-52, 54-65, 67-79, 81-92, 103-111
    ([0.9, 0.0, 0.0, 0.1], dict(top_p=0.3), [1.0, 0, 0, 0]),
    ([0.0, 0.5, 0.4, 0.1], dict(top_p=0.6), [0, 0.5556, 0.4444, 0]),
    ([0.0, 0.5, 0.4, 0.1], dict(top_p=0.95), [0, 0.5, 0.4, 0.1]),
    ([0.6, 0.0, 0.1, 0.3], dict(top_k=2), [0.6667, 0, 0, 0.3333]),
    ([0.9, 0.0, 0.0, 0.1], dict(min_p=0.05), [0.9, 0, 0, 0.1]),
])
def test_mlxlm_filtered_distributions(probs, kw, expected):
    # The reference estimates these from 4000 seeded draws (+-0.06); with
    # an even grid of uniforms the inverse-CDF draw gives them exactly.
    freq, _ = draw_frequencies(_ffi.SEM_MLXLM, log_probs(probs),
                               W.resolve_mlxlm(temperature=1.0, **kw))
    np.testing.assert_allclose(freq, expected, atol=2e-4 + 1.0 / 4096)


def test_mlxlm_min_p_keeps_only_the_high_token():
    # SampleTests.swift:94-101
    out = run(_ffi.SEM_MLXLM, np.tile([0.0, 0.0, 4.0], (10, 1)),
              W.resolve_mlxlm(temperature=1.0, min_p=0.95), uniforms=np.linspace(0, 0.99, 10))
    assert (out["tokens"] == 2).all()


# ---------------------------------------------- parameter resolution rules
def test_generate_parameters_choose_the_sampler():
    # SamplerPenaltyTests.swift:45-51, SampleTests.swift:113-117
    A, F, C = _ffi.KIND_ARGMAX, _ffi.KIND_FILTERED, _ffi.KIND_CATEGORICAL
    assert W.resolve_mlxlm(temperature=0.7)["kind"] == C
    assert W.resolve_mlxlm(temperature=0.7, top_p=1)["kind"] == C
    assert W.resolve_mlxlm(temperature=0.7, top_p=0)["kind"] == C
    assert W.resolve_mlxlm(temperature=0.7, top_p=0.9)["kind"] == F
    assert W.resolve_mlxlm(temperature=0, top_k=5)["kind"] == A
    assert W.resolve_mlxlm(temperature=0.7, top_k=40)["kind"] == F
    assert W.resolve_mlxlm(temperature=0.7, min_p=0.1)["kind"] == F
    assert W.resolve_mlxlm(temperature=0)["kind"] == A


# ------------------------------------------- CBv2 (LogitsPipelineV2) oracles
class SplitMixLogits:
    """CBv2SamplingTests.swift:44-78: SplitMix64 stream, logits on a 0.25
    grid in [-16, 16], distinct within a row."""
    M = (1 << 64) - 1

    def __init__(self, seed):
        self.state = seed & self.M

    def next(self):
        self.state = (self.state + 0x9E3779B97F4A7C15) & self.M
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & self.M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & self.M
        return z ^ (z >> 31)

    def logit(self, scale=4.0):
        u = np.float32(self.next() >> 40) / np.float32(1 << 24)
        v = (u * np.float32(2) - np.float32(1)) * np.float32(scale) * np.float32(4)
        r = np.float32(math.floor(abs(float(v)) + 0.5)) * np.float32(np.sign(v))
        return np.float32(r / np.float32(4))

    def logits(self, count):
        seen, out = set(), []
        while len(out) < count:
            v = self.logit()
            if float(v) not in seen:
                seen.add(float(v))
                out.append(v)
        return np.array(out, np.float32)

    def token(self, vocab):
        return int(self.next() % vocab)


def reference_transform(logits, spec):
    """CBv2SamplingTests.swift:82-115 (the reference test's own scalar
    oracle), evaluated in float32 like the Swift code."""
    f = np.float32
    x = np.array(logits, np.float32)
    for t, b in spec.get("bias", {}).items():
        if 0 <= t < len(x):
            x[t] = f(x[t] + f(b))
    rp, W_ = f(spec.get("rep", 1.0)), spec.get("rep_ctx", 64)
    if rp != f(1) and W_ > 0:
        hist = list(spec.get("prompt", [])) + list(spec.get("output", []))
        for t in set(hist[-W_:]):
            if 0 <= t < len(x):
                x[t] = f(x[t] / rp) if x[t] > 0 else f(x[t] * rp)
    fq, pr = f(spec.get("freq", 0.0)), f(spec.get("pres", 0.0))
    if fq != 0 or pr != 0:
        counts = np.zeros(len(x), np.float32)
        for t in spec.get("output", []):
            if 0 <= t < len(x):
                counts[t] += 1
        for i in range(len(x)):
            x[i] = f(x[i] - f(fq * counts[i]))
            x[i] = f(x[i] - f(pr * f(1 if counts[i] > 0 else 0)))
    T = f(spec.get("T", 0.0))
    if T >= f(1e-5) and T != f(1):
        x = (x / T).astype(np.float32)
    return x


def cbv2_run(specs, raw, vocab, uniforms=None):
    params, ents = [], []
    for s in specs:
        params.append(W.resolve_cbv2(temperature=s.get("T", 0.0), top_p=s.get("top_p", 1.0),
                                     top_k=s.get("top_k", 0), min_p=s.get("min_p", 0.0),
                                     repetition_penalty=s.get("rep", 1.0),
                                     repetition_context_size=s.get("rep_ctx", 64),
                                     frequency_penalty=s.get("freq", 0.0),
                                     presence_penalty=s.get("pres", 0.0), vocab=vocab))
        rep_on = s.get("rep", 1.0) != 1.0 and s.get("rep_ctx", 64) > 0
        counts_on = s.get("freq", 0.0) != 0.0 or s.get("pres", 0.0) != 0.0
        st = Cbv2RowState(prompt=s.get("prompt", []), output=s.get("output", []),
                          repetition_window=s.get("rep_ctx", 64), repetition_on=rep_on,
                          counts_on=counts_on, bias=s.get("bias"), vocab=vocab)
        for t in s.get("commit", []):
            st.commit(t)
        ents.append(st.entries())
    return run(_ffi.SEM_CBV2, np.stack(raw), params, entries=ents, uniforms=uniforms)


def test_cbv2_penalties_match_the_scalar_reference():
    # CBv2SamplingTests.swift:170-192 (testPenaltiesParityVsScalarReferenceOnRandomHistories)
    vocab = 16
    rng = SplitMixLogits(11)
    specs = []
    for i in range(4):
        prompt = [rng.token(vocab) for _ in range(10)]
        output = [rng.token(vocab) for _ in range(6)]
        specs.append(dict(T=[0, 0.7, 1.0, 1.3][i], rep=[1.5, 1.0, 2.0, 1.2][i],
                          rep_ctx=[4, 64, 3, 8][i], freq=[0.3, 0, 0.7, 0][i],
                          pres=[0.4, 0, 0, 1.1][i], bias={2: 5.5, 9: -3} if i == 1 else {},
                          prompt=prompt, output=output))
    raw = [rng.logits(vocab) for _ in specs]
    got = cbv2_run(specs, raw, vocab)["processed"]
    for r, s in enumerate(specs):
        np.testing.assert_allclose(got[r], reference_transform(raw[r], s), atol=1e-4,
                                   err_msg=f"row {r}")


def test_cbv2_incremental_commit_matches_rebuild_with_eviction():
    # CBv2SamplingTests.swift:195-229: window 2, tokens 5, 6, 5, 7 committed
    vocab = 16
    base = dict(T=1.0, rep=2.0, rep_ctx=2, freq=0.25, pres=0.5, prompt=[0, 1])
    raw = SplitMixLogits(13).logits(vocab)
    inc = cbv2_run([dict(base, commit=[5, 6, 5, 7])], [raw], vocab)["processed"][0]
    expected = reference_transform(raw, dict(base, output=[5, 6, 5, 7]))
    np.testing.assert_allclose(inc, expected, atol=1e-4)
    # only {5, 7} may carry the repetition penalty
    clean = reference_transform(raw, dict(base, rep=1.0, output=[5, 6, 5, 7]))
    np.testing.assert_allclose(inc[[0, 1, 6]], clean[[0, 1, 6]], atol=1e-4)


def test_cbv2_mid_flight_rebuild_matches_incremental_state():
    # CBv2SamplingTests.swift:231-257
    vocab = 16
    base = dict(T=1.0, rep=1.7, rep_ctx=3, freq=0.6, pres=0.2, prompt=[1, 2, 3, 4])
    raw = SplitMixLogits(17).logits(vocab)
    a = cbv2_run([dict(base, commit=[8, 9, 8])], [raw], vocab)["processed"][0]
    b = cbv2_run([dict(base, output=[8, 9, 8])], [raw], vocab)["processed"][0]
    np.testing.assert_allclose(a, b, atol=1e-5)


def test_cbv2_keep_sets_match_the_scalar_rule():
    # CBv2SamplingTests.swift:259-312: the test's own keep-set rule
    vocab = 16
    specs = [dict(T=1, top_k=3), dict(T=1, top_p=0.7), dict(T=1, min_p=0.25), dict(T=1)]
    rng = SplitMixLogits(19)
    raw = [rng.logits(vocab) for _ in specs]
    out = cbv2_run(specs, raw, vocab)
    for r, s in enumerate(specs):
        x = raw[r]
        order = sorted(range(vocab), key=lambda i: -float(x[i]))
        mx = np.float32(x.max())
        es = np.float32(0)
        for v in x:
            es = np.float32(es + np.float32(np.exp(np.float32(v - mx))))
        probs = [np.float32(np.float32(np.exp(np.float32(x[i] - mx))) / es) for i in order]
        keep, cum = set(), np.float32(0)
        for rank, tok in enumerate(order):
            p = probs[rank]
            kept = True
            if s.get("top_k", 0) > 0 and rank >= s["top_k"]:
                kept = False
            if s.get("top_p", 1.0) < 1 and cum > np.float32(s["top_p"]):
                kept = False
            if s.get("min_p", 0.0) > 0 and p < np.float32(s["min_p"]) * probs[0]:
                kept = False
            cum = np.float32(cum + p)
            if kept:
                keep.add(tok)
        assert order[0] in keep
        assert keep_set(out, r) == keep, f"row {r}"
        # kept tokens keep their value, the rest are excluded
        assert np.allclose(out["processed"][r][sorted(keep)], x[sorted(keep)], atol=1e-4)


def test_cbv2_greedy_rows_pass_through_and_draw_the_argmax():
    # CBv2SamplingTests.swift:314-328 and :392-402
    vocab = 16
    rng = SplitMixLogits(23)
    raw = [rng.logits(vocab) for _ in range(3)]
    out = cbv2_run([dict(), dict(), dict()], raw, vocab)
    assert np.array_equal(out["processed"].view(np.uint32), np.stack(raw).view(np.uint32))
    assert out["tokens"].tolist() == [int(np.argmax(x)) for x in raw]


def test_cbv2_top_k_one_is_the_argmax_at_high_temperature():
    # CBv2SamplingTests.swift:460-469
    vocab = 16
    for step in range(8):
        x = SplitMixLogits(1000 + step).logits(vocab)
        out = cbv2_run([dict(T=2.0, top_k=1)], [x], vocab, uniforms=[0.999])
        assert out["tokens"][0] == int(np.argmax(x))


def test_cbv2_mixed_batch_greedy_row_unaffected():
    # CBv2SamplingTests.swift:444-458
    vocab = 16
    rng = SplitMixLogits(37)
    raw = [rng.logits(vocab), rng.logits(vocab)]
    out = cbv2_run([dict(), dict(T=1.2)], raw, vocab, uniforms=[0.3, 0.6])
    assert out["tokens"][0] == int(np.argmax(raw[0]))
    assert 0 <= out["tokens"][1] < vocab


def test_cbv2_mask_precedes_top_k_and_survives_negative_penalty():
    # CBv2TokenConstraintSamplingTests.swift:313-345: only token 1 allowed
    bm = np.array([[1 << 1]], np.uint32)
    p = W.resolve_cbv2(temperature=1, top_k=1, vocab=4)
    out = run(_ffi.SEM_CBV2, [0, 1, 2, 100], p, bitmask=bm, mask_bits=4)
    assert out["tokens"][0] == 1
    # a negative repetition penalty on the masked maximum (token 3 in the window)
    st = Cbv2RowState(prompt=[3], output=[], repetition_window=64, repetition_on=True,
                      counts_on=False, vocab=4)
    p = W.resolve_cbv2(temperature=1, top_k=1, repetition_penalty=-1, vocab=4)
    out = run(_ffi.SEM_CBV2, [0, 1, 2, 100], p, entries=[st.entries()], bitmask=bm, mask_bits=4)
    assert out["tokens"][0] == 1
    assert out["processed"][0][3] == -np.inf


# ----------------------------------------------- suppressed ids, chain order
SUPPRESS_LOGITS = [0.5, 5.0, 1.0, 9.0, 2.0]


@pytest.mark.parametrize("semantics", [_ffi.SEM_MLXLM, _ffi.SEM_CBV2])
def test_suppress_masks_only_the_given_ids(semantics):
    # SuppressTokensTests.swift testSuppressTokensProcessorMasksOnlyGivenIds
    p = (W.resolve_mlxlm(temperature=1.0) if semantics == _ffi.SEM_MLXLM
         else W.resolve_cbv2(temperature=1.0, vocab=5))
    v = run(semantics, SUPPRESS_LOGITS, p, suppress_ids=[1, 3])["processed"][0]
    assert v.tolist() == [0.5, -np.inf, 1.0, -np.inf, 2.0]


def test_suppressed_token_is_never_the_argmax():
    # testSuppressedTokenIsNeverArgMax: 9.0 at id 3 suppressed -> id 1
    out = run(_ffi.SEM_MLXLM, SUPPRESS_LOGITS, W.resolve_mlxlm(temperature=0.0), suppress_ids=[3])
    assert out["tokens"][0] == 1


def test_suppress_ignores_out_of_range_and_negative_ids():
    # testSuppressTokensProcessorIgnoresOutOfRangeIds / AllOutOfRangeIsNoOp /
    # IgnoresNegativeIds
    p = W.resolve_mlxlm(temperature=1.0)
    v = run(_ffi.SEM_MLXLM, SUPPRESS_LOGITS, p, suppress_ids=[1, 258882, 258883])["processed"][0]
    assert v[1] == -np.inf and v[3] == 9.0
    v = run(_ffi.SEM_MLXLM, [0.5, 5.0, 1.0], p, suppress_ids=[258882, 258883])["processed"][0]
    assert v.tolist() == [0.5, 5.0, 1.0]
    v = run(_ffi.SEM_MLXLM, [0.5, 5.0, 1.0], p, suppress_ids=[-1, -106])["processed"][0]
    assert v.tolist() == [0.5, 5.0, 1.0]


def test_chained_suppressors_apply_both():
    # testChainedLogitProcessorAppliesAllProcessors: [1] then [3]
    v = run(_ffi.SEM_MLXLM, SUPPRESS_LOGITS, W.resolve_mlxlm(temperature=1.0),
            suppress_ids=[1, 3])["processed"][0]
    assert v[1] == -np.inf and v[3] == -np.inf and v[4] == 2.0


def test_mlxlm_custom_processor_runs_after_the_penalties():
    """SampleTests.swift:431-454 pins the chain order penalty -> custom
    (GenerationComponents.swift:112-124), there with a scaling processor.
    Here the custom processor is the grammar mask and suppression runs last
    (:126-141).  A negative repetition penalty on a masked / suppressed token
    tells the orders apart: applied after the penalty the token stays -inf;
    masked first, -inf * (-1.5) would come back as +inf and be drawn."""
    prompt = [1, 2, 3]
    ring = TokenRing(5)
    ring.load_prompt(prompt)
    pres = TokenRing(5)
    pres.load_prompt([1])
    ents = mlxlm_entries(ring, pres, None)
    p = W.resolve_mlxlm(temperature=0.0, repetition_penalty=-1.5, repetition_context_size=5,
                        presence_penalty=0.5, presence_context_size=5)
    bm = np.array([[0b1011]], np.uint32)  # token 2 forbidden by the mask
    out = run(_ffi.SEM_MLXLM, [1.0, 2.0, 3.0, 4.0], p, entries=[ents], bitmask=bm, mask_bits=4,
              suppress_ids=[3])
    v = out["processed"][0]
    # token 1: repetition x / -1.5 then presence -0.5 -> -1.8333; 2 masked; 3 suppressed
    np.testing.assert_allclose(v[:2], [1.0, 2.0 / -1.5 - 0.5], rtol=1e-6)
    assert v[2] == -np.inf and v[3] == -np.inf
    assert out["tokens"][0] == 0


# ------------------------------------------------------ grammar bitmask
def test_bitmask_lsb_first_allows_exactly_the_set_bits():
    # MaskRelocationTests.swift:15-33: vocab 8, only id 5 allowed
    bm = np.array([[1 << 5]], np.uint32)
    out = run(_ffi.SEM_CBV2, np.arange(8, dtype=np.float32), W.resolve_cbv2(temperature=0, vocab=8),
              bitmask=bm, mask_bits=8)
    pr = out["processed"][0]
    assert pr[5] == 5.0 and all(pr[i] == -np.inf for i in (0, 1, 2, 3, 4, 6, 7))
    assert out["tokens"][0] == 5


def test_bitmask_masked_maximum_is_never_drawn():
    # MaskRelocationTests.swift:35-57: 65 is the largest logit, only 123 allowed
    x = np.zeros(256, np.float32)
    x[123], x[65] = 10.0, 20.0
    words = np.zeros((1, 8), np.uint32)
    words[0, 123 // 32] |= np.uint32(1 << (123 % 32))
    out = run(_ffi.SEM_CBV2, x, W.resolve_cbv2(temperature=0, vocab=256), bitmask=words,
              mask_bits=256)
    assert out["tokens"][0] == 123


def test_bitmask_word_count_and_tail_policies():
    # MatcherTests.swift:25-140 word count (V+31)/32, LSB-first; ids past the
    # mask's bits follow the caller's tail policy
    V = 70
    words = np.zeros((1, (V + 31) // 32), np.uint32)
    for t in (0, 31, 32, 63):
        words[0, t // 32] |= np.uint32(1 << (t % 32))
    x = np.linspace(-1, 1, V).astype(np.float32)
    p = W.resolve_cbv2(temperature=1, vocab=V)
    keep = run(_ffi.SEM_CBV2, x, p, bitmask=words, mask_bits=64,
               mask_tail=_ffi.MASK_TAIL_KEEP)
    forbid = run(_ffi.SEM_CBV2, x, p, bitmask=words, mask_bits=64,
                 mask_tail=_ffi.MASK_TAIL_FORBID)
    allowed_keep = {0, 31, 32, 63} | set(range(64, V))
    assert set(np.nonzero(keep["processed"][0] > -np.inf)[0].tolist()) == allowed_keep
    assert set(np.nonzero(forbid["processed"][0] > -np.inf)[0].tolist()) == {0, 31, 32, 63}


def test_all_masked_row_fails_closed():
    bm = np.zeros((1, 1), np.uint32)
    out = run(_ffi.SEM_CBV2, [1, 2, 3], W.resolve_cbv2(temperature=1, vocab=3), bitmask=bm,
              mask_bits=3)
    assert out["tokens"][0] == -1 and out["row_flags"][0] & _ffi.ROW_EMPTY


# ------------------------------------------- argmax ordering (top-two rows)
TOP_TWO_ROWS = np.array([[7, 7, 7, -1, 0, 2], [np.nan, -np.inf, np.inf, np.nan, np.inf, 0],
                         [-0.0, 0.0, -1, -2, -3, -4], [1.0001, 1.0002, 1.0003, 1, 0, -1]],
                        np.float32)


@pytest.mark.parametrize("dtype", [_ffi.DTYPE_F32, _ffi.DTYPE_BF16, _ffi.DTYPE_F16])
def test_argmax_ties_to_lower_id_nan_last(dtype):
    # CBv2TopTwoTests.swift:9-53: value descending, NaN last, ties -> lower id
    # (-0 == +0).  The all-NaN row of that test is covered below.
    if dtype == _ffi.DTYPE_F32:
        x = TOP_TWO_ROWS
    elif dtype == _ffi.DTYPE_BF16:
        x = W.f32_to_bf16_bits(TOP_TWO_ROWS)
    else:
        x = TOP_TWO_ROWS.astype(np.float16).view(np.uint16)
    xf = TOP_TWO_ROWS if dtype != _ffi.DTYPE_BF16 else W.bf16_bits_to_f32(x)
    if dtype == _ffi.DTYPE_F16:
        xf = TOP_TWO_ROWS.astype(np.float16).astype(np.float32)
    out = run(_ffi.SEM_CBV2, x, W.resolve_cbv2(temperature=0, vocab=6), dtype=dtype)
    for r in range(len(xf)):
        order = sorted(range(6), key=lambda i: (np.isnan(xf[r, i]),
                                                -xf[r, i] if not np.isnan(xf[r, i]) else 0, i))
        assert out["tokens"][r] == order[0], f"row {r}"


def test_all_nan_row_is_flagged_and_empty():
    # Deliberate fail-closed rule of this build: NaN defines no token, so an
    # all-NaN row draws nothing and carries both the non-finite and the empty
    # flags (CBv2NonFiniteLogits.swift:30-34 flags such rows).
    out = run(_ffi.SEM_CBV2, np.full(6, np.nan, np.float32), W.resolve_cbv2(temperature=0, vocab=6))
    assert out["tokens"][0] == -1
    assert out["row_flags"][0] & _ffi.ROW_NONFINITE and out["row_flags"][0] & _ffi.ROW_EMPTY


# --------------------------------------------------- MTP typical acceptance
def test_typical_acceptance_pinned_mask():
    # CBv2MTPTypicalAcceptanceTests.swift:35-110: mask [T,F,F,T,T,T]
    target = np.array([[[10, 10, -30, -30], [20, 0, 0, 0], [1, 2, 3, 4]],
                       [[1, 5, 2, 0], [0, 0, 9, 0], [3, 3, 3, 3]],
                       [[2, 2, 2, -30], [3, 0, 0, 0], [0, 1, 0, 0]]], np.float32)
    drafts = np.array([[0, 1], [2, 2], [0, 0]], np.int32)
    params = W._params([W.resolve_cbv2(temperature=1, vocab=4),
                        W.resolve_cbv2(temperature=0, vocab=4),
                        W.resolve_cbv2(temperature=1, vocab=4)])
    out = O.verify(mode=_ffi.VERIFY_TYPICAL, target=target, draft=None, draft_tokens=drafts,
                   dtype=F32, params=params, uniforms=np.full((3, 3), 0.5, np.float32),
                   typical_delta=0.2)
    assert out["accept_mask"].reshape(-1).tolist() == [1, 0, 0, 1, 1, 1]


def test_typical_acceptance_uses_the_filtered_row():
    # CBv2MTPTypicalAcceptanceTests.swift:112-140: top-k 2 at T=0.5 rejects
    # the runner-up draft (p ~ 0.12 < floor ~ 0.14); T=1 without top-k accepts
    target = np.array([[[3, 2, 1, 0], [0, 0, 0, 9]]], np.float32)
    drafts = np.array([[1]], np.int32)
    u = np.full((1, 2), 0.5, np.float32)
    for (T, k), want in (((0.5, 2), 0), ((1.0, 0), 1)):
        params = W._params([W.resolve_cbv2(temperature=T, top_k=k, vocab=4)])
        out = O.verify(mode=_ffi.VERIFY_TYPICAL, target=target, draft=None, draft_tokens=drafts,
                       dtype=F32, params=params, uniforms=u, typical_delta=0.2)
        assert out["accept_mask"][0, 0] == want


def test_penalized_typical_verify_accepts_penalty_rows_exactly():
    # DefaultSamplerV2.swift:496-502: with penalties applied, rows whose
    # params carry a presence or frequency penalty (CBv2MTPVerifyPenalties.
    # applies, EngineLoopV2.swift:241-243) accept a draft only when it is the
    # target draw; the other sampled rows keep the typical rule.  The drafts
    # are the runner-up tokens, so the typical rule accepts where exact
    # acceptance does not.
    rng = np.random.default_rng(21)
    S, Wn, V = 6, 4, 64
    target = rng.normal(0, 0.3, (S, Wn, V)).astype(np.float32)
    target[:, :, :2] += 3.0                    # two near-equal favourites
    u = rng.random((S, Wn), dtype=np.float32)
    pen = dict(temperature=1.0, presence_penalty=0.2, frequency_penalty=0.1)
    plain = dict(temperature=1.0)
    params = W._params([W.resolve_cbv2(vocab=V, **(pen if s % 2 == 0 else plain))
                        for s in range(S)])
    outs = [[] for _ in range(S)]                # no confirmed outputs
    first = O.verify(mode=_ffi.VERIFY_EXACT, target=target, draft=None,
                     draft_tokens=np.zeros((S, Wn - 1), np.int32), dtype=F32, params=params,
                     uniforms=u, output_tokens=outs)
    # the favourite the target draw did not pick, at every position
    drafts = np.where(first["tokens"][:, :-1] == 0, 1, 0).astype(np.int32)
    out = O.verify(mode=_ffi.VERIFY_TYPICAL, target=target, draft=None, draft_tokens=drafts,
                   dtype=F32, params=params, uniforms=u, typical_delta=0.2, output_tokens=outs)
    exact = out["tokens"][:, :-1] == drafts
    typ = out["typical_margin"] > 0
    for s in range(S):
        if s % 2 == 0:
            assert np.array_equal(out["accept_mask"][s].astype(bool), exact[s]), s
        else:
            assert np.array_equal(out["accept_mask"][s].astype(bool), typ[s]), s
    # the rule matters here: on the plain rows the typical test accepts
    # runner-up drafts that exact acceptance rejects (the penalty rows, built
    # alike, would too under the typical rule)
    assert (typ & ~exact)[1::2].any()


@pytest.mark.parametrize("pkw", [dict(temperature=0.8, top_p=0.9), dict(temperature=0.0),
                                 dict(temperature=1.2, top_k=7, min_p=0.05)])
def test_exact_verify_is_the_ordinary_draw_at_every_position(pkw):
    # CBv2MTPTargetSamplingMatrixTests.swift:10-58: the verify window's target
    # token at position j is the token an ordinary step would sample from that
    # position's logits with the same uniform; accept iff it equals the draft
    rng = np.random.default_rng(77)
    S, Wn, V = 5, 4, 97
    target = rng.normal(0, 2, (S, Wn, V)).astype(np.float32)
    u = rng.random((S, Wn), dtype=np.float32)
    params = W._params([W.resolve_cbv2(vocab=V, **pkw)] * S)
    plain = O.sample(semantics=_ffi.SEM_CBV2, logits=target.reshape(S * Wn, V), dtype=F32,
                     params=np.repeat(params, Wn), uniforms=u.reshape(-1))["tokens"].reshape(S, Wn)
    drafts = plain[:, :-1].copy()
    drafts[::2, 1] = (drafts[::2, 1] + 1) % V  # even sequences diverge at position 1
    out = O.verify(mode=_ffi.VERIFY_EXACT, target=target, draft=None, draft_tokens=drafts,
                   dtype=F32, params=params, uniforms=u)
    assert np.array_equal(out["tokens"], plain)
    assert np.array_equal(out["accept_mask"].astype(bool), drafts == plain[:, :-1])
    want = np.argmin(np.concatenate([drafts == plain[:, :-1], np.zeros((S, 1), bool)], 1), 1)
    assert np.array_equal(out["accepted"], want)


# -------------------------------- speculative sampling: distribution invariant
def test_residual_speculative_sampling_preserves_the_target_distribution():
    """Leviathan et al. 2023 / Chen et al. 2023: with drafts x ~ p_d, accept
    x iff u < min(1, p_t(x)/p_d(x)), else draw from norm(max(0, p_t - p_d)),
    the emitted token is distributed as p_t.  Enumerated exactly over every
    draft and a grid of both uniforms, for a tiny vocabulary."""
    V, n = 5, 48
    rng = np.random.default_rng(5)
    t_logits = rng.normal(0, 1.5, V).astype(np.float32)
    d_logits = (t_logits + rng.normal(0, 1.0, V)).astype(np.float32)
    params = W.resolve_cbv2(temperature=1.0, vocab=V)
    # target / draft distributions as the oracle itself weighs them
    pt = draw_frequencies(_ffi.SEM_CBV2, t_logits, params, n=8192)[0]
    pd = draw_frequencies(_ffi.SEM_CBV2, d_logits, params, n=8192)[0]
    grid = ((np.arange(n) + 0.5) / n).astype(np.float32)
    S = V * n * n
    target = np.broadcast_to(np.stack([t_logits, t_logits]), (S, 2, V)).copy()
    draft = np.broadcast_to(d_logits, (S, 1, V)).copy()
    dtoks = np.repeat(np.arange(V, dtype=np.int32), n * n)[:, None]
    u = np.zeros((S, 2), np.float32)
    u[:, 0] = np.tile(np.repeat(grid, n), V)
    u[:, 1] = np.tile(np.tile(grid, n), V)
    out = O.verify(mode=_ffi.VERIFY_RESIDUAL, target=target, draft=draft, draft_tokens=dtoks,
                   dtype=F32, params=W._params([params] * S), uniforms=u, threads=8)
    first = out["tokens"][:, 0]
    weights = np.repeat(pd, n * n) / (n * n)
    emitted = np.bincount(first, weights=weights, minlength=V)
    np.testing.assert_allclose(emitted, pt, atol=4.0 / n)
    # accepted drafts are emitted as themselves, rejections carry a correction
    acc = out["accepted"] == 1
    assert np.array_equal(first[acc], dtoks[acc, 0])
    assert (out["tokens"][acc, 1] >= 0).all() and (out["tokens"][~acc, 1] == -1).all()


# ---------------------------------------------------- the draw (build rule)
def test_draw_is_monotone_and_exact_in_frequency():
    rng = np.random.default_rng(3)
    y = rng.normal(0, 2, 50).astype(np.float32)
    keep = (rng.random(50) < 0.6).astype(np.uint8)
    keep[int(np.argmax(y))] = 1
    n = 1 << 14
    toks = []
    for k in range(n):
        t, wsum = O.draw(y, keep, 1.0, (k + 0.5) / n)
        toks.append(t)
    toks = np.array(toks)
    assert (np.diff(toks) >= 0).all(), "inverse CDF in token-id order"
    assert keep[toks].all(), "only kept tokens are drawn"
    w = np.array([O.weight(v, y.max()) if keep[i] else 0 for i, v in enumerate(y)], np.float64)
    np.testing.assert_allclose(np.bincount(toks, minlength=50) / n, w / w.sum(), atol=2.0 / n)
    assert O.draw(y, keep, 1.0, 0.0)[0] == int(np.nonzero(keep)[0][0])
    assert O.draw(y, keep, 1.0, np.nextafter(np.float32(1), np.float32(0)))[0] == \
        int(np.nonzero(keep)[0][-1])


def test_dexp_accuracy():
    # within a few float ulps of e^d on (-80, 0]; zero at and below -80, where
    # any draw weight 2^40 e^d has long rounded to zero (d < -27.8)
    d = np.concatenate([np.linspace(-79.99, 0, 20001), -np.logspace(-8, 1.9, 2000)])
    d = d.astype(np.float32)
    got = np.array([O.dexp(v) for v in d], np.float64)
    want = np.exp(d.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 4e-7
    assert O.dexp(0.0) == 1.0 and O.dexp(-80.0) == 0.0 and O.dexp(-200.0) == 0.0


# --------------------------------------------------------------- Philox
@pytest.mark.parametrize("ctr,key,expected", [
    # Random123 known-answer vectors for philox4x32-10
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, expected):
    assert O.philox(ctr, key).tolist() == expected


def test_rng_uniform_is_uniform():
    keys = [O.rng_key(7, rid, 0) for rid in range(20000)]
    u = np.array([O.rng_uniform(k) for k in keys])
    assert ((u >= 0) & (u < 1)).all()
    hist = np.histogram(u, bins=20, range=(0, 1))[0]
    chi2 = ((hist - 1000.0) ** 2 / 1000.0).sum()
    assert chi2 < 45.0  # 19 degrees of freedom, p ~ 1e-3


# Published SplitMix64 outputs (the generator of Steele, Lea & Flood, "Fast
# splittable pseudorandom number generators", OOPSLA 2014, as listed for
# seed 1234567 by the Rosetta Code task "Pseudo-random numbers/Splitmix64"):
# the state advances by the golden gamma and each output mixes the new state.
_GAMMA = 0x9E3779B97F4A7C15
_SPLITMIX_1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                     4593380528125082431, 16408922859458223821]


def splitmix_known_answers():
    """(seed, id, step, key) for which each stage of SamplerV2.mix
    (SamplerV2.swift:183-191), splitmix(splitmix(splitmix(seed) ^ id) ^ step),
    lands on a published output.  splitmix(v) mixes v + gamma, so
    splitmix(1234567 + k * gamma) is output k: with seed = 1234567 + j * gamma,
    stage one gives output j, the id turns it into state j + 1 (output j + 1)
    and the step into state j + 2 (output j + 2)."""
    M = (1 << 64) - 1
    s, out = 1234567, _SPLITMIX_1234567
    cases = []
    for j in range(3):
        seed = (s + j * _GAMMA) & M
        rid = out[j] ^ ((s + (j + 1) * _GAMMA) & M)
        step = out[j + 1] ^ ((s + (j + 2) * _GAMMA) & M)
        cases.append((seed, rid, step, out[j + 2]))
    return cases


@pytest.mark.parametrize("seed,rid,step,key", splitmix_known_answers())
def test_rng_key_splitmix64_known_answer(seed, rid, step, key):
    """The key mix against the published SplitMix64 sequence: a wrong shift,
    multiplier, increment or composition order fails here."""
    assert O.rng_key(seed, rid, step) == key


def test_rng_key_depends_on_all_three_inputs():
    # CBv2SamplingTests.swift:471-476 (SamplerV2.mix)
    base = O.rng_key(1, 2, 3)
    assert base != O.rng_key(9, 2, 3) and base != O.rng_key(1, 9, 3) and base != O.rng_key(1, 2, 9)


# ----------------------------------------------------------- invariants
def test_rows_are_independent_of_their_batch():
    cfg = W.config2(rows=6, vocab=4096)
    full = O.sample(semantics=cfg["semantics"], logits=cfg["logits"], dtype=cfg["dtype"],
                    params=cfg["params"], row_ptr=cfg["row_ptr"], entries=cfg["entries"],
                    uniforms=cfg["uniforms"])
    for r in range(6):
        lo, hi = cfg["row_ptr"][r], cfg["row_ptr"][r + 1]
        one = O.sample(semantics=cfg["semantics"], logits=cfg["logits"][r:r + 1], dtype=cfg["dtype"],
                       params=cfg["params"][r:r + 1], row_ptr=np.array([0, hi - lo], np.int32),
                       entries=cfg["entries"][lo:hi], uniforms=cfg["uniforms"][r:r + 1])
        assert one["tokens"][0] == full["tokens"][r]


# ------------------------------------------------------- dtype conversions
def _dense_f32_patterns():
    """Every bfloat16 prefix with the low halves that decide rounding (ties to
    even and odd, one ulp either side, zero, all ones), plus random patterns:
    covers subnormals, both zeros, infinities and NaNs."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1000, 0x0FFF, 0x1001,
                     0x2000, 0x3000, 0x6000], np.uint32)
    grid = (hi[:, None] | lows[None, :]).reshape(-1)
    rnd = np.random.default_rng(77).integers(0, 1 << 32, 1 << 21, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([grid, rnd]).view(np.float32)


def test_f32_to_bf16_matches_torch():
    """The oracle's float32 -> bfloat16 rounding (used for mlx-lm penalties on
    16-bit logits) against torch's converter, bit for bit (NaN: any NaN)."""
    import torch
    x = _dense_f32_patterns()
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7F80) == 0x7F80).all() and ((got[nan] & 0x7F) != 0).all()


def test_f32_to_f16_matches_torch():
    import torch
    x = _dense_f32_patterns()
    got = O.f32_to_f16(x)
    want = torch.from_numpy(x.copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7C00) == 0x7C00).all() and ((got[nan] & 0x3FF) != 0).all()


def test_16bit_to_f32_all_patterns_match_torch():
    """All 2^16 bfloat16 and half patterns widen exactly as torch widens them."""
    import torch
    h = np.arange(1 << 16, dtype=np.uint16)
    bf = np.array([O.lib().lso_bf16_to_f32(int(v)) for v in h[::257]], np.float32)
    want_bf = torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    assert np.array_equal(bf.view(np.uint32), want_bf[::257].view(np.uint32))
    assert np.array_equal(W.bf16_bits_to_f32(h).view(np.uint32), want_bf.view(np.uint32))
    got = O.f16_to_f32(h)
    want = torch.from_numpy(h.view(np.int16).copy()).view(torch.float16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
