"""GPU tests of lsamp_step (CBv2DefaultSampler.sample, DefaultSamplerV2.swift:
84-181, as one call): draw, commit of the drawn tokens into the device
penalty table, and the raw log-probabilities of the drawn tokens and the top
k, against the same three steps made by separate calls with the penalty
entries rebuilt on the host, and replayed from a HIP graph.

When the draw runs the one-pass top-k kernel (16-bit logits, CBv2 top-k
rows), that kernel ranks the raw logits in the same pass (launch kind 3);
its log-probabilities are checked against the oracle's raw ranking
(LogitsPipelineV2.process :307-314, CBv2Logprobs.gather :534-549) and against
lsamp_logprobs: ids identical, values within the log-probability tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, csr
from rank_common import BF16, F16, F32, close_logprobs, to_bits

pytestmark = pytest.mark.gpu

V = 151936


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=V)
    yield c
    c.close()


def setup(seed, rows):
    import torch
    rng = np.random.default_rng(seed)
    prior = -1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))
    x = np.stack([rng.normal(0.0, 3.0, V) + prior[rng.permutation(V)] for _ in range(rows)])
    bits = W.f32_to_bf16_bits(x.astype(np.float32))
    lt = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
    p = W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, presence_penalty=0.5,
                       frequency_penalty=0.3, repetition_penalty=1.2, repetition_context_size=8,
                       vocab=V)
    prompts = [rng.integers(0, 300, 30).tolist() for _ in range(rows)]
    return rng, lt, W._params([p] * rows), prompts


def states(prompts):
    return [Cbv2RowState(pr, [], 8, repetition_on=True, counts_on=True, vocab=V) for pr in prompts]


def test_step_equals_separate_calls(ctx):
    import torch
    from lsamp.api import PenaltyTable
    rows = 8
    rng, lt, params, prompts = setup(1, rows)
    host = states(prompts)
    table = PenaltyTable(states(prompts), capacity=256, window_capacity=8)
    for step in range(6):
        u = rng.random(rows, dtype=np.float32)
        out = ctx.step(lt, params, table=table, uniforms=u, logprobs_top_k=5)
        # (the step's draw ranked the raw logits in its own pass)
        assert ctx.last_launch()["fused"] == 3
        rp, en = csr([h.entries() for h in host])
        ref = ctx.sample(lt, params, semantics=_ffi.SEM_CBV2, row_ptr=rp, entries=en, uniforms=u)
        lp = ctx.logprobs(lt, tokens=ref["tokens"], top_k=5)
        torch.cuda.synchronize()
        tok = out["tokens"].cpu().numpy()
        assert np.array_equal(tok, ref["tokens"].cpu().numpy()), f"step {step}"
        assert close_logprobs(out["chosen"].cpu().numpy(), lp["chosen"].cpu().numpy())
        assert np.array_equal(out["top_ids"].cpu().numpy(), lp["top_ids"].cpu().numpy())
        assert close_logprobs(out["top_values"].cpu().numpy(), lp["top_values"].cpu().numpy())
        assert not out["commit_flags"].cpu().numpy().any()
        for r in range(rows):
            host[r].commit(int(tok[r]))
    # the device table holds the host's entries after the six commits
    for r, (e, _, _, _) in enumerate(table.host_rows()):
        want = host[r].entries()
        assert e["token"].tolist() == want["token"].tolist()
        assert e["count"].tolist() == want["count"].tolist()
        assert e["flags"].tolist() == want["flags"].tolist()


def test_step_replays_from_a_graph(ctx):
    import torch
    from lsamp.api import PenaltyTable
    rows, steps = 8, 5
    rng, lt, params, prompts = setup(2, rows)
    u = torch.from_numpy(rng.random(rows, dtype=np.float32)).cuda()
    eager_t = PenaltyTable(states(prompts), capacity=256, window_capacity=8)
    graph_t = PenaltyTable(states(prompts), capacity=256, window_capacity=8)
    eager = ctx.prepare_step(lt, params, table=eager_t, uniforms=u, logprobs_top_k=3)
    graphed = ctx.prepare_step(lt, params, table=graph_t, uniforms=u, logprobs_top_k=3)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        graphed.launch(s.cuda_stream)
    torch.cuda.synchronize()
    for i in range(steps):
        eager.launch(s.cuda_stream)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        a, b = eager.outputs(), graphed.outputs()
        assert np.array_equal(a["tokens"].cpu().numpy(), b["tokens"].cpu().numpy()), f"replay {i}"
        assert np.array_equal(a["top_ids"].cpu().numpy(), b["top_ids"].cpu().numpy())
    ra, rb = eager_t.host_rows(), graph_t.host_rows()
    for r in range(rows):
        assert ra[r][0].tolist() == rb[r][0].tolist()


NAN, INF = float("nan"), float("inf")


def special_rows(x, rng):
    """Rows 1..8 of a batch get the raw ranking's edge cases."""
    V = x.shape[1]
    x[1, rng.choice(V, 5, replace=False)] = NAN            # NaN: log-sum-exp NaN
    x[2, rng.choice(V, 3, replace=False)] = INF            # +inf: log-sum-exp +inf
    x[3].fill(-INF)                                         # all -inf but two
    x[3, rng.choice(V, 2, replace=False)] = -3.0
    x[4].fill(1.5)                                          # every token tied
    x[5, [7, V // 2, V - 1]] = 50.0                         # ties across slices
    x[6].fill(NAN)                                          # all NaN (an EMPTY draw)
    np.minimum(x[7], 0.0, out=x[7])                         # signed zeros
    x[7, rng.choice(V, 40, replace=False)] = -0.0
    x[8, :V // 3] += 40.0                                   # one slice holds the top


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("vocab,k", [(151936, 0), (151936, 1), (151936, 20), (151936, 32),
                                     (40003, 20), (1001, 32)])
def test_step_logprobs_in_the_sampling_pass(ctx, dtype, vocab, k):
    """The top-k kernel's raw log-probabilities (launch kind 3) against the
    oracle's raw ranking and lsamp_logprobs: the raw logits before penalties,
    the grammar mask and the temperature; NaN, +inf, all -inf, tied, signed
    zero rows; rows that are not 16-byte aligned (odd vocabularies)."""
    import torch
    from lsamp.api import PenaltyTable
    rng = np.random.default_rng(vocab + 7 * k + dtype)
    rows = 12
    x = rng.normal(0.0, 3.0, (rows, vocab)).astype(np.float32)
    special_rows(x, rng)
    bits = to_bits(x, dtype)
    tdt = torch.bfloat16 if dtype == BF16 else torch.float16
    lt = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(tdt).cuda()
    p = W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, presence_penalty=0.5,
                       frequency_penalty=0.3, repetition_penalty=1.2, repetition_context_size=8,
                       vocab=vocab)
    params = W._params([p] * rows)
    prompts = [rng.integers(0, vocab, 30).tolist() for _ in range(rows)]
    table = PenaltyTable(states_v(prompts, vocab), capacity=256, window_capacity=8)
    # a grammar mask on the even rows (the raw log-probabilities ignore it)
    words = (vocab + 31) // 32
    mask = np.full((rows, words), 0xFFFFFFFF, np.uint32)
    mask[::2] = rng.integers(0, 1 << 32, (rows // 2 + rows % 2, words), dtype=np.uint64).astype(np.uint32)
    u = rng.random(rows, dtype=np.float32)
    out = ctx.step(lt, params, table=table, uniforms=u, logprobs_top_k=k, bitmask=mask,
                   mask_bits=vocab)
    torch.cuda.synchronize()
    assert ctx.last_launch()["fused"] == 3
    tok = out["tokens"].cpu().numpy()
    assert (tok[6] == -1), "an all-NaN row draws nothing"
    ref = O.rank(np.ascontiguousarray(bits).reshape(-1), dtype=dtype, k=k, raw_values=False,
                 rows=rows, vocab=vocab, row_stride=vocab, col_stride=1, tokens=tok)
    if k:
        ids = out["top_ids"].cpu().numpy()
        bad = np.nonzero((ids != ref["ids"]).any(axis=1))[0]
        assert bad.size == 0, f"ids differ in rows {bad}: {ids[bad[:2]]} vs {ref['ids'][bad[:2]]}"
        assert close_logprobs(out["top_values"].cpu().numpy(), ref["values"])
        # NaN, +inf and all-NaN rows have no finite log-sum-exp: they fail closed
        assert (ids[[1, 2, 6]] == -1).all() and (ids[[0, 3, 4, 5, 7, 8]] >= 0).all()
        assert np.isnan(out["top_values"].cpu().numpy()[[1, 2, 6]]).all()
    assert close_logprobs(out["chosen"].cpu().numpy(), ref["chosen"])
    # and the second-pass entry point on the same tokens agrees
    lp = ctx.logprobs(lt, tokens=out["tokens"], top_k=k)
    torch.cuda.synchronize()
    if k:
        assert np.array_equal(out["top_ids"].cpu().numpy(), lp["top_ids"].cpu().numpy())
        assert close_logprobs(out["top_values"].cpu().numpy(), lp["top_values"].cpu().numpy())
    assert close_logprobs(out["chosen"].cpu().numpy(), lp["chosen"].cpu().numpy())


def states_v(prompts, vocab):
    return [Cbv2RowState(pr, [], 8, repetition_on=True, counts_on=True, vocab=vocab)
            for pr in prompts]


def _fused_params(rows, vocab):
    """Rows the one-pass top-k kernel does not take (so the step runs the
    fused sampling kernel): wide nuclei (no top-k, the histogram path), top-k
    100 (its short list), and a greedy row."""
    kinds = [dict(temperature=0.9, top_p=0.9), dict(temperature=0.7, top_k=100, top_p=0.95),
             dict(temperature=1.1, top_p=0.8, min_p=0.02), dict(temperature=0.0)]
    return W._params([W.resolve_cbv2(repetition_penalty=1.2, repetition_context_size=8,
                                     presence_penalty=0.5, frequency_penalty=0.3, vocab=vocab,
                                     **kinds[r % len(kinds)]) for r in range(rows)])


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
@pytest.mark.parametrize("vocab,k,rows", [(151936, 0, 12), (151936, 20, 12), (151936, 32, 12),
                                          (40003, 1, 12), (40003, 20, 12), (151936, 20, 80)])
def test_step_logprobs_in_the_fused_pass(dtype, vocab, k, rows):
    """The fused sampling kernel's raw log-probabilities (launch kind 4: no
    second pass over the logits) against the oracle's raw ranking
    (LogitsPipelineV2.process :307-314, CBv2Logprobs.gather :534-549): the
    raw logits before penalties, the grammar mask and the temperature; NaN,
    +inf, all -inf, tied, signed-zero rows; rows that are not 16-byte aligned
    (odd vocabularies); 80 rows take the fused grid in several rounds (16-bit
    logits; fp32 steps that do not fit one round run split, with the second
    pass)."""
    import torch
    from lsamp.api import Context, PenaltyTable
    ctx = Context(0, max_rows=rows, max_vocab=vocab)
    try:
        rng = np.random.default_rng(vocab + 7 * k + dtype + rows)
        x = rng.normal(0.0, 3.0, (rows, vocab)).astype(np.float32)
        special_rows(x, rng)
        if dtype == F32:
            bits = x
            lt = torch.from_numpy(x).cuda()
        else:
            bits = to_bits(x, dtype)
            lt = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(
                torch.bfloat16).cuda()
        params = _fused_params(rows, vocab)
        prompts = [rng.integers(0, vocab, 30).tolist() for _ in range(rows)]
        table = PenaltyTable(states_v(prompts, vocab), capacity=256, window_capacity=8)
        words = (vocab + 31) // 32
        mask = np.full((rows, words), 0xFFFFFFFF, np.uint32)
        mask[::2] = rng.integers(0, 1 << 32, (rows // 2 + rows % 2, words),
                                 dtype=np.uint64).astype(np.uint32)
        u = rng.random(rows, dtype=np.float32)
        out = ctx.step(lt, params, table=table, uniforms=u, logprobs_top_k=k, bitmask=mask,
                       mask_bits=vocab)
        torch.cuda.synchronize()
        launch = ctx.last_launch()
        if dtype == F32 and rows == 80:
            assert launch["fused"] == 0, launch  # split, with lsamp_logprobs after it
        else:
            assert launch["fused"] == 4, launch
            assert rows != 80 or launch["rows_per_round"] < rows, launch
        tok = out["tokens"].cpu().numpy()
        ref = O.rank(np.ascontiguousarray(bits).reshape(-1), dtype=dtype, k=k, raw_values=False,
                     rows=rows, vocab=vocab, row_stride=vocab, col_stride=1, tokens=tok)
        if k:
            ids = out["top_ids"].cpu().numpy()
            bad = np.nonzero((ids != ref["ids"]).any(axis=1))[0]
            assert bad.size == 0, f"ids differ in rows {bad}: {ids[bad[:2]]} vs {ref['ids'][bad[:2]]}"
            assert close_logprobs(out["top_values"].cpu().numpy(), ref["values"])
            # NaN, +inf and all-NaN rows have no finite log-sum-exp: they fail closed
            assert (ids[[1, 2, 6]] == -1).all() and (ids[[0, 3, 4, 5, 7, 8]] >= 0).all()
        assert close_logprobs(out["chosen"].cpu().numpy(), ref["chosen"])
    finally:
        ctx.close()


@pytest.mark.parametrize("k", [0, 20])
def test_fp32_topk_batch_logprobs_take_the_fused_pass(k):
    """fp32 rows the one-pass top-k kernel would take (top-k 50, greedy): with
    raw log-probabilities the step runs the fused sampling kernel instead
    (launch kind 4), which ranks them in its own pass: its token equals the
    top-k kernel's draw and its log-probabilities match the oracle
    (LogitsPipelineV2.process :307-314, CBv2Logprobs.gather :534-549)."""
    import torch
    from lsamp.api import Context, PenaltyTable
    rows, vocab = 12, 151936
    ctx = Context(0, max_rows=rows, max_vocab=vocab)
    try:
        rng = np.random.default_rng(4242 + k)
        x = rng.normal(0.0, 3.0, (rows, vocab)).astype(np.float32)
        lt = torch.from_numpy(x).cuda()
        kinds = [dict(temperature=0.8, top_k=50, top_p=0.95), dict(temperature=0.0)]
        params = W._params([W.resolve_cbv2(repetition_penalty=1.1, repetition_context_size=8,
                                           vocab=vocab, **kinds[r % 2]) for r in range(rows)])
        prompts = [rng.integers(0, vocab, 30).tolist() for _ in range(rows)]
        table = PenaltyTable(states_v(prompts, vocab), capacity=256, window_capacity=8)
        rp, en = csr([h.entries() for h in states_v(prompts, vocab)])
        u = rng.random(rows, dtype=np.float32)
        plain = ctx.sample(lt, params, semantics=_ffi.SEM_CBV2, row_ptr=rp, entries=en, uniforms=u)
        torch.cuda.synchronize()
        assert ctx.last_launch()["fused"] == 2  # (the top-k kernel, no log-probabilities)
        out = ctx.step(lt, params, table=table, uniforms=u, logprobs_top_k=k)
        torch.cuda.synchronize()
        assert ctx.last_launch()["fused"] == 4, ctx.last_launch()
        tok = out["tokens"].cpu().numpy()
        assert np.array_equal(tok, plain["tokens"].cpu().numpy())
        ref = O.rank(x.reshape(-1), dtype=F32, k=k, raw_values=False, rows=rows, vocab=vocab,
                     row_stride=vocab, col_stride=1, tokens=tok)
        if k:
            assert np.array_equal(out["top_ids"].cpu().numpy(), ref["ids"])
            assert close_logprobs(out["top_values"].cpu().numpy(), ref["values"])
        assert close_logprobs(out["chosen"].cpu().numpy(), ref["chosen"])
    finally:
        ctx.close()


def test_fused_logprob_step_replays_from_a_graph():
    """lsamp_step on a batch the fused kernel takes, with log-probabilities
    (launch kind 4), captured in a HIP graph: every replay, with eager steps
    between them, gives the eager step's tokens, ids and values."""
    import torch
    from lsamp.api import Context, PenaltyTable
    rows, vocab = 16, 151936
    ctx = Context(0, max_rows=rows, max_vocab=vocab)
    try:
        rng = np.random.default_rng(77)
        x = rng.normal(0.0, 3.0, (rows, vocab)).astype(np.float32)
        lt = torch.from_numpy(to_bits(x, BF16).view(np.int16)).view(torch.bfloat16).cuda()
        params = _fused_params(rows, vocab)
        prompts = [rng.integers(0, vocab, 30).tolist() for _ in range(rows)]
        u = torch.from_numpy(rng.random(rows, dtype=np.float32)).cuda()
        eager_t = PenaltyTable(states_v(prompts, vocab), capacity=256, window_capacity=8)
        graph_t = PenaltyTable(states_v(prompts, vocab), capacity=256, window_capacity=8)
        eager = ctx.prepare_step(lt, params, table=eager_t, uniforms=u, logprobs_top_k=5)
        graphed = ctx.prepare_step(lt, params, table=graph_t, uniforms=u, logprobs_top_k=5)
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            graphed.launch(s.cuda_stream)
        torch.cuda.synchronize()
        assert ctx.last_launch()["fused"] == 4, ctx.last_launch()
        for i in range(4):
            eager.launch(s.cuda_stream)
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                g.replay()
            torch.cuda.synchronize()
            a, b = eager.outputs(), graphed.outputs()
            for key in ("tokens", "top_ids", "top_values", "chosen"):
                assert np.array_equal(a[key].cpu().numpy(), b[key].cpu().numpy(),
                                      equal_nan=key in ("top_values", "chosen")), (i, key)
    finally:
        ctx.close()
