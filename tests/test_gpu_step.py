"""GPU tests of lsamp_step (CBv2DefaultSampler.sample, DefaultSamplerV2.swift:
84-181, as one call): draw, commit of the drawn tokens into the device
penalty table, and the raw log-probabilities of the drawn tokens and the top
k, against the same three steps made by separate calls with the penalty
entries rebuilt on the host, and replayed from a HIP graph.
"""
from __future__ import annotations

import numpy as np
import pytest

from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, csr

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
        rp, en = csr([h.entries() for h in host])
        ref = ctx.sample(lt, params, semantics=_ffi.SEM_CBV2, row_ptr=rp, entries=en, uniforms=u)
        lp = ctx.logprobs(lt, tokens=ref["tokens"], top_k=5)
        torch.cuda.synchronize()
        tok = out["tokens"].cpu().numpy()
        assert np.array_equal(tok, ref["tokens"].cpu().numpy()), f"step {step}"
        assert np.array_equal(out["chosen"].cpu().numpy(), lp["chosen"].cpu().numpy())
        assert np.array_equal(out["top_ids"].cpu().numpy(), lp["top_ids"].cpu().numpy())
        assert np.array_equal(out["top_values"].cpu().numpy(), lp["top_values"].cpu().numpy())
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
