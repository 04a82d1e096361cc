"""GPU parity of the device-side penalty state (lsamp_commit on an
lsamp_penalty_table) against the oracle's dense restatement of
LogitsPipelineV2.commit, and of decode loops that sample from the table and
commit on the device against loops that rebuild the entries on the host.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from common import compare, run_oracle
from lsamp import _ffi
from lsamp import workloads as W
from lsamp.history import Cbv2RowState, csr

pytestmark = pytest.mark.gpu

BOTH = _ffi.STATE_COUNTS | _ffi.STATE_REPETITION


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=151936)
    yield c
    c.close()


def random_rows(rng, rows, vocab):
    specs = []
    for r in range(rows):
        mode = [_ffi.STATE_COUNTS, _ffi.STATE_REPETITION, BOTH, 0][r % 4]
        w = [1, 2, 5, 64][(r // 4) % 4]
        small = rng.integers(0, 40, rng.integers(0, 80)).tolist()   # many repeats
        prompt = small + rng.integers(0, vocab, rng.integers(0, 20)).tolist()
        output = rng.integers(0, 40, rng.integers(0, 10)).tolist()
        bias = {int(t): float(rng.normal()) for t in rng.integers(0, vocab, 3)} if r % 3 == 0 else {}
        specs.append((prompt, output, w, mode, bias))
    return specs


def states_of(specs, vocab):
    return [Cbv2RowState(p, o, w, repetition_on=bool(m & 2), counts_on=bool(m & 1), bias=b,
                         vocab=vocab) for p, o, w, m, b in specs]


def expected_entries(dense, mode, bias):
    """The sparse view of one row's dense state: {token: (count, flags, bias)}."""
    exp = {}
    toks = set(np.nonzero(dense.counts)[0]) | set(np.nonzero(dense.window_counts)[0]) | set(bias)
    for t in toks:
        cnt = int(dense.counts[t]) if mode & _ffi.STATE_COUNTS else 0
        fl = _ffi.PEN_REPETITION if (mode & 2) and dense.window_counts[t] > 0 else 0
        b = np.float32(bias.get(int(t), 0.0))
        if cnt or fl or b != 0:
            exp[int(t)] = (cnt, fl, float(b))
    return exp


def check_table(table, dense, specs, label):
    for r, (e, wc, win, ring) in enumerate(table.host_rows()):
        _, _, w, mode, bias = specs[r]
        got = {int(x["token"]): (int(x["count"]), int(x["flags"]), float(x["bias"])) for x in e}
        assert got == expected_entries(dense[r], mode, bias), f"{label}: row {r} entries"
        if mode & 2:
            assert win[:w].tolist() == dense[r].window.tolist(), f"{label}: row {r} window"
            assert ring == dense[r].ring_pos, f"{label}: row {r} ring position"
            for t, c in wc.items():
                assert c == int(dense[r].window_counts[t]), f"{label}: row {r} window count {t}"


@pytest.mark.parametrize("vocab", [1000, 151936])
def test_commit_sequence_matches_dense_state(ctx, vocab):
    import torch
    from lsamp.api import PenaltyTable
    rng = np.random.default_rng(vocab % 97)
    rows = 16
    specs = random_rows(rng, rows, vocab)
    table = PenaltyTable(states_of(specs, vocab), capacity=256, window_capacity=64)
    dense = [O.DenseRowState(vocab, p, o, w, m) for p, o, w, m, _ in specs]
    for step in range(40):
        tok = rng.integers(0, 40, rows).astype(np.int32)
        tok[step % rows] = -1                                  # an EMPTY row commits nothing
        if step % 5 == 0:                                      # re-add the token being evicted
            for r, (_, _, w, m, _) in enumerate(specs):
                if (m & 2) and dense[r].window[dense[r].ring_pos] >= 0:
                    tok[r] = dense[r].window[dense[r].ring_pos]
        flags = table.commit(ctx, torch.from_numpy(tok).cuda(), vocab)
        for r in range(rows):
            dense[r].commit(int(tok[r]))
        if step % 8 == 7 or step == 39:
            torch.cuda.synchronize()
            assert not flags.cpu().numpy().any()
            check_table(table, dense, specs, f"step {step}")


def test_capacity_overflow_is_reported(ctx):
    import torch
    from lsamp.api import PenaltyTable
    vocab = 1000
    specs = [([1, 2, 3], [], 4, BOTH, {}), ([5], [], 2, _ffi.STATE_COUNTS, {})]
    table = PenaltyTable(states_of(specs, vocab), capacity=3, window_capacity=4)
    flags = table.commit(ctx, torch.tensor([7, 9], dtype=torch.int32, device="cuda"), vocab)
    torch.cuda.synchronize()
    # row 0: {1, 2, 3} fill its three slots and 7 has none; row 1 (no
    # repetition, no output yet) takes 9 into an empty row
    assert flags.cpu().numpy().tolist() == [_ffi.ROW_OVERFLOW, 0]


def test_decode_loop_on_device_state_matches_host_rebuild(ctx):
    """Eight steps of sample -> commit with the table on the device against
    the same steps with entries rebuilt on the host from the histories, and
    against the oracle: identical tokens and processed logits at every step."""
    import torch
    from lsamp.api import PenaltyTable, params_array, stats_to_numpy, to_device_bytes
    rng = np.random.default_rng(3)
    rows, vocab = 8, 151936
    prior = -1.1 * np.log(np.arange(1, vocab + 1, dtype=np.float64))
    p = W.resolve_cbv2(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05, presence_penalty=0.5,
                       frequency_penalty=0.3, repetition_penalty=1.1, repetition_context_size=16,
                       vocab=vocab)
    params = [p] * rows
    prompts = [rng.integers(0, 500, 40).tolist() for _ in range(rows)]
    host = [Cbv2RowState(pr, [], 16, repetition_on=True, counts_on=True, vocab=vocab)
            for pr in prompts]
    table = PenaltyTable(host, capacity=512, window_capacity=16)
    pr_dev = to_device_bytes(params_array(W._params(params)), "cuda")
    for step in range(8):
        x = np.stack([rng.normal(0.0, 3.0, vocab) + prior[rng.permutation(vocab)]
                      for _ in range(rows)])
        # make recent history tokens attractive so the penalties decide draws
        for r in range(rows):
            x[r, host[r].window[0] if host[r].window[0] >= 0 else 0] += 8.0
        bits = W.f32_to_bf16_bits(x.astype(np.float32))
        lt = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).cuda()
        u = rng.random(rows, dtype=np.float32)
        dev = ctx.sample(lt, pr_dev, semantics=_ffi.SEM_CBV2, table=table, uniforms=u,
                         want_processed=True, want_keep=True, want_stats=True)
        rp, en = csr([h.entries() for h in host])
        ref = ctx.sample(lt, pr_dev, semantics=_ffi.SEM_CBV2, row_ptr=rp, entries=en, uniforms=u,
                         want_processed=True)
        torch.cuda.synchronize()
        tok_dev = dev["tokens"].cpu().numpy()
        assert np.array_equal(tok_dev, ref["tokens"].cpu().numpy()), f"step {step}"
        assert np.array_equal(dev["processed"].cpu().numpy(), ref["processed"].cpu().numpy())
        cfg = dict(semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_BF16, rows=rows, vocab=vocab,
                   logits=bits, params=W._params(params), uniforms=u, bitmask=None, mask_bits=0,
                   row_ptr=rp, entries=en)
        gpu = {"tokens": tok_dev, "row_flags": dev["row_flags"].cpu().numpy().astype(np.uint32),
               "processed": dev["processed"].cpu().numpy(), "keep": dev["keep"].cpu().numpy(),
               "stats": stats_to_numpy(dev["stats"])}
        compare(cfg, gpu, run_oracle(cfg), label=f"step {step}")
        flags = table.commit(ctx, dev["tokens"], vocab)
        for r in range(rows):
            host[r].commit(int(tok_dev[r]))
        torch.cuda.synchronize()
        assert not flags.cpu().numpy().any()


def test_rows_longer_than_the_register_scan(ctx):
    """Rows of about 3,000 entries: the sampled and evicted tokens and the
    run's last entry sit past the 1,024 entries the lanes hold in registers."""
    import torch
    from lsamp.api import PenaltyTable
    rng = np.random.default_rng(21)
    vocab, rows = 151936, 4
    specs = []
    for r in range(rows):
        hist = rng.permutation(vocab)[:3000].tolist()
        w = [64, 1500, 7, 1][r]
        # 2,500 distinct output tokens (counts), or a 1,500-token window
        specs.append((hist[:500], hist[500:], w, [BOTH, _ffi.STATE_REPETITION, BOTH,
                                                   _ffi.STATE_COUNTS][r], {}))
    table = PenaltyTable(states_of(specs, vocab), capacity=3200, window_capacity=1500)
    dense = [O.DenseRowState(vocab, p, o, w, m) for p, o, w, m, _ in specs]
    for step in range(30):
        tok = np.array([rng.choice(specs[r][1]) if step % 3 else rng.integers(0, vocab)
                        for r in range(rows)], np.int32)
        table.commit(ctx, torch.from_numpy(tok).cuda(), vocab)
        for r in range(rows):
            dense[r].commit(int(tok[r]))
    torch.cuda.synchronize()
    assert (table.row_len.cpu().numpy() > 1024).all()
    check_table(table, dense, specs, "long rows")
