"""Bounded waits that give up (the wait test hook, lsamp_test_set_spin_limit,
forced from the host: every wait's target becomes unreachable and its limit
a few polls, while every kernel still exits normally).

* The sampling kernel's fused arrangement hands work off instead of failing:
  a slice that gives up waiting leaves, and the row's last arriver at each
  exchange does the slice's remaining work from a re-read (its select; for a
  short-list row that falls back, its histogram too).  Every row is exact
  with the hook on, none fails closed: the reference always returns a token
  (SamplerV2.swift:85-107).
* The top-k kernel's finalizer waits only for slices that started before it;
  with the hook on it gives them up and fails its rows closed (token -1,
  LSAMP_ROW_TIMEOUT, in the same readback as the tokens, as the reference
  fails a row closed: CBv2NonFiniteLogits.swift:30-38).
* With the hook off, the next step is exact again (the counters recover)."""
from __future__ import annotations

import numpy as np
import pytest

from common import compare, run_gpu, run_oracle
from lsamp import _ffi
from lsamp import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=256, max_vocab=262144)
    yield c
    c.close()


def _hook(polls):
    lib = _ffi.load_library()
    _ffi.check(lib.lsamp_test_set_spin_limit(0, polls), "lsamp_test_set_spin_limit")


def _run_with_hook(ctx, cfg):
    ctx.read_status()  # clear
    _hook(16)
    try:
        g = run_gpu(ctx, cfg)
    finally:
        _hook(0)
    ctx.read_status()  # (waits that gave up set the sticky bit: clear it)
    return g


def _histogram_rows(params, V):
    """Rows that take the histogram path: filtered rows without an active
    top-k of at most 256."""
    k = params["top_k"]
    short = (params["kind"] == _ffi.KIND_ARGMAX) | ((k > 0) & (k < V) & (k <= 256))
    return ~short


@pytest.mark.parametrize("rows", [24, 160], ids=["one-round", "task-queue"])
def test_slices_that_give_up_leave_their_work_to_the_last_arriver(ctx, rows):
    cfg = W.config3(rows=rows)
    assert _histogram_rows(cfg["params"], cfg["vocab"]).any()
    o = run_oracle(cfg, threads=16)
    g = _run_with_hook(ctx, cfg)
    launch = ctx.last_launch()
    assert launch["fused"] == 1 and launch["slices"] > 1
    assert (rows > launch["rows_per_round"]) == (rows == 160), launch
    assert not (g["row_flags"] & _ffi.ROW_TIMEOUT).any()
    compare(cfg, g, o, label="hook on")
    for _ in range(2):
        compare(cfg, run_gpu(ctx, cfg), o, label="hook off")
    assert ctx.read_status() == 0


def test_fallback_histograms_of_slices_that_left(ctx):
    """Short-list rows that need the histogram path after all (+inf logits in
    two slices) with the hook on: the first exchange's last arriver builds
    the histograms of the slices that left, merges, and does every select."""
    cfg = W.config3(rows=16)
    V = cfg["vocab"]
    p = cfg["params"]
    k = p["top_k"]
    topk_rows = np.flatnonzero((p["kind"] == _ffi.KIND_FILTERED) & (k > 0) & (k <= 256))[:3]
    greedy_rows = np.flatnonzero(p["kind"] == _ffi.KIND_ARGMAX)[:1]
    assert len(topk_rows) == 3 and len(greedy_rows) == 1
    logits = cfg["logits"].copy()
    for r in np.concatenate([topk_rows, greedy_rows]):
        logits[r, [1000 + int(r), V // 2 + 7]] = 0x7F80  # bf16 +inf
    cfg = dict(cfg, logits=logits)
    o = run_oracle(cfg, threads=16)
    g = _run_with_hook(ctx, cfg)
    assert ctx.last_launch()["fused"] == 1
    assert not (g["row_flags"] & _ffi.ROW_TIMEOUT).any()
    compare(cfg, g, o, label="fallback, hook on")
    for r in np.concatenate([topk_rows, greedy_rows]):
        assert g["tokens"][r] in (1000 + int(r), V // 2 + 7)
    compare(cfg, run_gpu(ctx, cfg), o, label="fallback, hook off")
    assert ctx.read_status() == 0


def test_split_mode_never_waits(ctx):
    lib = _ffi.load_library()
    cfg = W.config3(rows=16)
    o = run_oracle(cfg, threads=16)
    ctx.set_mode(_ffi.MODE_SPLIT)
    _ffi.check(lib.lsamp_test_set_spin_limit(0, 16), "lsamp_test_set_spin_limit")
    try:
        g = run_gpu(ctx, cfg)
    finally:
        _ffi.check(lib.lsamp_test_set_spin_limit(0, 0), "lsamp_test_set_spin_limit")
        ctx.set_mode(_ffi.MODE_AUTO)
    compare(cfg, g, o, label="split with the hook on")
    assert not (g["row_flags"] & _ffi.ROW_TIMEOUT).any()


def test_topk_finalizer_timeout_fails_closed_and_recovers(ctx):
    """The top-k kernel: every row's finalizer waits (for its other slices'
    payloads, or, with one slice, through the hook alone), so with the hook
    on every row fails closed; with it off the same step is exact again (the
    tickets and epochs recover)."""
    lib = _ffi.load_library()
    cfg = W.config2(rows=16)
    o = run_oracle(cfg, threads=16)
    ctx.read_status()  # clear
    _ffi.check(lib.lsamp_test_set_spin_limit(0, 16), "lsamp_test_set_spin_limit")
    try:
        g = run_gpu(ctx, cfg)
        status = ctx.read_status()
    finally:
        _ffi.check(lib.lsamp_test_set_spin_limit(0, 0), "lsamp_test_set_spin_limit")
    assert ctx.last_launch()["fused"] == 2
    assert status & _ffi.STATUS_SPIN_TIMEOUT
    assert ((g["row_flags"] & _ffi.ROW_TIMEOUT) != 0).all(), g["row_flags"]
    assert (g["tokens"] == -1).all()
    for _ in range(2):
        compare(cfg, run_gpu(ctx, cfg), o, label="top-k after timeouts")
        assert ctx.last_launch()["fused"] == 2
    assert ctx.read_status() == 0
