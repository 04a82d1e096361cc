"""Fail-closed rows when a bounded wait gives up (the fused arrangement's
waits, and the top-k kernel's finalizer).

The wait test hook (lsamp_test_set_spin_limit) makes every wait's target
unreachable and its limit a few polls, forced from the host: every kernel
still exits normally.  A row whose path waited must come back as token -1
with LSAMP_ROW_TIMEOUT (the reference fails closed per row, in the same
readback as the tokens: CBv2NonFiniteLogits.swift:30-38); rows that never
waited must be exact; the next step, with the hook off, must be exact again
(the arrival counters recover)."""
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


def _waits(params, V):
    """Rows whose fused path waits for their other slices: filtered rows
    without an active top-k of at most 256 (the histogram path)."""
    k = params["top_k"]
    short = (params["kind"] == _ffi.KIND_ARGMAX) | ((k > 0) & (k < V) & (k <= 256))
    return ~short


def test_timed_out_rows_fail_closed_and_the_next_step_is_exact(ctx):
    lib = _ffi.load_library()
    cfg = W.config3(rows=24)
    o = run_oracle(cfg, threads=16)
    waits = _waits(cfg["params"], cfg["vocab"])
    assert waits.any() and (~waits).any()
    ctx.read_status()  # clear
    _ffi.check(lib.lsamp_test_set_spin_limit(0, 16), "lsamp_test_set_spin_limit")
    try:
        g = run_gpu(ctx, cfg)
        status = ctx.read_status()
    finally:
        _ffi.check(lib.lsamp_test_set_spin_limit(0, 0), "lsamp_test_set_spin_limit")
    assert ctx.last_launch()["fused"] == 1
    assert status & _ffi.STATUS_SPIN_TIMEOUT
    tmo = (g["row_flags"] & _ffi.ROW_TIMEOUT) != 0
    assert np.array_equal(tmo, waits), (tmo, waits)
    assert (g["tokens"][tmo] == -1).all()
    assert np.array_equal(g["tokens"][~tmo], o["tokens"][~tmo])
    # the hook is off: the same step is exact, counters included
    for _ in range(2):
        compare(cfg, run_gpu(ctx, cfg), o, label="after timeouts")
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
