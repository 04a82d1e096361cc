"""The two execution modes of lsamp_sample agree bit for bit.

Fused mode runs the whole step as one kernel whose work-groups hand their
row's histogram merge to each other; split mode runs it as two kernels.  Both
must give identical tokens, flags, processed logits, keep sets and statistics
(integer histogram and weight sums make the result independent of the order in
which work-groups finish), and a fused step must never leave the device's
spin-timeout status bit set.
"""
from __future__ import annotations

import numpy as np
import pytest

from common import run_gpu
from lsamp import _ffi
from lsamp import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=512, max_vocab=262144)
    yield c
    c.close()


def _both_modes(ctx, cfg):
    outs = {}
    for mode in (_ffi.MODE_FUSED, _ffi.MODE_SPLIT):
        ctx.set_mode(mode)
        try:
            outs[mode] = run_gpu(ctx, cfg)
        finally:
            ctx.set_mode(_ffi.MODE_AUTO)
        assert ctx.read_status() == 0, f"device status bits set after mode {mode}"
    return outs[_ffi.MODE_FUSED], outs[_ffi.MODE_SPLIT]


def _assert_same(a, b, label):
    assert np.array_equal(a["tokens"], b["tokens"]), f"{label}: tokens differ"
    assert np.array_equal(a["row_flags"], b["row_flags"]), f"{label}: flags differ"
    assert np.array_equal(a["processed"].view(np.uint32), b["processed"].view(np.uint32)), \
        f"{label}: processed logits differ"
    assert np.array_equal(a["keep"], b["keep"]), f"{label}: keep sets differ"
    assert a["stats"].tobytes() == b["stats"].tobytes(), f"{label}: stats differ"


@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_fused_equals_split_full_configs(ctx, n):
    cfg = W.WORKLOADS[n]()
    f, s = _both_modes(ctx, cfg)
    _assert_same(f, s, f"config{n}")


def _many_rounds_cfg(dtype):
    # 512 rows of a 40,001-token vocabulary: several rounds of the fused grid
    rng = np.random.default_rng(21)
    V, B = 40001, 512
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    params = [W.resolve_cbv2(temperature=[0.0, 0.7, 1.0, 1.3][r % 4],
                             top_k=[0, 40, 5, 400][(r // 4) % 4],
                             top_p=[1.0, 0.9, 0.5][r % 3], min_p=[0.0, 0.05][r % 2], vocab=V)
              for r in range(B)]
    logits = x if dtype == _ffi.DTYPE_F32 else W.f32_to_bf16_bits(x)
    return dict(semantics=_ffi.SEM_CBV2, dtype=dtype, rows=B, vocab=V, logits=logits,
                params=W._params(params), uniforms=rng.random(B, dtype=np.float32))


def test_fused_equals_split_many_rounds(ctx):
    cfg = _many_rounds_cfg(_ffi.DTYPE_BF16)
    f, s = _both_modes(ctx, cfg)
    _assert_same(f, s, "many rounds")
    ctx.set_mode(_ffi.MODE_FUSED)
    try:
        run_gpu(ctx, cfg)
        launch = ctx.last_launch()
    finally:
        ctx.set_mode(_ffi.MODE_AUTO)
    assert launch["fused"] == 1 and launch["rows_per_round"] < cfg["rows"], launch


def test_fp32_steps_of_several_rounds_run_split(ctx):
    """The fused kernel's several-rounds form is not built for the fp32 slab
    (it would not fit the registers): such steps take the split kernels, in
    every mode, with the same results."""
    cfg = _many_rounds_cfg(_ffi.DTYPE_F32)
    f, s = _both_modes(ctx, cfg)
    _assert_same(f, s, "fp32 many rounds")
    for mode in (_ffi.MODE_AUTO, _ffi.MODE_FUSED):
        ctx.set_mode(mode)
        try:
            run_gpu(ctx, cfg)
            assert ctx.last_launch()["fused"] == 0
        finally:
            ctx.set_mode(_ffi.MODE_AUTO)


def test_status_clear_after_default_mode(ctx):
    cfg = W.config2(rows=16)
    run_gpu(ctx, cfg)
    assert ctx.read_status() == 0


def test_fused_equals_split_past_the_row_order():
    # 1,100 rows: more than the fused kernel orders (histogram-path rows
    # first) at its start, so its work-groups take the tasks in row order
    import torch
    from lsamp.api import Context
    rng = np.random.default_rng(23)
    V, B = 8192, 1100
    c = Context(0, max_rows=B, max_vocab=V)
    try:
        x = rng.normal(0, 3, (B, V)).astype(np.float32)
        params = [W.resolve_cbv2(temperature=[0.0, 0.8, 1.1][r % 3], top_k=[0, 30, 300][(r // 3) % 3],
                                 top_p=[1.0, 0.9][r % 2], vocab=V) for r in range(B)]
        cfg = dict(semantics=_ffi.SEM_CBV2, dtype=_ffi.DTYPE_F32, rows=B, vocab=V, logits=x,
                   params=W._params(params), uniforms=rng.random(B, dtype=np.float32))
        f, s = _both_modes(c, cfg)
        _assert_same(f, s, "past the row order")
        assert c.last_launch()["fused"] == 0  # (the split launch ran last)
    finally:
        torch.cuda.synchronize()
        c.close()
