"""lsamp_sample_noalloc (the sampling step with its workspace in a file-scope
device array, for callers that cannot allocate) against lsamp_sample with a
context, through the C ABI: identical tokens, flags, processed logits, keep
sets and statistics, bit for bit, on two calls in a row, the second with a
smaller input, and a third back at the larger size (the array keeps the last
call's contents)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from common import to_torch_logits
from lsamp import _ffi
from lsamp import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    from lsamp.api import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, max_rows=64, max_vocab=262144)
    yield c
    c.close()


def _prepare(ctx, cfg, suppress=None):
    kw = dict(semantics=cfg["semantics"], row_ptr=cfg.get("row_ptr"), entries=cfg.get("entries"),
              uniforms=cfg["uniforms"], want_processed=True, want_keep=True, want_stats=True,
              suppress_ids=suppress)
    if cfg.get("bitmask") is not None:
        kw.update(bitmask=cfg["bitmask"], mask_bits=cfg["mask_bits"],
                  mask_tail=cfg.get("mask_tail", 0))
    return ctx.prepare_sample(to_torch_logits(cfg), cfg["params"], **kw)


def _outputs(prep):
    import torch
    torch.cuda.synchronize()
    o = prep.outputs()
    return {k: v.cpu().numpy() for k, v in o.items()}


def _run_both(ctx, cfg, suppress=None):
    import torch
    from lsamp.api import current_stream_handle
    lib = _ffi.load_library()
    a = _prepare(ctx, cfg, suppress)
    b = _prepare(ctx, cfg, suppress)
    a.launch()
    st = lib.lsamp_sample_noalloc(ctypes.byref(b.args),
                                  ctypes.c_void_p(current_stream_handle(torch.device("cuda", 0))))
    assert st == 0, _ffi.last_error()
    return _outputs(a), _outputs(b)


def _same(x, y, label):
    for k in ("tokens", "row_flags", "keep", "stats"):
        assert np.array_equal(x[k], y[k]), f"{label}: {k} differs"
    px, py = x["processed"], y["processed"]
    assert np.array_equal(px.view(np.uint32), py.view(np.uint32)), f"{label}: processed differs"


def test_no_alloc_equals_the_context_path(ctx):
    big = W.config2()                       # 64 rows x 151,936 bf16, penalties
    small = W.config4(rows=8, vocab=40000)  # 8 rows x 40,000 fp32, bitmask
    x, y = _run_both(ctx, big)
    _same(x, y, "first call (64 x 151,936)")
    x, y = _run_both(ctx, small, suppress=np.array([5, 77, 39999, 50000], np.int32))
    _same(x, y, "second call (8 x 40,000, suppressed ids)")
    x, y = _run_both(ctx, big)
    _same(x, y, "third call (64 x 151,936 again)")


def test_no_alloc_rejects_sizes_past_its_limits(ctx):
    import torch
    lib = _ffi.load_library()
    cfg = W.config2(rows=2, vocab=4096)
    prep = _prepare(ctx, cfg)
    args = _ffi.SampleArgs.from_buffer_copy(prep.args)
    args.rows = 65
    assert lib.lsamp_sample_noalloc(ctypes.byref(args), None) == _ffi.LSAMP_ERR_CAPACITY
    assert "no-allocation" in _ffi.last_error()
    args.rows, args.vocab = 2, 262145
    assert lib.lsamp_sample_noalloc(ctypes.byref(args), None) == _ffi.LSAMP_ERR_CAPACITY
    torch.cuda.synchronize()


def test_no_alloc_under_graph_capture(ctx):
    """A call captured in a HIP graph (after one eager call, which sets up the
    device's scratch address outside the capture) replays exactly: three
    replays with other work and synchronizations between them, each equal to
    the context path bit for bit.  The counters the call clears are cleared
    by a fill kernel, so the graph holds no memset node."""
    import torch
    from lsamp.api import current_stream_handle
    lib = _ffi.load_library()
    cfg = W.config2(rows=16)
    ref_prep = _prepare(ctx, cfg)
    ref_prep.launch()
    ref = _outputs(ref_prep)
    prep = _prepare(ctx, cfg)
    st = lib.lsamp_sample_noalloc(ctypes.byref(prep.args),
                                  ctypes.c_void_p(current_stream_handle(torch.device("cuda", 0))))
    assert st == 0, _ffi.last_error()
    _same(ref, _outputs(prep), "eager call before the capture")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=s):
        st = lib.lsamp_sample_noalloc(ctypes.byref(prep.args), ctypes.c_void_p(s.cuda_stream))
    assert st == 0, _ffi.last_error()
    other = W.config4(rows=8, vocab=40000)
    for i in range(3):
        # other work on the same scratch array between replays, and fresh
        # garbage in the outputs the replay must overwrite
        a, b = _run_both(ctx, other)
        _same(a, b, f"other work before replay {i}")
        prep.tokens.fill_(-7)
        prep.processed.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        _same(ref, _outputs(prep), f"replay {i}")
