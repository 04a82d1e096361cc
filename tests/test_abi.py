"""CPU tests of the C ABI (include/lsamp.h, lib/liblsamp.so) that need no
GPU: the library loads, exports every function the header declares, agrees on
struct layouts with the bindings, fails cleanly when no device is present,
and its host-side parameter resolution and RNG agree with the reference's
factory rules and with the oracle's independent restatement.
"""
from __future__ import annotations

import ctypes
import glob
import os
import re

import numpy as np
import pytest

import oracle as O
from lsamp import _ffi
from lsamp import workloads as W

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "lsamp.h")
HEADERS = sorted(glob.glob(os.path.join(REPO, "include", "*.h")))


@pytest.fixture(scope="module")
def lib():
    return _ffi.load_library()


def declared_functions():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lsamp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for required in ("lsamp_context_create", "lsamp_context_destroy", "lsamp_sample",
                     "lsamp_verify", "lsamp_last_error", "lsamp_version", "lsamp_penalize",
                     "lsamp_test_set_spin_limit"):
        assert required in names


def test_library_exports_every_declared_function(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


@pytest.mark.parametrize("name,struct", [
    ("lsamp_row_params", _ffi.RowParams), ("lsamp_penalty_entry", _ffi.PenaltyEntry),
    ("lsamp_row_stats", _ffi.RowStats), ("lsamp_sample_args", _ffi.SampleArgs),
    ("lsamp_verify_args", _ffi.VerifyArgs), ("lsamp_mask_assemble_args", _ffi.MaskAssembleArgs),
    ("lsamp_generate_parameters", _ffi.GenerateParameters),
    ("lsamp_cbv2_params", _ffi.Cbv2Params), ("lsamp_launch_info", _ffi.LaunchInfo),
    ("lsamp_penalize_args", _ffi.PenalizeArgs)])
def test_struct_layouts_agree(lib, name, struct):
    assert lib.lsamp_abi_sizeof(name.encode()) == ctypes.sizeof(struct)


def test_numpy_record_layouts_agree(lib):
    from lsamp.api import PARAMS_DTYPE, PENALTY_DTYPE, STATS_DTYPE
    assert PARAMS_DTYPE.itemsize == lib.lsamp_abi_sizeof(b"lsamp_row_params")
    assert PENALTY_DTYPE.itemsize == lib.lsamp_abi_sizeof(b"lsamp_penalty_entry")
    assert STATS_DTYPE.itemsize == lib.lsamp_abi_sizeof(b"lsamp_row_stats")
    assert lib.lsamp_abi_sizeof(b"no_such_struct") == -1


def test_version_string(lib):
    assert b"gfx950" in lib.lsamp_version()


def test_errors_without_a_device(lib):
    """Every call fails with a status and a message instead of crashing when
    no GPU is present (this container), or when handed NULL."""
    h = ctypes.c_void_p()
    st = lib.lsamp_context_create(0, 4, 1000, ctypes.byref(h))
    if st == 0:  # a GPU is visible: nothing to check here
        lib.lsamp_context_destroy(h)
        pytest.skip("a device is present")
    assert st == _ffi.LSAMP_ERR_DEVICE and not h.value
    assert lib.lsamp_last_error()
    assert lib.lsamp_sample(None, None, None) == _ffi.LSAMP_ERR_INVALID_ARGUMENT
    assert b"NULL" in lib.lsamp_last_error()
    assert lib.lsamp_verify(None, None, None) != 0
    assert lib.lsamp_context_set_mode(None, 0) == _ffi.LSAMP_ERR_INVALID_ARGUMENT
    lib.lsamp_context_destroy(None)


def test_context_shape_limits(lib):
    h = ctypes.c_void_p()
    assert lib.lsamp_context_create(0, 0, 1000, ctypes.byref(h)) == _ffi.LSAMP_ERR_SHAPE
    assert lib.lsamp_context_create(0, 4, 0, ctypes.byref(h)) == _ffi.LSAMP_ERR_SHAPE
    assert lib.lsamp_context_create(0, 4, 1 << 24, ctypes.byref(h)) == _ffi.LSAMP_ERR_SHAPE


# ---------------------------------------------------- parameter resolution
def gp(temperature=0.6, top_p=1.0, top_k=0, min_p=0.0, rep=None, rep_ctx=20, pres=None,
       pres_ctx=20, freq=None, freq_ctx=20):
    g = _ffi.GenerateParameters()
    g.temperature, g.top_p, g.top_k, g.min_p = temperature, top_p, top_k, min_p
    g.has_repetition_penalty = rep is not None
    g.repetition_penalty = rep or 0.0
    g.repetition_context_size = rep_ctx
    g.has_presence_penalty = pres is not None
    g.presence_penalty = pres or 0.0
    g.presence_context_size = pres_ctx
    g.has_frequency_penalty = freq is not None
    g.frequency_penalty = freq or 0.0
    g.frequency_context_size = freq_ctx
    return g


def resolve_gp(lib, **kw):
    out = _ffi.RowParams()
    ctx = ctypes.c_int32()
    assert lib.lsamp_resolve_generate_parameters(ctypes.byref(gp(**kw)), ctypes.byref(out),
                                                 ctypes.byref(ctx)) == 0
    return out, ctx.value


@pytest.mark.parametrize("kw,kind", [
    # SamplerPenaltyTests.swift:45-51; SampleTests.swift:113-117
    (dict(temperature=0.7), _ffi.KIND_CATEGORICAL),
    (dict(temperature=0.7, top_p=1), _ffi.KIND_CATEGORICAL),
    (dict(temperature=0.7, top_p=0), _ffi.KIND_CATEGORICAL),
    (dict(temperature=0.7, top_p=0.9), _ffi.KIND_FILTERED),
    (dict(temperature=0, top_k=5), _ffi.KIND_ARGMAX),
    (dict(temperature=0.7, top_k=40), _ffi.KIND_FILTERED),
    (dict(temperature=0.7, min_p=0.1), _ffi.KIND_FILTERED),
    (dict(temperature=0), _ffi.KIND_ARGMAX),
])
def test_generate_parameters_sampler_choice(lib, kw, kind):
    out, _ = resolve_gp(lib, **kw)
    assert out.kind == kind
    assert out.kind == W.resolve_mlxlm(**kw)["kind"]


@pytest.mark.parametrize("kw,contexts", [
    # SampleTests.swift:147-156, SamplerPenaltyTests.swift:260-276
    (dict(rep=1.1), 1), (dict(pres=0.5), 2), (dict(freq=0.5), 4),
    (dict(rep=1.1, pres=0.5, freq=0.5), 7),
    (dict(rep=1.5, rep_ctx=0), 0), (dict(pres=0.0), 0), (dict(pres=0.5, pres_ctx=0), 0),
    (dict(), 0), (dict(rep=1.0), 0),
])
def test_generate_parameters_processor_contexts(lib, kw, contexts):
    out, ctx = resolve_gp(lib, **kw)
    assert ctx == contexts
    py = W.resolve_mlxlm(repetition_penalty=kw.get("rep"), repetition_context_size=kw.get("rep_ctx", 20),
                         presence_penalty=kw.get("pres"), presence_context_size=kw.get("pres_ctx", 20),
                         frequency_penalty=kw.get("freq"), frequency_context_size=kw.get("freq_ctx", 20))
    assert out.repetition_penalty == pytest.approx(py["repetition_penalty"])
    assert out.presence_penalty == pytest.approx(py["presence_penalty"])
    assert out.frequency_penalty == pytest.approx(py["frequency_penalty"])


def resolve_cb(lib, vocab=1000, **kw):
    sp = _ffi.Cbv2Params()
    sp.temperature = kw.get("temperature", 1.0)
    sp.top_p = kw.get("top_p", 1.0)
    sp.top_k = kw.get("top_k", 0)
    sp.min_p = kw.get("min_p", 0.0)
    sp.repetition_penalty = kw.get("repetition_penalty", 1.0)
    sp.repetition_context_size = kw.get("repetition_context_size", 64)
    sp.frequency_penalty = kw.get("frequency_penalty", 0.0)
    sp.presence_penalty = kw.get("presence_penalty", 0.0)
    out = _ffi.RowParams()
    assert lib.lsamp_resolve_cbv2_params(ctypes.byref(sp), vocab, ctypes.byref(out)) == 0
    return out


@pytest.mark.parametrize("kw", [
    dict(temperature=0.0), dict(temperature=9e-6), dict(temperature=1e-5),
    dict(temperature=0.8, top_k=50, top_p=0.95, min_p=0.05),
    dict(temperature=1.0, top_k=1000), dict(temperature=1.0, top_k=5000),
    dict(temperature=1.0, top_p=0.0), dict(temperature=1.0, top_p=-1.0),
    dict(temperature=1.0, top_p=1.5), dict(temperature=1.0, min_p=3.0),
    dict(temperature=0.7, repetition_penalty=1.3, repetition_context_size=0),
    dict(temperature=0.7, repetition_penalty=1.3, repetition_context_size=16),
    dict(temperature=0.7, frequency_penalty=0.3), dict(temperature=0.7, presence_penalty=0.5),
])
def test_cbv2_resolution_matches_set_rows(lib, kw):
    # LogitsPipelineV2.swift:188-227: greedy iff T < 1e-5; top-k off unless
    # 0 < k < vocab; top-p off (2.0) unless 0 < p < 1, p <= 0 keeps the top
    # token only; min-p clamped to 1
    out = resolve_cb(lib, vocab=1000, **kw)
    py = W.resolve_cbv2(vocab=1000, **kw)
    for f, _ in _ffi.RowParams._fields_:
        assert getattr(out, f) == pytest.approx(py[f]), f
    greedy = np.float32(kw["temperature"]) < np.float32(1e-5)
    assert (out.kind == _ffi.KIND_ARGMAX) == greedy


# ------------------------------------------------------------------- RNG
def test_rng_key_matches_the_oracle(lib):
    rng = np.random.default_rng(9)
    for _ in range(200):
        s, i, t = (int(v) for v in rng.integers(0, 2**63, 3, dtype=np.uint64))
        assert lib.lsamp_rng_key(s, i, t) == O.rng_key(s, i, t)


def test_rng_key_splitmix64_known_answer(lib):
    # the published SplitMix64 outputs of seed 1234567, composed as
    # SamplerV2.mix composes them (SamplerV2.swift:183-191)
    from test_oracle_golden import splitmix_known_answers
    for seed, rid, step, key in splitmix_known_answers():
        assert lib.lsamp_rng_key(seed, rid, step) == key


def test_rng_uniform_matches_the_oracle(lib):
    rng = np.random.default_rng(10)
    for _ in range(200):
        k = int(rng.integers(0, 2**63, dtype=np.uint64))
        for purpose in (0, 1, 7):
            assert lib.lsamp_rng_uniform(k, purpose) == O.rng_uniform(k, purpose)
