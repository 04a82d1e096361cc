"""ctypes front end of the oracle (liblsamp_oracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg; never by the product path.
All arrays are host numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import sys
from ctypes import POINTER, Structure, c_double, c_float, c_int32, c_int64, c_uint8, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(REPO, "mlx-swift-lm_amd"))

from lsamp import _ffi  # noqa: E402  (struct layouts shared with the ABI)

LIB_PATH = os.path.join(HERE, "liblsamp_oracle.so")


class LsoSampleArgs(Structure):
    _fields_ = [
        ("semantics", c_int32), ("rows", c_int32), ("vocab", c_int32), ("dtype", c_int32),
        ("row_stride", c_int64), ("logits", c_void_p), ("params", c_void_p),
        ("penalty_row_ptr", c_void_p), ("penalty_entries", c_void_p),
        ("bitmask", c_void_p), ("mask_words", c_int32), ("mask_bits", c_int32),
        ("mask_tail", c_int32), ("uniforms", c_void_p), ("philox_keys", c_void_p),
        ("probe_tokens", c_void_p), ("threads", c_int32),
        ("tokens", c_void_p), ("row_flags", c_void_p), ("processed", c_void_p),
        ("keep", c_void_p), ("top_p_margin", c_void_p), ("min_p_margin", c_void_p),
        ("top_p_margin_exact", c_void_p), ("stats", c_void_p),
        ("suppress_ids", c_void_p), ("n_suppress", c_int32),
    ]


class LsoVerifyArgs(Structure):
    _fields_ = [
        ("mode", c_int32), ("sequences", c_int32), ("window", c_int32), ("vocab", c_int32),
        ("dtype", c_int32), ("target_logits", c_void_p), ("draft_logits", c_void_p),
        ("draft_tokens", c_void_p), ("params", c_void_p), ("uniforms", c_void_p),
        ("typical_delta", c_float), ("threads", c_int32), ("accepted", c_void_p),
        ("tokens", c_void_p), ("accept_mask", c_void_p), ("typical_margin", c_void_p),
        ("out_ptr", c_void_p), ("out_tokens", c_void_p), ("pen_drafts", c_void_p),
        ("pen_stride", c_int32), ("pen_offset", c_int32),
    ]


class LsoRankArgs(Structure):
    _fields_ = [
        ("rows", c_int32), ("vocab", c_int32), ("dtype", c_int32), ("row_stride", c_int64),
        ("col_stride", c_int64), ("logits", c_void_p), ("k", c_int32), ("raw_values", c_int32),
        ("tokens", c_void_p), ("chosen", c_void_p), ("values", c_void_p), ("ids", c_void_p),
        ("row_flags", c_void_p), ("lse", c_void_p),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.lso_sample.argtypes = [POINTER(LsoSampleArgs)]
        L.lso_sample.restype = c_int32
        L.lso_penalty_state_init.argtypes = [c_int32, c_void_p, c_int32, c_void_p, c_int32,
                                             c_int32, c_void_p, c_void_p, c_void_p,
                                             POINTER(c_int32)]
        L.lso_penalty_state_init.restype = None
        L.lso_penalty_commit.argtypes = [c_int32, c_uint32, c_int32, c_void_p, c_void_p,
                                         c_void_p, POINTER(c_int32), c_int32]
        L.lso_penalty_commit.restype = None
        L.lso_rank.argtypes = [POINTER(LsoRankArgs)]
        L.lso_rank.restype = c_int32
        L.lso_verify.argtypes = [POINTER(LsoVerifyArgs)]
        L.lso_verify.restype = c_int32
        L.lso_dexp.argtypes = [c_float]
        L.lso_dexp.restype = c_float
        L.lso_weight.argtypes = [c_float, c_float, c_float]
        L.lso_weight.restype = c_uint64
        L.lso_draw.argtypes = [c_int32, c_void_p, c_void_p, c_float, c_float, POINTER(c_uint64)]
        L.lso_draw.restype = c_int32
        L.lso_philox4x32_10.argtypes = [c_void_p, c_void_p, c_void_p]
        L.lso_philox4x32_10.restype = None
        L.lso_rng_key.argtypes = [c_uint64, c_uint64, c_uint64]
        L.lso_rng_key.restype = c_uint64
        L.lso_rng_uniform.argtypes = [c_uint64, c_uint32]
        L.lso_rng_uniform.restype = c_float
        L.lso_f32_to_bf16.argtypes = [c_float]
        L.lso_f32_to_bf16.restype = ctypes.c_uint16
        L.lso_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.lso_bf16_to_f32.restype = c_float
        for name in ("lso_f32_to_bf16_n", "lso_f32_to_f16_n", "lso_f16_to_f32_n"):
            getattr(L, name).argtypes = [c_void_p, c_void_p, c_int64]
            getattr(L, name).restype = None
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(c_void_p).value


def params_array(rows):
    """List of dicts / RowParams -> contiguous RowParams array."""
    arr = (_ffi.RowParams * len(rows))()
    for i, p in enumerate(rows):
        if isinstance(p, _ffi.RowParams):
            arr[i] = p
        else:
            for k, v in p.items():
                setattr(arr[i], k, v)
    return arr


PARAMS_DTYPE = np.dtype([
    ("kind", "<i4"), ("temperature", "<f4"), ("top_k", "<i4"), ("top_p", "<f4"),
    ("min_p", "<f4"), ("repetition_penalty", "<f4"), ("presence_penalty", "<f4"),
    ("frequency_penalty", "<f4")])


def _params_buffer(params):
    """Per-row params (structured array, RowParams array, or list of dicts /
    RowParams) -> contiguous numpy bytes in the lsamp_row_params layout."""
    if isinstance(params, np.ndarray):
        return np.ascontiguousarray(params)
    if isinstance(params, ctypes.Array):
        return np.frombuffer(bytes(params), dtype=PARAMS_DTYPE).copy()
    arr = params_array(params)
    return np.frombuffer(bytes(arr), dtype=PARAMS_DTYPE).copy()


def entries_array(entries):
    """Structured numpy array of PenaltyEntry (token, count, flags, bias)."""
    dt = np.dtype([("token", "<i4"), ("count", "<i4"), ("flags", "<u4"), ("bias", "<f4")])
    out = np.zeros(len(entries), dtype=dt)
    for i, e in enumerate(entries):
        out[i] = e
    return out


PENALTY_DTYPE = np.dtype([("token", "<i4"), ("count", "<i4"), ("flags", "<u4"), ("bias", "<f4")])
STATS_DTYPE = np.dtype([
    ("max_value", "<f4"), ("log_normalizer", "<f4"), ("kept", "<i4"), ("token", "<i4"),
    ("kept_weight", "<u8"), ("probe_weight", "<u8"), ("cut_value", "<f4"),
    ("kept_mass", "<f4"), ("kept_entropy", "<f4"), ("probe_prob", "<f4")])


def sample(*, semantics, logits, dtype, params, row_ptr=None, entries=None, bitmask=None,
           mask_bits=0, mask_tail=0, uniforms=None, philox_keys=None, probe_tokens=None,
           threads=1, want_processed=False, want_keep=False, want_margins=False,
           want_stats=False, vocab=None, row_stride=None, suppress_ids=None):
    """Run the oracle.  `logits` is a 2-D numpy array: float32, or uint16 bit
    patterns for bf16 / f16 (dtype says which)."""
    logits = np.ascontiguousarray(logits)
    rows = logits.shape[0]
    V = vocab if vocab is not None else logits.shape[1]
    stride = row_stride if row_stride is not None else logits.shape[1]
    params_keep = _params_buffer(params)
    out = {"tokens": np.zeros(rows, np.int32), "row_flags": np.zeros(rows, np.uint32)}
    if want_processed:
        out["processed"] = np.zeros((rows, V), np.float32)
    if want_keep:
        out["keep"] = np.zeros((rows, V), np.uint8)
    if want_margins:
        out["top_p_margin"] = np.zeros((rows, V), np.float32)
        out["min_p_margin"] = np.zeros((rows, V), np.float32)
        out["top_p_margin_exact"] = np.zeros((rows, V), np.float64)
    if want_stats:
        out["stats"] = np.zeros(rows, STATS_DTYPE)
    a = LsoSampleArgs()
    a.semantics = semantics
    a.rows = rows
    a.vocab = V
    a.dtype = dtype
    a.row_stride = stride
    a.logits = _ptr(logits)
    a.params = params_keep.ctypes.data_as(c_void_p).value
    if row_ptr is not None:
        row_ptr = np.ascontiguousarray(row_ptr, np.int32)
        entries = np.ascontiguousarray(entries, PENALTY_DTYPE)
        a.penalty_row_ptr = _ptr(row_ptr)
        a.penalty_entries = _ptr(entries) if len(entries) else _ptr(np.zeros(1, PENALTY_DTYPE))
    if bitmask is not None:
        bitmask = np.ascontiguousarray(bitmask, np.uint32)
        a.bitmask = _ptr(bitmask)
        a.mask_words = bitmask.shape[1]
        a.mask_bits = mask_bits
        a.mask_tail = mask_tail
    if uniforms is not None:
        uniforms = np.ascontiguousarray(uniforms, np.float32)
        a.uniforms = _ptr(uniforms)
    if philox_keys is not None:
        philox_keys = np.ascontiguousarray(philox_keys, np.uint64)
        a.philox_keys = _ptr(philox_keys)
    if probe_tokens is not None:
        probe_tokens = np.ascontiguousarray(probe_tokens, np.int32)
        a.probe_tokens = _ptr(probe_tokens)
    if suppress_ids is not None and len(suppress_ids) > 0:
        suppress_ids = np.ascontiguousarray(suppress_ids, np.int32)
        a.suppress_ids = _ptr(suppress_ids)
        a.n_suppress = len(suppress_ids)
    a.threads = threads
    for k in ("tokens", "row_flags", "processed", "keep", "top_p_margin", "min_p_margin",
              "top_p_margin_exact", "stats"):
        if k in out:
            setattr(a, k, _ptr(out[k]))
    st = lib().lso_sample(ctypes.byref(a))
    if st != 0:
        raise RuntimeError(f"lso_sample failed: {st}")
    return out


def verify(*, mode, target, draft, draft_tokens, dtype, params, uniforms, typical_delta=0.0,
           threads=1, output_tokens=None, pen_drafts=None, column_offset=0):
    """target [S, W, V], draft [S, W-1, V] (or None), draft_tokens [S, W-1].
    output_tokens: per sequence, the confirmed output tokens (penalty-aware
    windows); pen_drafts [S, n] the round's draft chain with the window's
    first column at chain position column_offset."""
    target = np.ascontiguousarray(target)
    S, W, V = target.shape
    if draft is not None:
        draft = np.ascontiguousarray(draft)
    draft_tokens = np.ascontiguousarray(draft_tokens, np.int32)
    uniforms = np.ascontiguousarray(uniforms, np.float32)
    params_keep = _params_buffer(params)
    out = {"accepted": np.zeros(S, np.int32), "tokens": np.zeros((S, W), np.int32),
           "accept_mask": np.zeros((S, W - 1), np.uint8),
           "typical_margin": np.zeros((S, W - 1), np.float64)}
    a = LsoVerifyArgs()
    a.mode = mode
    a.sequences = S
    a.window = W
    a.vocab = V
    a.dtype = dtype
    a.target_logits = _ptr(target)
    a.draft_logits = _ptr(draft)
    a.draft_tokens = _ptr(draft_tokens)
    a.params = params_keep.ctypes.data_as(c_void_p).value
    a.uniforms = _ptr(uniforms)
    a.typical_delta = typical_delta
    a.threads = threads
    a.accepted = _ptr(out["accepted"])
    a.tokens = _ptr(out["tokens"])
    a.accept_mask = _ptr(out["accept_mask"])
    a.typical_margin = _ptr(out["typical_margin"])
    keep = []
    if output_tokens is not None:
        optr = np.zeros(S + 1, np.int32)
        optr[1:] = np.cumsum([len(t) for t in output_tokens])
        otok = np.ascontiguousarray(np.concatenate([np.asarray(t, np.int32) for t in output_tokens])
                                    if optr[-1] else np.zeros(1, np.int32), np.int32)
        keep += [optr, otok]
        a.out_ptr = _ptr(optr)
        a.out_tokens = _ptr(otok)
        if pen_drafts is not None:
            pdr = np.ascontiguousarray(pen_drafts, np.int32)
            keep.append(pdr)
            a.pen_drafts = _ptr(pdr)
            a.pen_stride = pdr.shape[1]
            a.pen_offset = int(column_offset)
    st = lib().lso_verify(ctypes.byref(a))
    if st != 0:
        raise RuntimeError(f"lso_verify failed: {st}")
    return out


def rank(storage, *, dtype, k, raw_values, rows=None, vocab=None, row_stride=None,
         col_stride=1, tokens=None):
    """Exact top-k (and log-probabilities) of the [rows, vocab] view of
    `storage` (logit bits: uint16 for bf16 / f16, float32 for f32) with the
    given element strides.  Returns ids, values, chosen, row_flags, lse."""
    storage = np.ascontiguousarray(storage)
    if rows is None:
        rows, vocab = storage.shape
        row_stride = vocab
    if row_stride is None:
        row_stride = vocab
    out = {"ids": np.zeros((rows, k), np.int32), "values": np.zeros((rows, k), np.float32),
           "chosen": np.zeros(rows, np.float32), "row_flags": np.zeros(rows, np.uint32),
           "lse": np.zeros(rows, np.float64)}
    a = LsoRankArgs()
    a.rows, a.vocab, a.dtype = rows, vocab, dtype
    a.row_stride, a.col_stride = row_stride, col_stride
    a.logits = _ptr(storage)
    a.k = k
    a.raw_values = 1 if raw_values else 0
    tok = None
    if tokens is not None:
        tok = np.ascontiguousarray(tokens, np.int32)
        a.tokens = _ptr(tok)
        a.chosen = _ptr(out["chosen"])
    a.values = _ptr(out["values"])
    a.ids = _ptr(out["ids"])
    a.row_flags = _ptr(out["row_flags"])
    a.lse = _ptr(out["lse"])
    st = lib().lso_rank(ctypes.byref(a))
    if st != 0:
        raise RuntimeError(f"lso_rank failed: {st}")
    if tokens is None:
        del out["chosen"]
    return out


class DenseRowState:
    """One CBv2 row's dense penalty state (LogitsPipelineV2.swift:238-256,
    357-384), built and advanced by the oracle."""

    def __init__(self, vocab, prompt, output, window_size, mode):
        self.V, self.W, self.mode = int(vocab), int(window_size), int(mode)
        p = np.ascontiguousarray(prompt, np.int32)
        o = np.ascontiguousarray(output, np.int32)
        self.counts = np.zeros(self.V, np.float32)
        self.window_counts = np.zeros(self.V, np.float32)
        self.window = np.zeros(self.W, np.int32)
        pos = c_int32(0)
        lib().lso_penalty_state_init(self.V, _ptr(p), p.size, _ptr(o), o.size, self.W,
                                     _ptr(self.counts), _ptr(self.window_counts),
                                     _ptr(self.window), ctypes.byref(pos))
        self.ring_pos = pos.value

    def commit(self, token):
        pos = c_int32(self.ring_pos)
        lib().lso_penalty_commit(self.V, self.mode, self.W, _ptr(self.counts),
                                 _ptr(self.window_counts), _ptr(self.window), ctypes.byref(pos),
                                 int(token))
        self.ring_pos = pos.value


def dexp(d):
    return lib().lso_dexp(float(d))


def weight(y, y_max, scale=1.0):
    return lib().lso_weight(float(y), float(y_max), float(scale))


def draw(y, keep, scale, u):
    y = np.ascontiguousarray(y, np.float32)
    keep = np.ascontiguousarray(keep, np.uint8)
    tot = c_uint64(0)
    t = lib().lso_draw(len(y), _ptr(y), _ptr(keep), float(scale), float(u), ctypes.byref(tot))
    return t, tot.value


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    o = np.zeros(4, np.uint32)
    lib().lso_philox4x32_10(_ptr(c), _ptr(k), _ptr(o))
    return o


def rng_key(seed, rid, step):
    return lib().lso_rng_key(seed, rid, step)


def rng_uniform(key, purpose=0):
    return lib().lso_rng_uniform(key, purpose)


# ------------------------------------------------------------- grammar masks
def device_mask_words(allowed, vocab):
    """deviceMask(allowed:vocab:) (TokenConstraintSamplerV2.swift:187-193) as
    packed LSB-first uint32 words: bit t of word t // 32 set exactly for the
    allowed ids; an id outside [0, vocab) leaves the whole row false."""
    words = np.zeros((vocab + 31) // 32, np.uint32)
    allowed = [int(t) for t in allowed]
    if all(0 <= t < vocab for t in allowed):
        for t in allowed:
            words[t >> 5] |= np.uint32(1 << (t & 31))
    return words


def assemble_masks(plan, pool, vocab):
    """The step's bitmask from a lsamp.constraint.MaskPlan (the device
    assembly's rule): an open row (-1) is all ones (open, :195-200); a build
    row first stores device_mask_words of its ids in its pool row; every other
    row copies its pool row.  Returns (out [rows, words], flags [rows]) and
    updates `pool` [pool_rows, words] in place."""
    words = (vocab + 31) // 32
    out = np.zeros((plan.rows, words), np.uint32)
    flags = np.zeros(plan.rows, np.uint32)
    for r in range(plan.rows):
        s = int(plan.row_source[r])
        if s < 0:
            out[r] = np.uint32(0xFFFFFFFF)
            continue
        if plan.row_build[r]:
            ids = plan.ids[plan.ids_ptr[r]:plan.ids_ptr[r + 1]]
            pool[s] = device_mask_words(ids, vocab)
            if any(t < 0 or t >= vocab for t in ids):
                flags[r] = _ffi.MASK_ID_RANGE
        out[r] = pool[s]
    return out, flags


def f32_to_bf16(x):
    """The oracle's round-to-nearest-even float32 -> bfloat16 bits (uint16)."""
    a = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(a.shape, np.uint16)
    lib().lso_f32_to_bf16_n(_ptr(a), _ptr(out), a.size)
    return out


def f32_to_f16(x):
    """The oracle's round-to-nearest-even float32 -> IEEE half bits (uint16)."""
    a = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(a.shape, np.uint16)
    lib().lso_f32_to_f16_n(_ptr(a), _ptr(out), a.size)
    return out


def f16_to_f32(h):
    """The oracle's IEEE half bits -> float32."""
    a = np.ascontiguousarray(h, np.uint16).reshape(-1)
    out = np.empty(a.shape, np.float32)
    lib().lso_f16_to_f32_n(_ptr(a), _ptr(out), a.size)
    return out
