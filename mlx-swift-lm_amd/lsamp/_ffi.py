"""ctypes mirror of include/lsamp.h and the loader of liblsamp.so.

The structures below are field-for-field copies of the C declarations in
include/lsamp.h; `tests/test_abi_layout.py` checks their sizes against the
compiled library's own `sizeof` report so the two cannot drift apart.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int32,
                    c_int64, c_uint8, c_uint32, c_uint64, c_void_p)

PACKAGE_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PACKAGE_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "liblsamp.so")

# ---- constants (include/lsamp.h) ---------------------------------------------
LSAMP_OK = 0
LSAMP_ERR_INVALID_ARGUMENT = -1
LSAMP_ERR_SHAPE = -2
LSAMP_ERR_DTYPE = -3
LSAMP_ERR_CAPACITY = -4
LSAMP_ERR_DEVICE = -5

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
SEM_MLXLM, SEM_CBV2 = 0, 1
KIND_ARGMAX, KIND_FILTERED, KIND_CATEGORICAL = 0, 1, 2
MASK_TAIL_KEEP, MASK_TAIL_FORBID = 0, 1
PEN_REPETITION, PEN_PRESENCE = 1, 2
ROW_NONFINITE, ROW_EMPTY, ROW_OVERFLOW, ROW_TOKEN_RANGE, ROW_TIMEOUT = 1, 2, 4, 8, 16
STATUS_SPIN_TIMEOUT = 1
MAX_SUPPRESS = 65536
RANK_MAX_K = 32
VERIFY_RESIDUAL, VERIFY_EXACT, VERIFY_TYPICAL = 0, 1, 2
MODE_AUTO, MODE_FUSED, MODE_SPLIT = 0, 1, 2
STATE_COUNTS, STATE_REPETITION = 1, 2
STATUS_SPIN_TIMEOUT = 1
STATUS_PENALTY_CAPACITY = 2
MASK_ID_RANGE = 1
MASK_MAX_WORDS = 16000


class RowParams(Structure):
    _fields_ = [
        ("kind", c_int32),
        ("temperature", c_float),
        ("top_k", c_int32),
        ("top_p", c_float),
        ("min_p", c_float),
        ("repetition_penalty", c_float),
        ("presence_penalty", c_float),
        ("frequency_penalty", c_float),
    ]


class PenaltyEntry(Structure):
    _fields_ = [
        ("token", c_int32),
        ("count", c_int32),
        ("flags", c_uint32),
        ("bias", c_float),
    ]


class RowStats(Structure):
    _fields_ = [
        ("max_value", c_float),
        ("log_normalizer", c_float),
        ("kept", c_int32),
        ("token", c_int32),
        ("kept_weight", c_uint64),
        ("probe_weight", c_uint64),
        ("cut_value", c_float),
        ("kept_mass", c_float),
        ("kept_entropy", c_float),
        ("probe_prob", c_float),
    ]


class SampleArgs(Structure):
    _fields_ = [
        ("semantics", c_int32),
        ("rows", c_int32),
        ("vocab", c_int32),
        ("dtype", c_int32),
        ("row_stride", c_int64),
        ("logits", c_void_p),
        ("params", c_void_p),
        ("penalty_row_ptr", c_void_p),
        ("penalty_entries", c_void_p),
        ("bitmask", c_void_p),
        ("mask_words", c_int32),
        ("mask_bits", c_int32),
        ("mask_tail", c_int32),
        ("uniforms", c_void_p),
        ("philox_keys", c_void_p),
        ("probe_tokens", c_void_p),
        ("tokens", c_void_p),
        ("row_flags", c_void_p),
        ("processed", c_void_p),
        ("keep", c_void_p),
        ("stats", c_void_p),
        ("penalty_row_len", c_void_p),
        ("suppress_ids", c_void_p),
        ("n_suppress", c_int32),
        ("params_host", c_void_p),
    ]


class PenaltyTable(Structure):
    _fields_ = [
        ("rows", c_int32),
        ("capacity", c_int32),
        ("window_capacity", c_int32),
        ("entries", c_void_p),
        ("row_len", c_void_p),
        ("window_count", c_void_p),
        ("window", c_void_p),
        ("ring_pos", c_void_p),
        ("window_size", c_void_p),
        ("mode", c_void_p),
    ]


class CommitArgs(Structure):
    _fields_ = [
        ("table", PenaltyTable),
        ("vocab", c_int32),
        ("tokens", c_void_p),
        ("row_flags", c_void_p),
    ]


class PenalizeArgs(Structure):
    _fields_ = [
        ("rows", c_int32),
        ("vocab", c_int32),
        ("dtype", c_int32),
        ("row_stride", c_int64),
        ("logits", c_void_p),
        ("params", c_void_p),
        ("penalty_row_ptr", c_void_p),
        ("penalty_row_len", c_void_p),
        ("penalty_entries", c_void_p),
        ("out_dtype", c_int32),
        ("out", c_void_p),
    ]


class MaskAssembleArgs(Structure):
    _fields_ = [
        ("rows", c_int32),
        ("vocab", c_int32),
        ("words", c_int32),
        ("pool_rows", c_int32),
        ("pool", c_void_p),
        ("out", c_void_p),
        ("row_flags", c_void_p),
        ("row_source", c_void_p),
        ("row_build", c_void_p),
        ("ids_ptr", c_void_p),
        ("ids", c_void_p),
    ]


class VerifyArgs(Structure):
    _fields_ = [
        ("mode", c_int32),
        ("sequences", c_int32),
        ("window", c_int32),
        ("vocab", c_int32),
        ("dtype", c_int32),
        ("target_logits", c_void_p),
        ("draft_logits", c_void_p),
        ("draft_tokens", c_void_p),
        ("params", c_void_p),
        ("uniforms", c_void_p),
        ("typical_delta", c_float),
        ("accepted", c_void_p),
        ("tokens", c_void_p),
        ("accept_mask", c_void_p),
        ("penalty_row_ptr", c_void_p),
        ("penalty_row_len", c_void_p),
        ("penalty_entries", c_void_p),
        ("penalty_drafts", c_void_p),
        ("penalty_drafts_stride", c_int32),
        ("penalty_column_offset", c_int32),
        ("penalty_scratch", c_void_p),
        ("penalty_scratch_cap", c_int32),
    ]


class GenerateParameters(Structure):
    """lsamp_generate_parameters: the sampler/processor-driving subset of the
    reference's GenerateParameters (Evaluate.swift:127-289)."""
    _fields_ = [
        ("temperature", c_float),
        ("top_p", c_float),
        ("top_k", c_int32),
        ("min_p", c_float),
        ("has_repetition_penalty", c_int32),
        ("repetition_penalty", c_float),
        ("repetition_context_size", c_int32),
        ("has_presence_penalty", c_int32),
        ("presence_penalty", c_float),
        ("presence_context_size", c_int32),
        ("has_frequency_penalty", c_int32),
        ("frequency_penalty", c_float),
        ("frequency_context_size", c_int32),
    ]


class Cbv2Params(Structure):
    """lsamp_cbv2_params: CBv2SamplingParams subset (CBv2Contracts.swift:37-75)."""
    _fields_ = [
        ("temperature", c_float),
        ("top_p", c_float),
        ("top_k", c_int32),
        ("min_p", c_float),
        ("repetition_penalty", c_float),
        ("repetition_context_size", c_int32),
        ("frequency_penalty", c_float),
        ("presence_penalty", c_float),
    ]


_lib = None


class LaunchInfo(Structure):
    _fields_ = [("fused", c_int32), ("slices", c_int32), ("slice_len", c_int32),
                ("rows_per_round", c_int32), ("grid", c_int32)]


class StepArgs(Structure):
    _fields_ = [
        ("sample", SampleArgs),
        ("table", c_void_p),
        ("commit_flags", c_void_p),
        ("logprobs_top_k", c_int32),
        ("chosen_logprob", c_void_p),
        ("top_logprobs", c_void_p),
        ("top_ids", c_void_p),
    ]


class ProposeArgs(Structure):
    _fields_ = [
        ("rows", c_int32),
        ("vocab", c_int32),
        ("dtype", c_int32),
        ("row_stride", c_int64),
        ("logits", c_void_p),
        ("params", c_void_p),
        ("uniforms", c_void_p),
        ("philox_keys", c_void_p),
        ("tokens", c_void_p),
    ]


class Top2Args(Structure):
    _fields_ = [
        ("rows", c_int32),
        ("vocab", c_int32),
        ("dtype", c_int32),
        ("row_stride", c_int64),
        ("col_stride", c_int64),
        ("logits", c_void_p),
        ("ids", c_void_p),
        ("values", c_void_p),
    ]


class LogprobsArgs(Structure):
    _fields_ = [
        ("rows", c_int32),
        ("vocab", c_int32),
        ("dtype", c_int32),
        ("row_stride", c_int64),
        ("col_stride", c_int64),
        ("logits", c_void_p),
        ("top_k", c_int32),
        ("tokens", c_void_p),
        ("chosen", c_void_p),
        ("top_values", c_void_p),
        ("top_ids", c_void_p),
        ("row_flags", c_void_p),
    ]


class LibraryMissing(RuntimeError):
    pass


def load_library(path: str | None = None):
    """Load liblsamp.so.  Raises LibraryMissing if it has not been built:
    there is no fallback implementation of the kernels."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise LibraryMissing(
            f"{p} is missing: build it with `python __graft_entry__.py build` "
            "(hipcc --offload-arch=gfx950)")
    lib = ctypes.CDLL(p)
    lib.lsamp_context_create.argtypes = [c_int32, c_int32, c_int32, POINTER(c_void_p)]
    lib.lsamp_context_create.restype = c_int32
    lib.lsamp_context_destroy.argtypes = [c_void_p]
    lib.lsamp_context_destroy.restype = None
    lib.lsamp_sample.argtypes = [c_void_p, POINTER(SampleArgs), c_void_p]
    lib.lsamp_sample.restype = c_int32
    lib.lsamp_context_set_mode.argtypes = [c_void_p, c_int32]
    lib.lsamp_context_set_mode.restype = c_int32
    lib.lsamp_context_read_status.argtypes = [c_void_p, POINTER(c_uint32)]
    lib.lsamp_context_read_status.restype = c_int32
    lib.lsamp_sample_noalloc.argtypes = [POINTER(SampleArgs), c_void_p]
    lib.lsamp_sample_noalloc.restype = c_int32
    lib.lsamp_test_set_spin_limit.argtypes = [c_int32, c_int32]
    lib.lsamp_test_set_spin_limit.restype = c_int32
    lib.lsamp_context_last_launch.argtypes = [c_void_p, POINTER(LaunchInfo)]
    lib.lsamp_context_last_launch.restype = c_int32
    lib.lsamp_context_set_timing.argtypes = [c_void_p, c_int32]
    lib.lsamp_context_set_timing.restype = c_int32
    lib.lsamp_context_read_timing.argtypes = [c_void_p, POINTER(c_double), POINTER(c_double),
                                              POINTER(c_int64)]
    lib.lsamp_context_read_timing.restype = c_int32
    lib.lsamp_verify.argtypes = [c_void_p, POINTER(VerifyArgs), c_void_p]
    lib.lsamp_verify.restype = c_int32
    lib.lsamp_step.argtypes = [c_void_p, POINTER(StepArgs), c_void_p]
    lib.lsamp_step.restype = c_int32
    lib.lsamp_propose.argtypes = [c_void_p, POINTER(ProposeArgs), c_void_p]
    lib.lsamp_propose.restype = c_int32
    lib.lsamp_commit.argtypes = [c_void_p, POINTER(CommitArgs), c_void_p]
    lib.lsamp_commit.restype = c_int32
    lib.lsamp_penalize.argtypes = [c_void_p, POINTER(PenalizeArgs), c_void_p]
    lib.lsamp_penalize.restype = c_int32
    lib.lsamp_mask_assemble.argtypes = [c_void_p, POINTER(MaskAssembleArgs), c_void_p]
    lib.lsamp_mask_assemble.restype = c_int32
    lib.lsamp_top2.argtypes = [c_void_p, POINTER(Top2Args), c_void_p]
    lib.lsamp_top2.restype = c_int32
    lib.lsamp_logprobs.argtypes = [c_void_p, POINTER(LogprobsArgs), c_void_p]
    lib.lsamp_logprobs.restype = c_int32
    lib.lsamp_resolve_generate_parameters.argtypes = [
        POINTER(GenerateParameters), POINTER(RowParams), POINTER(c_int32)]
    lib.lsamp_resolve_generate_parameters.restype = c_int32
    lib.lsamp_resolve_cbv2_params.argtypes = [POINTER(Cbv2Params), c_int32, POINTER(RowParams)]
    lib.lsamp_resolve_cbv2_params.restype = c_int32
    lib.lsamp_rng_key.argtypes = [c_uint64, c_uint64, c_uint64]
    lib.lsamp_rng_key.restype = c_uint64
    lib.lsamp_rng_uniform.argtypes = [c_uint64, c_uint32]
    lib.lsamp_rng_uniform.restype = c_float
    lib.lsamp_last_error.argtypes = []
    lib.lsamp_last_error.restype = c_char_p
    lib.lsamp_version.argtypes = []
    lib.lsamp_version.restype = c_char_p
    lib.lsamp_abi_sizeof.argtypes = [c_char_p]
    lib.lsamp_abi_sizeof.restype = c_int64
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    lib = load_library()
    s = lib.lsamp_last_error()
    return s.decode() if s else ""


class LsampError(RuntimeError):
    def __init__(self, status: int, where: str):
        super().__init__(f"{where} failed with status {status}: {last_error()}")
        self.status = status


def check(status: int, where: str) -> None:
    if status != LSAMP_OK:
        raise LsampError(status, where)
