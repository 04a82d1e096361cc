"""torch-facing wrapper of the C ABI (include/lsamp.h).

Device memory and streams come from torch; every computation runs in the HIP
kernels of liblsamp.so.  Nothing here falls back to a CPU path: a missing
library raises _ffi.LibraryMissing.
"""
from __future__ import annotations

import ctypes
from typing import Iterable, Optional, Sequence

import numpy as np
import torch

from . import _ffi

PENALTY_DTYPE = np.dtype([("token", "<i4"), ("count", "<i4"), ("flags", "<u4"), ("bias", "<f4")])
PARAMS_DTYPE = np.dtype([
    ("kind", "<i4"), ("temperature", "<f4"), ("top_k", "<i4"), ("top_p", "<f4"),
    ("min_p", "<f4"), ("repetition_penalty", "<f4"), ("presence_penalty", "<f4"),
    ("frequency_penalty", "<f4")])
STATS_DTYPE = np.dtype([
    ("max_value", "<f4"), ("log_normalizer", "<f4"), ("kept", "<i4"), ("token", "<i4"),
    ("kept_weight", "<u8"), ("probe_weight", "<u8"), ("cut_value", "<f4"),
    ("kept_mass", "<f4"), ("kept_entropy", "<f4"), ("probe_prob", "<f4")])

TORCH_DTYPE = {_ffi.DTYPE_F32: torch.float32, _ffi.DTYPE_BF16: torch.bfloat16,
               _ffi.DTYPE_F16: torch.float16}
LSAMP_DTYPE = {v: k for k, v in TORCH_DTYPE.items()}


def params_array(rows: Iterable) -> np.ndarray:
    """Per-row parameters (dicts, RowParams or a structured array) -> numpy
    structured array in the lsamp_row_params layout."""
    if isinstance(rows, np.ndarray) and rows.dtype == PARAMS_DTYPE:
        return rows
    rows = list(rows)
    out = np.zeros(len(rows), PARAMS_DTYPE)
    for i, p in enumerate(rows):
        if isinstance(p, _ffi.RowParams):
            p = {f: getattr(p, f) for f, _ in _ffi.RowParams._fields_}
        for k, v in p.items():
            out[i][k] = v
    return out


def to_device_bytes(arr: np.ndarray, device) -> torch.Tensor:
    """Host numpy array -> device uint8 tensor holding the same bytes."""
    a = np.ascontiguousarray(arr)
    t = torch.from_numpy(a.view(np.uint8).reshape(-1).copy())
    return t.to(device)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def current_stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class Context:
    """Owns the device workspace (lsamp_context) for up to `max_rows` rows of
    up to `max_vocab` logits on `device`."""

    def __init__(self, device: int = 0, max_rows: int = 512, max_vocab: int = 262144):
        self.lib = _ffi.load_library()
        h = ctypes.c_void_p()
        _ffi.check(self.lib.lsamp_context_create(device, max_rows, max_vocab, ctypes.byref(h)),
                   "lsamp_context_create")
        self.handle = h
        self.device = device
        self.max_rows = max_rows
        self.max_vocab = max_vocab

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.lsamp_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_mode(self, mode: int) -> None:
        """_ffi.MODE_AUTO / MODE_FUSED / MODE_SPLIT."""
        _ffi.check(self.lib.lsamp_context_set_mode(self.handle, mode), "lsamp_context_set_mode")

    def read_status(self) -> int:
        v = ctypes.c_uint32()
        _ffi.check(self.lib.lsamp_context_read_status(self.handle, ctypes.byref(v)),
                   "lsamp_context_read_status")
        return v.value

    def last_launch(self) -> dict:
        """Shape of the last lsamp_sample launch: fused, slices, slice_len,
        rows_per_round, grid."""
        li = _ffi.LaunchInfo()
        _ffi.check(self.lib.lsamp_context_last_launch(self.handle, ctypes.byref(li)),
                   "lsamp_context_last_launch")
        return {f: getattr(li, f) for f, _ in _ffi.LaunchInfo._fields_}

    # ----------------------------------------------------------------- timing
    def set_timing(self, enable: bool) -> None:
        _ffi.check(self.lib.lsamp_context_set_timing(self.handle, 1 if enable else 0),
                   "lsamp_context_set_timing")

    def read_timing(self):
        """(first-kernel ms, second-kernel ms, timed calls) since the last read;
        a fused step has one kernel and an empty second interval."""
        a, b, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
        _ffi.check(self.lib.lsamp_context_read_timing(self.handle, ctypes.byref(a), ctypes.byref(b),
                                                      ctypes.byref(n)), "lsamp_context_read_timing")
        return a.value, b.value, n.value

    # ----------------------------------------------------------------- sample
    def prepare_sample(self, logits: torch.Tensor, params, *, semantics: int, vocab: Optional[int] = None,
                       row_ptr=None, entries=None, bitmask=None, mask_bits: Optional[int] = None,
                       mask_tail: int = _ffi.MASK_TAIL_KEEP, uniforms=None, philox_keys=None,
                       probe_tokens=None, want_processed: bool = False, want_keep: bool = False,
                       want_stats: bool = False, table: Optional["PenaltyTable"] = None,
                       suppress_ids=None) -> "PreparedSample":
        """`table`: read the penalty entries from a device PenaltyTable
        (instead of row_ptr / entries).  `suppress_ids`: token ids masked to
        -inf in every row (SuppressTokensProcessor, SuppressTokens.swift:67-81)."""
        row_len = None
        if table is not None:
            row_ptr, entries, row_len = table.row_ptr, table.entries, table.row_len
        return PreparedSample(self, logits, params, semantics=semantics, vocab=vocab,
                              row_ptr=row_ptr, entries=entries, row_len=row_len, bitmask=bitmask,
                              mask_bits=mask_bits, mask_tail=mask_tail, uniforms=uniforms,
                              philox_keys=philox_keys, probe_tokens=probe_tokens,
                              want_processed=want_processed, want_keep=want_keep,
                              want_stats=want_stats, suppress_ids=suppress_ids)

    def sample(self, logits: torch.Tensor, params, **kw) -> dict:
        prep = self.prepare_sample(logits, params, **kw)
        prep.launch()
        return prep.outputs()

    # ----------------------------------------------------------------- verify
    def prepare_step(self, logits: torch.Tensor, params, *, table: Optional["PenaltyTable"] = None,
                     uniforms=None, philox_keys=None, logprobs_top_k: int = -1,
                     **sample_kw) -> "PreparedStep":
        """One decode step (lsamp_step; CBv2DefaultSampler.sample,
        DefaultSamplerV2.swift:84-181): draw, commit into `table`, and the
        raw log-probabilities of the drawn tokens and the top k."""
        return PreparedStep(self, logits, params, table=table, uniforms=uniforms,
                            philox_keys=philox_keys, logprobs_top_k=logprobs_top_k, **sample_kw)

    def step(self, logits: torch.Tensor, params, **kw) -> dict:
        prep = self.prepare_step(logits, params, **kw)
        prep.launch()
        return prep.outputs()

    def propose(self, logits: torch.Tensor, params, *, uniforms=None, philox_keys=None,
                stream: Optional[int] = None) -> torch.Tensor:
        """Coupled MTP proposal (lsamp_propose; mtpCoupledProposal,
        DefaultSamplerV2.swift:310-374): [rows, vocab] draft logits of one
        chain position, drawn with the uniforms the verifier will use there."""
        if logits.dim() != 2 or logits.stride(1) != 1:
            raise ValueError("logits must be a [rows, vocab] view with contiguous rows")
        rows, V = logits.shape
        dev = logits.device
        keep = [logits]
        pr = params if isinstance(params, torch.Tensor) else to_device_bytes(params_array(params), dev)
        keep.append(pr)
        a = _ffi.ProposeArgs()
        a.rows, a.vocab, a.dtype = rows, V, LSAMP_DTYPE[logits.dtype]
        a.row_stride = logits.stride(0) if rows > 1 else V
        a.logits, a.params = logits.data_ptr(), pr.data_ptr()
        if uniforms is not None:
            u = (uniforms.to(dev).contiguous() if isinstance(uniforms, torch.Tensor)
                 else torch.from_numpy(np.ascontiguousarray(uniforms, np.float32)).to(dev))
            keep.append(u)
            a.uniforms = u.data_ptr()
        if philox_keys is not None:
            k = torch.from_numpy(np.asarray(philox_keys, np.uint64).view(np.int64)).to(dev)
            keep.append(k)
            a.philox_keys = k.data_ptr()
        tokens = torch.empty(rows, dtype=torch.int32, device=dev)
        a.tokens = tokens.data_ptr()
        s = stream if stream is not None else current_stream_handle(dev)
        st = self.lib.lsamp_propose(self.handle, ctypes.byref(a), ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_propose")
        self._last_propose_keep = keep
        return tokens

    def mask_pool(self, masks) -> torch.Tensor:
        """The device pool [pool_rows, words] (int32 view of the uint32
        words) of a lsamp.constraint.ConstraintMasks."""
        return torch.zeros((masks.pool_rows, masks.words), dtype=torch.int32,
                           device=f"cuda:{self.device}")

    def assemble_masks(self, plan, pool: torch.Tensor, vocab: int, out: Optional[torch.Tensor] = None,
                       row_flags: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """lsamp_mask_assemble (CBv2TokenConstraintSampler.mask,
        TokenConstraintSamplerV2.swift:131-182): the step's [rows, words]
        bitmask for lsamp_sample from a lsamp.constraint.MaskPlan."""
        words = (vocab + 31) // 32
        rows = plan.rows
        if pool.dim() != 2 or pool.shape[1] != words or pool.dtype != torch.int32:
            raise ValueError(f"pool must be int32 [pool_rows, {words}]")
        if out is None:
            out = torch.empty((rows, words), dtype=torch.int32, device=pool.device)
        src = np.ascontiguousarray(plan.row_source, np.int32)
        build = np.ascontiguousarray(plan.row_build, np.uint8)
        ptr = np.ascontiguousarray(plan.ids_ptr, np.int32)
        ids = np.ascontiguousarray(plan.ids, np.int32)
        a = _ffi.MaskAssembleArgs()
        a.rows, a.vocab, a.words, a.pool_rows = rows, vocab, words, pool.shape[0]
        a.pool, a.out = pool.data_ptr(), out.data_ptr()
        a.row_flags = _ptr(row_flags)
        a.row_source, a.row_build = src.ctypes.data, build.ctypes.data
        a.ids_ptr = ptr.ctypes.data
        a.ids = ids.ctypes.data if len(ids) else None
        s = stream if stream is not None else current_stream_handle(pool.device)
        _ffi.check(self.lib.lsamp_mask_assemble(self.handle, ctypes.byref(a), s),
                   "lsamp_mask_assemble")
        return out

    def prepare_top2(self, logits: torch.Tensor) -> "PreparedRank":
        return PreparedRank(self, logits, top2=True)

    def top2(self, logits: torch.Tensor) -> dict:
        """cbv2TopTwoRows (CBv2TopTwo.swift:191): ids [rows, 2] int32 and values
        [rows, 2] float32 of a [rows, vocab] (or [1, rows, vocab]) view."""
        p = self.prepare_top2(logits)
        p.launch()
        return p.outputs()

    def penalize(self, logits: torch.Tensor, params, *, row_ptr=None, entries=None,
                 row_len=None, out_dtype: Optional[torch.dtype] = None,
                 stream: Optional[int] = None) -> torch.Tensor:
        """PenaltyProcessor.process (Evaluate.swift:687-693) on its own
        (lsamp_penalize): [rows, vocab] logits in, the penalized logits out,
        in the logits' dtype or (out_dtype=torch.float32, as a frequency
        penalty promotes them) in float32."""
        if logits.dim() != 2:
            raise ValueError("logits must be [rows, vocab]")
        rows, V = logits.shape
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        dev = logits.device
        out_dtype = logits.dtype if out_dtype is None else out_dtype
        out = torch.empty((rows, V), dtype=out_dtype, device=dev)
        pr = params if isinstance(params, torch.Tensor) else to_device_bytes(params_array(params), dev)
        a = _ffi.PenalizeArgs()
        a.rows, a.vocab, a.dtype = rows, V, LSAMP_DTYPE[logits.dtype]
        a.row_stride = logits.stride(0) if rows > 1 else V
        a.logits = logits.data_ptr()
        a.params = pr.data_ptr()
        keep = [pr]
        if entries is not None:
            rp = torch.from_numpy(np.ascontiguousarray(row_ptr, np.int32)).to(dev)
            en = to_device_bytes(np.ascontiguousarray(entries, PENALTY_DTYPE), dev) \
                if len(entries) else torch.zeros(16, dtype=torch.uint8, device=dev)
            a.penalty_row_ptr, a.penalty_entries = rp.data_ptr(), en.data_ptr()
            keep += [rp, en]
            if row_len is not None:
                rl = torch.from_numpy(np.ascontiguousarray(row_len, np.int32)).to(dev)
                a.penalty_row_len = rl.data_ptr()
                keep.append(rl)
        a.out_dtype = LSAMP_DTYPE[out_dtype]
        a.out = out.data_ptr()
        s = stream if stream is not None else current_stream_handle(dev)
        st = self.lib.lsamp_penalize(self.handle, ctypes.byref(a), ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_penalize")
        out._lsamp_keep = keep  # the inputs stay alive until the output is consumed
        return out

    def prepare_logprobs(self, logits: torch.Tensor, *, tokens=None, top_k: int = 0) -> "PreparedRank":
        return PreparedRank(self, logits, top2=False, tokens=tokens, top_k=top_k)

    def logprobs(self, logits: torch.Tensor, *, tokens=None, top_k: int = 0) -> dict:
        """Raw log-probabilities (LogitsPipelineV2.swift:307-314) gathered for
        `tokens` and the top_k best tokens (CBv2Logprobs.gather, :534-549)."""
        p = self.prepare_logprobs(logits, tokens=tokens, top_k=top_k)
        p.launch()
        return p.outputs()

    def prepare_verify(self, target: torch.Tensor, draft: Optional[torch.Tensor], draft_tokens,
                       params, uniforms, *, mode: int = _ffi.VERIFY_RESIDUAL,
                       typical_delta: float = 0.0, penalty_row_ptr=None, penalty_entries=None,
                       penalty_row_len=None, penalty_drafts=None, column_offset: int = 0,
                       scratch_cap: int = 0) -> "PreparedVerify":
        """Penalty-aware verification (EXACT / TYPICAL): `penalty_row_ptr` /
        `penalty_entries` (/ `penalty_row_len`) hold each sequence's confirmed
        output counts; `penalty_drafts` [S, >= column_offset + W - 1] is the
        round's draft chain (default: draft_tokens, offset 0); `scratch_cap`
        entries per window position (default: the longest run + drafts)."""
        return PreparedVerify(self, target, draft, draft_tokens, params, uniforms, mode,
                              typical_delta, penalty_row_ptr, penalty_entries, penalty_row_len,
                              penalty_drafts, column_offset, scratch_cap)

    def verify(self, target: torch.Tensor, draft: Optional[torch.Tensor], draft_tokens, params,
               uniforms, **kw) -> dict:
        """MTP verification (lsamp_verify): target [S, W, V], draft [S, W-1, V]
        (RESIDUAL mode), draft_tokens [S, W-1], CBv2-resolved params [S],
        uniforms [S, W].  Returns accepted [S], tokens [S, W], accept_mask
        [S, W-1] as device tensors."""
        prep = self.prepare_verify(target, draft, draft_tokens, params, uniforms, **kw)
        prep.launch()
        return prep.outputs()


class PreparedSample:
    """A fully bound lsamp_sample call: every input and output buffer is a
    device tensor kept alive by this object, so `launch()` is one C call (and
    can be captured in a HIP graph)."""

    def __init__(self, ctx: Context, logits: torch.Tensor, params, *, semantics, vocab, row_ptr,
                 entries, bitmask, mask_bits, mask_tail, uniforms, philox_keys, probe_tokens,
                 want_processed, want_keep, want_stats, row_len=None, suppress_ids=None):
        dev = logits.device
        if logits.dim() != 2:
            raise ValueError("logits must be [rows, row_stride]")
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        rows = logits.shape[0]
        V = int(vocab) if vocab is not None else logits.shape[1]
        self.ctx = ctx
        self.keep_alive = [logits]
        self.params_host = None
        if isinstance(params, torch.Tensor):
            self.params = params
        else:
            # the host copy lets the library choose the kernel arrangement
            self.params_host = np.ascontiguousarray(params_array(params))
            self.params = to_device_bytes(self.params_host, dev)
        self.keep_alive.append(self.params)
        a = _ffi.SampleArgs()
        a.semantics = semantics
        a.rows = rows
        a.vocab = V
        a.dtype = LSAMP_DTYPE[logits.dtype]
        # a size-1 row axis may carry any stride (numpy [None, :] gives 0)
        a.row_stride = logits.stride(0) if rows > 1 else logits.shape[1]
        a.logits = logits.data_ptr()
        a.params = self.params.data_ptr()
        if self.params_host is not None and len(self.params_host) == rows:
            a.params_host = self.params_host.ctypes.data

        def dev_tensor(x, np_dtype, torch_dtype):
            if x is None:
                return None
            if isinstance(x, torch.Tensor):
                return x.to(dev)
            return torch.from_numpy(np.ascontiguousarray(x, np_dtype)).to(dev)

        if row_ptr is not None:
            rp = dev_tensor(row_ptr, np.int32, torch.int32)
            if isinstance(entries, torch.Tensor):
                en = entries.to(dev)
            else:
                e = np.ascontiguousarray(entries, PENALTY_DTYPE)
                if len(e) == 0:
                    e = np.zeros(1, PENALTY_DTYPE)
                en = to_device_bytes(e, dev)
            self.keep_alive += [rp, en]
            a.penalty_row_ptr = rp.data_ptr()
            a.penalty_entries = en.data_ptr()
            if row_len is not None:
                rl = dev_tensor(row_len, np.int32, torch.int32)
                self.keep_alive.append(rl)
                a.penalty_row_len = rl.data_ptr()
        if bitmask is not None:
            bm = dev_tensor(bitmask, np.uint32, torch.int32)
            if bm.dtype != torch.int32:
                bm = bm.view(torch.int32) if bm.element_size() == 4 else bm.to(torch.int32)
            self.keep_alive.append(bm)
            a.bitmask = bm.data_ptr()
            a.mask_words = bm.shape[-1]
            a.mask_bits = int(mask_bits) if mask_bits is not None else a.mask_words * 32
            a.mask_tail = mask_tail
        if uniforms is not None:
            u = dev_tensor(uniforms, np.float32, torch.float32)
            self.keep_alive.append(u)
            a.uniforms = u.data_ptr()
        if philox_keys is not None:
            k = dev_tensor(np.asarray(philox_keys, np.uint64).view(np.int64), np.int64, torch.int64)
            self.keep_alive.append(k)
            a.philox_keys = k.data_ptr()
        if probe_tokens is not None:
            pt = dev_tensor(probe_tokens, np.int32, torch.int32)
            self.keep_alive.append(pt)
            a.probe_tokens = pt.data_ptr()
        if suppress_ids is not None and len(suppress_ids) > 0:
            si = dev_tensor(suppress_ids, np.int32, torch.int32)
            if si.dtype != torch.int32:
                si = si.to(torch.int32)
            self.keep_alive.append(si)
            a.suppress_ids = si.data_ptr()
            a.n_suppress = int(si.numel())
        self.tokens = torch.empty(rows, dtype=torch.int32, device=dev)
        self.row_flags = torch.empty(rows, dtype=torch.int32, device=dev)
        a.tokens = self.tokens.data_ptr()
        a.row_flags = self.row_flags.data_ptr()
        self.processed = torch.empty((rows, V), dtype=torch.float32, device=dev) if want_processed else None
        self.keep = torch.empty((rows, V), dtype=torch.uint8, device=dev) if want_keep else None
        self.stats = (torch.empty(rows * STATS_DTYPE.itemsize, dtype=torch.uint8, device=dev)
                      if want_stats else None)
        a.processed = _ptr(self.processed)
        a.keep = _ptr(self.keep)
        a.stats = _ptr(self.stats)
        self.args = a
        self._byref = ctypes.byref(a)

    def launch(self, stream: Optional[int] = None) -> None:
        s = stream if stream is not None else current_stream_handle(self.tokens.device)
        st = self.ctx.lib.lsamp_sample(self.ctx.handle, self._byref, ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_sample")

    def outputs(self) -> dict:
        out = {"tokens": self.tokens, "row_flags": self.row_flags}
        if self.processed is not None:
            out["processed"] = self.processed
        if self.keep is not None:
            out["keep"] = self.keep
        if self.stats is not None:
            out["stats"] = self.stats
        return out

    def stats_numpy(self) -> np.ndarray:
        return self.stats.cpu().numpy().view(STATS_DTYPE)


class PreparedVerify:
    """A fully bound lsamp_verify call (device buffers kept alive here)."""

    def __init__(self, ctx: Context, target, draft, draft_tokens, params, uniforms, mode,
                 typical_delta, penalty_row_ptr=None, penalty_entries=None, penalty_row_len=None,
                 penalty_drafts=None, column_offset=0, scratch_cap=0):
        if target.dim() != 3 or not target.is_contiguous():
            raise ValueError("target must be a contiguous [S, W, V] tensor")
        S, W, V = target.shape
        dev = target.device
        self.ctx = ctx
        self.keep_alive = [target]
        a = _ffi.VerifyArgs()
        a.mode = mode
        a.sequences, a.window, a.vocab = S, W, V
        a.dtype = LSAMP_DTYPE[target.dtype]
        a.target_logits = target.data_ptr()
        if draft is not None:
            if tuple(draft.shape) != (S, W - 1, V) or not draft.is_contiguous():
                raise ValueError("draft must be a contiguous [S, W-1, V] tensor")
            if draft.dtype != target.dtype:
                raise ValueError("draft and target must share a dtype")
            self.keep_alive.append(draft)
            a.draft_logits = draft.data_ptr()

        def dev_tensor(x, np_dtype):
            if isinstance(x, torch.Tensor):
                return x.to(dev).contiguous()
            return torch.from_numpy(np.ascontiguousarray(x, np_dtype)).to(dev)

        dt = dev_tensor(draft_tokens, np.int32)
        u = dev_tensor(uniforms, np.float32)
        pr = params if isinstance(params, torch.Tensor) else to_device_bytes(params_array(params), dev)
        self.keep_alive += [dt, u, pr]
        a.draft_tokens = dt.data_ptr()
        a.uniforms = u.data_ptr()
        a.params = pr.data_ptr()
        a.typical_delta = typical_delta
        self.accepted = torch.empty(S, dtype=torch.int32, device=dev)
        self.tokens = torch.empty((S, W), dtype=torch.int32, device=dev)
        self.accept_mask = torch.empty((S, W - 1), dtype=torch.uint8, device=dev)
        a.accepted = self.accepted.data_ptr()
        a.tokens = self.tokens.data_ptr()
        a.accept_mask = self.accept_mask.data_ptr()
        if penalty_entries is not None:
            rp = dev_tensor(penalty_row_ptr, np.int32)
            if isinstance(penalty_entries, torch.Tensor):
                en = penalty_entries.to(dev)
                n_max = None
            else:
                e = np.ascontiguousarray(penalty_entries, PENALTY_DTYPE)
                rpn = np.asarray(penalty_row_ptr, np.int64)
                n_max = int((rpn[1:S + 1] - rpn[:S]).max()) if S else 0
                en = to_device_bytes(e if len(e) else np.zeros(1, PENALTY_DTYPE), dev)
            self.keep_alive += [rp, en]
            a.penalty_row_ptr = rp.data_ptr()
            a.penalty_entries = en.data_ptr()
            if penalty_row_len is not None:
                rl = dev_tensor(penalty_row_len, np.int32)
                self.keep_alive.append(rl)
                a.penalty_row_len = rl.data_ptr()
            if penalty_drafts is not None:
                pd = dev_tensor(penalty_drafts, np.int32)
                self.keep_alive.append(pd)
                a.penalty_drafts = pd.data_ptr()
                a.penalty_drafts_stride = pd.shape[-1]
                a.penalty_column_offset = int(column_offset)
            if n_max is None and not scratch_cap:
                raise ValueError("device penalty_entries need an explicit scratch_cap")
            cap = int(scratch_cap) or (n_max + int(column_offset) + W)
            self.scratch = torch.empty(S * W * cap * 16, dtype=torch.uint8, device=dev)
            a.penalty_scratch = self.scratch.data_ptr()
            a.penalty_scratch_cap = cap
        self.args = a
        self._byref = ctypes.byref(a)

    def launch(self, stream: Optional[int] = None) -> None:
        s = stream if stream is not None else current_stream_handle(self.tokens.device)
        st = self.ctx.lib.lsamp_verify(self.ctx.handle, self._byref, ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_verify")

    def outputs(self) -> dict:
        return {"accepted": self.accepted, "tokens": self.tokens, "accept_mask": self.accept_mask}


class PreparedStep:
    """A fully bound lsamp_step call (draw -> commit -> log-probabilities)."""

    def __init__(self, ctx: Context, logits, params, *, table, uniforms, philox_keys,
                 logprobs_top_k, draw_from_table: bool = True, **sample_kw):
        """`draw_from_table` False: the draw reads the penalty entries given
        in `sample_kw` (row_ptr / entries) and only the commit goes to `table`."""
        self.ctx = ctx
        self.sample = ctx.prepare_sample(logits, params, semantics=_ffi.SEM_CBV2,
                                         table=table if draw_from_table else None,
                                         uniforms=uniforms, philox_keys=philox_keys, **sample_kw)
        rows = logits.shape[0]
        dev = logits.device
        a = _ffi.StepArgs()
        a.sample = self.sample.args
        self.table = table
        if table is not None:
            a.table = ctypes.addressof(table._table)
            a.commit_flags = table.row_flags.data_ptr()
        a.logprobs_top_k = int(logprobs_top_k)
        self.chosen = self.top_values = self.top_ids = None
        if logprobs_top_k >= 0:
            k = int(logprobs_top_k)
            self.chosen = torch.empty(rows, dtype=torch.float32, device=dev)
            self.top_values = torch.empty((rows, k), dtype=torch.float32, device=dev)
            self.top_ids = torch.empty((rows, k), dtype=torch.int32, device=dev)
            a.chosen_logprob = self.chosen.data_ptr()
            a.top_logprobs = self.top_values.data_ptr() if k else None
            a.top_ids = self.top_ids.data_ptr() if k else None
        self.args = a
        self._byref = ctypes.byref(a)

    def launch(self, stream: Optional[int] = None) -> None:
        s = stream if stream is not None else current_stream_handle(self.sample.tokens.device)
        st = self.ctx.lib.lsamp_step(self.ctx.handle, self._byref, ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_step")

    def outputs(self) -> dict:
        out = self.sample.outputs()
        if self.table is not None:
            out["commit_flags"] = self.table.row_flags
        if self.chosen is not None:
            out.update(chosen=self.chosen, top_values=self.top_values, top_ids=self.top_ids)
        return out


class PenaltyTable:
    """Device-resident CBv2 penalty state (the lsamp_penalty_table of
    include/lsamp.h): per row a run of entries {token, output count,
    REPETITION while in the window, bias}, each entry's count in the window,
    and the repetition ring.  Built once from host histories
    (history.Cbv2RowState), advanced on the device by `commit` after each
    draw, and read by `Context.sample(..., table=...)`."""

    def __init__(self, states, *, capacity: int, window_capacity: int, device="cuda"):
        rows = len(states)
        cap, wcap = int(capacity), int(window_capacity)
        ent = np.zeros((rows, cap), PENALTY_DTYPE)
        wcnt = np.zeros((rows, cap), np.int32)
        win = np.full((rows, wcap), -1, np.int32)
        row_len = np.zeros(rows, np.int32)
        ring = np.zeros(rows, np.int32)
        wsize = np.ones(rows, np.int32)
        mode = np.zeros(rows, np.int32)
        for r, st in enumerate(states):
            e = st.entries()
            if len(e) > cap:
                raise ValueError(f"row {r}: {len(e)} entries exceed capacity {cap}")
            if st.W > wcap:
                raise ValueError(f"row {r}: window {st.W} exceeds window_capacity {wcap}")
            ent[r, :len(e)] = e
            row_len[r] = len(e)
            if st.repetition_on:
                in_win = [t for t in st.window if t >= 0]
                for j, t in enumerate(e["token"]):
                    wcnt[r, j] = in_win.count(int(t))
                win[r, :st.W] = st.window
            ring[r] = st.ring_pos
            wsize[r] = st.W
            mode[r] = (_ffi.STATE_COUNTS if st.counts_on else 0) | (
                _ffi.STATE_REPETITION if st.repetition_on else 0)
        t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)
        self.rows, self.capacity, self.window_capacity = rows, cap, wcap
        self.entries = to_device_bytes(ent.reshape(-1), device)
        self.window_count = t(wcnt)
        self.window = t(win)
        self.row_len = t(row_len)
        self.ring_pos = t(ring)
        self.window_size = t(wsize)
        self.mode = t(mode)
        self.row_ptr = t(np.arange(rows + 1, dtype=np.int32) * cap)
        tb = _ffi.PenaltyTable()
        tb.rows, tb.capacity, tb.window_capacity = rows, cap, wcap
        tb.entries = self.entries.data_ptr()
        tb.row_len = self.row_len.data_ptr()
        tb.window_count = self.window_count.data_ptr()
        tb.window = self.window.data_ptr()
        tb.ring_pos = self.ring_pos.data_ptr()
        tb.window_size = self.window_size.data_ptr()
        tb.mode = self.mode.data_ptr()
        self._table = tb
        self.row_flags = torch.zeros(rows, dtype=torch.int32, device=device)

    def commit(self, ctx: Context, tokens: torch.Tensor, vocab: int,
               stream: Optional[int] = None) -> torch.Tensor:
        """LogitsPipelineV2.commit for every row (lsamp_commit); returns the
        per-row flags (LSAMP_ROW_OVERFLOW)."""
        if tokens.dtype != torch.int32 or tokens.numel() != self.rows:
            raise ValueError("tokens must be an int32 tensor with one id per row")
        a = _ffi.CommitArgs()
        a.table = self._table
        a.vocab = int(vocab)
        a.tokens = tokens.data_ptr()
        a.row_flags = self.row_flags.data_ptr()
        s = stream if stream is not None else current_stream_handle(tokens.device)
        st = ctx.lib.lsamp_commit(ctx.handle, ctypes.byref(a), ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_commit")
        return self.row_flags

    def host_rows(self):
        """Per row: (entries sorted by token, window count by token, window,
        ring position)."""
        ent = self.entries.cpu().numpy().view(PENALTY_DTYPE).reshape(self.rows, self.capacity)
        wcnt = self.window_count.cpu().numpy()
        win = self.window.cpu().numpy()
        n = self.row_len.cpu().numpy()
        ring = self.ring_pos.cpu().numpy()
        out = []
        for r in range(self.rows):
            e = ent[r, :n[r]]
            order = np.argsort(e["token"], kind="stable")
            wc = {int(e["token"][j]): int(wcnt[r, j]) for j in range(n[r])}
            out.append((e[order], wc, win[r], int(ring[r])))
        return out


class PreparedRank:
    """A fully bound lsamp_top2 / lsamp_logprobs call over a 2-D view of
    logits with any strides (a [1, rows, vocab] view is taken as its rows)."""

    def __init__(self, ctx: Context, logits: torch.Tensor, *, top2: bool, tokens=None,
                 top_k: int = 0):
        if logits.dim() == 3 and logits.shape[0] == 1:
            logits = logits[0]
        if logits.dim() != 2:
            raise ValueError("logits must be [rows, vocab] or [1, rows, vocab]")
        rows, V = logits.shape
        dev = logits.device
        self.ctx = ctx
        self.top2 = top2
        self.keep_alive = [logits]
        dt = LSAMP_DTYPE[logits.dtype]
        rs, cs = logits.stride()
        if top2:
            a = _ffi.Top2Args()
            self.ids = torch.empty((rows, 2), dtype=torch.int32, device=dev)
            self.values = torch.empty((rows, 2), dtype=torch.float32, device=dev)
            a.ids, a.values = self.ids.data_ptr(), self.values.data_ptr()
        else:
            a = _ffi.LogprobsArgs()
            a.top_k = top_k
            self.ids = torch.empty((rows, top_k), dtype=torch.int32, device=dev)
            self.values = torch.empty((rows, top_k), dtype=torch.float32, device=dev)
            self.row_flags = torch.empty(rows, dtype=torch.int32, device=dev)
            a.top_ids = self.ids.data_ptr() if top_k > 0 else None
            a.top_values = self.values.data_ptr() if top_k > 0 else None
            a.row_flags = self.row_flags.data_ptr()
            self.chosen = None
            if tokens is not None:
                t = (tokens.to(dev, torch.int32).contiguous() if isinstance(tokens, torch.Tensor)
                     else torch.from_numpy(np.ascontiguousarray(tokens, np.int32)).to(dev))
                self.keep_alive.append(t)
                self.chosen = torch.empty(rows, dtype=torch.float32, device=dev)
                a.tokens, a.chosen = t.data_ptr(), self.chosen.data_ptr()
        a.rows, a.vocab, a.dtype = rows, V, dt
        a.row_stride, a.col_stride = rs, cs
        a.logits = logits.data_ptr()
        self.args = a
        self._byref = ctypes.byref(a)

    def launch(self, stream: Optional[int] = None) -> None:
        s = stream if stream is not None else current_stream_handle(self.ids.device)
        fn = self.ctx.lib.lsamp_top2 if self.top2 else self.ctx.lib.lsamp_logprobs
        st = fn(self.ctx.handle, self._byref, ctypes.c_void_p(s))
        if st != 0:
            raise _ffi.LsampError(st, "lsamp_top2" if self.top2 else "lsamp_logprobs")

    def outputs(self) -> dict:
        if self.top2:
            return {"ids": self.ids, "values": self.values}
        out = {"top_ids": self.ids, "top_values": self.values, "row_flags": self.row_flags}
        if self.chosen is not None:
            out["chosen"] = self.chosen
        return out


def stats_to_numpy(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(STATS_DTYPE)
