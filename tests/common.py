"""Shared helpers of the test suite: run one configuration through the HIP
library and through the oracle, and compare them under the parity rules:

* processed (filter-space) logits: equal values (fp32 bit patterns up to the
  sign of zero);
* keep sets: identical, except tokens whose top-p test sits within 1e-6 of
  cumulative mass of the boundary (the exclusive mass in exact arithmetic,
  which the oracle decides on), or whose min-p test sits within 1e-6 of its
  threshold (probability units in CBv2, log-probability units in mlx-lm).
  MLX's softmax / cumsum reduction order is not vendored, so these
  boundary positions are the ones no restatement can pin;
* drawn tokens: identical whenever the keep sets are identical (the
  fixed-point inverse-CDF draw is reproduced exactly by the oracle);
* row flags: identical.
"""
from __future__ import annotations

import numpy as np

import oracle as O
from lsamp import _ffi

TOP_P_TOL = 1e-6
MIN_P_TOL = 1e-6  # probability units (CBv2) / log units (mlx-lm)


def run_oracle(cfg, threads=8, uniforms=None, probe_tokens=None, philox_keys=None):
    """The oracle on cfg; with `philox_keys` it draws each row's uniform from
    its key (lso_rng_uniform) instead of cfg["uniforms"]."""
    if philox_keys is None and uniforms is None:
        uniforms = cfg["uniforms"]
    return O.sample(semantics=cfg["semantics"], logits=cfg["logits"], dtype=cfg["dtype"],
                    params=cfg["params"], row_ptr=cfg.get("row_ptr"), entries=cfg.get("entries"),
                    bitmask=cfg.get("bitmask"), mask_bits=cfg.get("mask_bits", 0),
                    mask_tail=cfg.get("mask_tail", 0),
                    uniforms=uniforms, philox_keys=philox_keys,
                    probe_tokens=probe_tokens, threads=threads, want_processed=True,
                    want_keep=True, want_margins=True, want_stats=True,
                    vocab=cfg.get("vocab"), row_stride=cfg.get("row_stride"),
                    suppress_ids=cfg.get("suppress_ids"))


def to_torch_logits(cfg, device="cuda"):
    import torch
    x = cfg["logits"]
    if cfg["dtype"] == _ffi.DTYPE_F32:
        t = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    elif cfg["dtype"] == _ffi.DTYPE_BF16:
        t = torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.int16)).view(torch.bfloat16)
    else:
        t = torch.from_numpy(np.ascontiguousarray(x, np.uint16).view(np.int16)).view(torch.float16)
    return t.to(device)


def run_gpu(ctx, cfg, uniforms=None, philox_keys=None, probe_tokens=None, logits_t=None):
    import torch
    from lsamp.api import stats_to_numpy
    lt = to_torch_logits(cfg) if logits_t is None else logits_t
    u = cfg["uniforms"] if (uniforms is None and philox_keys is None) else uniforms
    out = ctx.sample(lt, cfg["params"], semantics=cfg["semantics"], vocab=cfg.get("vocab"),
                     row_ptr=cfg.get("row_ptr"), entries=cfg.get("entries"),
                     bitmask=cfg.get("bitmask"), mask_bits=cfg.get("mask_bits"),
                     mask_tail=cfg.get("mask_tail", 0), uniforms=u, philox_keys=philox_keys,
                     probe_tokens=probe_tokens, want_processed=True, want_keep=True,
                     want_stats=True, suppress_ids=cfg.get("suppress_ids"))
    torch.cuda.synchronize()
    return {"tokens": out["tokens"].cpu().numpy(), "row_flags": out["row_flags"].cpu().numpy().astype(np.uint32),
            "processed": out["processed"].cpu().numpy(), "keep": out["keep"].cpu().numpy(),
            "stats": stats_to_numpy(out["stats"])}


def compare(cfg, gpu, ora, *, label="", uniforms=None):
    """Assert parity; return the list of rows that differ only at a documented
    boundary (their tokens are allowed to differ)."""
    rows = len(ora["tokens"])
    assert np.array_equal(gpu["row_flags"], ora["row_flags"]), \
        f"{label} row flags differ: gpu {gpu['row_flags']} oracle {ora['row_flags']}"
    gp, op = gpu["processed"], ora["processed"]
    bad = ~((gp == op) | (np.isnan(gp) & np.isnan(op)))
    if bad.any():
        r, i = np.argwhere(bad)[0]
        raise AssertionError(f"{label} processed logits differ at row {r} token {i}: "
                             f"gpu {gp[r, i]!r} oracle {op[r, i]!r} ({int(bad.sum())} tokens)")
    boundary_rows = []
    for r in range(rows):
        if ora["row_flags"][r] & (_ffi.ROW_EMPTY | _ffi.ROW_OVERFLOW):
            assert gpu["tokens"][r] == -1, f"{label} row {r}: empty row must give -1"
            continue
        gk, ok = gpu["keep"][r].astype(bool), ora["keep"][r].astype(bool)
        if np.array_equal(gk, ok):
            assert gpu["tokens"][r] == ora["tokens"][r], (
                f"{label} row {r}: same keep set ({int(ok.sum())} tokens) but token "
                f"gpu {gpu['tokens'][r]} != oracle {ora['tokens'][r]}")
            assert gpu["stats"]["kept_weight"][r] == ora["stats"]["kept_weight"][r], \
                f"{label} row {r}: kept weight differs"
            continue
        diff = np.nonzero(gk != ok)[0]
        tpx = ora["top_p_margin_exact"][r, diff]
        mpm = ora["min_p_margin"][r, diff]
        # within 1e-6 of cumulative mass of the top-p boundary (exact
        # arithmetic), or within 1e-6 of the min-p threshold
        near_p = np.abs(tpx) <= TOP_P_TOL
        near_m = np.abs(mpm) <= MIN_P_TOL
        ok_b = near_p | near_m
        assert ok_b.all(), (
            f"{label} row {r}: keep sets differ away from a boundary at tokens {diff[~ok_b][:8]} "
            f"(gpu keep {gk[diff[~ok_b][:8]]}, exact top-p margin {tpx[~ok_b][:8]}, "
            f"min-p margin {mpm[~ok_b][:8]})")
        # the draw itself must still be exact: redo it on the GPU's keep set
        u = float(np.asarray(cfg["uniforms"]).reshape(-1)[r]) if uniforms is None else float(uniforms[r])
        tok, wsum = O.draw(gpu["processed"][r], gk.astype(np.uint8), draw_scale(cfg, r), u)
        assert tok == gpu["tokens"][r], \
            f"{label} row {r}: gpu token {gpu['tokens'][r]} != draw on its keep set {tok}"
        assert wsum == gpu["stats"]["kept_weight"][r], f"{label} row {r}: kept weight differs"
        boundary_rows.append(r)
    return boundary_rows


def draw_scale(cfg, r):
    """Draw scale of row r: fl(1/T) for mlx-lm sampled rows, else 1."""
    p = cfg["params"][r]
    if cfg["semantics"] == _ffi.SEM_MLXLM and p["kind"] != _ffi.KIND_ARGMAX:
        return float(np.float32(1.0) / np.float32(p["temperature"]))
    return 1.0
