"""Shared parity criteria of the GPU tests.

Attention outputs are held to two bounds:
  - max-abs <= 1e-3, the tolerance stated for this path;
  - max-abs <= 1e-3 * max|want|, a relative bound.  At long contexts the
    outputs are small (std ~9e-3 at 32K tokens, ~5e-3 at 128K), so the
    absolute bound alone would pass a decode that dropped or misaddressed a
    16-token page (an error of ~1e-3 at 32K, ~3e-4 at 128K); such a page moves
    the relative error to ~1e-2 (tests/test_oracle.py plants one in the oracle
    to show it).  The kernels' measured error is ~1e-6 relative.
DeltaNet: outputs max-abs <= 1e-3; state relative <= 1e-4 (max and
Frobenius), as stated for this path.
"""
from __future__ import annotations

import contextlib

import numpy as np

TOL_ABS = 1e-3
TOL_REL = 1e-3
TOL_STATE_REL = 1e-4


def abs_rel(got, want) -> tuple[float, float]:
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    d = np.abs(got - want)
    err = float(np.max(d)) if d.size else 0.0
    scale = float(np.max(np.abs(want))) if np.size(want) else 0.0
    return err, (err / scale if scale > 0 else err)


def check_attn(margin, got, want, what: str = "out") -> None:
    err, rel = abs_rel(got, want)
    margin(f"{what} max-abs", err, TOL_ABS)
    margin(f"{what} rel", rel, TOL_REL)


def state_rel(got, want) -> tuple[float, float]:
    d = np.asarray(got, np.float64) - np.asarray(want, np.float64)
    return (float(np.max(np.abs(d)) / np.max(np.abs(want))),
            float(np.linalg.norm(d) / np.linalg.norm(want)))


def check_state(margin, got, want, what: str = "state") -> None:
    rel_max, rel_fro = state_rel(got, want)
    margin(f"{what} rel max", rel_max, TOL_STATE_REL)
    margin(f"{what} rel fro", rel_fro, TOL_STATE_REL)


@contextlib.contextmanager
def decode_split(ctx, tokens: int | None):
    """Fix the decode split size for the block (None: leave automatic)."""
    if tokens:
        ctx.set_decode_split(tokens)
    try:
        yield
    finally:
        if tokens:
            ctx.set_decode_split(0)
