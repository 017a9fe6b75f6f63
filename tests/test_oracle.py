"""The CPU restatement (oracle/) against the golden fixtures, closed forms and
invariants of tests/oracle_checks.py (CPU only)."""
import pytest

import oracle_checks as oc


@pytest.mark.parametrize("check", oc.CHECKS, ids=[c.__name__ for c in oc.CHECKS])
def test_oracle(check, ref, synth):
    msg = check(ref, synth)
    assert msg is None, msg


def test_relative_bound_catches_one_wrong_page(ref):
    """Why the GPU attention tests also hold outputs to 1e-3 * max|want|: at
    131072 cached tokens the outputs are so small that serving one 16-token
    page from the wrong place moves them by well under the absolute 1e-3;
    the relative bound rejects it.  The mistake is planted in the oracle's
    input, on the CPU."""
    import numpy as np
    from parity import TOL_ABS, TOL_REL, abs_rel
    rng = np.random.default_rng(0x51333890)
    P = 131072
    K = rng.standard_normal((P, 1024), dtype=np.float32)
    V = rng.standard_normal((P, 1024), dtype=np.float32)
    q = rng.standard_normal(6144, dtype=np.float32)
    want = ref.attn_heads(q, K, V, threads=8)
    page, other = 3000, 5000  # positions 48000..48015 read from 80000..80015
    K[page * 16:(page + 1) * 16] = K[other * 16:(other + 1) * 16]
    V[page * 16:(page + 1) * 16] = V[other * 16:(other + 1) * 16]
    bad = ref.attn_heads(q, K, V, threads=8)
    err, rel = abs_rel(bad, want)
    assert err < TOL_ABS, err      # the absolute bound alone would pass it
    assert rel > TOL_REL, rel      # the relative bound does not
