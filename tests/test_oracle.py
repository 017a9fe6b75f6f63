"""The CPU restatement (oracle/) against the golden fixtures, closed forms and
invariants of tests/oracle_checks.py (CPU only)."""
import pytest

import oracle_checks as oc


@pytest.mark.parametrize("check", oc.CHECKS, ids=[c.__name__ for c in oc.CHECKS])
def test_oracle(check, ref, synth):
    msg = check(ref, synth)
    assert msg is None, msg
