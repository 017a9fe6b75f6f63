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


def test_iq_grids_hold_the_lattice_values():
    """The IQ lattice grids (q38_iq_grids.h): each table's byte values are its
    format's levels (IQ2: 8, 25, 43; IQ3_XXS: 4..62; IQ3_S: odd 1..15; IQ1_S:
    -1, 0, 1), no entry repeats, and all but IQ1_S's are in ascending order;
    an eighth sign of even parity (ksigns_iq2xs) makes every 8-lane sign
    pattern's count of minus signs even."""
    import numpy as np
    g = oc._iq_grids()
    levels = {"Q38_IQ2XXS_GRID": {8, 25, 43}, "Q38_IQ2XS_GRID": {8, 25, 43}, "Q38_IQ2S_GRID": {8, 25, 43},
              "Q38_IQ3XXS_GRID": {4, 12, 20, 28, 36, 44, 52, 62}, "Q38_IQ3S_GRID": {1, 3, 5, 7, 9, 11, 13, 15},
              "Q38_IQ1S_GRID": {0, 1, 255}}
    sizes = {"Q38_IQ2XXS_GRID": 256, "Q38_IQ2XS_GRID": 512, "Q38_IQ2S_GRID": 1024, "Q38_IQ3XXS_GRID": 256,
             "Q38_IQ3S_GRID": 512, "Q38_IQ1S_GRID": 2048}
    for name, t in g.items():
        assert t.shape[0] == sizes[name], name
        assert set(np.unique(t).tolist()) == levels[name], name
        packed = [int.from_bytes(bytes(row.astype(np.uint8)), "little") for row in t]
        assert len(set(packed)) == len(packed), name
        if name != "Q38_IQ1S_GRID":
            assert packed == sorted(packed), name
    for i in range(128):
        assert np.sum(oc._ksign_mask(i) < 0) % 2 == 0


def test_iq_grids_equal_the_reference_tables():
    """q38_iq_grids.h holds exactly the values of the reference's copy of
    ggml's tables (src/kernel/iq_tables.rs, read as text); and the reference's
    KSIGNS_IQ2XS is i | parity(i) << 7, the rule the oracle and the kernels
    use in place of that table."""
    import os
    import re
    import numpy as np
    path = "/root/reference/src/kernel/iq_tables.rs"
    if not os.path.exists(path):
        pytest.skip("the reference's sources are not on this machine")
    text = open(path).read()
    g = oc._iq_grids()
    for name, bits, n in (("IQ2XXS_GRID", 64, 256), ("IQ2XS_GRID", 64, 512), ("IQ2S_GRID", 64, 1024),
                          ("IQ3XXS_GRID", 32, 256), ("IQ3S_GRID", 32, 512), ("IQ1S_GRID", 64, 2048)):
        body = re.search(r"pub const %s: \[u%d; %d\] = \[(.*?)\];" % (name, bits, n), text, re.S).group(1)
        want = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)]
        got = [int.from_bytes(bytes(row.astype(np.uint8)), "little") for row in g["Q38_" + name]]
        assert got == want, name
    body = re.search(r"pub const KSIGNS_IQ2XS: \[u8; 128\] = \[(.*?)\];", text, re.S).group(1)
    ks = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)]
    assert ks == [i | ((bin(i).count("1") & 1) << 7) for i in range(128)]
