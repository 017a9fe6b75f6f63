"""Each planted mistake in the restatement (q38_ref.c built with
-DQ38R_MUTANT=k) must be rejected by at least one check, so a plausible slip
in the oracle cannot pass unnoticed (CPU only)."""
import os
import subprocess

import pytest

import oracle_checks as oc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MUTANTS = {
    1: "query head h reads kv head h % 4 instead of h / 6",
    2: "value head vh reads q/k head vh / 3 instead of vh % 16",
    3: "RoPE angle pos * s^p instead of the f32 recurrence",
    4: "decay applied after the prediction",
    5: "score scale 1 instead of 1/16",
    6: "L2 norm without the 1e-6 floor",
    7: "softplus without the identity above 20",
    8: "RMSNorm without eps",
    9: "conv1d taps reversed",
    10: "output gate silu instead of sigmoid",
    11: "delta sign flipped",
    12: "DeltaNet readout without 1/sqrt(128)",
    13: "Q8_K rounding by truncation",
    14: "Q8_K scale signed by the last |maximum|",
    15: "Q4_K/Q5_K 6-bit scales with the wrong high bits",
    16: "Q6_K third quarter with the wrong high bits",
    17: "Q5_K fifth bit not advanced per chunk",
    18: "Q8_K group sums over the wrong groups",
    19: "Q3_K high bit read with the opposite sense",
    20: "IQ4_XS group scale without its -32 offset",
    21: "BF16 row dot reading neighbouring elements swapped",
    22: "Q2_K minimum from the scale nibble",
    23: "IQ4_NL low and high nibbles swapped",
    24: "IQ2_XXS group scale from the wrong nibble",
    25: "IQ2_XS the two scale nibbles of a group swapped",
    26: "IQ2_S high index bits of section s taken from the wrong pair",
    27: "IQ3_XXS without the 1/4 in d",
    28: "IQ3_S second index's high bit taken from the first index's bit",
    29: "IQ1_S delta sign flipped",
    30: "IQ1_M odd sections test the even sections' delta bit",
}


@pytest.mark.parametrize("mutant", sorted(MUTANTS), ids=[f"m{k}" for k in sorted(MUTANTS)])
def test_mutant_is_rejected(mutant, ref, synth, tmp_path):
    so = tmp_path / f"libq38ref_m{mutant}.so"
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-fPIC", "-shared", f"-DQ38R_MUTANT={mutant}",
                    "-I", os.path.join(ROOT, "qwen3.8_27b_in_rust_amd", "csrc"), "-o", str(so), os.path.join(ROOT, "oracle", "q38_ref.c"),
                    os.path.join(ROOT, "oracle", "q38_quant_ref.c"), "-lm", "-lpthread"], check=True)
    prev = ref.use_library(str(so))
    try:
        failures = []
        for check in oc.CHECKS:
            try:
                msg = check(ref, synth)
            except Exception as e:  # a crash of the check also rejects the mutant
                msg = f"raised {e!r}"
            if msg:
                failures.append(f"{check.__name__}: {msg}")
    finally:
        ref.restore_library(prev)
    assert failures, f"mutant {mutant} ({MUTANTS[mutant]}) passed every check"
    print(f"mutant {mutant} ({MUTANTS[mutant]}) rejected by {len(failures)} checks, e.g. {failures[0]}")
