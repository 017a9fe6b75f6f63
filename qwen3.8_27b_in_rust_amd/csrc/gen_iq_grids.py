"""Writes q38_iq_grids.h: the lattice grids of ggml's IQ weight formats.

The grids are format data, not code: a GGUF file's IQ1_S/IQ1_M, IQ2_XXS,
IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S blocks store indices into these fixed
tables (ggml-common.h, MIT licence), so a reader must hold exactly these
values.  They are taken here from the reference's copy,
src/kernel/iq_tables.rs, and written out as C initializer lists, one macro
per table, for the device code and the oracle to instantiate.
(ksigns_iq2xs and kmask_iq2xs are not copied: their entries are i | parity(i)
<< 7 and 1 << i, formed where they are used.)

    python3 gen_iq_grids.py [/root/reference/src/kernel/iq_tables.rs]
"""
import re
import sys
from pathlib import Path

TABLES = [  # (name in iq_tables.rs, macro, element bits, entries)
    ("IQ2XXS_GRID", "Q38_IQ2XXS_GRID", 64, 256),
    ("IQ2XS_GRID", "Q38_IQ2XS_GRID", 64, 512),
    ("IQ2S_GRID", "Q38_IQ2S_GRID", 64, 1024),
    ("IQ3XXS_GRID", "Q38_IQ3XXS_GRID", 32, 256),
    ("IQ3S_GRID", "Q38_IQ3S_GRID", 32, 512),
    ("IQ1S_GRID", "Q38_IQ1S_GRID", 64, 2048),
]


def read_tables(path):
    text = Path(path).read_text()
    out = {}
    for name, _, bits, n in TABLES:
        m = re.search(r"pub const %s: \[u%d; %d\] = \[(.*?)\];" % (name, bits, n), text, re.S)
        if m is None:
            raise SystemExit(f"{name}: not found in {path}")
        vals = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", m.group(1))]
        if len(vals) != n:
            raise SystemExit(f"{name}: {len(vals)} entries, expected {n}")
        out[name] = vals
    return out


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/kernel/iq_tables.rs"
    tables = read_tables(src)
    lines = [
        "/* Lattice grids of ggml's IQ weight formats (ggml-common.h, MIT licence):",
        " * the fixed tables a GGUF IQ block indexes.  Written by gen_iq_grids.py; one",
        " * initializer list per table, instantiated by the device code and the oracle. */",
        "#ifndef Q38_IQ_GRIDS_H",
        "#define Q38_IQ_GRIDS_H",
        "",
    ]
    for name, macro, bits, n in TABLES:
        vals = tables[name]
        width = 16 if bits == 64 else 8
        per_line = 4 if bits == 64 else 8
        lines.append(f"/* {name.lower()}: {n} entries of {bits // 8} bytes */")
        lines.append(f"#define {macro} {{ \\")
        for i in range(0, n, per_line):
            chunk = ", ".join(f"0x{v:0{width}x}" for v in vals[i:i + per_line])
            lines.append(f"    {chunk}, \\")
        lines.append("}")
        lines.append("")
    lines.append("#endif")
    Path(__file__).with_name("q38_iq_grids.h").write_text("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
