#!/usr/bin/env python3
"""Regenerate the IQ2 / IQ3 grid codebooks and the IQ4_NL value table from the
reference's vendored ggml header.

The IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS and IQ3_S formats index fixed codebooks
(third_party/ggml-common.h, ggml rev 8c63e709, MIT: iq2xxs_grid 256 x 8
bytes, iq2xs_grid 512 x 8, iq2s_grid 1024 x 8, iq3xxs_grid 256 x 4,
iq3s_grid 512 x 4), and IQ4_NL / IQ4_XS map nibbles through kvalues_iq4nl.
They are part of the on-disk formats, so they have to be identical.  Each
grid entry uses a small set of levels, so the tables are stored here in a
compact encoding of our own: one uint16 per entry holding the level index of
every element (2 bits per element for the IQ2 grids, 3 bits for IQ3), as
X-macro lists that host and device code expand into byte tables at compile
time.  The generator checks the level sets and that the sign table
ksigns_iq2xs is the even-parity completion i | parity(i) << 7, which the
kernels compute instead of storing.

Run from the repository root:  python oracle/gen_iq_grids.py
It reads /root/reference/third_party/ggml-common.h and writes
qwen3.8-27b-in-c_amd/csrc/q38_iq_grids.inc.
"""
import hashlib
import os
import re
import sys

HEADER = "/root/reference/third_party/ggml-common.h"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..",
                   "qwen3.8-27b-in-c_amd", "csrc", "q38_iq_grids.inc")

IQ2_LEVELS = (8, 25, 43)
IQ3XXS_LEVELS = (4, 12, 20, 28, 36, 44, 52, 62)
IQ3S_LEVELS = (1, 3, 5, 7, 9, 11, 13, 15)
# name, element bytes per entry, entries, levels, bits per element
GRIDS = (
    ("iq2xxs", 8, 256, IQ2_LEVELS, 2),
    ("iq2xs", 8, 512, IQ2_LEVELS, 2),
    ("iq2s", 8, 1024, IQ2_LEVELS, 2),
    ("iq3xxs", 4, 256, IQ3XXS_LEVELS, 3),
    ("iq3s", 4, 512, IQ3S_LEVELS, 3),
)


def table_text(text, ctype, name):
    match = re.search(r"GGML_TABLE_BEGIN\(%s, %s, [^)]*\)(.*?)GGML_TABLE_END\(\)" % (ctype, name), text, re.S)
    if not match:
        raise RuntimeError("%s not found" % name)
    return match.group(1)


def read_reference_tables(path=HEADER):
    """{name: list of entries, each a list of element values}, plus the
    IQ4_NL values."""
    text = open(path, encoding="utf-8").read()
    grids = {}
    for name, width, count, _, _ in GRIDS:
        ctype = "uint64_t" if width == 8 else "uint32_t"
        digits = 16 if width == 8 else 8
        words = [int(w, 16) for w in re.findall(r"0x([0-9a-fA-F]{%d})" % digits,
                                                 table_text(text, ctype, name + "_grid"))]
        if len(words) != count:
            raise RuntimeError("%s: expected %d entries, found %d" % (name, count, len(words)))
        grids[name] = [[(w >> (8 * k)) & 0xFF for k in range(width)] for w in words]
    values = [int(v) for v in re.findall(r"-?\d+", table_text(text, "int8_t", "kvalues_iq4nl"))]
    signs = [int(v) for v in re.findall(r"\d+", table_text(text, "uint8_t", "ksigns_iq2xs"))]
    return grids, values, signs


def encode(entries, levels, bits):
    codes = []
    for entry in entries:
        code = 0
        for k, value in enumerate(entry):
            if value not in levels:
                raise RuntimeError("grid value %d outside the level set" % value)
            code |= levels.index(value) << (bits * k)
        codes.append(code)
    return codes


def decode(codes, levels, bits, width):
    mask = (1 << bits) - 1
    return [[levels[(c >> (bits * k)) & mask] for k in range(width)] for c in codes]


def expanded_sha(grids, values):
    h = hashlib.sha256()
    for name, _, _, _, _ in GRIDS:
        h.update(bytes(b for entry in grids[name] for b in entry))
    h.update(bytes(v & 0xFF for v in values))
    return h.hexdigest()


def main():
    grids, values, signs = read_reference_tables()
    if len(values) != 16:
        raise RuntimeError("kvalues_iq4nl must hold 16 values")
    if signs != [i | (bin(i).count("1") & 1) << 7 for i in range(128)]:
        raise RuntimeError("ksigns_iq2xs is not the even-parity completion")
    lines = [
        "/* IQ2 / IQ3 grid codebooks and IQ4_NL values: the tables the GGUF IQ2_XXS,",
        " * IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_NL and IQ4_XS formats index",
        " * (third_party/ggml-common.h, ggml rev 8c63e709: iq2xxs_grid, iq2xs_grid,",
        " * iq2s_grid, iq3xxs_grid, iq3s_grid, kvalues_iq4nl).",
        " * Encoding: entry e of a grid is one code; element k of it is the level",
        " * with index (code >> (B * k)) & (2^B - 1), B = 2 for the IQ2 grids",
        " * (levels 8, 25, 43; 8 elements) and B = 3 for the IQ3 grids (IQ3_XXS",
        " * levels 4, 12, 20, 28, 36, 44, 52, 62; IQ3_S levels 1, 3, .., 15; 4",
        " * elements).  Lists are X-macros: Q38_IQ2XXS_CODES(X) expands X(code) per",
        " * entry.  The sign table of the IQ2/IQ3 formats is i | parity(i) << 7.",
        " * SHA-256 of the expanded tables (grids in the order above, entry-major,",
        " * then the 16 values as bytes):",
        " *   " + expanded_sha(grids, values),
        " * Generated by oracle/gen_iq_grids.py; do not edit. */",
        "",
        "#define Q38_IQ4NL_VALUES " + ", ".join(str(v) for v in values),
        "",
    ]
    for name, width, count, levels, bits in GRIDS:
        codes = encode(grids[name], levels, bits)
        if decode(codes, levels, bits, width) != grids[name]:
            raise RuntimeError("round trip failed for " + name)
        lines.append("#define Q38_%s_CODES(X) \\" % name.upper())
        for i in range(0, count, 10):
            chunk = " ".join("X(0x%04x)" % c for c in codes[i:i + 10])
            lines.append("    " + chunk + (" \\" if i + 10 < count else ""))
        lines.append("")
    with open(OUT, "w") as f:
        f.write("\n".join(lines))
    print("wrote", os.path.relpath(OUT))


if __name__ == "__main__":
    sys.exit(main())
