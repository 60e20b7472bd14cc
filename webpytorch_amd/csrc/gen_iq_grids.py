"""Write iq_grids.h: the codebooks of the llama.cpp i-quant GGUF block types (IQ2_XXS, IQ2_XS,
IQ2_S, IQ3_XXS, IQ3_S, IQ1_S / IQ1_M). They are part of the file format -- a block stores
indices into them -- so they have to be the format's own values; the reference carries them
as data in `webtorch/iqtables.py` (extracted there from ggml's `ggml-common.h`). This script
reads that file as text (nothing in it is executed), re-encodes the tables and writes the
header. It runs only where the reference tree is present; the header is committed.

Encodings in the header:
  * IQ2 grids: one uint64 per entry, byte j = value j (each 8, 25 or 43);
  * IQ3 grids: one uint32 per entry, byte j = value j (4, 12, ..., 62);
  * IQ1 grid: one uint16 per entry, bits 2j..2j+1 = value j + 1 (values -1, 0, 1).
The sign tables of IQ2_XXS / IQ2_XS / IQ3_XXS are not stored: a 7-bit sign index s stands for
the byte s | (parity of s) << 7, computed in the kernels.

Usage: python webpytorch_amd/csrc/gen_iq_grids.py [reference_iqtables.py]
"""
import hashlib
import os
import re
import sys

import numpy as np

SRC = "/root/reference/webtorch/iqtables.py"
HERE = os.path.dirname(os.path.abspath(__file__))

# (table name in the source, header name, entry dtype)
TABLES = (("IQ2XXS_GRID", "kIQ2XXS", np.uint64), ("IQ2XS_GRID", "kIQ2XS", np.uint64),
          ("IQ2S_GRID", "kIQ2S", np.uint64), ("IQ3XXS_GRID", "kIQ3XXS", np.uint32),
          ("IQ3S_GRID", "kIQ3S", np.uint32), ("IQ1S_GRID", "kIQ1S", np.uint64))


def read_tables(path):
    text = open(path).read()
    out = {}
    for src, _, dt in TABLES:
        m = re.search(r"^%s = np\.array\(\[(.*?)\], dtype=np\.(\w+)\)" % src, text, re.S | re.M)
        if not m:
            raise SystemExit("table %s not found in %s" % (src, path))
        vals = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", m.group(1))]
        out[src] = np.array(vals, dt)
    return out


def expanded(tables):
    """The values the format defines, as int8 arrays (entries, values per entry): what the
    digests below are taken of."""
    ex = {}
    for src, _, dt in TABLES:
        t = tables[src]
        per = 8 if dt == np.uint64 else 4
        ex[src] = t.view(np.uint8).reshape(-1, per).view(np.int8).copy()
    return ex


def digests(ex):
    return {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() for k, v in ex.items()}


def iq1_packed(t):
    v = t.view(np.uint8).reshape(-1, 8).view(np.int8).astype(np.int32) + 1
    if v.min() < 0 or v.max() > 2:
        raise SystemExit("IQ1 grid values outside -1..1")
    return (v << (2 * np.arange(8))).sum(axis=1).astype(np.uint16)


def emit(tables):
    ex = expanded(tables)
    lines = ["// Codebooks of the llama.cpp i-quant GGUF block types, written by gen_iq_grids.py from the",
             "// format's tables (values, not code). IQ2 grids: byte j of an entry is value j; IQ3 grids:",
             "// likewise, 4 values per entry; IQ1 grid: bits 2j..2j+1 of an entry are value j + 1.",
             "// SHA-256 of the values (int8 per value, entries in order):"]
    for k, h in digests(ex).items():
        lines.append("//   %s %s" % (k, h))
    lines += ["#pragma once", "#include <stdint.h>", "", "namespace miq {", "namespace iq {", ""]
    for src, name, dt in TABLES:
        t = tables[src]
        if src == "IQ1S_GRID":
            t, ctype, width, per_line = iq1_packed(t), "uint16_t", 4, 16
        elif dt == np.uint64:
            ctype, width, per_line = "uint64_t", 16, 4
        else:
            ctype, width, per_line = "uint32_t", 8, 8
        lines.append("__device__ __constant__ %s %s[%d] = {" % (ctype, name, t.size))
        for i in range(0, t.size, per_line):
            row = ", ".join("0x%0*x%s" % (width, int(v), "ull" if ctype == "uint64_t" else "u") for v in t[i:i + per_line])
            lines.append("    " + row + ",")
        lines.append("};")
        lines.append("")
    lines += ["}  // namespace iq", "}  // namespace miq", ""]
    return "\n".join(lines)


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else SRC
    tables = read_tables(src)
    sizes = {k: v.size for k, v in tables.items()}
    want = {"IQ2XXS_GRID": 256, "IQ2XS_GRID": 512, "IQ2S_GRID": 1024, "IQ3XXS_GRID": 256, "IQ3S_GRID": 512,
            "IQ1S_GRID": 2048}
    if sizes != want:
        raise SystemExit("unexpected table sizes %s" % sizes)
    with open(os.path.join(HERE, "iq_grids.h"), "w") as f:
        f.write(emit(tables))
    for k, h in digests(expanded(tables)).items():
        print(k, h)


if __name__ == "__main__":
    main()
