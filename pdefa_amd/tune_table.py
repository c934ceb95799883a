"""Builds a launch-shape table (pdefa_amd/tuning/<arch>.txt) from record files.

A process run with PDEFA_TUNE_RECORD=<file> appends every conv launch-shape
choice it measures on the device (single convs and grouped launches) to that
file.  This merges such records, and an existing table, into one table: one
`device <arch> <CUs>` header per device kind, then its `conv` and `group`
lines, the first choice seen for a shape winning (a table, once committed,
keeps its choices; new shapes are added).

    PDEFA_TUNE_RECORD=/tmp/rec.txt python bench.py
    PDEFA_TUNE_RECORD=/tmp/rec.txt PDEFA_TUNE_TABLE=/tmp/rec.txt python -m pytest tests -m gpu
    python -m pdefa_amd.tune_table pdefa_amd/tuning/gfx950.txt /tmp/rec.txt
"""
from __future__ import annotations

import os
import sys
from typing import Dict, List, Tuple


def _key(line: str) -> Tuple[str, ...]:
    """The shape part of a conv / group line (everything but the choice)."""
    f = line.split()
    if f[0] == "conv":
        return tuple(f[:-3])
    if f[0] == "group":
        return tuple(f[:-3])
    raise ValueError(f"not a table line: {line!r}")


def read(path: str) -> Dict[Tuple[str, int], List[str]]:
    """{(arch, cus): lines in file order} of a table or record file."""
    out: Dict[Tuple[str, int], List[str]] = {}
    dev = None
    with open(path) as f:
        for raw in f:
            line = raw.strip()
            if not line or line.startswith("#"):
                continue
            f_ = line.split()
            if f_[0] == "device":
                dev = (f_[1], int(f_[2]))
                out.setdefault(dev, [])
            elif dev is not None and f_[0] in ("conv", "group"):
                out[dev].append(line)
    return out


def merge(table: str, records: List[str]) -> int:
    """Merges `records` into `table` (created if missing); returns the number
    of lines added."""
    merged: Dict[Tuple[str, int], Dict[Tuple[str, ...], str]] = {}
    sources = ([table] if os.path.exists(table) else []) + records
    before = 0
    for i, src in enumerate(sources):
        for dev, lines in read(src).items():
            d = merged.setdefault(dev, {})
            for line in lines:
                d.setdefault(_key(line), line)
        if i == 0 and os.path.exists(table):
            before = sum(len(v) for v in merged.values())
    os.makedirs(os.path.dirname(os.path.abspath(table)), exist_ok=True)
    with open(table, "w") as f:
        f.write("# pdefa conv launch-shape table: measured choices per device kind (see pdefa_amd/tune_table.py)\n")
        for (arch, cus), lines in sorted(merged.items()):
            f.write(f"device {arch} {cus}\n")
            convs = sorted(l for l in lines.values() if l.startswith("conv "))
            groups = sorted(l for l in lines.values() if l.startswith("group "))
            for line in convs + groups:
                f.write(line + "\n")
    return sum(len(v) for v in merged.values()) - before


if __name__ == "__main__":
    if len(sys.argv) < 3:
        sys.exit(__doc__)
    n = merge(sys.argv[1], sys.argv[2:])
    print(f"{sys.argv[1]}: {n} lines added")
