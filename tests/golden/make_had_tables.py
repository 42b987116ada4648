"""Write signrot_amd/functional/had_tables.json from the reference's ±1 tables.

The reference keeps its known Hadamard factors as Python list literals in
signrot/functional/hadamard_matrices.py (get_had12 ... get_had172, lines
8-4200).  This script reads that file as text, evaluates only the list
literals (ast.literal_eval, nothing is imported or executed), checks that each
table is a Hadamard matrix (entries ±1, H Hᵀ = K·I), and stores each row as a
hex bit mask (bit j set ⇔ entry j is +1).  It also writes the SHA-256 of the
decoded tables to tests/golden/had_tables.sha256 so the test suite can pin the
committed tables without the reference present.

Run once, in a container where /root/reference exists:
    python tests/golden/make_had_tables.py
"""
import ast
import hashlib
import json
import pathlib
import re
import sys

import numpy as np

REF = pathlib.Path("/root/reference/signrot/functional/hadamard_matrices.py")
ROOT = pathlib.Path(__file__).resolve().parents[2]
OUT = ROOT / "signrot_amd" / "functional" / "had_tables.json"
SHA = ROOT / "tests" / "golden" / "had_tables.sha256"


def parse(text):
    tables = {}
    for m in re.finditer(r"def get_had(\d+)\(\):\s*return torch\.FloatTensor\(", text):
        k = int(m.group(1))
        start = m.end()
        depth = 0
        for i in range(start, len(text)):
            c = text[i]
            if c == "[":
                depth += 1
            elif c == "]":
                depth -= 1
                if depth == 0:
                    lit = text[start:i + 1]
                    break
        # comments inside the literal are not valid in literal_eval input
        lit = re.sub(r"#[^\n]*", "", lit)
        h = np.array(ast.literal_eval(lit), dtype=np.int64)
        # get_had148 wraps its rows in one extra list level ([1, 148, 148]);
        # the reference's `hadK @ x` broadcasts it, so the leading 1 is dropped
        tables[k] = h.reshape(h.shape[-2], h.shape[-1])
    return tables


def digest(tables):
    h = hashlib.sha256()
    for k in sorted(tables):
        h.update(str(k).encode())
        h.update(np.ascontiguousarray(tables[k], dtype=np.int8).tobytes())
    return h.hexdigest()


def main():
    tables = parse(REF.read_text())
    out = {}
    for k, h in sorted(tables.items()):
        assert h.shape == (k, k), (k, h.shape)
        assert np.all(np.abs(h) == 1), k
        assert np.array_equal(h @ h.T, k * np.eye(k, dtype=np.int64)), k
        rows = []
        for r in h:
            bits = 0
            for j, v in enumerate(r):
                if v > 0:
                    bits |= 1 << j
            rows.append(format(bits, "x"))
        out[str(k)] = rows
    OUT.write_text(json.dumps(out, indent=0) + "\n")
    SHA.write_text(digest(tables) + "\n")
    print("wrote", OUT, "K =", sorted(tables))


if __name__ == "__main__":
    sys.exit(main())
