"""The known Hadamard factors (K = 12 ... 172) of the reference's
signrot/functional/hadamard_matrices.py:8-4200 (from N. J. A. Sloane's
library of Hadamard matrices).

The ±1 tables are kept bit-for-bit -- parity of the rotation needs the same
matrices -- but stored in our own compact encoding: had_tables.json holds,
per K, one hexadecimal bit mask per row (bit j set <=> entry j is +1),
generated and checked (H Hᵀ = K·I) by tests/golden/make_had_tables.py.
"""
import functools
import json
import pathlib

import torch

_PATH = pathlib.Path(__file__).resolve().parent / "had_tables.json"


@functools.lru_cache(maxsize=None)
def _rows(k):
    return tuple(json.loads(_PATH.read_text())[str(k)])


def _table(k):
    rows = _rows(k)
    bits = torch.tensor([[(int(h, 16) >> j) & 1 for j in range(k)] for h in rows],
                        dtype=torch.float32)
    return bits * 2 - 1


def get_had12():
    return _table(12)


def get_had20():
    return _table(20)


def get_had28():
    return _table(28)


def get_had36():
    return _table(36)


def get_had40():
    return _table(40)


def get_had52():
    return _table(52)


def get_had60():
    return _table(60)


def get_had108():
    return _table(108)


def get_had140():
    return _table(140)


def get_had148():
    return _table(148)


def get_had156():
    return _table(156)


def get_had172():
    return _table(172)
