"""Loader for the golden vectors written by tests/golden/make_golden.py."""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden", "golden_reference.npz")

if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle.qflash_oracle import Consts, Flags  # noqa: E402


class GoldenCase(dict):
    name: str

    @property
    def consts(self) -> Consts:
        return Consts(*[int(x) for x in self["consts"]])

    @property
    def flags(self) -> Flags:
        f = [int(x) for x in self["flags"]]
        return Flags(bool(f[0]), bool(f[1]), bool(f[2]), f[3], f[4])

    @property
    def masked(self) -> bool:
        return "bias_i32" in self

    @property
    def has_fp(self) -> bool:
        return "q_fp" in self


def load_cases() -> dict[str, GoldenCase]:
    z = np.load(GOLDEN, allow_pickle=False)
    raw = {k: z[k] for k in z.files}
    cases: dict[str, GoldenCase] = {}
    for key, val in raw.items():
        if val.dtype.kind == "U" and val.ndim == 0 and str(val).startswith("@"):
            val = raw[str(val)[1:]]
        name, field = key.split("/", 1)
        c = cases.setdefault(name, GoldenCase())
        c.name = name
        c[field] = val
    return cases
