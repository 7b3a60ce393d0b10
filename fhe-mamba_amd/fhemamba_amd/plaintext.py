"""Plaintext bounds for the compact (single-residue) encoding route.

compact_plaintext_fits follows native/fideslib_stage0/include/
plaintext_rns.hpp:15-25: every coefficient of the inverse special FFT is
bounded by mean(|slot|), so when mean(|slot|) * scale + 1 < q0 / 4 the
rounded coefficients are determined by their residue mod q0 alone.  The sum
is formed in x87 extended precision (numpy.longdouble), as the reference's
long double is on x86-64.
"""
from __future__ import annotations

import math
from typing import Iterable

import numpy as np


def compact_plaintext_fits(values: Iterable[float], slots: int, scale: float,
                           q0: int) -> bool:
    values = [float(v) for v in values]
    slots, q0 = int(slots), int(q0)
    if (not slots or len(values) > slots or not math.isfinite(scale) or scale <= 0
            or q0 < 4 or q0 >= 1 << 61):
        return False
    total = np.longdouble(0)
    for v in values:
        if not math.isfinite(v):
            return False
        total += abs(np.longdouble(v))
    lhs = total * np.longdouble(scale) / np.longdouble(slots) + np.longdouble(1)
    return bool(lhs < np.longdouble(q0) / np.longdouble(4))
