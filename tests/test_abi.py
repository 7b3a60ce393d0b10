"""C-ABI library checks that need no GPU: it loads, exports exactly the
entry points include/fhecore.h declares, host-only parameter selection
agrees with the oracle, and failures come back as status codes."""
import os
import re

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fhecore.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(fhe_[a-z0-9_]+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from fhemamba_amd import _lib
    names = declared_symbols()
    assert len(names) >= 40
    for name in names:
        assert hasattr(_lib.lib, name), name
    assert set(_lib.SIGNATURES) | {"fhe_last_error"} == set(names)
    assert _lib.lib.fhe_abi_version() == 1


@pytest.mark.parametrize("log_n,depth,sb,fb,dnum",
                         [(17, 44, 59, 60, 4), (16, 23, 59, 60, 3), (13, 7, 50, 60, 2)])
def test_gen_moduli_matches_oracle(log_n, depth, sb, fb, dnum):
    import fhemamba_amd as F
    assert F.gen_moduli(log_n, depth, sb, fb, dnum) == O.gen_moduli(log_n, depth, sb, fb, dnum)


def test_gen_moduli_rejects_bad_arguments():
    import fhemamba_amd as F
    with pytest.raises(ValueError):
        F.gen_moduli(3, 4, 40, 60, 2)
    with pytest.raises(ValueError):
        F.gen_moduli(12, 4, 61, 60, 2)


def test_context_failure_is_a_status_not_a_crash():
    """Bad moduli are rejected before touching a device; without a device
    the HIP error is reported through fhe_last_error."""
    import fhemamba_amd as F
    from fhemamba_amd._lib import FheError
    with pytest.raises(ValueError, match="not a prime"):
        F.Context(12, [12289 * 3], [], 1)  # composite
    q, p = O.gen_moduli(12, 3, 40, 60, 2)
    try:
        ctx = F.Context(12, q, p, 2)
    except FheError as e:
        assert e.code == 2 and "hip" in str(e).lower()
    else:
        ctx.close()


def test_galois_elements_match_oracle():
    import fhemamba_amd as F
    for n in (1 << 12, 1 << 16):
        for step in (1, -1, 7, -64, n // 4 - 1):
            assert F.galois_element(step, n) == O.galois_elt(step, n)
        assert F.conjugation_element(n) == 2 * n - 1
