"""fhemamba_amd: MI355X (gfx950) CKKS-RNS evaluation core.

The compute path is libfhecore.so (HIP) behind the C ABI in
include/fhecore.h; this package binds it with ctypes and mirrors the
fhemamba CKKS backend interface on top.
"""
from .core import Context, Key, Poly, conjugation_element, galois_element, gen_moduli

__all__ = ["Context", "Key", "Poly", "conjugation_element", "galois_element", "gen_moduli"]
