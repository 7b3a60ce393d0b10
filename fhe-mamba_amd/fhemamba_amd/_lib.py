"""ctypes binding of libfhecore.so (declarations: include/fhecore.h).

The library is the only compute path: importing this module fails loudly
if the shared object has not been built, and every call that returns a
non-zero status raises FheError with the library's message.
"""
from __future__ import annotations

import atexit
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("FHEMAMBA_LIB", os.path.join(HERE, "libfhecore.so"))

_u32, _u64, _i64, _int = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_int
_p = ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)
_dbl = ctypes.c_double

FHE_OK, FHE_ERR_ARG, FHE_ERR_HIP, FHE_ERR_RANGE, FHE_ERR_STATE, FHE_ERR_INTERNAL = range(6)


class FheError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"fhecore error {code}: {message}")
        self.code = code


class FheArgumentError(FheError, ValueError):
    pass


class FheRangeError(FheError, OverflowError):
    pass


# name -> argtypes (all functions return int unless noted)
SIGNATURES = {
    "fhe_abi_version": [],
    "fhe_gen_moduli": [_u32, _u32, _u32, _u32, _u32, _p, _p, _u32, _p],
    "fhe_context_create": [_u32, _p, _u32, _p, _u32, _u32, _int, _pp],
    "fhe_context_destroy": [_p],
    "fhe_context_info": [_p, _p],
    "fhe_alloc_count": [_p],
    "fhe_context_moduli": [_p, _p, _p],
    "fhe_context_set_stream": [_p, _p],
    "fhe_sync": [_p],
    "fhe_profile_begin": [_p],
    "fhe_profile_end": [_p, ctypes.c_char_p, ctypes.c_size_t],
    "fhe_ntt_forward": [_p, _p, _u32, _u32, _u32],
    "fhe_ntt_inverse": [_p, _p, _u32, _u32, _u32],
    "fhe_mac": [_p, _p, _p, _u32, _u32, _p],
    "fhe_poly_create": [_p, _u32, _u32, _pp],
    "fhe_poly_destroy": [_p],
    "fhe_poly_shape": [_p, _p, _p],
    "fhe_poly_data": [_p, _pp],
    "fhe_poly_upload": [_p, _p, _u32, _u32],
    "fhe_poly_download": [_p, _p],
    "fhe_poly_copy": [_p, _p],
    "fhe_drop_limbs": [_p, _p, _u32],
    "fhe_add": [_p, _p, _p],
    "fhe_sub": [_p, _p, _p],
    "fhe_negate": [_p, _p],
    "fhe_mul_plain": [_p, _p, _p],
    "fhe_add_plain": [_p, _p, _p],
    "fhe_mul_const": [_p, _p, _p],
    "fhe_add_const": [_p, _p, _p],
    "fhe_mul_int": [_p, _p, _i64],
    "fhe_rescale": [_p, _p],
    "fhe_rescale_many": [_p, _p, _u32],
    "fhe_tensor": [_p, _p, _p],
    "fhe_key_load": [_p, _p, _pp],
    "fhe_key_download": [_p, _p],
    "fhe_key_destroy": [_p],
    "fhe_keyswitch": [_p, _p, _p],
    "fhe_relinearize": [_p, _p, _p],
    "fhe_relinearize_many": [_p, _p, _u32, _p],
    "fhe_rotate": [_p, _p, _p, _u32],
    "fhe_rotate_noalloc": [_p, _p, _p, _u32],
    "fhe_rotation_precompute": [_p, _pp],
    "fhe_rotate_hoisted": [_p, _p, _p, _p, _u32, _p],
    "fhe_linear_transform": [_p, _p, _p, _u32, _u32, _p, _p, _p, _u32],
    "fhe_linear_transform_hoisted": [_p, _p, _p, _u32, _u32, _p, _p, _p, _p, _u32],
    "fhe_linear_transform_hoisted_many": [_p, _p, _u32, _p, _u32, _u32, _p, _p, _p, _p, _u32],
    "fhe_rotate_many": [_p, _p, _p, _p, _u32],
    "fhe_mod_raise": [_p, _p, _u32],
    "fhe_encode": [_p, _p, _p, _u32, _u32, _dbl, _u32, _p],
    "fhe_encode_many": [_p, _p, _p, _u32, _u32, _u32, _dbl, _u32, _p],
    "fhe_linear_wsum": [_p, _p, _p, _u32, _u32],
    "fhe_decode": [_p, _p, _u32, _dbl, _p, _p],
    "fhe_context_set_sampling": [_p, _int, _p],
    "fhe_keygen_secret": [_p, _u64, _p],
    "fhe_keygen_secret_sparse": [_p, _u64, _u32, _p],
    "fhe_keygen_public": [_p, _p, _u64, _p],
    "fhe_keygen_relin": [_p, _p, _u64, _pp],
    "fhe_keygen_galois": [_p, _p, _u32, _u64, _pp],
    "fhe_encrypt": [_p, _p, _p, _u64],
    "fhe_decrypt": [_p, _p, _p],
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libfhecore.so not found at {LIB_PATH}; build it with "
            "`python fhe-mamba_amd/build.py` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.fhe_last_error.restype = ctypes.c_char_p
    lib.fhe_last_error.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _int
    return lib


lib = _load()

# Finalizers stop calling into the library once interpreter shutdown begins
# (objects still alive then are reclaimed with the process).
alive = True


def _shutdown() -> None:
    global alive
    alive = False


atexit.register(_shutdown)


def check(rc: int) -> None:
    if rc != FHE_OK:
        msg = lib.fhe_last_error().decode(errors="replace")
        if rc == FHE_ERR_ARG:
            raise FheArgumentError(rc, msg)
        if rc == FHE_ERR_RANGE:
            raise FheRangeError(rc, msg)
        raise FheError(rc, msg)


def call(name: str, *args) -> None:
    check(getattr(lib, name)(*args))


def device_free_bytes(device: int | None = None) -> int | None:
    """Free memory of HIP device `device` (default: the current one;
    hipMemGetInfo from the HIP runtime the library links, with that device
    current for the call), or None when it cannot be read."""
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
        prev = ctypes.c_int(0)
        if device is not None:
            if hip.hipGetDevice(ctypes.byref(prev)) != 0 or hip.hipSetDevice(device) != 0:
                return None
        try:
            if hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) != 0:
                return None
        finally:
            if device is not None:
                hip.hipSetDevice(prev.value)
        return int(free.value)
    except OSError:
        return None
