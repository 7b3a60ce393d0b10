"""ctypes/numpy view of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline
leg, always as the checker.  The library product never imports it.
See ckks_oracle.h for what each function restates and how it is pinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libckks_oracle.so")
REF_DRIVER = os.path.join(HERE, "_ref", "ref_headers")

_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_p = ctypes.c_void_p


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "orc_mulmod": (_u64, [_u64, _u64, _u64]),
        "orc_powmod": (_u64, [_u64, _u64, _u64]),
        "orc_invmod": (_u64, [_u64, _u64]),
        "orc_is_prime": (ctypes.c_int, [_u64]),
        "orc_first_prime": (_u64, [_u32, _u64]),
        "orc_previous_prime": (_u64, [_u64, _u64]),
        "orc_next_prime": (_u64, [_u64, _u64]),
        "orc_root_of_unity": (_u64, [_u64, _u64]),
        "orc_gen_moduli": (ctypes.c_int, [_u32, _u32, _u32, _u32, _u32, _p, _p, _u32]),
        "orc_num_special_primes": (ctypes.c_int, [_p, _u32, _u32, _u32]),
        "orc_ntt_fwd": (None, [_p, _u32, _u64, _u64]),
        "orc_ntt_inv": (None, [_p, _u32, _u64, _u64]),
        "orc_ntt_naive": (None, [_p, _p, _u32, _u64, _u64]),
        "orc_negacyclic_schoolbook": (None, [_p, _p, _p, _u32, _u64]),
        "orc_automorph_ntt": (None, [_p, _p, _u32, _u32]),
        "orc_automorph_coeff": (None, [_p, _p, _u32, _u32, _u64]),
        "orc_galois_elt": (_u32, [ctypes.c_int32, _u32]),
        "orc_switch_basis": (None, [_p, _p, _u32, _p, _p, _u32, _u32]),
        "orc_ctx_create": (_p, [_u32, _p, _u32, _p, _u32, _u32]),
        "orc_ctx_destroy": (None, [_p]),
        "orc_ctx_psi": (_u64, [_p, _u32]),
        "orc_ctx_ntt_fwd": (None, [_p, _p, _u32]),
        "orc_ctx_ntt_inv": (None, [_p, _p, _u32]),
        "orc_ntt_fwd_batch": (None, [_p, _p, _u32, _u32, _u32, ctypes.c_int]),
        "orc_ntt_inv_batch": (None, [_p, _p, _u32, _u32, _u32, ctypes.c_int]),
        "orc_mac_batch": (None, [_p, _p, _p, _u32, _u32, _p, ctypes.c_int]),
        "orc_add": (None, [_p, _p, _p, _u32, _u32, _p]),
        "orc_num_digits": (_u32, [_p, _u32]),
        "orc_modup": (None, [_p, _p, _u32, _p]),
        "orc_ksk_inner": (None, [_p, _p, _u32, _p, _p]),
        "orc_moddown": (None, [_p, _p, _u32, _p]),
        "orc_keyswitch": (None, [_p, _p, _u32, _p, _p]),
        "orc_rotate": (None, [_p, _p, _u32, _p, _u32, _p]),
        "orc_rotate_hoisted": (None, [_p, _p, _u32, _p, _p, _u32, _p]),
        "orc_rescale": (None, [_p, _p, _u32, _u32, _p]),
        "orc_tensor": (None, [_p, _p, _p, _u32, _p]),
        "orc_relinearize": (None, [_p, _p, _u32, _p, _p]),
        "orc_draw": (_u64, [_u64, _u64]),
        "orc_stream_key": (_u64, [_u64, _u64, _u64]),
        "orc_sample_uniform": (None, [_u64, _u64, _p, _u32]),
        "orc_sample_ternary": (None, [_u64, _p, _u32]),
        "orc_sample_cbd": (None, [_u64, _p, _u32]),
        "orc_signed_to_eval": (None, [_p, _p, _u32, _u32, _p]),
        "orc_chacha20_block": (None, [_p, _u32, _p, _p]),
        "orc_set_sampling_key": (None, [_p]),
        "orc_stream_word": (_u64, [_u64, _u64, _u64, _u64]),
        "orc_keygen_secret": (None, [_u64, _u32, _p]),
        "orc_keygen_secret_sparse": (None, [_u64, _u32, _u32, _p]),
        "orc_keygen_public": (None, [_p, _p, _u64, _p]),
        "orc_keygen_switch": (None, [_p, _p, _p, _u64, _u64, _p]),
        "orc_keygen_galois": (None, [_p, _p, _u32, _u64, _p]),
        "orc_keygen_relin": (None, [_p, _p, _u64, _p]),
        "orc_encrypt_pk": (None, [_p, _p, _p, _u32, _u64, _p]),
        "orc_decrypt": (None, [_p, _p, _u32, _u32, _p, _p]),
        "orc_fft_special_inv": (None, [_p, _p, _u32]),
        "orc_fft_special": (None, [_p, _p, _u32]),
        "orc_encode": (ctypes.c_int, [_p, _p, _p, _u32, _u32, ctypes.c_double, _u32, _p]),
        "orc_decode": (None, [_p, _p, _u32, _u32, ctypes.c_double, _p, _p]),
        "orc_crt_centered": (None, [_p, _p, _u32, _p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class sampling_key:
    """Context manager: the ChaCha20 sampling family under `key` (32 bytes)
    for the oracle's key generation and encryption inside the block; the
    seeded family (the oracle's default) again afterwards."""

    def __init__(self, key: bytes):
        if len(key) != 32:
            raise ValueError("the ChaCha20 sampling key is 32 bytes")
        self.key = ctypes.create_string_buffer(bytes(key), 32)

    def __enter__(self):
        lib.orc_set_sampling_key(self.key)
        return self

    def __exit__(self, *exc):
        lib.orc_set_sampling_key(None)
        return False


def chacha20_block(key: bytes, counter: int, nonce: bytes) -> bytes:
    """RFC 8439 ChaCha20 block: 64 bytes of keystream."""
    k = np.frombuffer(bytes(key), dtype="<u4").astype(np.uint32).copy()
    nc = np.frombuffer(bytes(nonce), dtype="<u4").astype(np.uint32).copy()
    out = np.zeros(16, dtype=np.uint32)
    lib.orc_chacha20_block(k.ctypes.data, counter, nc.ctypes.data, out.ctypes.data)
    return out.astype("<u4").tobytes()


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def u64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint64)


# ---------------------------------------------------------------- moduli
def gen_moduli(log_n: int, depth: int, scale_bits: int, first_bits: int, dnum: int):
    q = np.zeros(depth + 1, dtype=np.uint64)
    p = np.zeros(64, dtype=np.uint64)
    k = lib.orc_gen_moduli(log_n, depth, scale_bits, first_bits, dnum, ptr(q), ptr(p), 64)
    if k < 0:
        raise ValueError("moduli generation failed")
    return [int(x) for x in q], [int(x) for x in p[:k]]


def ntt_friendly_primes(log_n: int, bits: int, count: int, skip=()):
    """Descending primes q = 1 mod 2N below 2^bits."""
    m = 2 << log_n
    out, q = [], lib.orc_first_prime(bits, m)
    while len(out) < count:
        q = lib.orc_previous_prime(q, m)
        if q >= (1 << bits) or q in skip:
            continue
        out.append(int(q))
    return out


# ---------------------------------------------------------------- context
class Ctx:
    """Oracle context over Q = q[0..L) and P = p[0..K)."""

    def __init__(self, log_n: int, q, p, dnum: int):
        self.log_n, self.n = log_n, 1 << log_n
        self.q, self.p = [int(x) for x in q], [int(x) for x in p]
        self.L, self.K = len(self.q), len(self.p)
        self.mods = self.q + self.p
        self.alpha = -(-self.L // dnum)
        self.dnum = -(-self.L // self.alpha)
        qa, pa = u64(self.q), u64(self.p if self.p else [0])
        self.h = lib.orc_ctx_create(log_n, ptr(qa), self.L, ptr(pa), self.K, dnum)

    def __del__(self):
        h, self.h = getattr(self, "h", None), None
        if h:
            lib.orc_ctx_destroy(h)

    def psi(self, idx):
        return int(lib.orc_ctx_psi(self.h, idx))

    def ntt_fwd(self, a, idx):
        a = u64(a).copy()
        lib.orc_ctx_ntt_fwd(self.h, ptr(a), idx)
        return a

    def ntt_inv(self, a, idx):
        a = u64(a).copy()
        lib.orc_ctx_ntt_inv(self.h, ptr(a), idx)
        return a

    def ntt_fwd_batch(self, data, limb0=0, nthreads=1):
        d = u64(data).copy()
        npoly, nlimb = int(np.prod(d.shape[:-2])) if d.ndim > 2 else 1, d.shape[-2]
        lib.orc_ntt_fwd_batch(self.h, ptr(d), npoly, limb0, nlimb, nthreads)
        return d

    def ntt_inv_batch(self, data, limb0=0, nthreads=1):
        d = u64(data).copy()
        npoly, nlimb = int(np.prod(d.shape[:-2])) if d.ndim > 2 else 1, d.shape[-2]
        lib.orc_ntt_inv_batch(self.h, ptr(d), npoly, limb0, nlimb, nthreads)
        return d

    def mac(self, x, w, nthreads=1):
        x, w = u64(x), u64(w)
        ncts, nq = x.shape[0], x.shape[2]
        acc = np.zeros((2, nq, self.n), dtype=np.uint64)
        lib.orc_mac_batch(self.h, ptr(x), ptr(w), ncts, nq, ptr(acc), nthreads)
        return acc

    def add(self, a, b):
        """a + b mod q_l limb by limb for polys [..., nq, N] (EvalAdd)."""
        a, b = u64(a), u64(b)
        nq = a.shape[-2]
        npoly = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
        out = np.zeros_like(a)
        lib.orc_add(self.h, ptr(a), ptr(b), npoly, nq, ptr(out))
        return out

    def num_digits(self, nq):
        return int(lib.orc_num_digits(self.h, nq))

    def modup(self, a):
        a = u64(a)
        nq = a.shape[0]
        out = np.zeros((self.num_digits(nq), nq + self.K, self.n), dtype=np.uint64)
        lib.orc_modup(self.h, ptr(a), nq, ptr(out))
        return out

    def ksk_inner(self, digits, key):
        digits, key = u64(digits), u64(key)
        nq = digits.shape[1] - self.K
        out = np.zeros((2, nq + self.K, self.n), dtype=np.uint64)
        lib.orc_ksk_inner(self.h, ptr(digits), nq, ptr(key), ptr(out))
        return out

    def moddown(self, ext):
        ext = u64(ext)
        nq = ext.shape[0] - self.K
        out = np.zeros((nq, self.n), dtype=np.uint64)
        lib.orc_moddown(self.h, ptr(ext), nq, ptr(out))
        return out

    def keyswitch(self, a, key):
        a, key = u64(a), u64(key)
        out = np.zeros((2, a.shape[0], self.n), dtype=np.uint64)
        lib.orc_keyswitch(self.h, ptr(a), a.shape[0], ptr(key), ptr(out))
        return out

    def rotate(self, ct, key, galois):
        ct, key = u64(ct), u64(key)
        out = np.zeros_like(ct)
        lib.orc_rotate(self.h, ptr(ct), ct.shape[1], ptr(key), galois, ptr(out))
        return out

    def rotate_hoisted(self, ct, digits, key, galois):
        """One rotation of a hoisted set: digits = self.modup(ct[1])."""
        ct, digits, key = u64(ct), u64(digits), u64(key)
        out = np.zeros_like(ct)
        lib.orc_rotate_hoisted(self.h, ptr(ct), ct.shape[1], ptr(digits), ptr(key), galois,
                               ptr(out))
        return out

    def rescale(self, x):
        x = u64(x)
        npoly, nq = x.shape[0], x.shape[1]
        out = np.zeros((npoly, nq - 1, self.n), dtype=np.uint64)
        lib.orc_rescale(self.h, ptr(x), npoly, nq, ptr(out))
        return out

    def tensor(self, a, b):
        a, b = u64(a), u64(b)
        out = np.zeros((3, a.shape[1], self.n), dtype=np.uint64)
        lib.orc_tensor(self.h, ptr(a), ptr(b), a.shape[1], ptr(out))
        return out

    def relinearize(self, ct3, key):
        ct3, key = u64(ct3), u64(key)
        out = np.zeros((2, ct3.shape[1], self.n), dtype=np.uint64)
        lib.orc_relinearize(self.h, ptr(ct3), ct3.shape[1], ptr(key), ptr(out))
        return out

    # ------------------------------------------------------------ keys
    def secret(self, seed):
        s = np.zeros(self.n, dtype=np.int64)
        lib.orc_keygen_secret(seed, self.n, ptr(s))
        return s

    def secret_sparse(self, seed, h):
        """Sparse-ternary secret with exactly h coefficients +-1."""
        s = np.zeros(self.n, dtype=np.int64)
        lib.orc_keygen_secret_sparse(seed, self.n, h, ptr(s))
        return s

    def signed_to_eval(self, coef, idx0, nlimb):
        coef = np.ascontiguousarray(coef, dtype=np.int64)
        out = np.zeros((nlimb, self.n), dtype=np.uint64)
        lib.orc_signed_to_eval(self.h, ptr(coef), idx0, nlimb, ptr(out))
        return out

    def public_key(self, s, seed):
        s = np.ascontiguousarray(s, dtype=np.int64)
        pk = np.zeros((2, self.L, self.n), dtype=np.uint64)
        lib.orc_keygen_public(self.h, ptr(s), seed, ptr(pk))
        return pk

    def galois_key(self, s, galois, seed):
        s = np.ascontiguousarray(s, dtype=np.int64)
        key = np.zeros((self.dnum, 2, self.L + self.K, self.n), dtype=np.uint64)
        lib.orc_keygen_galois(self.h, ptr(s), galois, seed, ptr(key))
        return key

    def relin_key(self, s, seed):
        s = np.ascontiguousarray(s, dtype=np.int64)
        key = np.zeros((self.dnum, 2, self.L + self.K, self.n), dtype=np.uint64)
        lib.orc_keygen_relin(self.h, ptr(s), seed, ptr(key))
        return key

    def encrypt(self, pk, m, seed):
        pk, m = u64(pk), u64(m)
        ct = np.zeros((2, m.shape[0], self.n), dtype=np.uint64)
        lib.orc_encrypt_pk(self.h, ptr(pk), ptr(m), m.shape[0], seed, ptr(ct))
        return ct

    def decrypt(self, ct, s):
        ct = u64(ct)
        s = np.ascontiguousarray(s, dtype=np.int64)
        m = np.zeros((ct.shape[1], self.n), dtype=np.uint64)
        lib.orc_decrypt(self.h, ptr(ct), ct.shape[0], ct.shape[1], ptr(s), ptr(m))
        return m

    # ------------------------------------------------------------ encoding
    def encode(self, values, slots, scale, nq):
        v = np.asarray(values)
        re = np.ascontiguousarray(np.real(v), dtype=np.float64)
        im = np.ascontiguousarray(np.imag(v), dtype=np.float64)
        out = np.zeros((nq, self.n), dtype=np.uint64)
        st = lib.orc_encode(self.h, ptr(re), ptr(im), len(v), slots, scale, nq, ptr(out))
        if st != 0:
            raise ValueError("encode: value out of range")
        return out

    def decode(self, poly, slots, scale):
        poly = u64(poly)
        re = np.zeros(slots)
        im = np.zeros(slots)
        lib.orc_decode(self.h, ptr(poly), poly.shape[0], slots, scale, ptr(re), ptr(im))
        return re + 1j * im

    def crt_centered(self, coef):
        coef = u64(coef)
        out = np.zeros(self.n)
        lib.orc_crt_centered(self.h, ptr(coef), coef.shape[0], ptr(out))
        return out


def galois_elt(step: int, n: int) -> int:
    return int(lib.orc_galois_elt(step, n))


def fft_special_inv(values):
    v = np.asarray(values, dtype=np.complex128)
    re, im = np.ascontiguousarray(v.real), np.ascontiguousarray(v.imag)
    lib.orc_fft_special_inv(ptr(re), ptr(im), len(v))
    return re + 1j * im


def fft_special(values):
    v = np.asarray(values, dtype=np.complex128)
    re, im = np.ascontiguousarray(v.real), np.ascontiguousarray(v.imag)
    lib.orc_fft_special(ptr(re), ptr(im), len(v))
    return re + 1j * im


def ref_driver_available() -> bool:
    return os.path.exists(REF_DRIVER)


def ref_driver(lines):
    """Run the reference-header driver (only where it was built)."""
    out = subprocess.run([REF_DRIVER], input="\n".join(lines) + "\n", capture_output=True,
                         text=True, check=True).stdout
    return out.splitlines()
