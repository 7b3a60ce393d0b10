"""Thin object layer over the C ABI: contexts, device polys and keys.

Arrays cross the boundary as numpy uint64 in the limb-major layout
[poly][limb][N]; device work runs on the context's HIP stream and every
download synchronises.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import call

_u64p = ctypes.POINTER(ctypes.c_uint64)


def _ptr(a: np.ndarray) -> int:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


def gen_moduli(log_n: int, depth: int, scale_bits: int, first_bits: int, dnum: int):
    """FLEXIBLEAUTO Q chain (depth+1 primes) and HYBRID P primes (host only)."""
    q = np.zeros(depth + 1, dtype=np.uint64)
    p = np.zeros(64, dtype=np.uint64)
    k = ctypes.c_uint32(0)
    call("fhe_gen_moduli", log_n, depth, scale_bits, first_bits, dnum, _ptr(q), _ptr(p), 64,
         ctypes.byref(k))
    return [int(x) for x in q], [int(x) for x in p[: k.value]]


class Context:
    """Device context over Q = q[0..L) and P = p[0..K) for ring 2^log_n."""

    def __init__(self, log_n: int, q, p, dnum: int, device: int = 0,
                 sampling: str = "chacha20", sampling_key: bytes | None = None):
        """sampling: "chacha20" (default; keys and encryption samples from
        ChaCha20 under a 32-byte master key, `sampling_key` or fresh OS
        entropy) or "seeded" (the seed of each call alone fixes its samples:
        reproducible for parity tests, not secure)."""
        qa = np.ascontiguousarray(q, dtype=np.uint64)
        pa = np.ascontiguousarray(p if len(p) else [0], dtype=np.uint64)
        h = ctypes.c_void_p()
        call("fhe_context_create", log_n, _ptr(qa), len(qa), _ptr(pa), len(p), dnum, device,
             ctypes.byref(h))
        self._h = h
        self.device = device
        self.set_sampling(sampling, sampling_key)
        info = np.zeros(5, dtype=np.uint32)
        call("fhe_context_info", h, _ptr(info))
        self.log_n, self.L, self.K, self.dnum, self.alpha = (int(x) for x in info)
        self.n = 1 << self.log_n
        mods = np.zeros(self.L + self.K, dtype=np.uint64)
        psi = np.zeros(self.L + self.K, dtype=np.uint64)
        call("fhe_context_moduli", h, _ptr(mods), _ptr(psi))
        self.mods = [int(x) for x in mods]
        self.psi = [int(x) for x in psi]
        self.q, self.p = self.mods[: self.L], self.mods[self.L:]

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("context is closed")
        return self._h

    def set_sampling(self, sampling: str = "chacha20", key: bytes | None = None):
        if sampling == "chacha20":
            if key is not None and len(key) != 32:
                raise ValueError("the ChaCha20 sampling key is 32 bytes")
            buf = None if key is None else ctypes.create_string_buffer(bytes(key), 32)
            call("fhe_context_set_sampling", self.handle, 0, buf)
        elif sampling == "seeded":
            if key is not None:
                raise ValueError("the seeded sampling family takes no key")
            call("fhe_context_set_sampling", self.handle, 1, None)
        else:
            raise ValueError(f"unknown sampling family {sampling!r}")
        self.sampling = sampling

    def close(self):
        if getattr(self, "_h", None):
            call("fhe_context_destroy", self._h)
            self._h = None

    def __del__(self):
        if _lib.alive:
            try:
                self.close()
            except Exception:
                pass

    def sync(self):
        call("fhe_sync", self.handle)

    def set_stream(self, stream_ptr: int | None):
        call("fhe_context_set_stream", self.handle, stream_ptr)

    # ---------------------------------------------------------------- polys
    def poly(self, npoly: int, nlimb: int) -> "Poly":
        return Poly(self, npoly, nlimb)

    def upload(self, array) -> "Poly":
        a = np.ascontiguousarray(array, dtype=np.uint64)
        if a.ndim == 2:
            a = a[None]
        p = Poly(self, a.shape[0], a.shape[1])
        call("fhe_poly_upload", p.handle, _ptr(a), a.shape[0], a.shape[1])
        return p

    def load_key(self, array) -> "Key":
        a = np.ascontiguousarray(array, dtype=np.uint64)
        if a.shape != (self.dnum, 2, self.L + self.K, self.n):
            raise ValueError(f"key shape {a.shape} != {(self.dnum, 2, self.L + self.K, self.n)}")
        h = ctypes.c_void_p()
        call("fhe_key_load", self.handle, _ptr(a), ctypes.byref(h))
        return Key(self, h)

    # ------------------------------------------------------------- profiling
    def profile_begin(self):
        call("fhe_profile_begin", self.handle)

    def profile_end(self) -> dict:
        """Per-kernel {name: (launches, total_ms)} from HIP events."""
        import json
        buf = ctypes.create_string_buffer(1 << 16)
        call("fhe_profile_end", self.handle, buf, len(buf))
        return {k: (int(v[0]), float(v[1])) for k, v in json.loads(buf.value.decode()).items()}

    # ----------------------------------------------------------- raw batches
    def ntt_forward_dev(self, dev_ptr: int, npoly: int, nlimb: int, limb0: int = 0):
        call("fhe_ntt_forward", self.handle, ctypes.c_void_p(dev_ptr), npoly, nlimb, limb0)

    def ntt_inverse_dev(self, dev_ptr: int, npoly: int, nlimb: int, limb0: int = 0):
        call("fhe_ntt_inverse", self.handle, ctypes.c_void_p(dev_ptr), npoly, nlimb, limb0)

    def mac_dev(self, x_ptr: int, w_ptr: int, count: int, nq: int, acc_ptr: int):
        call("fhe_mac", self.handle, ctypes.c_void_p(x_ptr), ctypes.c_void_p(w_ptr), count, nq,
             ctypes.c_void_p(acc_ptr))

    # ------------------------------------------------------------ arithmetic
    def _out(self, out, npoly, nlimb):
        return out if out is not None else Poly(self, npoly, nlimb)

    def add(self, a, b, out=None):
        out = self._out(out, a.npoly, a.nlimb)
        call("fhe_add", out.handle, a.handle, b.handle)
        return out

    def sub(self, a, b, out=None):
        out = self._out(out, a.npoly, a.nlimb)
        call("fhe_sub", out.handle, a.handle, b.handle)
        return out

    def negate(self, a, out=None):
        out = self._out(out, a.npoly, a.nlimb)
        call("fhe_negate", out.handle, a.handle)
        return out

    def mul_plain(self, ct, pt, out=None):
        out = self._out(out, ct.npoly, ct.nlimb)
        call("fhe_mul_plain", out.handle, ct.handle, pt.handle)
        return out

    def add_plain(self, ct, pt, out=None):
        out = self._out(out, ct.npoly, ct.nlimb)
        call("fhe_add_plain", out.handle, ct.handle, pt.handle)
        return out

    def linear_wsum(self, terms, weights, nlimb: int, out=None):
        """sum_i weights[i] * terms[i] (Python integers, |w| < 2^126) over the
        first nlimb limbs of 2-poly ciphertexts, in one pass."""
        if len(terms) != len(weights) or not terms:
            raise ValueError("linear_wsum needs matching, non-empty terms and weights")
        w = np.zeros(2 * len(weights), dtype=np.uint64)
        for i, m in enumerate(weights):
            m = int(m)
            if m.bit_length() > 126:
                raise ValueError("weight does not fit 127 bits")
            w[2 * i] = m & 0xFFFFFFFFFFFFFFFF
            w[2 * i + 1] = (m >> 64) & 0xFFFFFFFFFFFFFFFF
        out = self._out(out, 2, nlimb)
        hs = (ctypes.c_void_p * len(terms))(*[t.handle.value for t in terms])
        call("fhe_linear_wsum", out.handle, hs, _ptr(w), len(terms), nlimb)
        return out

    def mul_const(self, a, consts, out=None):
        c = np.ascontiguousarray(consts, dtype=np.uint64)
        out = self._out(out, a.npoly, a.nlimb)
        call("fhe_mul_const", out.handle, a.handle, _ptr(c))
        return out

    def add_const(self, a, consts, out=None):
        c = np.ascontiguousarray(consts, dtype=np.uint64)
        out = self._out(out, a.npoly, a.nlimb)
        call("fhe_add_const", out.handle, a.handle, _ptr(c))
        return out

    def mul_int(self, a, value: int, out=None):
        out = self._out(out, a.npoly, a.nlimb)
        call("fhe_mul_int", out.handle, a.handle, int(value))
        return out

    def drop_limbs(self, a, nlimb: int, out=None):
        out = self._out(out, a.npoly, nlimb)
        call("fhe_drop_limbs", out.handle, a.handle, nlimb)
        return out

    def mod_raise(self, a, nlimb: int, out=None):
        """Limb 0 of every poly, centred mod q0, lifted to nlimb limbs."""
        out = self._out(out, a.npoly, nlimb)
        call("fhe_mod_raise", out.handle, a.handle, nlimb)
        return out

    def rescale(self, a, out=None):
        out = self._out(out, a.npoly, a.nlimb - 1)
        call("fhe_rescale", out.handle, a.handle)
        return out

    def rescale_many(self, polys, outs=None):
        """Rescale every poly set of `polys` (one shape) in shared launches;
        the same polys as rescale() of each."""
        count = len(polys)
        outs = outs if outs is not None else [Poly(self, a.npoly, a.nlimb - 1) for a in polys]
        ah = (ctypes.c_void_p * max(count, 1))(*([a.handle.value for a in polys] or [None]))
        oh = (ctypes.c_void_p * max(count, 1))(*([o.handle.value for o in outs] or [None]))
        call("fhe_rescale_many", oh, ah, count)
        return outs

    def tensor(self, a, b):
        out = Poly(self, 3, a.nlimb)
        call("fhe_tensor", out.handle, a.handle, b.handle)
        return out

    def keyswitch(self, a, key, out=None):
        out = self._out(out, 2, a.nlimb)
        call("fhe_keyswitch", out.handle, a.handle, key.handle)
        return out

    def relinearize(self, ct3, key, out=None):
        out = self._out(out, 2, ct3.nlimb)
        call("fhe_relinearize", out.handle, ct3.handle, key.handle)
        return out

    def relinearize_many(self, ct3s, key, outs=None):
        """Relinearize every 3-poly tensor of `ct3s` (one level) in one
        batched key switch; the same polys as relinearize() of each."""
        count = len(ct3s)
        outs = outs if outs is not None else [Poly(self, 2, t.nlimb) for t in ct3s]
        th = (ctypes.c_void_p * max(count, 1))(*([t.handle.value for t in ct3s] or [None]))
        oh = (ctypes.c_void_p * max(count, 1))(*([o.handle.value for o in outs] or [None]))
        call("fhe_relinearize_many", oh, th, count, key.handle)
        return outs

    def rotate(self, ct, key, galois: int, out=None):
        out = self._out(out, 2, ct.nlimb)
        call("fhe_rotate", out.handle, ct.handle, key.handle, galois)
        return out

    def rotation_precompute(self, ct) -> "Poly":
        h = ctypes.c_void_p()
        call("fhe_rotation_precompute", ct.handle, ctypes.byref(h))
        return Poly(self, handle=h)

    def rotate_hoisted(self, ct, digits, keys, galois, outs=None):
        count = len(keys)
        outs = outs if outs is not None else [Poly(self, 2, ct.nlimb) for _ in range(count)]
        kh = (ctypes.c_void_p * count)(*[k.handle.value for k in keys])
        oh = (ctypes.c_void_p * count)(*[o.handle.value for o in outs])
        ga = np.ascontiguousarray(galois, dtype=np.uint32)
        call("fhe_rotate_hoisted", ct.handle, digits.handle, kh, _ptr(ga), count, oh)
        return outs

    def rotate_many(self, cts, keys, galois, outs=None):
        """Rotate cts[r] by keys[r] / galois[r] in one batched key switch."""
        count = len(cts)
        outs = outs if outs is not None else [Poly(self, 2, c.nlimb) for c in cts]
        ch = (ctypes.c_void_p * count)(*[c.handle.value for c in cts])
        kh = (ctypes.c_void_p * count)(*[k.handle.value for k in keys])
        oh = (ctypes.c_void_p * count)(*[o.handle.value for o in outs])
        ga = np.ascontiguousarray(galois, dtype=np.uint32)
        call("fhe_rotate_many", oh, ch, kh, _ptr(ga), count)
        return outs

    def linear_transform(self, ct, pts, bstep: int, baby_keys, baby_galois, giant_key=None,
                         giant_galois: int = 1, out=None):
        """BSGS transform: sum_g rot_giant^g(sum_b pts[g*bstep+b] * rot_b(ct)).

        pts: list of one-poly plaintexts or None (zero diagonal), already
        pre-rotated for their giant step; baby_keys / baby_galois: bstep - 1
        entries (None where unused); giant_key rotates by bstep strides."""
        count = len(pts)
        out = self._out(out, 2, ct.nlimb)
        ph = (ctypes.c_void_p * count)(*[p.handle.value if p is not None else None
                                         for p in pts])
        nb = max(1, bstep - 1)
        bk = (ctypes.c_void_p * nb)(*([k.handle.value if k is not None else None
                                       for k in baby_keys] + [None] * (nb - len(baby_keys))))
        bg = np.zeros(nb, dtype=np.uint32)
        bg[: len(baby_galois)] = baby_galois
        call("fhe_linear_transform", out.handle, ct.handle, ph, count, bstep, bk, _ptr(bg),
             giant_key.handle if giant_key is not None else None, giant_galois)
        return out

    def linear_transform_hoisted(self, ct, pts, bstep: int, baby_keys, baby_galois,
                                 giant_keys=(), giant_galois=(), out=None):
        """The same sum with baby b = ct rotated by baby_keys[b] (b = 0 ..
        min(bstep, count) - 1; baby_keys[0] None: baby 0 is ct, else it is
        ct's offset rotation and the other keys include the offset), all
        from one ModUp; giant_keys: one key (Horner's rule) or one per giant
        step g = 1 .. G - 1 (rotations by g giant strides, one batch)."""
        count = len(pts)
        out = self._out(out, 2, ct.nlimb)
        ph = (ctypes.c_void_p * count)(*[p.handle.value if p is not None else None
                                         for p in pts])
        nb = max(1, min(bstep, count))
        bk = (ctypes.c_void_p * nb)(*([k.handle.value if k is not None else None
                                       for k in baby_keys] + [None] * (nb - len(baby_keys))))
        bg = np.ones(nb, dtype=np.uint32)
        bg[: len(baby_galois)] = baby_galois
        ng = len(giant_keys)
        gk = (ctypes.c_void_p * max(ng, 1))(*([k.handle.value for k in giant_keys] or [None]))
        gg = np.ones(max(ng, 1), dtype=np.uint32)
        gg[:ng] = giant_galois
        call("fhe_linear_transform_hoisted", out.handle, ct.handle, ph, count, bstep, bk,
             _ptr(bg), gk, _ptr(gg), ng)
        return out

    def linear_transform_hoisted_many(self, cts, pts, bstep: int, baby_keys, baby_galois,
                                      giant_keys=(), giant_galois=(), outs=None) -> list:
        """linear_transform_hoisted of every ciphertext of `cts` (one limb
        count) with the same diagonals and keys, in shared launches; the
        same polys as one call per ciphertext."""
        count, m = len(pts), len(cts)
        outs = list(outs) if outs is not None else [Poly(self, 2, c.nlimb) for c in cts]
        ch = (ctypes.c_void_p * m)(*[c.handle.value for c in cts])
        oh = (ctypes.c_void_p * m)(*[o.handle.value for o in outs])
        ph = (ctypes.c_void_p * count)(*[p.handle.value if p is not None else None
                                         for p in pts])
        nb = max(1, min(bstep, count))
        bk = (ctypes.c_void_p * nb)(*([k.handle.value if k is not None else None
                                       for k in baby_keys] + [None] * (nb - len(baby_keys))))
        bg = np.ones(nb, dtype=np.uint32)
        bg[: len(baby_galois)] = baby_galois
        ng = len(giant_keys)
        gk = (ctypes.c_void_p * max(ng, 1))(*([k.handle.value for k in giant_keys] or [None]))
        gg = np.ones(max(ng, 1), dtype=np.uint32)
        gg[:ng] = giant_galois
        call("fhe_linear_transform_hoisted_many", oh, ch, m, ph, count, bstep, bk, _ptr(bg),
             gk, _ptr(gg), ng)
        return outs

    # -------------------------------------------------------------- encoding
    def encode(self, values, slots: int, scale: float, nlimb: int, out=None) -> "Poly":
        v = np.asarray(values)
        re = np.ascontiguousarray(np.real(v), dtype=np.float64)
        im = np.ascontiguousarray(np.imag(v), dtype=np.float64)
        out = self._out(out, 1, nlimb)
        call("fhe_encode", self.handle, _ptr(re), _ptr(im), len(v), slots, float(scale), nlimb,
             out.handle)
        return out

    def encode_many(self, rows, slots: int, scale: float, nlimb: int) -> list:
        """One encode per row of `rows` (equal-length value vectors) in shared
        launches; the same polys as encode() of each row."""
        v = np.asarray(rows)
        if v.ndim != 2:
            raise ValueError("encode_many takes a 2-D array of rows")
        re = np.ascontiguousarray(np.real(v), dtype=np.float64)
        im = np.ascontiguousarray(np.imag(v), dtype=np.float64) if np.iscomplexobj(v) else None
        outs = [Poly(self, 1, nlimb) for _ in range(v.shape[0])]
        hs = (ctypes.c_void_p * max(len(outs), 1))(*([o.handle.value for o in outs] or [None]))
        call("fhe_encode_many", self.handle, _ptr(re), _ptr(im) if im is not None else None,
             v.shape[1], v.shape[0], slots, float(scale), nlimb, hs)
        return outs

    def decode(self, pt, slots: int, scale: float) -> np.ndarray:
        re = np.zeros(slots)
        im = np.zeros(slots)
        call("fhe_decode", self.handle, pt.handle, slots, float(scale), _ptr(re), _ptr(im))
        return re + 1j * im

    # ---------------------------------------------------------- key material
    def keygen_secret(self, seed: int) -> np.ndarray:
        s = np.zeros(self.n, dtype=np.int64)
        call("fhe_keygen_secret", self.handle, seed, _ptr(s))
        return s

    def keygen_secret_sparse(self, seed: int, h: int) -> np.ndarray:
        """Sparse-ternary secret: exactly h coefficients +-1, the rest 0."""
        s = np.zeros(self.n, dtype=np.int64)
        call("fhe_keygen_secret_sparse", self.handle, seed, h, _ptr(s))
        return s

    def keygen_public(self, s, seed: int) -> "Poly":
        s = np.ascontiguousarray(s, dtype=np.int64)
        pk = Poly(self, 2, self.L)
        call("fhe_keygen_public", self.handle, _ptr(s), seed, pk.handle)
        return pk

    def keygen_relin(self, s, seed: int) -> "Key":
        s = np.ascontiguousarray(s, dtype=np.int64)
        h = ctypes.c_void_p()
        call("fhe_keygen_relin", self.handle, _ptr(s), seed, ctypes.byref(h))
        return Key(self, h)

    def keygen_galois(self, s, galois: int, seed: int) -> "Key":
        s = np.ascontiguousarray(s, dtype=np.int64)
        h = ctypes.c_void_p()
        call("fhe_keygen_galois", self.handle, _ptr(s), galois, seed, ctypes.byref(h))
        return Key(self, h)

    def encrypt(self, pk, pt, seed: int) -> "Poly":
        ct = Poly(self, 2, pt.nlimb)
        call("fhe_encrypt", ct.handle, pk.handle, pt.handle, seed)
        return ct

    def decrypt(self, ct, s) -> "Poly":
        s = np.ascontiguousarray(s, dtype=np.int64)
        pt = Poly(self, 1, ct.nlimb)
        call("fhe_decrypt", pt.handle, ct.handle, _ptr(s))
        return pt


class Poly:
    """Device-resident RNS poly set [npoly][nlimb][N] owned by a Context."""

    def __init__(self, ctx: Context, npoly: int = 0, nlimb: int = 0, handle=None):
        self.ctx = ctx
        if handle is None:
            handle = ctypes.c_void_p()
            call("fhe_poly_create", ctx.handle, npoly, nlimb, ctypes.byref(handle))
        self._h = handle

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("poly is closed")
        return self._h

    @property
    def shape(self):
        a, b = ctypes.c_uint32(), ctypes.c_uint32()
        call("fhe_poly_shape", self.handle, ctypes.byref(a), ctypes.byref(b))
        return a.value, b.value

    @property
    def npoly(self):
        return self.shape[0]

    @property
    def nlimb(self):
        return self.shape[1]

    def data_ptr(self) -> int:
        d = ctypes.c_void_p()
        call("fhe_poly_data", self.handle, ctypes.byref(d))
        return d.value or 0

    def numpy(self) -> np.ndarray:
        npoly, nlimb = self.shape
        out = np.zeros((npoly, nlimb, self.ctx.n), dtype=np.uint64)
        call("fhe_poly_download", self.handle, _ptr(out))
        return out

    def copy(self) -> "Poly":
        p = Poly(self.ctx, 0, 0)
        call("fhe_poly_copy", p.handle, self.handle)
        return p

    def close(self):
        if getattr(self, "_h", None):
            call("fhe_poly_destroy", self._h)
            self._h = None

    def __del__(self):
        if _lib.alive:
            try:
                self.close()
            except Exception:
                pass


class Key:
    """Hybrid switching key resident in HBM."""

    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self._h = handle

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("key is closed")
        return self._h

    def numpy(self) -> np.ndarray:
        """The key's residues [dnum][2][L+K][N] in the form load_key takes."""
        c = self.ctx
        out = np.empty((c.dnum, 2, c.L + c.K, c.n), dtype=np.uint64)
        call("fhe_key_download", self.handle, _ptr(out))
        return out

    def close(self):
        if getattr(self, "_h", None):
            call("fhe_key_destroy", self._h)
            self._h = None

    def __del__(self):
        if _lib.alive:
            try:
                self.close()
            except Exception:
                pass


def galois_element(step: int, n: int) -> int:
    """5^step mod 2N (negative steps use 5^-1), OpenFHE's rotation index map."""
    order = n // 2
    return pow(5, step % order, 2 * n)


def conjugation_element(n: int) -> int:
    return 2 * n - 1
