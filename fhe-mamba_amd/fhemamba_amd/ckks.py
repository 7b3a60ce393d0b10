"""OpenFHE-shaped CKKS interface over the device library.

The names, argument meanings and error behaviour follow the OpenFHE /
FIDESlib surface that the reference drives:
  * parameters and context: src/fhemamba/ckks_probes.py:167-201 and
    native/fideslib_stage0/src/packed_fideslib.cpp:1060-1090
    (CCParamsCKKSRNS setters, GenCryptoContext, Enable, KeyGen,
    EvalMultKeyGen, EvalRotateKeyGen);
  * evaluation: packed_fideslib.cpp:117-270 (EvalAdd/EvalSub/EvalMult with
    ciphertexts, plaintexts and doubles, EvalMultMutableInPlace,
    EvalSquareInPlace, EvalRotate(InPlace), EvalFastRotationPrecompute /
    EvalFastRotation, RescaleInPlace, GetLevel / SetLevel /
    GetNoiseScaleDeg), patches/fideslib-v2.1.0-conjugate-api.patch
    (EvalConjugate) and patches/fideslib-v2.1.0-linear-transform-api.patch
    (LinearTransformInPlace).

Only what that path uses is provided: CKKS-RNS with HYBRID key switching
and FLEXIBLEAUTO scaling.  Scale bookkeeping (FLEXIBLEAUTO):
  * sf[0] is the last Q prime and sf[l] = sf[l-1]^2 / q_{L-l}: a degree-1
    ciphertext at level l (l limbs dropped) carries scale sf[l], degree 2
    carries sf[l]^2, and rescaling degree 2 at level l gives sf[l+1];
  * EvalMult rescales degree-2 operands first, then brings both to one
    level; multiplying by a double scales it by sf[level];
  * EvalAdd / EvalSub bring the operands to one level, degree and scale:
    the operand with more limbs is multiplied by the integer nearest to the
    scale ratio (times the prime it then drops) and rescaled;
  * RescaleInPlace rescales while the degree is 2 (a degree-1 ciphertext
    is left as it is).
The exact rounding of OpenFHE's scale adjustments, its PRNG and its
serialisation are not reproduced; results agree to CKKS precision.
"""
from __future__ import annotations

import enum
import math
import os
from typing import Iterable, Sequence

import numpy as np

from .core import Context, Poly, conjugation_element, galois_element, gen_moduli
from .rotation import bsgs_rotations  # noqa: F401
from .serial import (BINARY, JSON, DeserializeCiphertext, DeserializeCryptoContext,  # noqa: F401
                     DeserializePrivateKey, DeserializePublicKey, SerializeToFile, SerType)

__all__ = [
    "CCParamsCKKSRNS", "GenCryptoContext", "CryptoContext", "Ciphertext", "Plaintext",
    "KeyPair", "PublicKey", "PrivateKey", "ScalingTechnique", "KeySwitchTechnique",
    "SecretKeyDist", "SecurityLevel", "PKESchemeFeature",
]


class ScalingTechnique(enum.Enum):
    FIXEDMANUAL = 0
    FIXEDAUTO = 1
    FLEXIBLEAUTO = 2
    FLEXIBLEAUTOEXT = 3
    NORESCALE = 4
    COMPOSITESCALINGAUTO = 5
    COMPOSITESCALINGMANUAL = 6


class KeySwitchTechnique(enum.Enum):
    BV = 1
    HYBRID = 2


class SecretKeyDist(enum.Enum):
    GAUSSIAN = 0
    UNIFORM_TERNARY = 1
    SPARSE_TERNARY = 2


# Nonzero coefficients of a SPARSE_TERNARY secret (+-1 each, the rest 0).
SPARSE_HAMMING_WEIGHT = 192


class SecurityLevel(enum.Enum):
    HEStd_128_classic = 0
    HEStd_192_classic = 1
    HEStd_256_classic = 2
    HEStd_128_quantum = 3
    HEStd_192_quantum = 4
    HEStd_256_quantum = 5
    HEStd_NotSet = 6


class PKESchemeFeature(enum.Enum):
    PKE = 0x01
    KEYSWITCH = 0x02
    PRE = 0x04
    LEVELEDSHE = 0x08
    ADVANCEDSHE = 0x10
    MULTIPARTY = 0x20
    FHE = 0x40
    SCHEMESWITCH = 0x80


# Largest log2(Q*P) per ring dimension for a uniform-ternary secret
# (HomomorphicEncryption.org standard, classical attacks), used to pick or
# check the ring dimension as GenCryptoContext does.
_HE_STD_MAX_LOGQ = {
    SecurityLevel.HEStd_128_classic: {1024: 27, 2048: 54, 4096: 109, 8192: 218, 16384: 438,
                                      32768: 881, 65536: 1747, 131072: 3523},
    SecurityLevel.HEStd_192_classic: {1024: 19, 2048: 37, 4096: 75, 8192: 152, 16384: 305,
                                      32768: 611},
    SecurityLevel.HEStd_256_classic: {1024: 14, 2048: 29, 4096: 58, 8192: 118, 16384: 237,
                                      32768: 476},
}


class CCParamsCKKSRNS:
    """Parameter set; setter / getter names as OpenFHE's CCParams."""

    _FIELDS = {
        "MultiplicativeDepth": 1,
        "ScalingModSize": 50,
        "FirstModSize": 60,
        "RingDim": 0,
        "BatchSize": 0,
        "NumLargeDigits": 0,
        "KeySwitchTechnique": KeySwitchTechnique.HYBRID,
        "ScalingTechnique": ScalingTechnique.FLEXIBLEAUTO,
        "SecretKeyDist": SecretKeyDist.UNIFORM_TERNARY,
        "SecurityLevel": SecurityLevel.HEStd_128_classic,
    }

    def __init__(self):
        self._v = dict(self._FIELDS)

    def __getattr__(self, name):
        fields = type(self)._FIELDS
        if name.startswith("Set") and name[3:] in fields:
            return lambda value: self._v.__setitem__(name[3:], value)
        if name.startswith("Get") and name[3:] in fields:
            return lambda: self._v[name[3:]]
        raise AttributeError(name)

    def __repr__(self):
        return "CCParamsCKKSRNS(" + ", ".join(f"{k}={v}" for k, v in self._v.items()) + ")"


def _num_large_digits(requested: int, depth: int) -> int:
    """HYBRID digit count: the requested value, else 3 above depth 3, 2 for
    depth 1..3, 1 for depth 0."""
    if requested > 0:
        return int(requested)
    if depth > 3:
        return 3
    return 2 if depth > 0 else 1


def _log2_qp(q, p) -> float:
    return sum(math.log2(x) for x in list(q) + list(p))


# Classical-128 bound on the bit length of Q*P for a uniform-ternary secret
# with error sigma 3.19 (2024 Security Guidelines, Table 5.2), as the
# reference tabulates it: native/fideslib_stage0/src/fideslib_security.hpp:18-30.
CLASSICAL128_MAX_QP_BITS = {1024: 26, 2048: 53, 4096: 106, 8192: 214, 16384: 430, 32768: 868,
                            65536: 1747, 131072: 3523}
# Standard deviation of the encryption error.  OpenFHE samples a discrete
# Gaussian with sigma 3.19; this library draws a centred binomial with
# eta = 21 (variance 21 / 2, sigma 3.24), never narrower.
ERROR_SIGMA = math.sqrt(21 / 2)


def audit_chain(ring: int, q, p, dnum: int, *, security_level: "SecurityLevel",
                secret_dist: "SecretKeyDist", sigma: float = ERROR_SIGMA) -> dict:
    """Classical-128 audit of a HYBRID chain, the fields and rule of the
    reference's CkksSecurityAudit (fideslib_security.hpp:33-80): exact bit
    lengths of Q, P and Q*P (not sums of per-prime sizes), the guideline
    bound for the ring dimension, and a pass only for HEStd_128_classic
    with a uniform-ternary secret, sigma >= 3.19 and Q*P within the bound."""
    qprod, pprod = math.prod(int(x) for x in q), math.prod(int(x) for x in p)
    a = {
        "ring_dimension": int(ring),
        "q_bits": qprod.bit_length(),
        "p_bits": pprod.bit_length(),
        "qp_bits": (qprod * pprod).bit_length(),
        "q_towers": len(q),
        "p_towers": len(p),
        "hybrid_digits": int(dnum),
        "error_sigma": float(sigma),
        "guideline_max_qp_bits": CLASSICAL128_MAX_QP_BITS.get(int(ring), 0),
        "library_classical128": security_level == SecurityLevel.HEStd_128_classic,
        "uniform_ternary": secret_dist == SecretKeyDist.UNIFORM_TERNARY,
        "hybrid": True,
    }
    a["passed"] = bool(a["library_classical128"] and a["uniform_ternary"] and a["hybrid"]
                       and math.isfinite(sigma) and sigma >= 3.19
                       and a["guideline_max_qp_bits"] and a["q_towers"] and a["p_towers"]
                       and a["qp_bits"] <= a["guideline_max_qp_bits"])
    a["basis"] = "2024 Security Guidelines Table 5.2; classical RLWE parameter bound"
    return a


def flexibleauto_scaling_factors(q) -> list[float]:
    """FLEXIBLEAUTO scaling factor per level (limbs dropped) of the Q chain:
    sf[0] = q_{L-1} and sf[l] = sf[l-1]^2 / q_{L-l}, in double precision, so
    that rescaling a degree-2 ciphertext at level l lands on sf[l+1]."""
    L = len(q)
    sf = [float(q[-1])]
    for lev in range(1, L):
        sf.append(sf[-1] * sf[-1] / float(q[L - lev]))
    return sf


def select_chain(params: CCParamsCKKSRNS):
    """(ring dimension, Q primes, P primes, dnum) for a parameter set.

    With RingDim set, the chain is built for it and checked against the
    security table (unless HEStd_NotSet); otherwise the smallest tabulated
    ring dimension whose log2(Q*P) is within the bound is chosen."""
    g = params._v
    if g["KeySwitchTechnique"] != KeySwitchTechnique.HYBRID:
        raise NotImplementedError("only HYBRID key switching is implemented")
    if g["ScalingTechnique"] != ScalingTechnique.FLEXIBLEAUTO:
        raise NotImplementedError("only FLEXIBLEAUTO scaling is implemented")
    if g["SecretKeyDist"] not in (SecretKeyDist.UNIFORM_TERNARY, SecretKeyDist.SPARSE_TERNARY):
        raise NotImplementedError("only UNIFORM_TERNARY and SPARSE_TERNARY secrets are implemented")
    depth, sbits, fbits = (int(g["MultiplicativeDepth"]), int(g["ScalingModSize"]),
                           int(g["FirstModSize"]))
    if depth < 0 or not 20 <= sbits <= 60 or not sbits <= fbits <= 60:
        raise ValueError("need depth >= 0 and 20 <= ScalingModSize <= FirstModSize <= 60")
    dnum = _num_large_digits(int(g["NumLargeDigits"]), depth)
    ring, level = int(g["RingDim"]), g["SecurityLevel"]
    table = _HE_STD_MAX_LOGQ.get(level)
    if table is None and level != SecurityLevel.HEStd_NotSet:
        raise NotImplementedError(f"security level {level.name} is not tabulated")
    if ring:
        if ring & (ring - 1) or not 16 <= ring <= 1 << 17:
            raise ValueError("RingDim must be a power of two in [16, 2^17]")
        q, p = gen_moduli(ring.bit_length() - 1, depth, sbits, fbits, dnum)
        if table is not None and _log2_qp(q, p) > table.get(ring, 0):
            raise ValueError(f"RingDim {ring} does not give {level.name} for "
                             f"log2(QP) = {_log2_qp(q, p):.1f}")
        return ring, q, p, dnum
    if table is None:
        raise ValueError("RingDim must be set when the security level is HEStd_NotSet")
    for ring in sorted(table):
        try:
            q, p = gen_moduli(ring.bit_length() - 1, depth, sbits, fbits, dnum)
        except Exception:
            continue
        if _log2_qp(q, p) <= table[ring]:
            return ring, q, p, dnum
    raise ValueError("no tabulated ring dimension is large enough for this chain")


def GenCryptoContext(params: CCParamsCKKSRNS, seed: int | None = None,
                     device: int = 0) -> "CryptoContext":  # noqa: N802 - OpenFHE name
    """Build the prime chain, key-switching primes and device context.

    Without `seed` (the default) every key and encryption sample comes from
    ChaCha20 under a 256-bit master key drawn from OS entropy.  A `seed`
    selects the seeded sampling family instead: it fixes every sample drawn
    through this context, which makes runs reproducible for tests and
    benchmarks and is NOT secure (the public key reveals the seed)."""
    return CryptoContext(params, seed=seed, device=device)


class CryptoContext:
    def __init__(self, params: CCParamsCKKSRNS, seed: int | None = None, device: int = 0):
        g = params._v
        ring, q, p, self._dnum = select_chain(params)
        self._params = params
        self._ctx = Context(ring.bit_length() - 1, q, p, self._dnum, device,
                            sampling="chacha20" if seed is None else "seeded")
        self.n = ring
        self.L = len(q)
        batch = int(g["BatchSize"]) or ring // 2
        if batch & (batch - 1) or batch > ring // 2:
            raise ValueError("BatchSize must be a power of two <= RingDim / 2")
        self._slots = batch
        self._sf = flexibleauto_scaling_factors(q)
        self._features: set = set()
        self._relin = None
        self._galois: dict = {}
        # Per-call stream labels.  With ChaCha20 sampling they are public
        # nonces (the secrecy is the library's master key).
        self._seed = int.from_bytes(os.urandom(8), "little") if seed is None else int(seed)
        self._draws = 0
        self._cache: dict = {}
        self._boot = None
        self._secret_dist = g["SecretKeyDist"]
        from . import serial
        serial.register(self)

    # ------------------------------------------------------------ set-up
    def _next_seed(self) -> int:
        self._draws += 1
        x = (self._seed + self._draws * 0x9E3779B97F4A7C15) & (2**64 - 1)
        x ^= x >> 31
        return (x * 0xBF58476D1CE4E5B9) & (2**64 - 1)

    def Enable(self, feature):  # noqa: N802
        self._features.add(feature)

    def GetRingDimension(self) -> int:  # noqa: N802
        return self.n

    def GetCyclotomicOrder(self) -> int:  # noqa: N802
        return 2 * self.n

    def GetBatchSize(self) -> int:  # noqa: N802
        return self._slots

    def GetScalingFactorReal(self, level: int = 0) -> float:  # noqa: N802
        return self._sf[level]

    def GetModuli(self) -> tuple[list[int], list[int]]:  # noqa: N802
        return list(self._ctx.q), list(self._ctx.p)

    def SecurityAudit(self) -> dict:  # noqa: N802
        """This context's classical-128 audit (audit_chain; the reference's
        audit_ckks_context, fideslib_security.hpp:57-78)."""
        q, p = self.GetModuli()
        g = self._params._v
        return audit_chain(self.n, q, p, self._dnum, security_level=g["SecurityLevel"],
                           secret_dist=g["SecretKeyDist"])

    def RequireClassical128(self) -> dict:  # noqa: N802
        """The audit, or ValueError when it fails (require_classical128,
        fideslib_security.hpp:37-41)."""
        a = self.SecurityAudit()
        if not a["passed"]:
            raise ValueError("classical-128 CKKS audit failed: require HEStd_128_classic, "
                             "uniform ternary, sigma >= 3.19 and actual HYBRID Q*P within "
                             "the published dimension bound")
        return a

    @property
    def device(self) -> Context:
        """The underlying device context (raw residue-level operations)."""
        return self._ctx

    # ------------------------------------------------------------ keys
    def secret_hamming_weight(self) -> float:
        """Expected number of nonzero secret coefficients: h for a sparse
        secret, 2N/3 for a uniform-ternary one."""
        if self._secret_dist == SecretKeyDist.SPARSE_TERNARY:
            return float(SPARSE_HAMMING_WEIGHT)
        return 2.0 * self.n / 3.0

    def KeyGen(self) -> "KeyPair":  # noqa: N802
        if self._secret_dist == SecretKeyDist.SPARSE_TERNARY:
            s = self._ctx.keygen_secret_sparse(self._next_seed(),
                                               min(SPARSE_HAMMING_WEIGHT, self.n))
        else:
            s = self._ctx.keygen_secret(self._next_seed())
        sk = PrivateKey(self, s)
        pk = PublicKey(self, self._ctx.keygen_public(s, self._next_seed()))
        return KeyPair(pk, sk)

    def EvalMultKeyGen(self, secret_key: "PrivateKey"):  # noqa: N802
        self._relin = self._ctx.keygen_relin(secret_key.s, self._next_seed())

    def _galois_keygen(self, secret_key, elements):
        for g in elements:
            if g not in self._galois:
                self._galois[g] = self._ctx.keygen_galois(secret_key.s, g, self._next_seed())

    def EvalRotateKeyGen(self, secret_key: "PrivateKey", index_list: Iterable[int]):  # noqa: N802
        self._galois_keygen(secret_key, [galois_element(int(i), self.n) for i in index_list])

    EvalAtIndexKeyGen = EvalRotateKeyGen

    def EvalConjugateKeyGen(self, secret_key: "PrivateKey"):  # noqa: N802
        self._galois_keygen(secret_key, [conjugation_element(self.n)])

    def EvalAutomorphismKeyGen(self, secret_key: "PrivateKey", elements: Iterable[int]):  # noqa: N802
        self._galois_keygen(secret_key, [int(g) for g in elements])

    # ------------------------------------------------------------ key files
    def SerializeEvalMultKey(self, path: str, sertype=SerType.BINARY) -> bool:  # noqa: N802
        """The relinearisation key to a file (fhemamba_amd.serial)."""
        from . import serial
        serial._binary(sertype)
        return serial._ok(serial.save_eval_mult_key, path, self)

    def DeserializeEvalMultKey(self, path: str, sertype=SerType.BINARY) -> bool:  # noqa: N802
        from . import serial
        serial._binary(sertype)
        return serial._ok(serial.load_eval_mult_key, path, self)

    def SerializeEvalAutomorphismKey(self, path: str, sertype=SerType.BINARY) -> bool:  # noqa: N802
        """Every rotation / conjugation key of this context to one file."""
        from . import serial
        serial._binary(sertype)
        return serial._ok(serial.save_eval_automorphism_keys, path, self)

    def DeserializeEvalAutomorphismKey(self, path: str, sertype=SerType.BINARY) -> bool:  # noqa: N802
        from . import serial
        serial._binary(sertype)
        return serial._ok(serial.load_eval_automorphism_keys, path, self)

    def HasRotationKeys(self, index_list: Iterable[int]) -> bool:  # noqa: N802
        """Whether a rotation key for every index is present (generated or
        loaded)."""
        return all(galois_element(int(i), self.n) in self._galois for i in index_list)

    def HasConjugationKey(self) -> bool:  # noqa: N802
        return conjugation_element(self.n) in self._galois

    def _key_for(self, galois: int):
        try:
            return self._galois[galois]
        except KeyError:
            raise KeyError(f"no rotation key for automorphism index {galois}; "
                           "call EvalRotateKeyGen first") from None

    def _rotation_key(self, index: int):
        return self._key_for(galois_element(int(index), self.n))

    # ------------------------------------------------------------ encoding
    def _encode(self, values, level: int, deg: int, slots: int) -> "Plaintext":
        if not 0 <= level < self.L:
            raise ValueError(f"level {level} outside [0, {self.L - 1}]")
        if deg not in (1, 2):
            raise ValueError("noise scale degree must be 1 or 2")
        v = np.asarray(values, dtype=np.complex128).ravel()
        if len(v) > slots:
            raise ValueError(f"{len(v)} values do not fit {slots} slots")
        nq = self.L - level
        sf = self._sf[level]
        poly = self._ctx.encode(v, slots, sf, nq)
        scale = sf
        if deg == 2:
            c = int(round(sf))
            self._ctx.mul_const(poly, self._const_residues(c, nq), out=poly)
            scale = sf * c
        return Plaintext(self, poly, level, deg, scale, slots, v)

    def MakeCKKSPackedPlaintext(self, values, noiseScaleDeg: int = 1, level: int = 0,  # noqa: N802,N803
                                params=None, slots: int = 0) -> "Plaintext":
        return self._encode(values, int(level), int(noiseScaleDeg), int(slots) or self._slots)

    def MakeCKKSPackedPlaintexts(self, rows, noiseScaleDeg: int = 1, level: int = 0,  # noqa: N802,N803
                                 slots: int = 0) -> list:
        """MakeCKKSPackedPlaintext of every vector in `rows` at one level and
        degree, encoded in shared launches (fhe_encode_many): the same
        plaintexts as one call per vector."""
        level, deg, slots = int(level), int(noiseScaleDeg), int(slots) or self._slots
        if not 0 <= level < self.L:
            raise ValueError(f"level {level} outside [0, {self.L - 1}]")
        if deg not in (1, 2):
            raise ValueError("noise scale degree must be 1 or 2")
        vals = [np.asarray(r).ravel() for r in rows]
        if not vals:
            return []
        width = max(len(v) for v in vals)
        if width > slots:
            raise ValueError(f"{width} values do not fit {slots} slots")
        cplx = any(np.iscomplexobj(v) for v in vals)
        mat = np.zeros((len(vals), width), dtype=np.complex128 if cplx else np.float64)
        for i, v in enumerate(vals):
            mat[i, :len(v)] = v
        nq = self.L - level
        sf = self._sf[level]
        polys = self._ctx.encode_many(mat, slots, sf, nq)
        scale = sf
        if deg == 2:
            c = int(round(sf))
            res = self._const_residues(c, nq)
            for p in polys:
                self._ctx.mul_const(p, res, out=p)
            scale = sf * c
        return [Plaintext(self, p, level, deg, scale, slots, v) for p, v in zip(polys, vals)]

    def _const_residues(self, c: int, nq: int) -> np.ndarray:
        return np.array([c % qi for qi in self._ctx.q[:nq]], dtype=np.uint64)

    # ------------------------------------------------------------ encryption
    def Encrypt(self, a, b) -> "Ciphertext":  # noqa: N802
        pk, pt = (a, b) if isinstance(a, PublicKey) else (b, a)
        if not isinstance(pk, PublicKey) or not isinstance(pt, Plaintext):
            raise TypeError("Encrypt(publicKey, plaintext)")
        poly = self._ctx.encrypt(pk.poly, pt.poly, self._next_seed())
        return Ciphertext(self, poly, pt.level, pt.deg, pt.scale, pt.slots)

    def Decrypt(self, a, b) -> "Plaintext":  # noqa: N802
        sk, ct = (a, b) if isinstance(a, PrivateKey) else (b, a)
        if not isinstance(sk, PrivateKey) or not isinstance(ct, Ciphertext):
            raise TypeError("Decrypt(ciphertext, privateKey)")
        m = self._ctx.decrypt(ct.poly, sk.s)
        values = self._ctx.decode(m, ct.slots, ct.scale)
        return Plaintext(self, m, ct.level, ct.deg, ct.scale, ct.slots, values)

    # ------------------------------------------------------------ scale helpers
    def _wrap(self, poly: Poly, level: int, deg: int, scale: float, slots: int) -> "Ciphertext":
        return Ciphertext(self, poly, level, deg, scale, slots)

    def _rescaled(self, ct: "Ciphertext") -> "Ciphertext":
        if ct.poly.nlimb < 2:
            raise ValueError("no limb left to rescale")
        q_top = self._ctx.q[ct.poly.nlimb - 1]
        return self._wrap(self._ctx.rescale(ct.poly), ct.level + 1, ct.deg - 1,
                          ct.scale / q_top, ct.slots)

    def _rescaled_many(self, cts: list) -> list:
        """[_rescaled(ct) for ct in cts], the ciphertexts of one shape
        rescaled in shared launches (fhe_rescale_many)."""
        out: list = [None] * len(cts)
        groups: dict = {}
        for idx, ct in enumerate(cts):
            if ct.poly.nlimb < 2:
                raise ValueError("no limb left to rescale")
            groups.setdefault((ct.poly.npoly, ct.poly.nlimb), []).append(idx)
        for (_, nlimb), idxs in groups.items():
            q_top = self._ctx.q[nlimb - 1]
            polys = (self._ctx.rescale_many([cts[i].poly for i in idxs]) if len(idxs) > 1
                     else [self._ctx.rescale(cts[idxs[0]].poly)])
            for i, poly in zip(idxs, polys):
                ct = cts[i]
                out[i] = self._wrap(poly, ct.level + 1, ct.deg - 1, ct.scale / q_top, ct.slots)
        return out

    def _times_int(self, ct: "Ciphertext", c: int) -> "Ciphertext":
        nq = ct.poly.nlimb
        poly = self._ctx.mul_const(ct.poly, self._const_residues(c, nq))
        return self._wrap(poly, ct.level, ct.deg + 1, ct.scale * c, ct.slots)

    def _dropped(self, ct: "Ciphertext", level: int) -> "Ciphertext":
        if level == ct.level:
            return ct
        if level < ct.level:
            raise ValueError("cannot raise a ciphertext's level")
        poly = self._ctx.drop_limbs(ct.poly, self.L - level)
        return self._wrap(poly, level, ct.deg, ct.scale, ct.slots)

    def _lift_to(self, lo: "Ciphertext", hi: "Ciphertext") -> "Ciphertext":
        """Bring degree-1 `lo` (more limbs) to hi's level, degree and scale."""
        if hi.deg == 1:
            q_top = self._ctx.q[lo.poly.nlimb - 1]
            c = int(round(hi.scale * q_top / lo.scale))
            out = self._rescaled(self._times_int(lo, c))
        else:
            out = self._times_int(lo, int(round(hi.scale / lo.scale)))
        out = self._dropped(out, hi.level)
        out.scale = hi.scale
        return out

    def _align_add(self, a: "Ciphertext", b: "Ciphertext"):
        for _ in range(4):
            if a.level == b.level:
                if a.deg == b.deg:
                    return a, b
                if a.deg < b.deg:
                    a = self._times_int(a, int(round(b.scale / a.scale)))
                    a.scale = b.scale
                else:
                    b = self._times_int(b, int(round(a.scale / b.scale)))
                    b.scale = a.scale
                return a, b
            swap = a.level > b.level
            lo, hi = (b, a) if swap else (a, b)
            if lo.deg >= 2:
                lo = self._rescaled(lo)
            else:
                lo = self._lift_to(lo, hi)
            a, b = (hi, lo) if swap else (lo, hi)
        raise RuntimeError("level alignment did not converge")

    def _align_mult(self, a: "Ciphertext", b: "Ciphertext"):
        if a.deg >= 2:
            a = self._rescaled(a)
        if b.deg >= 2:
            b = self._rescaled(b)
        if a.level < b.level:
            a = self._lift_to(a, b)
        elif b.level < a.level:
            b = self._lift_to(b, a)
        return a, b

    def _plain_for_add(self, ct: "Ciphertext", pt: "Plaintext") -> "Plaintext":
        """pt at ct's limbs and scale (re-encoded from its values if needed)."""
        if pt.level <= ct.level and pt.deg == ct.deg and \
                abs(pt.scale / ct.scale - 1.0) < 1e-12:
            return pt
        if ct.deg > 2:
            raise ValueError("cannot add a plaintext to a degree > 2 ciphertext")
        return self._encode(pt.values, ct.level, ct.deg, pt.slots)

    @staticmethod
    def _is_number(x) -> bool:
        return isinstance(x, (int, float, np.integer, np.floating))

    # ------------------------------------------------------------ addition
    def _add(self, a, b, negate_b: bool) -> "Ciphertext":
        if self._is_number(a) and isinstance(b, Ciphertext):
            if negate_b:
                return self._add(self.EvalNegate(b), float(a), False)
            return self._add(b, a, False)
        if isinstance(a, Plaintext) and isinstance(b, Ciphertext):
            if negate_b:
                return self._add(self.EvalNegate(b), a, False)
            return self._add(b, a, False)
        if not isinstance(a, Ciphertext):
            raise TypeError("EvalAdd / EvalSub need a ciphertext operand")
        if isinstance(b, Ciphertext):
            x, y = self._align_add(a, b)
            f = self._ctx.sub if negate_b else self._ctx.add
            return self._wrap(f(x.poly, y.poly), x.level, x.deg, x.scale, x.slots)
        if isinstance(b, Plaintext):
            p = self._plain_for_add(a, b)
            poly = p.poly
            if negate_b:
                poly = self._ctx.negate(poly)
            return self._wrap(self._ctx.add_plain(a.poly, poly), a.level, a.deg, a.scale,
                              a.slots)
        if self._is_number(b):
            v = -float(b) if negate_b else float(b)
            c = int(round(v * a.scale))
            poly = self._ctx.add_const(a.poly, self._const_residues(c, a.poly.nlimb))
            return self._wrap(poly, a.level, a.deg, a.scale, a.slots)
        raise TypeError(f"unsupported operand {type(b).__name__}")

    def EvalAdd(self, a, b) -> "Ciphertext":  # noqa: N802
        return self._add(a, b, False)

    def EvalSub(self, a, b) -> "Ciphertext":  # noqa: N802
        return self._add(a, b, True)

    def EvalAddInPlace(self, a: "Ciphertext", b) -> None:  # noqa: N802
        a._assign(self._add(a, b, False))

    def EvalSubInPlace(self, a: "Ciphertext", b) -> None:  # noqa: N802
        a._assign(self._add(a, b, True))

    def EvalNegate(self, a: "Ciphertext") -> "Ciphertext":  # noqa: N802
        return self._wrap(self._ctx.negate(a.poly), a.level, a.deg, a.scale, a.slots)

    def EvalNegateInPlace(self, a: "Ciphertext") -> None:  # noqa: N802
        a._assign(self.EvalNegate(a))

    # ------------------------------------------------------------ multiplication
    def _relin_key(self):
        if self._relin is None:
            raise KeyError("no relinearization key; call EvalMultKeyGen first")
        return self._relin

    def _mult_ct(self, a: "Ciphertext", b: "Ciphertext") -> "Ciphertext":
        key = self._relin_key()
        same = a is b
        a, b = self._align_mult(a, b)
        t = self._ctx.tensor(a.poly, a.poly if same else b.poly)
        out = self._ctx.relinearize(t, key)
        return self._wrap(out, a.level, a.deg + b.deg, a.scale * b.scale, a.slots)

    def _mult(self, a, b) -> "Ciphertext":
        if not isinstance(a, Ciphertext):
            a, b = b, a
        if not isinstance(a, Ciphertext):
            raise TypeError("EvalMult needs a ciphertext operand")
        if isinstance(b, Ciphertext):
            return self._mult_ct(a, b)
        if a.deg >= 2:
            a = self._rescaled(a)
        if isinstance(b, Plaintext):
            if b.level > a.level:
                a = self._dropped(a, b.level)
            poly = self._ctx.mul_plain(a.poly, b.poly)
            return self._wrap(poly, a.level, a.deg + b.deg, a.scale * b.scale, a.slots)
        if self._is_number(b):
            sf = self._sf[a.level]
            c = int(round(float(b) * sf))
            poly = self._ctx.mul_const(a.poly, self._const_residues(c, a.poly.nlimb))
            return self._wrap(poly, a.level, a.deg + 1, a.scale * sf, a.slots)
        raise TypeError(f"unsupported operand {type(b).__name__}")

    def EvalMult(self, a, b) -> "Ciphertext":  # noqa: N802
        return self._mult(a, b)

    def EvalMultMany(self, pairs) -> list:  # noqa: N802
        """[EvalMult(a, b) for a, b in pairs] with the ciphertext products
        of one level relinearized together (fhe_relinearize_many): the
        same ciphertexts, fewer and larger key-switch launches.  A pair
        whose operands are one object is a square, as in EvalMult."""
        out: list = [None] * len(pairs)
        groups: dict = {}
        # the degree-2 operands, rescaled together (each once) as
        # _align_mult would rescale them one at a time
        deep = {}
        for a, b in pairs:
            if isinstance(a, Ciphertext) and isinstance(b, Ciphertext):
                for x in (a, b):
                    if x.deg >= 2:
                        deep.setdefault(id(x), x)
        settled = dict(zip(deep, self._rescaled_many(list(deep.values()))))
        for idx, (a, b) in enumerate(pairs):
            if not (isinstance(a, Ciphertext) and isinstance(b, Ciphertext)):
                out[idx] = self._mult(a, b)
                continue
            same = a is b
            a, b = settled.get(id(a), a), settled.get(id(b), b)
            a, b = self._align_mult(a, b)
            t = self._ctx.tensor(a.poly, a.poly if same else b.poly)
            groups.setdefault(t.nlimb, []).append((idx, t, a, b))
        key = self._relin_key() if groups else None
        for items in groups.values():
            polys = self._ctx.relinearize_many([t for _, t, _, _ in items], key)
            for (idx, _, a, b), poly in zip(items, polys):
                out[idx] = self._wrap(poly, a.level, a.deg + b.deg, a.scale * b.scale, a.slots)
        return out

    def EvalMultInPlace(self, a: "Ciphertext", b) -> None:  # noqa: N802
        a._assign(self._mult(a, b))

    def EvalMultMutableInPlace(self, a: "Ciphertext", b: "Ciphertext") -> None:  # noqa: N802
        a._assign(self._mult(a, b))

    def EvalSquare(self, a: "Ciphertext") -> "Ciphertext":  # noqa: N802
        return self._mult_ct(a, a)

    def EvalSquareInPlace(self, a: "Ciphertext") -> None:  # noqa: N802
        a._assign(self._mult_ct(a, a))

    def EvalLinearWSum(self, cts: Sequence["Ciphertext"], weights) -> "Ciphertext":  # noqa: N802
        """sum_i weights[i] * cts[i] as one degree-2 ciphertext at the
        deepest input level with scale sf[t]^2 (so that its rescale lands
        on the FLEXIBLEAUTO table): each input is rescaled if needed, has
        limbs dropped to level t (free) and is multiplied by the integer
        round(w_i sf[t]^2 / scale_i), so every product carries the same
        scale and the sum needs no alignment products."""
        items = [(c if c.deg < 2 else self._rescaled(c), float(w))
                 for c, w in zip(cts, weights)]
        if not items:
            raise ValueError("EvalLinearWSum needs at least one ciphertext")
        t = max(c.level for c, _ in items)
        target = self._sf[t] * self._sf[t]
        nq = self.L - t
        terms, ms = [], []
        for c, w in items:
            m = int(round(w * target / c.scale))
            if m != 0:
                terms.append(c.poly)
                ms.append(m)
        # one pass over the terms' first nq limbs (no limb drops, no
        # per-term products)
        acc = self._ctx.linear_wsum(terms, ms, nq) if terms else None
        if acc is None:
            c0 = items[0][0]
            x = c0.poly if c0.level == t else self._ctx.drop_limbs(c0.poly, nq)
            acc = self._ctx.mul_const(x, self._const_residues(0, nq))
        return self._wrap(acc, t, 2, target, items[0][0].slots)

    def MultByInteger(self, a: "Ciphertext", value: int) -> "Ciphertext":  # noqa: N802
        """Multiply by a small integer without changing the scale
        (multIntScalar, native/fideslib_stage0/src/fideslib_refresh_correction.hpp:37)."""
        return self._wrap(self._ctx.mul_int(a.poly, int(value)), a.level, a.deg, a.scale,
                          a.slots)

    # ------------------------------------------------------------ levels
    def Rescale(self, a: "Ciphertext") -> "Ciphertext":  # noqa: N802
        return self._rescaled(a) if a.deg >= 2 else a.Clone()

    def RescaleMany(self, cts) -> list:  # noqa: N802
        """[Rescale(ct) for ct in cts], the rescales of one shape sharing
        their launches (fhe_rescale_many): the same ciphertexts."""
        out = [ct if ct.deg >= 2 else ct.Clone() for ct in cts]
        deep = [i for i, ct in enumerate(cts) if ct.deg >= 2]
        for i, r in zip(deep, self._rescaled_many([cts[i] for i in deep])):
            out[i] = r
        return out

    def RescaleInPlace(self, a: "Ciphertext") -> None:  # noqa: N802
        if a.deg >= 2:
            a._assign(self._rescaled(a))

    ModReduce = Rescale
    ModReduceInPlace = RescaleInPlace

    def LevelReduce(self, a: "Ciphertext", evalKey=None, levels: int = 1) -> "Ciphertext":  # noqa: N802,N803
        return self._dropped(a, a.level + int(levels))

    def LevelReduceInPlace(self, a: "Ciphertext", evalKey=None, levels: int = 1) -> None:  # noqa: N802,N803
        a._assign(self._dropped(a, a.level + int(levels)))

    def AlignToLevel(self, a: "Ciphertext", level: int) -> "Ciphertext":  # noqa: N802
        """`a` as a degree-1 ciphertext at `level` on that level's standard
        scale (an extension of the OpenFHE API): rescaled first if degree 2,
        then, if still shallower, FLEXIBLEAUTO's alignment of a shallower
        operand (a product by an integer onto the target scale, a rescale
        and a limb drop, as EvalAdd / EvalMult apply to the shallower of
        two operands).  Operands met at varying levels reach one level, so
        plaintexts encoded for it are reused."""
        x = self._rescaled(a) if a.deg >= 2 else a
        level = int(level)
        if not x.level <= level < self.L:
            raise ValueError(f"cannot align level {x.level} to level {level}")
        if level == x.level:
            return x
        target = self._sf[level]
        q_top = self._ctx.q[x.poly.nlimb - 1]
        out = self._rescaled(self._times_int(x, int(round(target * q_top / x.scale))))
        out = self._dropped(out, level)
        out.scale = target
        return out

    # ------------------------------------------------------------ rotations
    def EvalRotate(self, a: "Ciphertext", index: int) -> "Ciphertext":  # noqa: N802
        g = galois_element(int(index), self.n)
        if g == 1:
            return a.Clone()
        poly = self._ctx.rotate(a.poly, self._key_for(g), g)
        return self._wrap(poly, a.level, a.deg, a.scale, a.slots)

    EvalAtIndex = EvalRotate

    def EvalRotateInPlace(self, a: "Ciphertext", index: int) -> None:  # noqa: N802
        a._assign(self.EvalRotate(a, index))

    def EvalRotateMany(self, cts: Sequence["Ciphertext"], index) -> list:  # noqa: N802
        """Rotate several ciphertexts (one index for all, or one each) in one
        batched key switch; ciphertexts at different levels are grouped."""
        idx = list(index) if isinstance(index, (list, tuple, np.ndarray)) else [index] * len(cts)
        if len(idx) != len(cts):
            raise ValueError("one rotation index per ciphertext")
        outs: list = [None] * len(cts)
        by_level: dict = {}
        for j, (c, i) in enumerate(zip(cts, idx)):
            g = galois_element(int(i), self.n)
            if g == 1:
                outs[j] = c.Clone()
            else:
                by_level.setdefault(c.level, []).append((j, g))
        for level, items in by_level.items():
            polys = self._ctx.rotate_many([cts[j].poly for j, _ in items],
                                          [self._key_for(g) for _, g in items],
                                          [g for _, g in items])
            for (j, _), p in zip(items, polys):
                c = cts[j]
                outs[j] = self._wrap(p, c.level, c.deg, c.scale, c.slots)
        return outs

    def EvalConjugate(self, a: "Ciphertext") -> "Ciphertext":  # noqa: N802
        g = conjugation_element(self.n)
        poly = self._ctx.rotate(a.poly, self._key_for(g), g)
        return self._wrap(poly, a.level, a.deg, a.scale, a.slots)

    def EvalConjugateMany(self, cts: Sequence["Ciphertext"]) -> list:  # noqa: N802
        """[EvalConjugate(ct) for ct in cts], the conjugations at one level
        in one batched key switch (fhe_rotate_many): the same ciphertexts."""
        cts = list(cts)
        if len(cts) == 1:
            return [self.EvalConjugate(cts[0])]
        g = conjugation_element(self.n)
        key = self._key_for(g)
        outs: list = [None] * len(cts)
        by_level: dict = {}
        for j, c in enumerate(cts):
            by_level.setdefault(c.level, []).append(j)
        for idx in by_level.values():
            polys = self._ctx.rotate_many([cts[j].poly for j in idx], [key] * len(idx),
                                          [g] * len(idx))
            for j, p in zip(idx, polys):
                c = cts[j]
                outs[j] = self._wrap(p, c.level, c.deg, c.scale, c.slots)
        return outs

    def EvalFastRotationPrecompute(self, a: "Ciphertext") -> "FastRotationPrecompute":  # noqa: N802
        return FastRotationPrecompute(a, self._ctx.rotation_precompute(a.poly))

    def EvalFastRotation(self, a: "Ciphertext", index, m: int,  # noqa: N802
                         precomp: "FastRotationPrecompute"):
        """One index -> one ciphertext; a list of indices -> a list, all from
        the one precompute (the FIDESlib vector overload)."""
        if m != 2 * self.n:
            raise ValueError(f"cyclotomic order must be {2 * self.n}")
        if precomp.ct is not a and precomp.level != a.level:
            raise ValueError("precompute belongs to another ciphertext level")
        single = not isinstance(index, (list, tuple, np.ndarray))
        idx = [int(index)] if single else [int(i) for i in index]
        outs: list = [None] * len(idx)
        todo = []
        for j, i in enumerate(idx):
            g = galois_element(i, self.n)
            if g == 1:
                outs[j] = a.Clone()
            else:
                todo.append((j, g))
        if todo:
            polys = self._ctx.rotate_hoisted(a.poly, precomp.digits,
                                             [self._key_for(g) for _, g in todo],
                                             [g for _, g in todo])
            for (j, _), p in zip(todo, polys):
                outs[j] = self._wrap(p, a.level, a.deg, a.scale, a.slots)
        return outs[0] if single else outs

    # ------------------------------------------------------------ linear maps
    def LinearTransformInPlace(self, ct: "Ciphertext", rowSize: int, bStep: int,  # noqa: N802,N803
                               pts: Sequence, stride: int = 1, offset: int = 0) -> None:
        """ct <- sum_g rot(sum_b pts[g*bStep+b] * rot(ct, b*stride), g*bStep*stride).

        pts[k] (None for a zero diagonal) must already be rotated by
        -(k // bStep) * bStep * stride, as the reference's pre-rotated
        masks are.  A nonzero offset first rotates ct by `offset`.

        The key set decides the schedule (`bsgs_rotations` lists the keys of
        the fast one): with keys for offset + b*stride the offset rotation
        joins the babies' shared ModUp instead of costing a key switch of
        its own, and with keys for every multiple g*bStep*stride the giant
        steps run as one batch of independent rotations instead of Horner's
        rule; otherwise the offset is one rotation and the giants use the
        bStep*stride key.  All schedules give the same sum."""
        self.LinearTransformManyInPlace([ct], rowSize, bStep, pts, stride, offset)

    def LinearTransformManyInPlace(self, cts: Sequence["Ciphertext"], rowSize: int,  # noqa: N802,N803
                                   bStep: int, pts: Sequence, stride: int = 1,  # noqa: N803
                                   offset: int = 0) -> None:
        """LinearTransformInPlace of every ciphertext of `cts` with the same
        diagonals (an extension of the OpenFHE API): ciphertexts that meet
        at one level share their ModUps and key-switch launches
        (fhe_linear_transform_hoisted_many); the same results as one call
        each."""
        cts = list(cts)
        count, bstep = int(rowSize), int(bStep)
        if len(pts) < count:
            raise ValueError("fewer plaintexts than rowSize")
        pts = list(pts[:count])
        present = [p for p in pts if p is not None]
        if not present:
            raise ValueError("linear transform has no nonzero diagonal")
        nb = min(bstep, count)
        giants = -(-count // bstep)
        used = sorted({k % bstep for k in range(count) if pts[k] is not None})
        has = lambda r: galois_element(int(r), self.n) in self._galois  # noqa: E731
        fold = bool(offset) and all(has(offset + b * stride) for b in used)
        batch = giants > 2 and all(has(g * bstep * stride) for g in range(1, giants))
        if offset and not fold:
            for ct, r in zip(cts, self.EvalRotateMany(cts, offset)):
                ct._assign(r)
        off = offset if fold else 0
        deep = [ct for ct in cts if ct.deg >= 2]
        for ct, r in zip(deep, self._rescaled_many(deep)):
            ct._assign(r)
        deg, scale = present[0].deg, present[0].scale
        if any(p.deg != deg or abs(p.scale / scale - 1) > 1e-12 for p in present):
            raise ValueError("diagonals must share one scale and degree")
        plevel = max(p.level for p in present)
        for ct in cts:
            if plevel > ct.level:
                ct._assign(self._dropped(ct, plevel))
        baby_keys, baby_gal = [None] * nb, [1] * nb
        for b in used:
            if b or off:
                g = galois_element(off + b * stride, self.n)
                baby_keys[b], baby_gal[b] = self._key_for(g), g
        steps = range(1, giants) if batch else ([1] if giants > 1 else [])
        gal = [galois_element(g * bstep * stride, self.n) for g in steps]
        gkeys = [self._key_for(g) for g in gal]
        ppolys = [None if p is None else p.poly for p in pts]
        by_level: dict = {}
        for ct in cts:
            by_level.setdefault(ct.level, []).append(ct)
        for group in by_level.values():
            if len(group) == 1:
                polys = [self._ctx.linear_transform_hoisted(
                    group[0].poly, ppolys, bstep, baby_keys, baby_gal, gkeys, gal)]
            else:
                polys = self._ctx.linear_transform_hoisted_many(
                    [ct.poly for ct in group], ppolys, bstep, baby_keys, baby_gal, gkeys, gal)
            for ct, poly in zip(group, polys):
                ct._assign(self._wrap(poly, ct.level, ct.deg + deg, ct.scale * scale,
                                      ct.slots))

    # ------------------------------------------------------------ bootstrapping
    def _monomial(self, power: int, nq: int) -> Poly:
        """X^power (power mod 2N) in evaluation form on nq limbs."""
        key = ("monomial", power, nq)
        if key not in self._cache:
            n, q = self.n, self._ctx.q[:nq]
            coef = np.zeros((1, nq, n), dtype=np.uint64)
            k = power % (2 * n)
            for j, qj in enumerate(q):
                coef[0, j, k % n] = 1 if k < n else qj - 1
            poly = self._ctx.upload(coef)
            self._ctx.ntt_forward_dev(poly.data_ptr(), 1, nq, 0)
            self._cache[key] = poly
        return self._cache[key]

    def MultByMonomial(self, a: "Ciphertext", power: int) -> "Ciphertext":  # noqa: N802
        """a * X^power.  Slot j is multiplied by zeta^(power * 5^j) for the
        primitive 2N-th root zeta; X^(N/2) multiplies every slot by i and
        X^(3N/2) by -i.  Exact: no level, scale or noise change."""
        poly = self._ctx.mul_plain(a.poly, self._monomial(int(power), a.poly.nlimb))
        return self._wrap(poly, a.level, a.deg, a.scale, a.slots)

    def ModRaise(self, a: "Ciphertext") -> "Ciphertext":  # noqa: N802
        """Lift a one-limb ciphertext to every limb (level 0).  It then
        decrypts to t = m + q0 * I with small integer I; its scale is set to
        sf[0], so its slots decode to Decode(t) / sf[0]."""
        if a.deg >= 2:
            a = self._rescaled(a)
        if a.poly.nlimb != 1:
            raise ValueError("ModRaise needs a ciphertext with one limb left")
        poly = self._ctx.mod_raise(a.poly, self.L)
        return self._wrap(poly, 0, 1, self._sf[0], a.slots)

    def EvalBootstrapSetup(self, levelBudget=(5, 5), dim1=(0, 0), slots: int = 0,  # noqa: N802,N803
                           correctionFactor: int = 0, precompute: bool = True, *,
                           s2c_first: bool = False, real_slots: bool = False) -> None:
        """Plan CoeffToSlot / SlotToCoeff for `slots`-slot ciphertexts (full
        or sparse packing) with levelBudget = (levels for CoeffToSlot, levels
        for SlotToCoeff).  correctionFactor 0 picks the message scale-down
        automatically.  s2c_first: the SlotToCoeff-first ordering of the
        reference's patched EvalBootstrapSetup (packed_fideslib.cpp:1084-1086;
        full packing; the input must sit SlotToCoeff levels lower, the output
        keeps them); real_slots: the caller's slots are real, so S2C-first
        runs EvalMod on the real part only."""
        from .bootstrap import BootstrapConfig, CKKSBootstrapper
        slots = int(slots) or self._slots
        cfg = BootstrapConfig.for_ring(self.n, tuple(int(b) for b in levelBudget),
                                       int(correctionFactor),
                                       hamming_weight=self.secret_hamming_weight())
        self._boot = CKKSBootstrapper(self, cfg, slots, s2c_first=s2c_first,
                                      real_slots=real_slots)

    def _bootstrapper(self):
        if self._boot is None:
            raise RuntimeError("call EvalBootstrapSetup first")
        return self._boot

    def EvalBootstrapKeyGen(self, secretKey: "PrivateKey", slots: int = 0) -> None:  # noqa: N802,N803
        """Rotation keys of the CoeffToSlot / SlotToCoeff plans and the
        conjugation key."""
        boot = self._bootstrapper()
        self.EvalRotateKeyGen(secretKey, boot.rotation_indices())
        self.EvalConjugateKeyGen(secretKey)

    def GetBootstrapDepth(self) -> int:  # noqa: N802
        """Levels one EvalBootstrap consumes after ModRaise."""
        return self._bootstrapper().depth()

    def GetBootstrapInputCeiling(self) -> int:  # noqa: N802
        """Deepest level an EvalBootstrap input may sit at."""
        return self._bootstrapper().input_ceiling()

    def EvalBootstrap(self, ct: "Ciphertext", numIterations: int = 1,  # noqa: N802,N803
                      precision: int = 0, *, scale: float = 1.0,
                      coeff_bound: float = 1.0) -> "Ciphertext":
        """Refresh `ct` to level GetBootstrapDepth() (slot values kept to
        bootstrapping precision).  numIterations = 2 runs a second pass on
        the scaled residual of the first (precision = log2 of that scale;
        0 picks 12).  `scale` (an extension of the OpenFHE call) admits
        slots in [-scale, scale]: the division and the multiplication back
        ride on the bootstrap's own scale-down and SlotToCoeff constants,
        so they cost no level.  `coeff_bound` (also an extension; the
        ordinary order): a public bound on the message's coefficients
        relative to its slot bound (bootstrap.coefficient_bound of the
        slots), which lets the first pass scale the message down less; 1,
        the default, is the worst case."""
        boot = self._bootstrapper()
        scale = float(scale)
        if not scale > 0:
            raise ValueError("bootstrap scale must be positive")
        out = boot.bootstrap(ct, pre=1.0 / scale, post=scale, coeff_bound=float(coeff_bound))
        if int(numIterations) <= 1:
            return out
        if int(numIterations) != 2:
            raise ValueError("numIterations must be 1 or 2")
        bits = int(precision) or 12
        residual = self.EvalSub(ct, out)
        fix = boot.bootstrap(residual, pre=2.0 ** bits / scale, post=scale * 2.0 ** -bits)
        return self.EvalAdd(out, fix)

    def EvalBootstrapMany(self, cts: Sequence["Ciphertext"], numIterations: int = 1,  # noqa: N802,N803
                          precision: int = 0, *, scale: float = 1.0,
                          real_slots: bool | None = None) -> list:
        """[EvalBootstrap(ct, numIterations, precision, scale=scale) for ct
        in cts] (an extension of the OpenFHE API): under S2C-first the
        ciphertexts go through every stage in step, sharing their key
        switches, rescales and EvalMod products; the same ciphertexts as
        one call each.  `real_slots` False (S2C-first) refreshes complex
        slots whatever the setup's mode, e.g. two real values packed as
        a + i b."""
        boot = self._bootstrapper()
        scale = float(scale)
        if not scale > 0:
            raise ValueError("bootstrap scale must be positive")
        if int(numIterations) > 2:
            raise ValueError("numIterations must be 1 or 2")
        cts = list(cts)
        outs = boot.bootstrap_many(cts, pre=1.0 / scale, post=scale, real_slots=real_slots)
        if int(numIterations) <= 1:
            return outs
        bits = int(precision) or 12
        residuals = [self.EvalSub(ct, out) for ct, out in zip(cts, outs)]
        fixes = boot.bootstrap_many(residuals, pre=2.0 ** bits / scale,
                                    post=scale * 2.0 ** -bits, real_slots=real_slots)
        return [self.EvalAdd(o, f) for o, f in zip(outs, fixes)]


class FastRotationPrecompute:
    """ModUp'd digits of a ciphertext's c1 (EvalFastRotationPrecompute)."""

    def __init__(self, ct: "Ciphertext", digits: Poly):
        self.ct = ct
        self.level = ct.level
        self.digits = digits


class PublicKey:
    def __init__(self, cc: CryptoContext, poly: Poly):
        self.cc = cc
        self.poly = poly


class PrivateKey:
    def __init__(self, cc: CryptoContext, s: np.ndarray):
        self.cc = cc
        self.s = s


class KeyPair:
    def __init__(self, publicKey: PublicKey, secretKey: PrivateKey):  # noqa: N803
        self.publicKey = publicKey
        self.secretKey = secretKey

    def good(self) -> bool:
        return self.publicKey is not None and self.secretKey is not None


class Plaintext:
    def __init__(self, cc: CryptoContext, poly: Poly, level: int, deg: int, scale: float,
                 slots: int, values):
        self.cc = cc
        self.poly = poly
        self.level = level
        self.deg = deg
        self.scale = scale
        self.slots = slots
        self.values = np.asarray(values, dtype=np.complex128)
        self._length = slots

    def GetLevel(self) -> int:  # noqa: N802
        return self.level

    def GetNoiseScaleDeg(self) -> int:  # noqa: N802
        return self.deg

    def GetScalingFactor(self) -> float:  # noqa: N802
        return self.scale

    def GetSlots(self) -> int:  # noqa: N802
        return self.slots

    def SetLength(self, length: int) -> None:  # noqa: N802
        self._length = int(length)

    def GetLength(self) -> int:  # noqa: N802
        return self._length

    def _padded(self) -> np.ndarray:
        v = np.zeros(self.slots, dtype=np.complex128)
        v[: min(len(self.values), self.slots)] = self.values[: self.slots]
        return v[: self._length]

    def GetCKKSPackedValue(self) -> list:  # noqa: N802
        return list(self._padded())

    def GetRealPackedValue(self) -> list:  # noqa: N802
        return [float(x) for x in self._padded().real]

    def __repr__(self):
        head = ", ".join(f"{x:.6g}" for x in self._padded().real[:8])
        return f"Plaintext(level={self.level}, deg={self.deg}, slots={self.slots}, [{head}, ...])"


class Ciphertext:
    def __init__(self, cc: CryptoContext, poly: Poly, level: int, deg: int, scale: float,
                 slots: int):
        self.cc = cc
        self.poly = poly
        self.level = level
        self.deg = deg
        self.scale = scale
        self.slots = slots

    def _assign(self, other: "Ciphertext") -> None:
        self.poly, self.level, self.deg, self.scale, self.slots = \
            other.poly, other.level, other.deg, other.scale, other.slots

    def Clone(self) -> "Ciphertext":  # noqa: N802
        return Ciphertext(self.cc, self.poly.copy(), self.level, self.deg, self.scale,
                          self.slots)

    def GetLevel(self) -> int:  # noqa: N802
        return self.level

    def SetLevel(self, level: int) -> None:  # noqa: N802
        """Drop limbs down to `level` (scale unchanged), as the reference's
        level alignment uses it (packed_fideslib.cpp:123-127)."""
        self._assign(self.cc._dropped(self, int(level)))

    def GetNoiseScaleDeg(self) -> int:  # noqa: N802
        return self.deg

    def SetNoiseScaleDeg(self, deg: int) -> None:  # noqa: N802
        self.deg = int(deg)

    def GetScalingFactor(self) -> float:  # noqa: N802
        return self.scale

    def SetScalingFactor(self, scale: float) -> None:  # noqa: N802
        self.scale = float(scale)

    def GetSlots(self) -> int:  # noqa: N802
        return self.slots

    def GetCryptoContext(self) -> CryptoContext:  # noqa: N802
        return self.cc

    def residues(self) -> np.ndarray:
        """Limb-major residues [2][L - level][N] (evaluation form)."""
        return self.poly.numpy()

    def __repr__(self):
        return (f"Ciphertext(level={self.level}, deg={self.deg}, scale=2^"
                f"{math.log2(self.scale):.2f}, slots={self.slots})")
