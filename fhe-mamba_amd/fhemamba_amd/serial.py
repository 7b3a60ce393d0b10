"""Contexts, keys and ciphertexts on disk, for the process-separated
client / server decode: the Serial::SerializeToFile / DeserializeFromFile,
SerializeEvalMultKey / DeserializeEvalMultKey and
SerializeEvalAutomorphismKey / DeserializeEvalAutomorphismKey calls of
native/fideslib_stage0/src/fideslib_handoff.cpp:28-90 and
src/stage1_mamba2_decode_fideslib.cpp:879-892, :1248-1275, :1446-1481,
under openfhe-python's names (SerializeToFile(path, obj, BINARY) -> bool,
DeserializeCryptoContext(path, BINARY) -> (cc, bool), ...).

Wire format "fhecore-wire-v1", one object per file, little-endian:
  8 bytes   magic b"FHECORE1"
  u64       header length H
  H bytes   header, UTF-8 JSON: {"kind", "context" (fingerprint), the
            object's metadata, "arrays": [{"dtype", "shape", "crc32"}, ...]}
  then each array's raw words in order (uint64 residues, or int64 secret
  coefficients), CRC-32 checked on reading.
A context file holds the parameter set and the prime chain (the server
rebuilds the context from them and checks the chain); it never holds a
sampling seed, so a context deserialised on the server draws from ChaCha20
under fresh OS entropy.  Keys are stored in the standard evaluation form
[dnum][2][L+K][N] that fhe_key_load takes; ciphertexts as their limb-major
residues with level, noise-scale degree, scaling factor (exact float hex)
and slot count.  Objects other than contexts name their context by the
fingerprint of its ring dimension, chain and digit count and attach to the
context with that fingerprint that this process built or loaded last (or to
the one passed as `cc`).

OpenFHE's own BINARY (cereal) encoding is not reproduced: these files
interchange with this library only.
"""
from __future__ import annotations

import enum
import hashlib
import json
import os
import weakref
import zlib

import numpy as np

MAGIC = b"FHECORE1"
_CONTEXTS: "weakref.WeakValueDictionary" = weakref.WeakValueDictionary()
_last_error = ""


class SerType(enum.Enum):
    BINARY = "BINARY"
    JSON = "JSON"


BINARY = SerType.BINARY
JSON = SerType.JSON


class SerialError(ValueError):
    pass


def last_error() -> str:
    """Why the last Serialize*/Deserialize* call returned False."""
    return _last_error


# ----------------------------------------------------------------- fingerprints
def fingerprint(cc) -> str:
    q, p = cc.GetModuli()
    blob = json.dumps({"ring": cc.GetRingDimension(), "q": [int(x) for x in q],
                       "p": [int(x) for x in p], "dnum": int(cc._dnum)}, sort_keys=True)
    return hashlib.sha256(blob.encode()).hexdigest()[:32]


def register(cc) -> str:
    """Make `cc` the context that objects with its fingerprint attach to
    (every context registers when it is built or deserialised; the latest
    live one wins)."""
    fp = fingerprint(cc)
    _CONTEXTS[fp] = cc
    return fp


def _context_for(fp: str, cc=None):
    if cc is not None:
        if fingerprint(cc) != fp:
            raise SerialError("the object belongs to another crypto context")
        return cc
    found = _CONTEXTS.get(fp)
    if found is None:
        raise SerialError("no crypto context with this object's parameters is loaded; "
                          "deserialize the context first")
    return found


# ----------------------------------------------------------------- file layout
def _write(path: str, header: dict, arrays) -> None:
    """Write the header and then the arrays; `arrays` may be a generator
    (large key sets are downloaded and written one key at a time), so the
    CRCs go in a header placeholder patched after the data."""
    specs = header.setdefault("arrays", [])
    with open(path, "wb") as f:
        f.write(MAGIC)
        # reserve room for the header with its CRCs: fixed-width fields
        for spec in specs:
            spec["crc32"] = "00000000"
        text = json.dumps(header).encode()
        f.write(len(text).to_bytes(8, "little"))
        start = f.tell()
        f.write(text)
        for i, a in enumerate(arrays):
            a = np.ascontiguousarray(a)
            spec = specs[i]
            if str(a.dtype) != spec["dtype"] or list(a.shape) != spec["shape"]:
                raise SerialError("array does not match its header entry")
            raw = a.view(np.uint8).reshape(-1)
            spec["crc32"] = f"{zlib.crc32(raw) & 0xFFFFFFFF:08x}"
            f.write(memoryview(raw))
        text2 = json.dumps(header).encode()
        if len(text2) != len(text):
            raise SerialError("header size changed while writing")
        f.seek(start)
        f.write(text2)


class _Reader:
    def __init__(self, path: str):
        self.f = open(path, "rb")
        if self.f.read(8) != MAGIC:
            self.f.close()
            raise SerialError(f"{path}: not an fhecore-wire-v1 file")
        n = int.from_bytes(self.f.read(8), "little")
        if n <= 0 or n > 1 << 26:
            self.f.close()
            raise SerialError(f"{path}: bad header length")
        try:
            self.header = json.loads(self.f.read(n).decode())
        except (UnicodeDecodeError, json.JSONDecodeError) as exc:
            self.f.close()
            raise SerialError(f"{path}: unreadable header") from exc
        self.path = path
        self.i = 0

    def kind(self, want: str) -> dict:
        if self.header.get("kind") != want:
            raise SerialError(f"{self.path}: holds a {self.header.get('kind')}, not a {want}")
        return self.header

    def array(self) -> np.ndarray:
        specs = self.header.get("arrays", [])
        if self.i >= len(specs):
            raise SerialError(f"{self.path}: fewer arrays than the object needs")
        spec = specs[self.i]
        self.i += 1
        dtype = np.dtype(spec["dtype"])
        if dtype not in (np.dtype(np.uint64), np.dtype(np.int64)):
            raise SerialError(f"{self.path}: unexpected array type {dtype}")
        shape = tuple(int(d) for d in spec["shape"])
        # Shapes come from the file: check them against the bytes the file
        # still holds before allocating anything.
        if len(shape) > 4 or any(d < 0 for d in shape):
            raise SerialError(f"{self.path}: bad array shape {shape}")
        nbytes = int(np.prod(shape, dtype=object)) * dtype.itemsize
        left = os.fstat(self.f.fileno()).st_size - self.f.tell()
        if nbytes > left:
            raise SerialError(f"{self.path}: truncated ({nbytes} array bytes, {left} left)")
        a = np.empty(shape, dtype=dtype)
        got = self.f.readinto(memoryview(a.view(np.uint8).reshape(-1)))
        if got != a.nbytes:
            raise SerialError(f"{self.path}: truncated")
        if f"{zlib.crc32(a.view(np.uint8).reshape(-1)) & 0xFFFFFFFF:08x}" != spec["crc32"]:
            raise SerialError(f"{self.path}: checksum mismatch")
        return a

    def close(self):
        self.f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _spec(a_shape, dtype="uint64") -> dict:
    return {"dtype": dtype, "shape": [int(d) for d in a_shape]}


# ----------------------------------------------------------------- objects
def _params_json(cc) -> dict:
    out = {}
    for k, v in cc._params._v.items():
        out[k] = {"enum": type(v).__name__, "name": v.name} if isinstance(v, enum.Enum) else v
    return out


def _params_from_json(d: dict):
    from . import ckks
    params = ckks.CCParamsCKKSRNS()
    for k, v in d.items():
        if k not in ckks.CCParamsCKKSRNS._FIELDS:
            raise SerialError(f"unknown context parameter {k}")
        if isinstance(v, dict):
            etype = getattr(ckks, v.get("enum", ""), None)
            if not (isinstance(etype, type) and issubclass(etype, enum.Enum)) or \
                    v.get("name") not in etype.__members__:
                raise SerialError(f"bad value for context parameter {k}")
            v = etype[v["name"]]
        params._v[k] = v
    return params


def save_context(path: str, cc) -> None:
    q, p = cc.GetModuli()
    header = {"kind": "crypto-context", "context": fingerprint(cc), "format": "fhecore-wire-v1",
              "params": _params_json(cc), "ring_dim": cc.GetRingDimension(),
              "q": [int(x) for x in q], "p": [int(x) for x in p], "dnum": int(cc._dnum),
              "features": sorted(f.name for f in cc._features)}
    _write(path, header, [])


def load_context(path: str):
    from . import ckks
    with _Reader(path) as r:
        h = r.kind("crypto-context")
    cc = ckks.GenCryptoContext(_params_from_json(h["params"]))
    q, p = cc.GetModuli()
    if [int(x) for x in q] != h["q"] or [int(x) for x in p] != h["p"] or \
            cc.GetRingDimension() != h["ring_dim"] or int(cc._dnum) != h["dnum"]:
        raise SerialError(f"{path}: the parameters rebuild a different prime chain")
    for name in h.get("features", []):
        if name not in ckks.PKESchemeFeature.__members__:
            raise SerialError(f"{path}: unknown feature {name}")
        cc.Enable(ckks.PKESchemeFeature[name])
    if register(cc) != h["context"]:
        raise SerialError(f"{path}: context fingerprint mismatch")
    return cc


def save_public_key(path: str, pk) -> None:
    a = pk.poly.numpy()
    _write(path, {"kind": "public-key", "context": fingerprint(pk.cc), "arrays": [_spec(a.shape)]},
           [a])


def load_public_key(path: str, cc=None):
    from . import ckks
    with _Reader(path) as r:
        h = r.kind("public-key")
        cc = _context_for(h["context"], cc)
        a = r.array()
    if a.shape != (2, cc.L, cc.n):
        raise SerialError(f"{path}: public key shape {a.shape}")
    return ckks.PublicKey(cc, cc.device.upload(a))


def save_private_key(path: str, sk) -> None:
    s = np.ascontiguousarray(sk.s, dtype=np.int64)
    _write(path, {"kind": "private-key", "context": fingerprint(sk.cc),
                  "arrays": [_spec(s.shape, "int64")]}, [s])


def load_private_key(path: str, cc=None):
    from . import ckks
    with _Reader(path) as r:
        h = r.kind("private-key")
        cc = _context_for(h["context"], cc)
        s = r.array()
    if s.shape != (cc.n,) or np.any(np.abs(s) > 1):
        raise SerialError(f"{path}: not a ternary secret of this ring")
    return ckks.PrivateKey(cc, s)


def save_ciphertext(path: str, ct) -> None:
    a = ct.poly.numpy()
    _write(path, {"kind": "ciphertext", "context": fingerprint(ct.cc), "level": int(ct.level),
                  "noise_scale_deg": int(ct.deg), "scaling_factor": float(ct.scale).hex(),
                  "slots": int(ct.slots), "arrays": [_spec(a.shape)]}, [a])


def load_ciphertext(path: str, cc=None):
    from . import ckks
    with _Reader(path) as r:
        h = r.kind("ciphertext")
        cc = _context_for(h["context"], cc)
        a = r.array()
    level, deg, slots = int(h["level"]), int(h["noise_scale_deg"]), int(h["slots"])
    if a.ndim != 3 or a.shape[0] != 2 or a.shape[1] != cc.L - level or a.shape[2] != cc.n or \
            not 1 <= deg <= 2 or not 1 <= slots <= cc.n // 2 or slots & (slots - 1):
        raise SerialError(f"{path}: ciphertext metadata does not fit the context")
    qs = np.array(cc.GetModuli()[0][: a.shape[1]], dtype=np.uint64)
    if np.any(a >= qs[None, :, None]):
        raise SerialError(f"{path}: residue out of range")
    return ckks.Ciphertext(cc, cc.device.upload(a), level, deg, float.fromhex(h["scaling_factor"]),
                           slots)


def _key_shape(cc):
    d = cc.device
    return (d.dnum, 2, d.L + d.K, d.n)


def _check_key(path, cc, a):
    if a.shape != _key_shape(cc):
        raise SerialError(f"{path}: key shape {a.shape}")
    mods = np.array(list(cc.GetModuli()[0]) + list(cc.GetModuli()[1]), dtype=np.uint64)
    if np.any(a >= mods[None, None, :, None]):
        raise SerialError(f"{path}: key residue out of range")


def save_eval_mult_key(path: str, cc) -> None:
    if cc._relin is None:
        raise SerialError("no multiplication key to serialise; call EvalMultKeyGen first")
    shape = _key_shape(cc)
    _write(path, {"kind": "eval-mult-key", "context": fingerprint(cc), "arrays": [_spec(shape)]},
           [cc._relin.numpy()])


def load_eval_mult_key(path: str, cc) -> None:
    with _Reader(path) as r:
        h = r.kind("eval-mult-key")
        _context_for(h["context"], cc)
        a = r.array()
    _check_key(path, cc, a)
    cc._relin = cc.device.load_key(a)


def save_eval_automorphism_keys(path: str, cc) -> None:
    galois = sorted(int(g) for g in cc._galois)
    shape = _key_shape(cc)
    header = {"kind": "eval-automorphism-keys", "context": fingerprint(cc), "galois": galois,
              "arrays": [_spec(shape) for _ in galois]}
    _write(path, header, (cc._galois[g].numpy() for g in galois))


def load_eval_automorphism_keys(path: str, cc) -> int:
    with _Reader(path) as r:
        h = r.kind("eval-automorphism-keys")
        _context_for(h["context"], cc)
        galois = [int(g) for g in h.get("galois", [])]
        if len(galois) != len(h.get("arrays", [])) or len(set(galois)) != len(galois) or \
                any(g <= 0 or g >= 2 * cc.n or g % 2 == 0 for g in galois):
            raise SerialError(f"{path}: bad automorphism index list")
        for g in galois:
            a = r.array()
            _check_key(path, cc, a)
            cc._galois[g] = cc.device.load_key(a)
    return len(galois)


# ----------------------------------------------------------------- OpenFHE-shaped API
def _ok(fn, *args) -> bool:
    global _last_error
    try:
        fn(*args)
        _last_error = ""
        return True
    except (SerialError, OSError, ValueError, KeyError) as exc:
        _last_error = str(exc)
        return False


def _loaded(fn, *args):
    global _last_error
    try:
        obj = fn(*args)
        _last_error = ""
        return obj, True
    except (SerialError, OSError, ValueError, KeyError) as exc:
        _last_error = str(exc)
        return None, False


def _binary(sertype):
    if sertype not in (SerType.BINARY, "BINARY"):
        raise SerialError("only the BINARY serialisation type is provided")


def SerializeToFile(path: str, obj, sertype=SerType.BINARY) -> bool:  # noqa: N802
    """Serialize a CryptoContext, PublicKey, PrivateKey or Ciphertext."""
    from . import ckks
    _binary(sertype)
    for cls, fn in ((ckks.CryptoContext, save_context), (ckks.PublicKey, save_public_key),
                    (ckks.PrivateKey, save_private_key), (ckks.Ciphertext, save_ciphertext)):
        if isinstance(obj, cls):
            return _ok(fn, path, obj)
    raise TypeError(f"cannot serialise a {type(obj).__name__}")


def DeserializeCryptoContext(path: str, sertype=SerType.BINARY):  # noqa: N802
    _binary(sertype)
    return _loaded(load_context, path)


def DeserializePublicKey(path: str, sertype=SerType.BINARY, cc=None):  # noqa: N802
    _binary(sertype)
    return _loaded(load_public_key, path, cc)


def DeserializePrivateKey(path: str, sertype=SerType.BINARY, cc=None):  # noqa: N802
    _binary(sertype)
    return _loaded(load_private_key, path, cc)


def DeserializeCiphertext(path: str, sertype=SerType.BINARY, cc=None):  # noqa: N802
    _binary(sertype)
    return _loaded(load_ciphertext, path, cc)


def serialized_bytes(obj) -> bytes:
    """The file image of a ciphertext (for in-memory transport and tests)."""
    import os
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "obj.bin")
        if not SerializeToFile(path, obj):
            raise SerialError(last_error())
        with open(path, "rb") as f:
            return f.read()


__all__ = ["SerType", "BINARY", "JSON", "SerialError", "SerializeToFile",
           "DeserializeCryptoContext", "DeserializePublicKey", "DeserializePrivateKey",
           "DeserializeCiphertext", "last_error", "fingerprint"]
