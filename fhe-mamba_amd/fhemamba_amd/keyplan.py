"""Rotation-key planning by a dry run over symbolic ciphertexts.

A server that holds no secret key cannot generate rotation keys on demand,
so the client generates every key the server's circuit will ask for before
the handoff (the reference builds its rotation key set from the payload
dimensions before key generation, stage1_mamba2_decode_fideslib.cpp:
1125-1149, :1290-1293).
Here the list comes from running the circuit itself, on KeyPlanContext: the
CryptoContext surface that fhemamba_amd.packed.PackedEvaluator and
fhemamba_amd.mamba2_decode.EncryptedMamba2Decoder use, over ciphertexts
that carry only a level and a noise-scale degree.  The evaluators request
rotation keys through EvalRotateKeyGen before every rotation, and which
offsets a circuit rotates by depends on its dimensions, never on slot
values, so the recorded set is the set the real run requests (bootstrap
keys come from the real context's bootstrapping plan).
"""
from __future__ import annotations


class _SymPlain:
    def __init__(self, level: int, deg: int = 1):
        self.level, self.deg = level, deg


class _SymCt:
    def __init__(self, level: int = 0, deg: int = 1, scale: float = 1.0):
        self.level, self.deg, self.scale = level, deg, scale

    def Clone(self):  # noqa: N802
        return _SymCt(self.level, self.deg, self.scale)

    def _assign(self, other):
        self.level, self.deg, self.scale = other.level, other.deg, other.scale

    def GetLevel(self):  # noqa: N802
        return self.level

    def SetLevel(self, level):  # noqa: N802
        self.level = max(self.level, int(level))

    def GetNoiseScaleDeg(self):  # noqa: N802
        return self.deg

    def GetScalingFactor(self):  # noqa: N802
        return self.scale

    def SetScalingFactor(self, scale):  # noqa: N802
        self.scale = float(scale)


class _Sync:
    @staticmethod
    def sync():
        pass


class _NoBoot:
    @staticmethod
    def rotation_indices():
        return []


class KeyPlanContext:
    """Symbolic stand-in for a CryptoContext with `slots` slots, ring
    dimension `ring_dim`, `limbs` Q primes and a bootstrap that returns
    values at `boot_level` (input ceiling `boot_ceiling`).  Records every
    rotation index passed to EvalRotateKeyGen."""

    def __init__(self, slots: int, ring_dim: int, limbs: int, boot_level: int,
                 boot_ceiling: int):
        self.slots, self.n, self.limbs = int(slots), int(ring_dim), int(limbs)
        self.boot_level, self.boot_ceiling = int(boot_level), int(boot_ceiling)
        self.rotations: set = set()
        self.device = _Sync()

    # ---- parameters
    def GetBatchSize(self):  # noqa: N802
        return self.slots

    def GetRingDimension(self):  # noqa: N802
        return self.n

    def GetModuli(self):  # noqa: N802
        return [0] * self.limbs, []

    def GetScalingFactorReal(self, level=0):  # noqa: N802
        return 1.0

    # ---- keys
    def EvalRotateKeyGen(self, secret_key, index_list):  # noqa: N802
        self.rotations.update(int(i) % self.slots for i in index_list)

    def EvalBootstrapSetup(self, *args, **kw):  # noqa: N802
        pass

    def EvalBootstrapKeyGen(self, *args, **kw):  # noqa: N802
        pass

    def _bootstrapper(self):
        return _NoBoot()

    def GetBootstrapInputCeiling(self):  # noqa: N802
        return self.boot_ceiling

    # ---- level bookkeeping
    @staticmethod
    def _settled(ct):
        out = ct.Clone()
        while out.deg >= 2:
            out.deg -= 1
            out.level += 1
        return out

    def Rescale(self, ct):  # noqa: N802
        return self._settled(ct)

    def RescaleInPlace(self, ct):  # noqa: N802
        ct._assign(self._settled(ct))

    def AlignToLevel(self, ct, level):  # noqa: N802
        s = self._settled(ct)
        if not s.level <= level < self.limbs:
            raise ValueError(f"cannot align level {s.level} to level {level}")
        return _SymCt(int(level))

    def MakeCKKSPackedPlaintext(self, values, deg=1, level=0, slots=0):  # noqa: N802
        return _SymPlain(int(level), int(deg))

    def MakeCKKSPackedPlaintexts(self, rows, deg=1, level=0, slots=0):  # noqa: N802
        return [_SymPlain(int(level), int(deg)) for _ in rows]

    def Encrypt(self, key, pt):  # noqa: N802
        return _SymCt(pt.level)

    def _binary(self, a, b, product: bool):
        if not isinstance(a, _SymCt):
            a, b = b, a
        if product:
            a = self._settled(a)
            if isinstance(b, _SymCt):
                b = self._settled(b)
                return _SymCt(max(a.level, b.level), a.deg + b.deg)
            if isinstance(b, _SymPlain):
                return _SymCt(max(a.level, b.level), a.deg + b.deg)
            return _SymCt(a.level, a.deg + 1)
        if isinstance(b, _SymCt):
            return _SymCt(max(a.level, b.level), max(a.deg, b.deg))
        return a.Clone()

    def EvalMult(self, a, b):  # noqa: N802
        return self._binary(a, b, True)

    def EvalSquare(self, a):  # noqa: N802
        return self._binary(a, a, True)

    def EvalAdd(self, a, b):  # noqa: N802
        return self._binary(a, b, False)

    def EvalSub(self, a, b):  # noqa: N802
        return self._binary(a, b, False)

    def MultByInteger(self, a, k):  # noqa: N802
        return a.Clone()

    def EvalRotate(self, a, k):  # noqa: N802
        return a.Clone()

    def EvalRotateMany(self, cts, k):  # noqa: N802
        return [c.Clone() for c in cts]

    def EvalFastRotationPrecompute(self, a):  # noqa: N802
        return a

    def EvalFastRotation(self, a, index, m, pre):  # noqa: N802
        return [a.Clone() for _ in index]

    def LinearTransformInPlace(self, ct, rows, bstep, pts, stride=1, offset=0):  # noqa: N802
        s = self._settled(ct)
        lv = max([s.level] + [p.level for p in pts if p is not None])
        ct._assign(_SymCt(lv, s.deg + 1))

    def EvalBootstrap(self, ct, passes=1, precision=0, *, scale=1.0):  # noqa: N802
        s = self._settled(ct)
        if s.level > self.boot_ceiling:
            raise ValueError("bootstrap input too deep")
        return _SymCt(self.boot_level)


class _PlanKeys:
    publicKey = object()
    secretKey = object()


def plan_decoder_rotations(chain, *, slots: int, ring_dim: int, limbs: int, boot_level: int,
                           boot_ceiling: int, s2c_first: bool, bootstrap_passes: int = 2) -> set:
    """Every rotation index (mod slots) the encrypted Mamba-2 decode of
    `chain` asks for beyond the bootstrapping keys: two tokens (zero state,
    then carried state) of the chain's first layer and the final norm on
    KeyPlanContext.  Every layer of a chain has one set of dimensions, so
    the first layer's rotations are every layer's."""
    import numpy as np

    from .mamba2_decode import EncryptedMamba2Decoder
    from .mamba2_payload import ChainPayload
    one = ChainPayload(1, chain.n_test_tokens, chain.final_norm_eps, chain.final_norm_w,
                       chain.input_embeddings, chain.expected_final, chain.expected_poly_final,
                       chain.layers[:1], chain.final_norm_poly)
    plan = KeyPlanContext(slots, ring_dim, limbs, boot_level, boot_ceiling)
    dec = EncryptedMamba2Decoder(plan, _PlanKeys(), one, bootstrap_passes=bootstrap_passes,
                                 s2c_first=s2c_first)
    states = dec.initial_states()
    for _ in range(2):
        _, states = dec.step(np.zeros(one.layers[0].d_model), states)
    return set(plan.rotations)


def decoder_rotations(cc, chain, *, s2c_first: bool, bootstrap_passes: int = 2) -> set:
    """plan_decoder_rotations for a real context whose bootstrapping is set
    up (EvalBootstrapSetup)."""
    return plan_decoder_rotations(
        chain, slots=cc.GetBatchSize(), ring_dim=cc.GetRingDimension(),
        limbs=len(cc.GetModuli()[0]), boot_level=cc.GetBootstrapDepth(),
        boot_ceiling=cc.GetBootstrapInputCeiling(), s2c_first=s2c_first,
        bootstrap_passes=bootstrap_passes)
