"""Test helpers for the packed-program executor: a numpy program builder
that writes the `fhemamba-packed-v1/v2` text format (header, one line per
node, one per output, as src/fhemamba/packed_program.py:323-342 writes it)
with plaintext references, and a slot-level stand-in for the CKKS context
(values instead of ciphertexts, level bookkeeping kept) so the executor's
node semantics can be checked on the CPU."""
from __future__ import annotations

import numpy as np


class ProgramBuilder:
    def __init__(self, slots: int, bound: float = 64.0, extended: bool = False):
        self.slots, self.bound, self.extended = slots, bound, extended
        self.nodes: list = []     # (op, size, bound, parents, data)
        self.values: list = []
        self.outputs: list = []

    def _node(self, op, parents, data, value, bound=None):
        value = np.asarray(value, dtype=np.float64).ravel()
        self.nodes.append((op, value.size, bound or self.bound, list(parents),
                           np.asarray(data, dtype=np.float64).ravel()))
        self.values.append(value)
        return len(self.nodes) - 1

    def input(self, v):
        return self._node("input", [], v, v)

    def public(self, v):
        return self._node("public", [], v, v)

    def add(self, a, b):
        return self._node("add", [a, b], [], self.values[a] + self.values[b])

    def mul(self, a, b):
        return self._node("mul", [a, b], [], self.values[a] * self.values[b])

    def addp(self, a, v):
        return self._node("addp", [a], v, self.values[a] + np.asarray(v))

    def mulp(self, a, v):
        return self._node("mulp", [a], v, self.values[a] * np.asarray(v))

    def linear(self, a, W):
        W = np.asarray(W, dtype=np.float64)
        return self._node("linear", [a], W, W @ self.values[a])

    def linear_ref(self, a, weight_node):
        op, m, _, parents, W = self.nodes[weight_node]
        W = W.reshape(m, -1)
        return self._node("linear_ref", [a], [weight_node], W @ self.values[a])

    def gather(self, a, idx):
        idx = np.asarray(idx)
        return self._node("gather", [a], idx, self.values[a][idx])

    def scatter(self, a, idx, size):
        out = np.zeros(size)
        out[np.asarray(idx)] = self.values[a]
        return self._node("scatter", [a], idx, out)

    def repeat(self, a, outer, inner, rep):
        v = self.values[a].reshape(outer, 1, inner)
        out = np.broadcast_to(v, (outer, rep, inner))
        return self._node("repeat", [a], [outer, inner, rep], out)

    def sum(self, a, width):
        v = self.values[a].reshape(-1, width).sum(-1)
        return self._node("sum", [a], [width], v)

    def cheb(self, a, lo, hi, coeffs):
        u = (2 * self.values[a] - (lo + hi)) / (hi - lo)
        v = np.polynomial.chebyshev.chebval(u, coeffs)
        return self._node("cheb", [a], [lo, hi, *coeffs], v)

    def feedback(self, a, value):
        return self._node("feedback", [a], [], value)

    def output(self, node, exact=None):
        v = self.values[node]
        self.outputs.append((node, v, v if exact is None else np.asarray(exact)))

    def text(self) -> str:
        lines = [f"fhemamba-packed-v{2 if self.extended else 1} {self.slots} "
                 f"{self.bound:.17g} {len(self.nodes)} {len(self.outputs)}"]
        for op, size, bound, parents, data in self.nodes:
            f = [op, str(size)]
            if self.extended:
                f.append(format(bound, ".17g"))
            f += [str(len(parents)), *map(str, parents), str(len(data))]
            f += [format(float(v), ".17g") for v in data]
            lines.append(" ".join(f))
        for node, poly, exact in self.outputs:
            f = [str(node), str(len(poly))] + [format(float(v), ".17g")
                                               for v in [*poly, *exact]]
            lines.append(" ".join(f))
        return "\n".join(lines) + "\n"


# ---------------------------------------------------------------- slot backend
class SlotCt:
    def __init__(self, z, level=0, deg=1):
        self.z, self.level, self.deg = np.asarray(z, dtype=complex), level, deg

    def Clone(self):  # noqa: N802
        return SlotCt(self.z.copy(), self.level, self.deg)

    def GetLevel(self):  # noqa: N802
        return self.level

    def GetNoiseScaleDeg(self):  # noqa: N802
        return self.deg

    def _assign(self, other):
        self.z, self.level, self.deg = other.z, other.level, other.deg


class SlotKeys:
    publicKey = "pk"
    secretKey = "sk"


class SlotContext:
    """Slot vectors with the CryptoContext method names the executor uses.
    Levels follow the FLEXIBLEAUTO rules (a product is degree 2 until the
    next rescale); EvalBootstrap returns the values at level `boot_depth`.
    Rotations need keys, as on the GPU."""

    def __init__(self, slots: int, L: int = 45, boot_depth: int = 21):
        self.slots, self.L, self.boot_depth = slots, L, boot_depth
        self.n = 2 * slots          # ring dimension stand-in (cyclotomic order 2n)
        self.keys: set = set()
        self.bootstraps = 0

    def GetRingDimension(self):  # noqa: N802
        return self.n

    def GetBatchSize(self):  # noqa: N802
        return self.slots

    def GetModuli(self):  # noqa: N802
        return [0] * self.L, []

    def _plain(self, v):
        return SlotCt(np.asarray(v, dtype=complex))

    def MakeCKKSPackedPlaintext(self, values, deg=1, level=0, params=None, slots=0):  # noqa: N802
        v = np.zeros(self.slots, dtype=complex)
        vals = np.asarray(values, dtype=complex).ravel()
        v[: len(vals)] = vals
        return ("pt", v, level)

    def Encrypt(self, pk, pt):  # noqa: N802
        return SlotCt(pt[1])

    def Decrypt(self, ct, sk):  # noqa: N802
        return _SlotPlain(ct.z)

    def _rescaled(self, a):
        if a.deg >= 2:
            a = SlotCt(a.z, a.level + 1, a.deg - 1)
        return a

    def Rescale(self, a):  # noqa: N802
        return self._rescaled(a)

    def RescaleInPlace(self, a):  # noqa: N802
        a._assign(self._rescaled(a))

    def _check(self, level):
        assert level <= self.L - 1, f"level {level} beyond the chain"

    def AlignToLevel(self, a, level):  # noqa: N802
        x = self._rescaled(a)
        if not x.level <= level < self.L:
            raise ValueError(f"cannot align level {x.level} to level {level}")
        return x if level == x.level else SlotCt(x.z, level, 1)

    def EvalAdd(self, a, b):  # noqa: N802
        if isinstance(b, SlotCt):
            lv = max(a.level, b.level)
            return SlotCt(a.z + b.z, lv, max(a.deg, b.deg))
        if isinstance(b, tuple):
            return SlotCt(a.z + b[1], a.level, a.deg)
        return SlotCt(a.z + float(b), a.level, a.deg)

    def EvalSub(self, a, b):  # noqa: N802
        if isinstance(b, SlotCt):
            return SlotCt(a.z - b.z, max(a.level, b.level), max(a.deg, b.deg))
        return SlotCt(a.z - float(b), a.level, a.deg)

    def EvalMult(self, a, b):  # noqa: N802
        a = self._rescaled(a)
        if isinstance(b, SlotCt):
            b = self._rescaled(b)
            out = SlotCt(a.z * b.z, max(a.level, b.level), 2)
        elif isinstance(b, tuple):
            out = SlotCt(a.z * b[1], max(a.level, b[2]), 2)
        else:
            out = SlotCt(a.z * float(b), a.level, 2)
        self._check(out.level + 1)
        return out

    def EvalSquare(self, a):  # noqa: N802
        return self.EvalMult(a, a)

    def EvalLinearWSum(self, cts, weights):  # noqa: N802
        cts = [self._rescaled(c) for c in cts]
        lv = max(c.level for c in cts)
        self._check(lv + 1)
        return SlotCt(sum(float(w) * c.z for c, w in zip(cts, weights)), lv, 2)

    def MultByInteger(self, a, v):  # noqa: N802
        return SlotCt(a.z * int(v), a.level, a.deg)

    def EvalRotateKeyGen(self, sk, idx):  # noqa: N802
        self.keys.update(int(i) % self.slots for i in idx)

    def _rot(self, a, k):
        k %= self.slots
        assert k == 0 or k in self.keys, f"no key for rotation {k}"
        return SlotCt(np.roll(a.z, -k), a.level, a.deg)

    def EvalRotate(self, a, k):  # noqa: N802
        return self._rot(a, k)

    def EvalRotateMany(self, cts, k):  # noqa: N802
        self.rotate_many_calls = getattr(self, "rotate_many_calls", 0) + 1
        idx = list(k) if isinstance(k, (list, tuple)) else [k] * len(cts)
        return [self._rot(c, i) for c, i in zip(cts, idx)]

    def EvalFastRotationPrecompute(self, a):  # noqa: N802
        return a

    def EvalFastRotation(self, a, idx, m, pre):  # noqa: N802
        return [self._rot(a, k) for k in idx]

    def LinearTransformInPlace(self, ct, rows, bstep, pts, stride=1, offset=0):  # noqa: N802
        """The schedules of CryptoContext.LinearTransformInPlace, chosen the
        same way by the keys present (each rotation asserts its key)."""
        used = sorted({k % bstep for k in range(rows) if pts[k] is not None})
        giants = -(-rows // bstep)
        have = lambda r: r % self.slots == 0 or r % self.slots in self.keys  # noqa: E731
        fold = bool(offset) and all(have(offset + b * stride) for b in used)
        batch = giants > 2 and all(have(g * bstep * stride) for g in range(1, giants))
        x = self._rescaled(ct if fold or not offset else self._rot(ct, offset))
        off = offset if fold else 0
        lv = x.level
        inners = []
        for g in range(giants):
            inner = np.zeros(self.slots, dtype=complex)
            for b in range(bstep):
                k = g * bstep + b
                if k < rows and pts[k] is not None:
                    inner += pts[k][1] * self._rot(x, off + b * stride).z
                    lv = max(lv, pts[k][2])
            inners.append(inner)
        if batch:                          # every giant rotation from its own key
            out = inners[0].copy()
            for g in range(1, giants):
                out += self._rot(SlotCt(inners[g]), g * bstep * stride).z
        else:                              # Horner's rule: one giant key
            out = inners[-1]
            for inner in reversed(inners[:-1]):
                out = self._rot(SlotCt(out), bstep * stride).z + inner
        ct._assign(SlotCt(out, lv, 2))

    def EvalBootstrapSetup(self, budget, dims, slots, correction=0, precompute=True, *,  # noqa: N802
                           s2c_first=False, real_slots=False):
        # S2C-first moves the SlotToCoeff levels from the output to the input
        self.boot_s2c_levels = int(budget[1]) if s2c_first else 0

    def GetBootstrapInputCeiling(self):  # noqa: N802
        return self.L - 2 - getattr(self, "boot_s2c_levels", 0)

    def EvalBootstrapKeyGen(self, sk, slots):  # noqa: N802
        pass

    def _bootstrapper(self):
        class _B:
            @staticmethod
            def rotation_indices():
                return []
        return _B()

    def EvalBootstrap(self, ct, passes=1, precision=0, *, scale=1.0):  # noqa: N802
        ct = self._rescaled(ct)
        assert ct.level <= self.GetBootstrapInputCeiling(), "bootstrap input too deep"
        # the refresh bound must bring every slot into [-1, 1]
        top = np.max(np.abs(ct.z)) / scale
        assert top <= 1.0 + 1e-9, f"bootstrap input {top}"
        self.bootstraps += passes
        return SlotCt(ct.z, self.boot_depth - getattr(self, "boot_s2c_levels", 0), 1)

    def EvalBootstrapMany(self, cts, passes=1, precision=0, *, scale=1.0,  # noqa: N802
                          real_slots=None):
        self.bootstrap_many_calls = getattr(self, "bootstrap_many_calls", []) + [len(cts)]
        outs = [self.EvalBootstrap(ct, passes, precision, scale=scale) for ct in cts]
        if real_slots is None or real_slots:
            for o in outs:
                o.z = o.z.real.astype(complex)
        return outs

    def MultByMonomial(self, a, power):  # noqa: N802
        # X^(N/2) multiplies every slot by i, X^(3N/2) by -i (N = self.n)
        p = int(power) % (2 * self.n)
        if p not in (self.n // 2, 3 * self.n // 2):
            raise NotImplementedError("slot stand-in: only X^(N/2) and X^(3N/2)")
        return SlotCt(a.z * (1j if p == self.n // 2 else -1j), a.level, a.deg)

    def EvalConjugateMany(self, cts):  # noqa: N802
        return [SlotCt(np.conj(c.z), c.level, c.deg) for c in cts]


class _SlotPlain:
    def __init__(self, z):
        self.z = z
        self.n = len(z)

    def SetLength(self, n):  # noqa: N802
        self.n = n

    def GetRealPackedValue(self):  # noqa: N802
        return list(self.z.real[: self.n])
