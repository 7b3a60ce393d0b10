"""CKKS bootstrapping (full and sparse packing) over the CKKS interface.

Pipeline of EvalBootstrap as the reference drives it
(native/fideslib_stage0/src/packed_fideslib.cpp:235-270,
src/stage1_mamba2_decode_fideslib.cpp:2127-2297):
  1. scale the input down by 2^-c (the correction that keeps the message
     small against q0) and drop it to one limb;
  2. ModRaise (fhe_mod_raise): the decryption becomes t = P + q0 I;
  3. CoeffToSlot: the inverse special FFT (the encoder's, without its final
     bit reversal), so slot s holds (t_j + i t_{j+n}) / q0 for j =
     brv(s), scaled by 1/(2K);
  4. EvalMod on the real and imaginary parts (split by conjugation):
     sin(2 pi u) / (2 pi) ~ u - round(u) from a Chebyshev interpolant of
     cos(2 pi (u - 1/4) / 2^r) on [-K, K] and r double-angle steps;
  5. SlotToCoeff: the forward special FFT stages on the bit-reversed input,
     scaled back by q0 2^c / (2 pi scale).
The FFTs are factored into their radix-2 stages, grouped by the level
budget; each group is one baby-step giant-step linear transform over the
diagonals of the group's product (LinearTransformInPlace).

S2C-first ordering (EvalBootstrapSetup(..., s2c_first=True), the
reference's --s2c-first circuit, packed_fideslib.cpp:1084-1086, :1131-1134;
full packing only): SlotToCoeff runs first, on the input at its low level,
so that the plaintext's coefficients j and j + n become the real and
imaginary parts of slot brv(j); then scale-down, ModRaise, CoeffToSlot and
EvalMod leave the message in the slots with no transform after EvalMod.
The input needs the SlotToCoeff levels before the drop to one limb (a
lower refresh ceiling) and the output keeps them (a higher refreshed
level).  For real slots (real_slots=True) the imaginary half carries no
message: one EvalMod on the real part and a projection onto the real
part (one conjugation) are the whole result.

The stage structure follows the encoder's special FFT (oracle/ckks_oracle.c
fft_special / fft_special_inv: roots zeta^(5^j) of order 4 * slots).
OpenFHE's exact bootstrapping (its level-budget split of the FFT, its sine
approximation and scaling constants, the sparse-secret key) is not
reproduced: the result is checked by decryption, not residue by residue.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .ckks_probes import cheb_ps_depth, chebyshev_ps_many
from .ptcache import PlaintextCache
from .rotation import bsgs_rotations

Diag = dict  # rotation offset -> complex diagonal vector


# ----------------------------------------------------------------- FFT stages
def _rot_group(n: int) -> np.ndarray:
    m = 4 * n
    out = np.empty(n, dtype=np.int64)
    p = 1
    for j in range(n):
        out[j] = p
        p = p * 5 % m
    return out


def _twiddle(k: int, m: int) -> complex:
    a = 2.0 * math.pi * k / m
    return complex(math.cos(a), math.sin(a))


def forward_stage(n: int, length: int) -> Diag:
    """Stage `length` of the decode FFT: for each block and j < h,
    out[x] = a[x] + w_j a[x+h], out[x+h] = a[x] - w_j a[x+h]."""
    m, h = 4 * n, length // 2
    lenq, rot = 4 * length, _rot_group(n)
    gap = m // lenq
    w = np.array([_twiddle(int(rot[j] % lenq) * gap, m) for j in range(h)])
    x = np.arange(n)
    j = x % length
    top = j < h
    d0 = np.where(top, 1.0 + 0j, -w[np.where(top, 0, j - h)])
    dp = np.where(top, w[np.where(top, j, 0)], 0j)
    dm = np.where(top, 0j, 1.0 + 0j)
    return _merge({0: d0, h % n: dp}, {(-h) % n: dm})


def inverse_stage(n: int, length: int) -> Diag:
    """Stage `length` of the encode FFT: out[x] = a[x] + a[x+h],
    out[x+h] = conj(w_j) (a[x] - a[x+h])."""
    m, h = 4 * n, length // 2
    lenq, rot = 4 * length, _rot_group(n)
    gap = m // lenq
    wc = np.array([_twiddle(int((lenq - rot[j] % lenq) * gap), m) for j in range(h)])
    x = np.arange(n)
    j = x % length
    top = j < h
    wb = wc[np.where(top, 0, j - h)]
    d0 = np.where(top, 1.0 + 0j, -wb)
    dp = np.where(top, 1.0 + 0j, 0j)
    dm = np.where(top, 0j, wb)
    return _merge({0: d0, h % n: dp}, {(-h) % n: dm})


def _merge(a: Diag, b: Diag) -> Diag:
    out = {k: v.copy() for k, v in a.items()}
    for k, v in b.items():
        out[k] = out[k] + v if k in out else v.copy()
    return out


def compose(A: Diag, B: Diag, n: int) -> Diag:
    """Diagonals of A(B(.)): sum over k + m = s of A_k * rot(B_m, k)."""
    out: Diag = {}
    for k, da in A.items():
        for mo, db in B.items():
            s = (k + mo) % n
            term = da * np.roll(db, -k)
            out[s] = out[s] + term if s in out else term
    return out


def apply_diags(D: Diag, a: np.ndarray) -> np.ndarray:
    out = np.zeros_like(a, dtype=complex)
    for k, d in D.items():
        out += d * np.roll(a, -k)
    return out


def split_budget(stages: int, budget: int) -> list[int]:
    """Stage counts per group, as even as possible, larger groups first."""
    budget = max(1, min(budget, stages))
    base, extra = divmod(stages, budget)
    return [base + (1 if i < extra else 0) for i in range(budget)]


def fft_groups(n: int, budget: int, inverse: bool) -> list[Diag]:
    """The encode (inverse=True: stages n..2) or decode (stages 2..n) FFT
    without bit reversal, as `budget` composed groups in application order."""
    lengths = [1 << k for k in range(1, int(math.log2(n)) + 1)]
    if inverse:
        lengths = lengths[::-1]
    stages = [inverse_stage(n, L) if inverse else forward_stage(n, L) for L in lengths]
    groups, i = [], 0
    for size in split_budget(len(stages), budget):
        D = stages[i]
        for s in stages[i + 1:i + size]:
            D = compose(s, D, n)
        groups.append(D)
        i += size
    return groups


@dataclass
class GroupPlan:
    """One linear transform: out = sum_k pts[k] (.) rot(in, offset + k stride)."""
    offset: int
    stride: int
    diags: list            # complex vectors (None for zero), index k
    bstep: int

    @property
    def rows(self) -> int:
        return len(self.diags)

    def rotations(self) -> list[int]:
        """Keys of LinearTransformInPlace's fast schedule (the offset folded
        into the babies' shared ModUp, the giant steps as one batch)."""
        used = sorted({k % self.bstep for k, d in enumerate(self.diags) if d is not None})
        return bsgs_rotations(self.rows, self.bstep, self.stride, self.offset, used)

    def prerotated(self) -> list:
        """pts[k] rotated by -(k // bstep) * bstep * stride (LinearTransformInPlace)."""
        out = []
        for k, d in enumerate(self.diags):
            if d is None:
                out.append(None)
            else:
                out.append(np.roll(d, (k // self.bstep) * self.bstep * self.stride))
        return out


def plan_group(D: Diag, n: int, tol: float = 1e-12) -> GroupPlan:
    """Lay a group's nonzero diagonals on an arithmetic progression of
    rotation offsets (symmetric offsets -r..r of the smallest stride)."""
    offs = [k for k, v in D.items() if np.max(np.abs(v)) > tol]
    signed = sorted(((k + n // 2) % n) - n // 2 for k in offs)
    nz = [abs(s) for s in signed if s]
    stride = min(nz) if nz else 1
    lo, hi = signed[0], signed[-1]
    rows = (hi - lo) // stride + 1
    diags = [None] * rows
    for k in offs:
        s = ((k + n // 2) % n) - n // 2
        idx = (s - lo) // stride
        diags[idx] = D[k] if diags[idx] is None else diags[idx] + D[k]
    bstep = max(1, 1 << int(math.ceil(math.log2(max(1, math.isqrt(rows))))))
    return GroupPlan(offset=lo, stride=stride, diags=diags, bstep=bstep)


# ----------------------------------------------------------------- EvalMod
@dataclass(frozen=True)
class SineApprox:
    """sin(2 pi u) for u in [-K, K] as cos(2 pi (u - 1/4) / 2^r) (Chebyshev
    interpolant of degree `degree` in v = u / K) and r double-angle steps
    cos(2x) = 2 cos(x)^2 - 1."""
    K: float
    r: int
    degree: int

    @property
    def coeffs(self) -> list[float]:
        f = lambda v: np.cos(2 * np.pi * (v * self.K - 0.25) / 2 ** self.r)  # noqa: E731
        return [float(c) for c in np.polynomial.chebyshev.chebinterpolate(f, self.degree)]

    def plain(self, u: np.ndarray) -> np.ndarray:
        c = np.polynomial.chebyshev.chebval(np.asarray(u) / self.K, self.coeffs)
        for _ in range(self.r):
            c = 2 * c * c - 1
        return c

    def depth(self) -> int:
        return cheb_ps_depth(self.degree) + self.r


def uniform_ternary_bound(ring_dim: int) -> float:
    """Power of two K bounding |I| in t = m + q0 I after ModRaise for a
    uniform-ternary secret: each coefficient of I is a sum of about 2N/3 + 1
    terms uniform in [-1/2, 1/2] (standard deviation sqrt(N / 18)); K covers
    8 standard deviations."""
    return float(1 << math.ceil(math.log2(8.0 * math.sqrt(ring_dim / 18.0))))


def secret_bound(hamming_weight: float) -> float:
    """K for a secret with `hamming_weight` nonzero +-1 coefficients: I is a
    sum of hamming_weight + 1 terms uniform in [-1/2, 1/2], standard
    deviation sqrt((h + 1) / 12); K covers 8 of them (h = 2N/3 gives
    uniform_ternary_bound; h = 192 gives 64)."""
    return float(1 << math.ceil(math.log2(8.0 * math.sqrt((hamming_weight + 1.0) / 12.0))))


NOISE_MODEL_OFFSET_BITS = 4.0


def coefficient_bound(values) -> float:
    """max |m_k| / max |z_j| for the message polynomial m whose n slots are
    `values`: z_j = m(psi^(5^j)), psi = exp(i pi / 2n), over the subring of
    degree 2n (a sparse message's coefficients sit at multiples of N / 2n
    with these values).  m_k = (1 / 2n) sum over odd e of m(psi^e) psi^(-ek),
    the values at the odd powers being z_j at 5^j and conj(z_j) at -5^j
    (mod 4n): one FFT of length 2n.  A client that knows its slots computes
    this before encrypting; every message has it in (0, 1]."""
    z = np.asarray(values, dtype=np.complex128).ravel()
    n = len(z)
    if n < 1 or n & (n - 1):
        raise ValueError("coefficient_bound needs a power-of-two number of slots")
    top = float(np.max(np.abs(z)))
    if top == 0.0:
        return 1.0
    m = 2 * n
    e = np.array([pow(5, j, 2 * m) for j in range(n)])
    w = np.zeros(2 * m, dtype=np.complex128)
    w[e] = z
    w[(-e) % (2 * m)] = np.conj(z)
    coef = np.exp(-1j * np.pi * np.arange(m) / m) * np.fft.fft(w[1::2]) / m
    return float(min(1.0, np.max(np.abs(coef.real)) / top))


def correction_bits_for(ring_dim: int, sine: SineApprox, in_scale: float, q0: float,
                        scale: float, slots: int = 0, hamming_weight: float = 0.0,
                        coeff_bound: float = 1.0) -> int:
    """Scale-down c (the message enters ModRaise times 2^-c) balancing the
    two errors of one bootstrap, in message units for a coefficient of size 1:
      * noise: rescale / key-switch rounding of about sqrt(N h / 12) per
        coefficient (h nonzero secret coefficients; N / sqrt(18) for a
        uniform-ternary secret, h = 2N/3, the default) at the working scale,
        times K (v = u / K), 2^r (double angles), sqrt(slots) (SlotToCoeff
        gain) and q0 / (2 pi in_scale) (the way back), all times 2^c; the
        offset NOISE_MODEL_OFFSET_BITS is measured (N = 2^12 and 2^16,
        59-bit scale, uniform ternary);
      * the sine's cubic term: (2 pi a)^2 / 6 relative, a = 2^-c b in_scale / q0
        for coefficients at most b (coeff_bound, 1 by default: a constant
        slot vector puts its whole mass in one coefficient) times the slot
        bound.
    Equal at 3c = log2((2 pi rho)^2 / 6) - e0, rho = b in_scale / q0."""
    if not 0.0 < coeff_bound <= 1.0:
        raise ValueError("coeff_bound must lie in (0, 1]")
    rho = coeff_bound * in_scale / q0
    h = float(hamming_weight) or 2.0 * ring_dim / 3.0
    e0 = (math.log2(math.sqrt(ring_dim * h / 12.0) / scale) + math.log2(sine.K) + sine.r
          + 0.5 * math.log2(slots or ring_dim // 2)
          + math.log2(q0 / (2 * math.pi * in_scale))
          + NOISE_MODEL_OFFSET_BITS)
    c = (math.log2((2 * math.pi * rho) ** 2 / 6.0) - e0) / 3.0
    return max(0, min(30, int(round(c))))


@dataclass
class BootstrapConfig:
    level_budget: tuple = (3, 3)
    correction_bits: int = 0            # 0: chosen by correction_bits_for()
    sine: SineApprox = field(default_factory=lambda: SineApprox(K=128.0, r=5, degree=59))
    hamming_weight: float = 0.0         # nonzero secret coefficients; 0: uniform ternary

    @classmethod
    def for_ring(cls, ring_dim: int, level_budget=(3, 3), correction_bits: int = 0,
                 hamming_weight: float = 0.0):
        """K from the secret's bound (uniform ternary unless hamming_weight
        is given); r = log2 K - 2 double angles bring the interpolated
        cosine down to K / 2^r = 4 periods over [-K, K], interpolated with
        degree 59: within 2^-38 (K = 64) ... 2^-32 (K = 512) of the sine
        over [-K, K] after the double angles.  For K = 512 this spends the
        same levels as 6 double angles and degree 89, with 5 fewer
        relinearizations per EvalMod and a smaller error."""
        h = float(hamming_weight) or 2.0 * ring_dim / 3.0
        K = secret_bound(h)
        sine = SineApprox(K=K, r=max(0, int(math.log2(K)) - 2), degree=59)
        return cls(level_budget=tuple(level_budget), correction_bits=int(correction_bits),
                   sine=sine, hamming_weight=h)


class CKKSBootstrapper:
    """Bootstrapping of `slots`-slot ciphertexts for a CryptoContext of this
    package (driven by CryptoContext.EvalBootstrapSetup / EvalBootstrap).

    Sparse packing (slots n < N/2): the message lies in the subring of
    X^(N/2n) and its slots repeat with period n over the N/2 evaluation
    points.  After ModRaise the sum of rotations by n, 2n, ..., N/4 (the
    trace onto that subring) turns t = m + q0 I into R (m + q0 I'), R =
    N / 2n, where I' keeps I's coefficients at multiples of N/2n; the n-point
    transforms then act on the n slots as they do at full packing, and 1/R
    joins the CoeffToSlot constant."""

    def __init__(self, cc, config: BootstrapConfig | None = None, slots: int = 0,
                 pt_cache_bytes: int = 16 << 30, s2c_first: bool = False,
                 real_slots: bool = False):
        self.cc = cc
        self.cfg = config or BootstrapConfig.for_ring(cc.GetRingDimension())
        self.N = cc.GetRingDimension()
        self.n = int(slots) or self.N // 2
        if self.n < 2 or self.n & (self.n - 1) or self.n > self.N // 2:
            raise ValueError(f"bootstrapping slots must be a power of two in [2, {self.N // 2}]")
        if s2c_first and self.n != self.N // 2:
            raise ValueError("S2C-first bootstrapping requires full packing")
        self.s2c_first = bool(s2c_first)
        self.real_slots = bool(real_slots)
        self.R = self.N // (2 * self.n)
        self.c2s = [plan_group(D, self.n) for D in
                    fft_groups(self.n, self.cfg.level_budget[0], inverse=True)]
        self.s2c = [plan_group(D, self.n) for D in
                    fft_groups(self.n, self.cfg.level_budget[1], inverse=False)]
        self._coeffs = self.cfg.sine.coeffs
        self._pts = PlaintextCache(self.N, pt_cache_bytes)

    def trace_rotations(self) -> list[int]:
        """Rotations n, 2n, ..., N/4 of the subring trace (empty at full packing)."""
        return [self.n << k for k in range(int(math.log2(self.R)))]

    def rotation_indices(self) -> list[int]:
        out = set()
        for g in self.c2s + self.s2c:
            out.update(i % self.n for i in g.rotations())
        return sorted(i for i in out if i) + self.trace_rotations()

    def depth(self) -> int:
        """Levels from ModRaise (level 0) to the output."""
        return len(self.c2s) + self.cfg.sine.depth() + (0 if self.s2c_first else len(self.s2c))

    def input_ceiling(self) -> int:
        """Deepest input level (limbs consumed) EvalBootstrap accepts:
        L - 2, less the SlotToCoeff levels under S2C-first."""
        return len(self.cc.GetModuli()[0]) - 2 - (len(self.s2c) if self.s2c_first else 0)

    def correction_bits(self, in_scale: float, q0: float, scale: float,
                        coeff_bound: float = 1.0) -> int:
        if self.cfg.correction_bits:
            return self.cfg.correction_bits
        return correction_bits_for(self.N, self.cfg.sine, in_scale, q0, scale, self.n,
                                   self.cfg.hamming_weight, coeff_bound)

    # --------------------------------------------------------------- helpers
    def _group_pts(self, which: str, idx: int, plan: GroupPlan, level: int, factor: float):
        key = (which, idx, level, factor)
        pts = self._pts.get(key)
        if pts is None:
            diags = plan.prerotated()
            rows = [d * factor for d in diags if d is not None]
            batch = getattr(self.cc, "MakeCKKSPackedPlaintexts", None)
            many = batch(rows, 1, level, slots=self.n) if batch else \
                [self.cc.MakeCKKSPackedPlaintext(r, 1, level, slots=self.n) for r in rows]
            it = iter(many)
            pts = [None if d is None else next(it) for d in diags]
            self._pts.put(key, pts)
        return pts

    @staticmethod
    def group_factors(total: float, groups: int, power_last: bool = False) -> list[float]:
        """Per-group constants whose product is `total`: spread evenly, or
        (power_last) the mantissa m of |total| = m 2^e spread as
        (m 2^(groups-1))^(1/groups) and the rest of the power of two on the
        last group, so that totals sharing a mantissa share the diagonals
        of every group but the last."""
        mag = abs(total)
        if mag == 0.0:
            raise ValueError("transform constant must be non-zero")
        if power_last:
            fr, ex = math.frexp(mag)                          # mag = fr 2^ex, fr in [1/2, 1)
            base = (2.0 * fr * 2.0 ** (groups - 1)) ** (1.0 / groups)
            out = [base] * groups
            out[-1] = base * 2.0 ** (ex - groups)
        else:
            out = [mag ** (1.0 / groups)] * groups
        if total < 0:
            out[0] = -out[0]
        return out

    def _transform(self, ct, plans: list, which: str, total: float, power_last: bool = False):
        """Apply the groups in order, their diagonals scaled by
        group_factors(total)."""
        factors = self.group_factors(total, len(plans), power_last)
        for idx, plan in enumerate(plans):
            if ct.GetNoiseScaleDeg() >= 2:
                self.cc.RescaleInPlace(ct)
            pts = self._group_pts(which, idx, plan, ct.GetLevel(), factors[idx])
            # offsets mod n: rotations act on the n slots (5^-h and 5^(n-h)
            # differ as automorphisms once n < N/2)
            self.cc.LinearTransformInPlace(ct, plan.rows, plan.bstep, pts, plan.stride,
                                           plan.offset % self.n)
        self.cc.RescaleInPlace(ct)
        return ct

    def _transform_many(self, cts: list, plans: list, which: str, total: float,
                        power_last: bool = False) -> list:
        """_transform of every ciphertext of `cts` in step: each group's
        rescales share their launches and the ciphertexts at one level go
        through one multi-ciphertext linear transform."""
        cc = self.cc
        factors = self.group_factors(total, len(plans), power_last)
        cts = list(cts)
        for idx, plan in enumerate(plans):
            # the degree-2 ones rescaled together (the others are used as
            # they are, as RescaleInPlace leaves them)
            deep = [i for i, ct in enumerate(cts) if ct.GetNoiseScaleDeg() >= 2]
            for i, r in zip(deep, cc.RescaleMany([cts[i] for i in deep])):
                cts[i] = r
            by_level: dict = {}
            for ct in cts:
                by_level.setdefault(ct.GetLevel(), []).append(ct)
            for level, group in by_level.items():
                pts = self._group_pts(which, idx, plan, level, factors[idx])
                cc.LinearTransformManyInPlace(group, plan.rows, plan.bstep, pts, plan.stride,
                                              plan.offset % self.n)
        return cc.RescaleMany(cts)

    def _squares(self, cs: list) -> list:
        """EvalSquare of each (one batched relinearization for several)."""
        many = getattr(self.cc, "EvalMultMany", None)
        if many is not None and len(cs) > 1:
            return many([(c, c) for c in cs])
        return [self.cc.EvalSquare(c) for c in cs]

    def _eval_mod(self, vs: list, gain: int = 1) -> list:
        """sin(2 pi u) * gain for each v = u / K of `vs` (independent
        inputs, evaluated in lockstep); the integer gain rides on the last
        double angle (gain (2 y^2 - 1) = (2 gain) y^2 - gain by an integer
        product, no level)."""
        cs = chebyshev_ps_many(self.cc, [(v, self._coeffs, 1e-14, None) for v in vs])
        r = self.cfg.sine.r
        for step in range(r):
            sqs = self._squares(cs)
            if step == r - 1 and gain != 1:
                cs = [self.cc.EvalSub(self.cc.MultByInteger(sq, 2 * gain), float(gain))
                      for sq in sqs]
            else:
                cs = [self.cc.EvalSub(self.cc.EvalAdd(sq, sq), 1.0) for sq in sqs]
        if r == 0 and gain != 1:
            cs = [self.cc.MultByInteger(c, gain) for c in cs]
        return cs

    def _eval_mod_amplitude(self, vs: list, amp: float) -> list:
        """amp sin(2 pi u) for each v = u / K of `vs` (in lockstep) and any
        real amp > 0: the interpolant carries a_0 = amp^(2^-r) and each
        double angle y <- 2 y^2 - a_(k+1) with a_(k+1) = a_k^2, so y_k =
        a_k cos(2^k x) and y_r = amp cos(2^r x) with integer products only."""
        r = self.cfg.sine.r
        a = amp ** (2.0 ** -r)
        # the floor scales with a: the same terms as the unscaled interpolant
        coeffs = [a * x for x in self._coeffs]
        cs = chebyshev_ps_many(self.cc, [(v, coeffs, 1e-14 * a, None) for v in vs])
        for _ in range(r):
            a = a * a
            cs = [self.cc.EvalSub(self.cc.EvalAdd(sq, sq), a) for sq in self._squares(cs)]
        return cs

    # --------------------------------------------------------------- bootstrap
    def bootstrap(self, ct, pre: float = 1.0, post: float = 1.0, coeff_bound: float = 1.0):
        """Refresh ct; the slots are multiplied by `pre` on the way in (in
        the scale-down step) and by `post` on the way out (in SlotToCoeff),
        so a residual pass spends no extra level.  `coeff_bound` (the
        ordinary order only): a public bound b on the message's
        coefficients relative to its slot bound (coefficient_bound of the
        slots); EvalMod sees those coefficients, so c is sized for b
        instead of the worst case 1.  Under S2C-first EvalMod sees the slot
        values themselves and b has no effect."""
        if self.s2c_first:
            return self._bootstrap_s2c_first(ct, pre, post)
        cc, n, N = self.cc, self.n, self.N
        L = len(cc.GetModuli()[0])
        q0 = float(cc.GetModuli()[0][0])
        x = ct.Clone()
        cc.RescaleInPlace(x)
        if x.GetLevel() > L - 2:
            raise ValueError(f"EvalBootstrap needs the input at level <= {L - 2}")
        x.SetLevel(L - 2)
        in_scale = cc.GetScalingFactorReal(L - 1)
        c = self.correction_bits(in_scale, q0, cc.GetScalingFactorReal(0), coeff_bound)
        # The product by sf[L-2] / scale(x) makes the rescaled scale
        # sf[L-2]^2 / q1 = sf[L-1] whatever level x came from, so the
        # constants below (and their cached diagonals) depend on pre and
        # post alone.
        x = cc.EvalMult(x, pre * 2.0 ** -c * cc.GetScalingFactorReal(L - 2) / x.GetScalingFactor())
        cc.RescaleInPlace(x)                                  # one limb left
        x.SetScalingFactor(in_scale)
        raised = cc.ModRaise(x)                               # decrypts to t = P + q0 I
        for r in self.trace_rotations():                      # sparse: R (P + q0 I')
            raised = cc.EvalAdd(raised, cc.EvalRotate(raised, r))
        # Slots of `raised` are Decode(t) / sf0; the encode stages map them
        # to n * (t_j + i t_{j+n}) / sf0 at slot brv(j) (coefficient index
        # j N/2n under sparse packing).  Scaled so that each part of
        # u = (t_j + i t_{j+n}) / q0 arrives divided by 2K.
        K = self.cfg.sine.K
        y = self._transform(raised, self.c2s, "c2s",
                            raised.GetScalingFactor() / (q0 * n * 2 * K * self.R))
        yc = cc.EvalConjugate(y)
        re = cc.EvalAdd(y, yc)                                # Re(u) / K
        im = cc.MultByMonomial(cc.EvalSub(y, yc), 3 * N // 2)  # (2i Im(u) / 2K) * -i
        # The decode stages of (P_j + i P_{j+n}) / in_scale at slot brv(j)
        # give the message times 2^-c.  A power of two of the way-back factor
        # moves into EvalMod so that each SlotToCoeff group's diagonals stay
        # within 2 (times the scale) of the 62-bit encoding limit.
        back = q0 / (2 * math.pi * in_scale) * 2.0 ** c * post
        gain = 1 << max(0, math.ceil(math.log2(max(back, 1.0))) - len(self.s2c))
        re_m, im_m = self._eval_mod([re, im], gain)           # gain sin(2 pi u)
                                                              #   ~ gain 2 pi P / q0
        w = cc.EvalAdd(re_m, cc.MultByMonomial(im_m, N // 2))
        return self._transform(w, self.s2c, "s2c", back / gain, power_last=True)

    def bootstrap_many(self, cts, pre: float = 1.0, post: float = 1.0,
                       real_slots: bool | None = None) -> list:
        """bootstrap(ct, pre, post) of every ciphertext of `cts`, in step
        under S2C-first (each stage's key switches, rescales and EvalMod
        products of all of them share their launches; the same ciphertexts
        as one call each); the ordinary order refreshes them in turn.
        `real_slots` (S2C-first) overrides the setup's slot mode for this
        call: False refreshes complex slots (two real ciphertexts packed as
        a + i b, say) with both EvalMods."""
        cts = list(cts)
        real = self.real_slots if real_slots is None else bool(real_slots)
        if not self.s2c_first or (len(cts) <= 1 and real == self.real_slots):
            return [self.bootstrap(ct, pre, post) for ct in cts]
        cc, n, N = self.cc, self.n, self.N
        L = len(cc.GetModuli()[0])
        q0 = float(cc.GetModuli()[0][0])
        top = self.input_ceiling()
        xs = cc.RescaleMany(cts)
        for x in xs:
            if x.GetLevel() > top:
                raise ValueError(f"S2C-first EvalBootstrap needs the input at level <= {top}")
            x.SetLevel(top)
        in_scale = cc.GetScalingFactorReal(L - 1)
        c = self.correction_bits(in_scale, q0, cc.GetScalingFactorReal(0))
        amp = q0 / (2 * math.pi * in_scale) * 2.0 ** c * post
        k = post * q0 / (amp * 2 * math.pi * in_scale)
        ys = self._transform_many(xs, self.s2c, "s2c_first", k, power_last=True)
        ys = cc.RescaleMany([cc.EvalMult(y, pre * cc.GetScalingFactorReal(L - 2)
                                         / y.GetScalingFactor()) for y in ys])
        for y in ys:
            y.SetScalingFactor(in_scale)
        raised = [cc.ModRaise(y) for y in ys]
        K = self.cfg.sine.K
        zs = self._transform_many(raised, self.c2s, "c2s",
                                  raised[0].GetScalingFactor() / (q0 * n * 2 * K))
        zcs = cc.EvalConjugateMany(zs)
        if real:
            outs = self._eval_mod_amplitude([cc.EvalAdd(z, zc) for z, zc in zip(zs, zcs)],
                                            amp / 2)
            outs = cc.RescaleMany(outs)
            return [cc.EvalAdd(o, oc) for o, oc in zip(outs, cc.EvalConjugateMany(outs))]
        m = len(zs)
        ims = [cc.MultByMonomial(cc.EvalSub(z, zc), 3 * N // 2) for z, zc in zip(zs, zcs)]
        res = self._eval_mod_amplitude([cc.EvalAdd(z, zc) for z, zc in zip(zs, zcs)] + ims,
                                       amp)
        outs = [cc.EvalAdd(res[i], cc.MultByMonomial(res[m + i], N // 2)) for i in range(m)]
        return cc.RescaleMany(outs)

    def _bootstrap_s2c_first(self, ct, pre: float, post: float):
        """SlotToCoeff, scale-down, ModRaise, CoeffToSlot, EvalMod.

        The SlotToCoeff constant k and the scale-down's `pre` make the
        one-limb plaintext's coefficients P_j + i P_{j+n} = in_scale k
        v[brv(j)] for v = pre m; EvalMod with amplitude A returns
        A 2 pi P / q0 = pre post m when k = post q0 / (A 2 pi in_scale).  A
        is the ordinary pipeline's way-back factor q0 2^c post /
        (2 pi in_scale), so k = 2^-c and |P / q0| (the sine's argument) has
        the same size as there; A, whatever real value, rides on the
        double-angle constants (_eval_mod_amplitude), no level.  The input
        is first dropped
        to the fixed level input_ceiling(), so the SlotToCoeff diagonals are
        encoded at one level whatever level the input came from."""
        cc, n, N = self.cc, self.n, self.N
        L = len(cc.GetModuli()[0])
        q0 = float(cc.GetModuli()[0][0])
        x = ct.Clone()
        cc.RescaleInPlace(x)
        top = self.input_ceiling()
        if x.GetLevel() > top:
            raise ValueError(f"S2C-first EvalBootstrap needs the input at level <= {top}")
        x.SetLevel(top)
        in_scale = cc.GetScalingFactorReal(L - 1)
        c = self.correction_bits(in_scale, q0, cc.GetScalingFactorReal(0))
        amp = q0 / (2 * math.pi * in_scale) * 2.0 ** c * post        # EvalMod's amplitude
        k = post * q0 / (amp * 2 * math.pi * in_scale)               # = 2^-c
        y = self._transform(x, self.s2c, "s2c_first", k, power_last=True)
        # level L - 2: times pre (which may be large: a plain constant has
        # no encoding limit) to one limb at scale sf[L-1], as the ordinary
        # scale-down
        y = cc.EvalMult(y, pre * cc.GetScalingFactorReal(L - 2) / y.GetScalingFactor())
        cc.RescaleInPlace(y)
        y.SetScalingFactor(in_scale)
        raised = cc.ModRaise(y)
        K = self.cfg.sine.K
        z = self._transform(raised, self.c2s, "c2s", raised.GetScalingFactor() / (q0 * n * 2 * K))
        zc = cc.EvalConjugate(z)
        if self.real_slots:
            # EvalMod turns the conjugation's key-switch noise in Re(u) / K
            # into imaginary slot noise amp 2 pi K times larger, which a
            # second pass would not see and high-degree polynomials would
            # fold back into the real parts: the result is projected onto
            # its real part, (y + conj(y)) / 2 with the 1/2 in the amplitude
            out = self._eval_mod_amplitude([cc.EvalAdd(z, zc)], amp / 2)[0]
            cc.RescaleInPlace(out)
            out = cc.EvalAdd(out, cc.EvalConjugate(out))             # pre post Re(m)
        else:
            im = cc.MultByMonomial(cc.EvalSub(z, zc), 3 * N // 2)
            out, im_m = self._eval_mod_amplitude([cc.EvalAdd(z, zc), im], amp)
            out = cc.EvalAdd(out, cc.MultByMonomial(im_m, N // 2))
            cc.RescaleInPlace(out)
        return out


def main(argv=None) -> int:
    """Time EvalBootstrap on one seeded full-packing ciphertext:
    python -m fhemamba_amd.bootstrap [--log-n 16] [--depth 44] [--secret
    sparse|uniform] [--order s2c-first|ordinary] [--passes 1|2]
    [--repeat K] [--warmup W].  Prints one JSON line (ms per call, its
    launches when profiling, the decrypted error)."""
    import argparse
    import json
    import time

    import numpy as np

    from .ckks_probes import build_toy_context

    ap = argparse.ArgumentParser(prog="python -m fhemamba_amd.bootstrap")
    ap.add_argument("--log-n", type=int, default=16)
    ap.add_argument("--depth", type=int, default=44)
    ap.add_argument("--secret", choices=("sparse", "uniform"), default="sparse")
    ap.add_argument("--order", choices=("s2c-first", "ordinary"), default="s2c-first")
    ap.add_argument("--passes", type=int, choices=(1, 2), default=1)
    ap.add_argument("--repeat", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--correction-factor", type=int, default=0,
                    help="message scale-down exponent c (OpenFHE's correctionFactor; "
                         "0 picks it from the ring, secret and order)")
    args = ap.parse_args(argv)
    n = 1 << args.log_n
    slots = n // 2
    s2c = args.order == "s2c-first"
    cc, keys = build_toy_context(ring_dimension=n, batch=slots, depth=args.depth, scale_bits=59,
                                 first_mod_bits=60, seed=21,
                                 secret_dist="SPARSE_TERNARY" if args.secret == "sparse"
                                 else "UNIFORM_TERNARY")
    cc.EvalBootstrapSetup([4, 4], [0, 0], slots, args.correction_factor, s2c_first=s2c,
                          real_slots=s2c)
    cc.EvalBootstrapKeyGen(keys.secretKey, slots)
    x = np.random.default_rng(8).uniform(-1, 1, slots)
    ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(x)))
    ct.SetLevel(cc.GetBootstrapInputCeiling())
    for _ in range(args.warmup):
        cc.EvalBootstrap(ct, args.passes)
    cc.device.sync()
    t0 = time.perf_counter()
    for _ in range(args.repeat):
        out = cc.EvalBootstrap(ct, args.passes)
    cc.device.sync()
    ms = (time.perf_counter() - t0) / max(args.repeat, 1) * 1e3
    cc.device.profile_begin()
    cc.EvalBootstrap(ct, args.passes)
    prof = cc.device.profile_end()
    pt = cc.Decrypt(out, keys.secretKey)
    pt.SetLength(slots)
    err = float(np.max(np.abs(np.asarray(pt.GetRealPackedValue()) - x)))
    print(json.dumps({
        "ring_dimension": n, "depth": args.depth, "secret": args.secret, "order": args.order,
        "passes": args.passes, "correction_factor": args.correction_factor or "auto",
        "ms_per_call": ms,
        "kernel_ms_per_call": sum(v[1] for v in prof.values()),
        "launches_per_call": sum(v[0] for v in prof.values()),
        "max_abs_err": err, "output_level": int(out.GetLevel()),
    }))
    return 0


if __name__ == "__main__":
    import sys

    sys.exit(main())
