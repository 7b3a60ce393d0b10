"""Bootstrapping plan on the CPU: the factored special FFT against the
oracle's encode / decode FFT, the baby-step giant-step layout of each group,
the sine approximation, and the whole circuit on a slot-level simulation
(ModRaise simulated through the oracle's coefficient encoding)."""
import math

import numpy as np
import pytest

import oracle as O
from fhemamba_amd import bootstrap as B


def brv_perm(n):
    bits = n.bit_length() - 1
    return np.array([int(format(i, f"0{bits}b")[::-1], 2) if bits else 0 for i in range(n)])


@pytest.mark.parametrize("n", [2, 4, 16, 128, 1024])
@pytest.mark.parametrize("budget", [1, 2, 3, 4])
def test_fft_groups_match_oracle_fft(n, budget):
    rng = np.random.default_rng(n + budget)
    z = rng.normal(size=n) + 1j * rng.normal(size=n)
    coef = np.array(O.fft_special_inv(z))           # encode FFT (with its 1/n and bitrev)
    # encode stages without bit reversal: n * coef at slot brv(j)
    y = z.copy()
    for g in B.fft_groups(n, budget, inverse=True):
        y = B.apply_diags(g, y)
    assert np.max(np.abs(y - n * coef[brv_perm(n)])) < 1e-12 * n
    # decode stages on bit-reversed input give back the slots
    w = coef[brv_perm(n)].copy()
    for g in B.fft_groups(n, budget, inverse=False):
        w = B.apply_diags(g, w)
    assert np.max(np.abs(w - z)) < 1e-12 * n
    assert np.allclose(np.array(O.fft_special(coef)), z)


def test_stage_diagonals_are_sparse():
    n = 64
    for L in (2, 4, 64):
        for D in (B.forward_stage(n, L), B.inverse_stage(n, L)):
            assert sorted(D) == sorted({0, L // 2 % n, (-L // 2) % n})


def test_split_budget():
    assert B.split_budget(15, 4) == [4, 4, 4, 3]
    assert B.split_budget(15, 1) == [15]
    assert B.split_budget(3, 5) == [1, 1, 1]
    assert sum(B.split_budget(11, 3)) == 11


def simulate_linear_transform(ct, plan):
    """LinearTransformInPlace semantics: rotate by offset, then
    sum_g rot(sum_b pts[g*bs+b] * rot(ct, b*stride), g*bs*stride)."""
    rot = lambda v, k: np.roll(v, -k)  # noqa: E731
    x = rot(ct, plan.offset)
    pts = plan.prerotated()
    out = np.zeros_like(x)
    for g in range((plan.rows + plan.bstep - 1) // plan.bstep):
        inner = np.zeros_like(x)
        for b in range(plan.bstep):
            k = g * plan.bstep + b
            if k < plan.rows and pts[k] is not None:
                inner += pts[k] * rot(x, b * plan.stride)
        out += rot(inner, g * plan.bstep * plan.stride)
    return out


@pytest.mark.parametrize("n,budget", [(256, 3), (1024, 4), (2048, 3), (32768, 4)])
def test_group_plans_reproduce_groups(n, budget):
    rng = np.random.default_rng(7)
    x = rng.normal(size=n) + 1j * rng.normal(size=n)
    for inverse in (True, False):
        groups = B.fft_groups(n, budget, inverse) if n <= 2048 else \
            B.fft_groups(n, budget, inverse)[:1]
        for D in groups:
            plan = B.plan_group(D, n)
            assert plan.rows <= 2 ** (max(B.split_budget(int(math.log2(n)), budget)) + 1) - 1
            assert np.max(np.abs(simulate_linear_transform(x, plan) - B.apply_diags(D, x))) \
                < 1e-9
            # every rotation the transform makes is in its key list
            assert all(r % n for r in plan.rotations())


def test_uniform_ternary_bound():
    assert B.uniform_ternary_bound(2 ** 12) == 128
    assert B.uniform_ternary_bound(2 ** 16) == 512


def test_secret_bound_and_sparse_plan():
    """K from the secret's Hamming weight: 2N/3 reproduces the uniform
    bound; h = 192 (sparse ternary) gives K = 64, four double angles and a
    degree-59 cosine, three levels fewer than the uniform plan at N=2^16
    (K = 512, seven double angles, degree 59)."""
    for ring in (2 ** 12, 2 ** 16):
        assert B.secret_bound(2 * ring / 3) == B.uniform_ternary_bound(ring)
    assert B.secret_bound(192) == 64
    sparse = B.BootstrapConfig.for_ring(2 ** 16, (4, 4), hamming_weight=192).sine
    dense = B.BootstrapConfig.for_ring(2 ** 16, (4, 4)).sine
    assert (sparse.K, sparse.r, sparse.degree) == (64, 4, 59)
    assert (dense.K, dense.r, dense.degree) == (512, 7, 59)
    assert dense.depth() - sparse.depth() == 3
    # a sparse secret's smaller rounding noise (and smaller K) leaves room
    # for a larger scale-down, which shrinks the sine's cubic term
    c_sparse = B.correction_bits_for(2 ** 16, sparse, 2.0 ** 59, 2.0 ** 60, 2.0 ** 59,
                                     hamming_weight=192)
    c_dense = B.correction_bits_for(2 ** 16, dense, 2.0 ** 59, 2.0 ** 60, 2.0 ** 59)
    assert (c_sparse, c_dense) == (10, 7)


@pytest.mark.parametrize("ring,hw", [(2 ** 10, 0), (2 ** 12, 0), (2 ** 16, 0), (2 ** 16, 192)])
def test_sine_approximation(ring, hw):
    s = B.BootstrapConfig.for_ring(ring, hamming_weight=hw).sine
    K = int(s.K)
    u = (np.arange(-K + 1, K)[:, None] + np.linspace(-2 ** -10, 2 ** -10, 17)[None, :]).ravel()
    assert np.max(np.abs(s.plain(u) - np.sin(2 * np.pi * u))) < 1e-9
    # the interpolant stays inside [-1, 1] (T_i stay bounded)
    v = np.linspace(-1, 1, 20001)
    assert np.max(np.abs(np.polynomial.chebyshev.chebval(v, s.coeffs))) <= 1 + 1e-9


# ---------------------------------------------------------------- slot simulation
class SimCt:
    def __init__(self, z, level, deg=1):
        self.z, self.level, self.deg = np.asarray(z, dtype=complex), level, deg

    def Clone(self):  # noqa: N802
        return SimCt(self.z.copy(), self.level, self.deg)

    def GetLevel(self):  # noqa: N802
        return self.level

    def SetLevel(self, level):  # noqa: N802
        self.level = level

    def GetNoiseScaleDeg(self):  # noqa: N802
        return self.deg


class SimCC:
    """Slot vectors (all N/2 evaluation points) in place of ciphertexts.
    ModRaise goes through the oracle's encoding: the coefficients
    t = Encode(z) * scale gain q0 * I for random integers |I| < K / 2 (at
    every coefficient, also outside a sparse message's subring) and are
    decoded at scale sf0."""

    def __init__(self, log_n, L, q0_bits=60, sf_bits=59, seed=0):
        self.N, self.L = 1 << log_n, L
        self.q0 = float(2 ** q0_bits - 2 ** 20 + 1)
        self.sf = [2.0 ** sf_bits] * L
        self.rng = np.random.default_rng(seed)
        self.ibound = 0

    def GetRingDimension(self):  # noqa: N802
        return self.N

    def GetModuli(self):  # noqa: N802
        return [int(self.q0)] + [1] * (self.L - 1), []

    def GetScalingFactorReal(self, level):  # noqa: N802
        return self.sf[level]

    def RescaleInPlace(self, ct):  # noqa: N802
        while ct.deg >= 2:
            ct.deg -= 1
            ct.level += 1
        assert ct.level < self.L

    @staticmethod
    def _val(x):
        return x.z if isinstance(x, SimCt) else x

    def _bin(self, a, b, f, deg_add):
        level = max(a.level, b.level) if isinstance(b, SimCt) else a.level
        deg = a.deg + (b.deg if isinstance(b, SimCt) else 1) if deg_add else a.deg
        return SimCt(f(a.z, self._val(b)), level, deg)

    def EvalAdd(self, a, b):  # noqa: N802
        return self._bin(a, b, np.add, False)

    def EvalSub(self, a, b):  # noqa: N802
        return self._bin(a, b, np.subtract, False)

    def EvalMult(self, a, b):  # noqa: N802
        a = a.Clone()
        self.RescaleInPlace(a)
        if isinstance(b, SimCt):
            b = b.Clone()
            self.RescaleInPlace(b)
        return self._bin(a, b, np.multiply, True)

    def EvalSquare(self, a):  # noqa: N802
        return self.EvalMult(a, a)

    def MultByInteger(self, a, value):  # noqa: N802
        return SimCt(a.z * int(value), a.level, a.deg)

    def EvalConjugate(self, a):  # noqa: N802
        return SimCt(np.conj(a.z), a.level, a.deg)

    def MultByMonomial(self, a, power):  # noqa: N802
        n = self.N // 2
        rot = np.array([pow(5, j, 2 * self.N) for j in range(n)], dtype=object)
        e = np.array([int(power * r % (2 * self.N)) for r in rot], dtype=float)
        return SimCt(a.z * np.exp(1j * np.pi * e / self.N), a.level, a.deg)

    def MakeCKKSPackedPlaintext(self, values, deg=1, level=0, slots=0):  # noqa: N802
        v = np.asarray(values, dtype=complex)
        return np.tile(v, (self.N // 2) // len(v))         # sparse slots repeat

    def EvalRotate(self, a, k):  # noqa: N802
        return SimCt(np.roll(a.z, -k), a.level, a.deg)

    def LinearTransformInPlace(self, ct, rows, bstep, pts, stride, offset):  # noqa: N802
        plan = B.GroupPlan(offset=offset, stride=stride, diags=[None] * rows, bstep=bstep)
        plan.prerotated = lambda: pts
        self.RescaleInPlace(ct)
        ct.z = simulate_linear_transform(ct.z, plan)
        ct.deg += 1

    def ModRaise(self, x):  # noqa: N802
        assert x.level == self.L - 1
        coef = np.array(O.fft_special_inv(x.z))          # t / scale as complex pairs
        t = np.round(coef * self.sf[self.L - 1])
        I = self.rng.integers(-self.ibound, self.ibound + 1, size=(2, len(t)))
        t = t + self.q0 * (I[0] + 1j * I[1])
        return SimCt(np.array(O.fft_special(t / self.sf[0])), 0)

    def GetScalingFactor(self, ct):
        return self.sf[ct.level]


SimCt.GetScalingFactor = lambda self: 2.0 ** 59
SimCt.SetScalingFactor = lambda self, scale: None


@pytest.mark.parametrize("log_n,budget", [(8, (2, 2)), (10, (3, 3)), (11, (4, 2))])
def test_bootstrap_circuit_on_slots(log_n, budget):
    cc = SimCC(log_n, L=40)
    cfg = B.BootstrapConfig.for_ring(1 << log_n, budget)
    cc.ibound = int(cfg.sine.K) // 2
    boot = B.CKKSBootstrapper(cc, cfg)
    n = cc.N // 2
    rng = np.random.default_rng(log_n)
    m = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    out = boot.bootstrap(SimCt(m, 5))
    assert out.level == boot.depth()
    err = np.max(np.abs(out.z - m))
    # noise-free: the sine's cubic term at |P / q0| <= 2^-(c+1) bounds the error
    c = boot.correction_bits(2.0 ** 59, cc.q0, 2.0 ** 59)
    assert c == B.correction_bits_for(cc.N, cfg.sine, 2.0 ** 59, cc.q0, 2.0 ** 59) >= 9
    assert err < 1e-5, err


def test_coefficient_bound_matches_the_encode_fft():
    """coefficient_bound against the oracle's encode FFT (the coefficients
    of the message, as complex pairs): random real and complex slots at
    full packing and a constant vector (all mass in one coefficient)."""
    for n in (2, 16, 512, 4096):
        rng = np.random.default_rng(n)
        for z in (rng.uniform(-1, 1, n), rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n),
                  np.full(n, -0.25)):
            v = np.asarray(O.fft_special_inv(z))
            want = max(np.max(np.abs(v.real)), np.max(np.abs(v.imag))) / np.max(np.abs(z))
            assert B.coefficient_bound(z) == pytest.approx(want, rel=1e-12, abs=1e-15)
    assert B.coefficient_bound(np.zeros(8)) == 1.0
    with pytest.raises(ValueError):
        B.coefficient_bound(np.ones(6))


def test_correction_bits_with_a_coefficient_bound():
    """c falls by (2/3) log2(1/b) for a coefficient bound b (the cubic term
    is sized for coefficients b times the slot bound); b = 1 is the
    default's worst case, and b outside (0, 1] is refused."""
    sine = B.BootstrapConfig.for_ring(2 ** 16).sine
    args = (2 ** 16, sine, 2.0 ** 59, 2.0 ** 60, 2.0 ** 59)
    c1 = B.correction_bits_for(*args)
    assert B.correction_bits_for(*args, coeff_bound=1.0) == c1 == 7
    assert B.correction_bits_for(*args, coeff_bound=2.0 ** -6) == c1 - 4
    assert B.correction_bits_for(*args, coeff_bound=2.0 ** -3) == c1 - 2
    for bad in (0.0, -0.5, 1.5):
        with pytest.raises(ValueError):
            B.correction_bits_for(*args, coeff_bound=bad)


@pytest.mark.parametrize("log_n,budget", [(10, (3, 3)), (11, (4, 2))])
def test_bootstrap_circuit_with_a_coefficient_bound(log_n, budget):
    """Noise-free, the smaller scale-down that a coefficient bound allows
    keeps the sine's cubic term at the size the worst case has: the same
    error bound as without it."""
    cc = SimCC(log_n, L=40)
    cfg = B.BootstrapConfig.for_ring(1 << log_n, budget)
    cc.ibound = int(cfg.sine.K) // 2
    boot = B.CKKSBootstrapper(cc, cfg)
    n = cc.N // 2
    rng = np.random.default_rng(log_n + 7)
    m = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    b = B.coefficient_bound(m)
    assert boot.correction_bits(2.0 ** 59, cc.q0, 2.0 ** 59, b) <= \
        boot.correction_bits(2.0 ** 59, cc.q0, 2.0 ** 59) - 2
    out = boot.bootstrap(SimCt(m, 5), coeff_bound=b)
    assert np.max(np.abs(out.z - m)) < 1e-5


def test_correction_bits_model():
    """c grows with the room the noise leaves: 10 at N = 2^12 and 7 at
    N = 2^16 for a 59-bit scale over a 60-bit q0; 0 at a 50-bit scale."""
    for ring, sbits, want in ((2 ** 12, 59, 10), (2 ** 16, 59, 7), (2 ** 12, 50, 0)):
        sine = B.BootstrapConfig.for_ring(ring).sine
        assert B.correction_bits_for(ring, sine, 2.0 ** sbits, 2.0 ** 60, 2.0 ** sbits) == want


@pytest.mark.parametrize("log_n,slots", [(10, 64), (11, 8), (11, 512)])
def test_sparse_bootstrap_circuit_on_slots(log_n, slots):
    """Sparse packing: the trace after ModRaise removes I's coefficients
    outside the subring, so only the n slots' own coefficients reach EvalMod."""
    cc = SimCC(log_n, L=40, seed=slots)
    cfg = B.BootstrapConfig.for_ring(1 << log_n, (2, 2))
    cc.ibound = int(cfg.sine.K) // 2
    boot = B.CKKSBootstrapper(cc, cfg, slots)
    assert boot.trace_rotations() == [slots << k for k in range(int(math.log2(boot.R)))]
    rng = np.random.default_rng(slots)
    m = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    out = boot.bootstrap(SimCt(np.tile(m, boot.R), 5))
    assert np.max(np.abs(out.z - np.tile(m, boot.R))) < 1e-5
    with pytest.raises(ValueError):
        B.CKKSBootstrapper(cc, cfg, 3)


def test_bootstrap_rejects_a_fresh_top_level_input():
    cc = SimCC(8, L=30)
    boot = B.CKKSBootstrapper(cc, B.BootstrapConfig.for_ring(256, (2, 2)))
    with pytest.raises(ValueError):
        boot.bootstrap(SimCt(np.zeros(128), 29))


@pytest.mark.parametrize("total", [37.25, -37.25, 3.0e-5, 1.0, 16.0, -0.75])
@pytest.mark.parametrize("groups", [1, 2, 3, 4])
def test_group_factors(total, groups):
    """The group constants multiply to the total (even spread or power of
    two on the last group); with the power on the last group, totals that
    differ by a power of two share every other group's constant, and a
    total in (2^(g-1), 2^g) is spread evenly."""
    for power_last in (False, True):
        f = B.CKKSBootstrapper.group_factors(total, groups, power_last)
        assert len(f) == groups
        assert math.isclose(math.prod(f), total, rel_tol=1e-12)
    f = B.CKKSBootstrapper.group_factors(total, groups, True)
    for k in (-13, -1, 3):
        g = B.CKKSBootstrapper.group_factors(total * 2.0 ** k, groups, True)
        assert g[:-1] == f[:-1]
        assert g[-1] == f[-1] * 2.0 ** k
    inside = 1.5 * 2.0 ** (groups - 1)
    even = B.CKKSBootstrapper.group_factors(inside, groups, False)
    split = B.CKKSBootstrapper.group_factors(inside, groups, True)
    assert all(math.isclose(a, b, rel_tol=1e-14) for a, b in zip(even, split))
    with pytest.raises(ValueError):
        B.CKKSBootstrapper.group_factors(0.0, groups)


@pytest.mark.parametrize("log_n,budget", [(8, (2, 2)), (10, (3, 3)), (11, (2, 4))])
@pytest.mark.parametrize("real", [False, True])
def test_s2c_first_bootstrap_circuit_on_slots(log_n, budget, real):
    """S2C-first ordering: SlotToCoeff on the input, ModRaise, CoeffToSlot,
    EvalMod.  The output holds the message (complex, or with real_slots
    the real message from one EvalMod) at depth len(c2s) + sine depth; the
    input ceiling is the SlotToCoeff levels lower; the residual pass's
    pre / post constants ride through as in the ordinary order."""
    cc = SimCC(log_n, L=40)
    cfg = B.BootstrapConfig.for_ring(1 << log_n, budget)
    cc.ibound = int(cfg.sine.K) // 2
    boot = B.CKKSBootstrapper(cc, cfg, s2c_first=True, real_slots=real)
    plain = B.CKKSBootstrapper(cc, cfg)
    assert boot.depth() == plain.depth() - budget[1]
    assert boot.input_ceiling() == plain.input_ceiling() - budget[1] == 40 - 2 - budget[1]
    n = cc.N // 2
    rng = np.random.default_rng(log_n)
    m = rng.uniform(-1, 1, n) + (0 if real else 1j * rng.uniform(-1, 1, n))
    out = boot.bootstrap(SimCt(m, 5))
    assert out.level == boot.depth()
    assert np.max(np.abs(out.z - m)) < 1e-5
    if real:
        assert np.max(np.abs(out.z.imag)) < 1e-12
    # a residual-style pass: slots scaled up by 2^12 on the way in, down on the way out
    r = 1e-4 * m
    out = boot.bootstrap(SimCt(r, 5), pre=2.0 ** 12, post=2.0 ** -12)
    assert np.max(np.abs(out.z - r)) < 1e-9
    with pytest.raises(ValueError, match="level"):
        boot.bootstrap(SimCt(m, boot.input_ceiling() + 1))
    with pytest.raises(ValueError, match="full packing"):
        B.CKKSBootstrapper(cc, cfg, n // 2, s2c_first=True)


def test_s2c_first_residual_pass_with_a_small_bound():
    """A residual pass for a small refresh bound (pre = 2^12 / 2^-10): pre
    rides on the scale-down constant, not on the SlotToCoeff diagonals,
    whose constants stay those of every other bound."""
    cc = SimCC(10, L=40)
    cfg = B.BootstrapConfig.for_ring(1 << 10, (2, 2))
    cc.ibound = int(cfg.sine.K) // 2
    boot = B.CKKSBootstrapper(cc, cfg, s2c_first=True, real_slots=True)
    m = np.random.default_rng(3).uniform(-1, 1, 512) * 2.0 ** -22
    out = boot.bootstrap(SimCt(m, 5), pre=2.0 ** 22, post=2.0 ** -22)
    assert np.max(np.abs(out.z - m)) < 2.0 ** -40
    keys = {k for k in boot._pts._d if k[0] == "s2c_first"}
    assert keys
    boot.bootstrap(SimCt(m * 2.0 ** 8, 5), pre=2.0 ** 14, post=2.0 ** -14)
    assert {k for k in boot._pts._d if k[0] == "s2c_first"} == keys
