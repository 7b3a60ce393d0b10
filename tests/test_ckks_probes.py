"""Circuit helpers (the ckks_probes interface) on array and depth-ledger
backends, and the parameter / chain selection of the OpenFHE-shaped API.
Host only: no device work."""
import math
import sys
from types import SimpleNamespace

import numpy as np
import pytest

from fhemamba_amd import ckks
from fhemamba_amd.ckks_probes import (CkksPrimitives, affine, build_toy_context, ceil_log2,
                                      cheb_baby_size, cheb_eval64, cheb_ps_depth,
                                      chebyshev_ps, chebyshev_ps_many, floor_coeffs)


class ArrayBackend:
    """Plain numpy arrays in place of ciphertexts (no encryption)."""

    def MakeCKKSPackedPlaintext(self, values):  # noqa: N802
        return np.asarray(values)

    def Encrypt(self, key, values):  # noqa: N802
        return values.copy()

    def EvalMult(self, left, right):  # noqa: N802
        return left * right

    def EvalAdd(self, left, right):  # noqa: N802
        return left + right

    def EvalSub(self, left, right):  # noqa: N802
        return left - right


class DepthBackend:
    """Ciphertexts are their consumed depth: a product (ciphertext or
    double) costs one level, additions take the maximum."""

    def __init__(self):
        self.mults = 0

    def MakeCKKSPackedPlaintext(self, values):  # noqa: N802
        return ("pt",)

    def Encrypt(self, key, pt):  # noqa: N802
        return 0

    def EvalMult(self, a, b):  # noqa: N802
        self.mults += 1
        return max(a, b if isinstance(b, int) and not isinstance(b, bool) and
                   not isinstance(b, float) else 0) + 1

    def EvalAdd(self, a, b):  # noqa: N802
        return max(a, b) if isinstance(b, int) else a

    def EvalSub(self, a, b):  # noqa: N802
        return max(a, b) if isinstance(b, int) else a


DEGREES = [0, 1, 2, 3, 7, 8, 15, 16, 31, 32, 59, 79, 119]


@pytest.mark.parametrize("degree", DEGREES)
def test_chebyshev_matches_numpy(degree):
    he = CkksPrimitives(ArrayBackend(), SimpleNamespace(publicKey=None), batch=37)
    x = np.linspace(-0.95, 0.95, 37)
    c = np.random.default_rng(degree).normal(size=degree + 1)
    if degree > 2:
        c[2] = 1e-15  # below the floor: skipped by the circuit, zeroed here
    c = floor_coeffs(c)
    np.testing.assert_allclose(he.eval_chebyshev(x, c), cheb_eval64(c, x), rtol=1e-10,
                               atol=1e-10)
    np.testing.assert_array_equal(he.eval_chebyshev(x, [0.0] * 8), np.zeros(37))


class LockstepBackend(ArrayBackend):
    """ArrayBackend with EvalMultMany; counts the ciphertext products and
    the steps they are issued in (one per EvalMultMany call or lone
    ciphertext product)."""

    def __init__(self):
        self.products = self.steps = 0

    def EvalMult(self, left, right):  # noqa: N802
        if isinstance(right, np.ndarray):
            self.products += 1
            self.steps += 1
        return left * right

    def EvalMultMany(self, pairs):  # noqa: N802
        self.products += len(pairs)
        self.steps += 1
        return [a * b for a, b in pairs]


@pytest.mark.parametrize("degrees", [(59,), (96, 64, 64), (3, 31, 119), (0, 8, 15), (59, 59)])
def test_lockstep_series_equal_one_at_a_time(degrees):
    """chebyshev_ps_many gives each series exactly what chebyshev_ps gives
    it alone; in lockstep the products of every series go out in as many
    steps as the deepest series alone needs."""
    rng = np.random.default_rng(sum(degrees))
    xs = [rng.uniform(-0.95, 0.95, 29) for _ in degrees]
    cs = [floor_coeffs(rng.normal(size=d + 1)) for d in degrees]
    const = lambda v: np.full(29, v)  # noqa: E731
    alone = [chebyshev_ps(ArrayBackend(), x, c, 1e-12, const) for x, c in zip(xs, cs)]
    many = LockstepBackend()
    got = chebyshev_ps_many(many, [(x, c, 1e-12, const) for x, c in zip(xs, cs)])
    for a, g, x, c in zip(alone, got, xs, cs):
        np.testing.assert_array_equal(g, a)
        np.testing.assert_allclose(g, cheb_eval64(c, x), rtol=1e-9, atol=1e-9)
    singles = []
    for x, c in zip(xs, cs):
        b = LockstepBackend()
        chebyshev_ps_many(b, [(x, c, 1e-12, const)])
        singles.append(b)
    assert many.products == sum(b.products for b in singles)
    assert many.steps == max(b.steps for b in singles)


@pytest.mark.parametrize("degree", [d for d in DEGREES if d >= 1])
def test_ps_depth_ledger_matches_circuit(degree):
    """cheb_ps_depth equals the depth the circuit actually consumes when
    every coefficient is present, and is at least ceil(log2(degree + 1))."""
    be = DepthBackend()
    he = CkksPrimitives(be, SimpleNamespace(publicKey=None), batch=4)
    got = he.eval_chebyshev(0, [1.0] * (degree + 1))
    assert got == cheb_ps_depth(degree)
    assert cheb_ps_depth(degree) >= ceil_log2(degree + 1)


def test_small_helpers():
    assert affine(2, 6) == (0.5, -2.0)
    a, b = affine(-3.0, 5.0)
    assert a * -3.0 + b == -1.0 and a * 5.0 + b == 1.0
    assert [ceil_log2(v) for v in (1, 2, 3, 4, 5, 1024, 1025)] == [0, 1, 2, 2, 3, 10, 11]
    assert [cheb_baby_size(d) for d in (1, 3, 7, 15, 31, 63)] == [2, 2, 4, 4, 8, 8]
    assert floor_coeffs([1e-13, -1e-11, 0.5], 1e-12) == [0.0, -1e-11, 0.5]
    # brute force on the definition: 2^ceil(levels/2) with levels from d + 1
    for d in range(1, 300):
        levels = max(1, math.ceil(math.log2(d + 1)))
        assert cheb_baby_size(d) == 2 ** math.ceil(levels / 2)


def test_padding_and_newton():
    he = CkksPrimitives(ArrayBackend(), SimpleNamespace(publicKey=None), batch=4)
    np.testing.assert_array_equal(he.encrypt(np.array([1.0, 2.0]), fill=-0.25),
                                  [1, 2, -0.25, -0.25])
    x, y = np.array([1.0, 2.0, 3.0, 4.0]), np.full(4, 0.6)
    want = y.copy()
    for _ in range(3):
        want = 1.5 * want - 0.5 * x * want ** 3
    np.testing.assert_allclose(he.newton_refine(y, -0.5 * x, 3), want)
    # converges to 1/sqrt(x) from a close start
    z = he.newton_refine(1 / np.sqrt(x) * 1.05, -0.5 * x, 6)
    np.testing.assert_allclose(z, 1 / np.sqrt(x), rtol=1e-12)
    np.testing.assert_allclose(he.affine_ct(np.array([2.0]), 0.5, -1.0), [0.0])
    np.testing.assert_allclose(he.const_ct(3.5), np.full(4, 3.5))


def test_build_toy_context_calls(monkeypatch):
    calls = {}

    class Params:
        def __getattr__(self, name):
            return lambda value: calls.update({name: value})

    context = SimpleNamespace(
        Enable=lambda feature: calls.setdefault("features", []).append(feature),
        KeyGen=lambda: SimpleNamespace(secretKey="secret"),
        EvalMultKeyGen=lambda key: calls.update(mult_key=key),
        EvalRotateKeyGen=lambda key, rotations: calls.update(rotations=rotations),
    )
    backend = SimpleNamespace(
        CCParamsCKKSRNS=Params,
        GenCryptoContext=lambda params: context,
        KeySwitchTechnique=SimpleNamespace(HYBRID="hybrid"),
        ScalingTechnique=SimpleNamespace(FLEXIBLEAUTO="flexible"),
        SecretKeyDist=SimpleNamespace(UNIFORM_TERNARY="ternary"),
        SecurityLevel=SimpleNamespace(HEStd_NotSet="not-set"),
        PKESchemeFeature=SimpleNamespace(PKE=1, KEYSWITCH=2, LEVELEDSHE=3, ADVANCEDSHE=4,
                                         FHE=5),
    )
    cc, _ = build_toy_context(ring_dimension=16384, batch=8192, depth=40, scale_bits=59,
                              first_mod_bits=60, rotations=[1, -1], backend=backend)
    assert cc is context
    assert calls == {
        "SetSecretKeyDist": "ternary", "SetSecurityLevel": "not-set", "SetRingDim": 16384,
        "SetScalingTechnique": "flexible", "SetFirstModSize": 60, "SetScalingModSize": 59,
        "SetKeySwitchTechnique": "hybrid", "SetMultiplicativeDepth": 40,
        "SetBatchSize": 8192, "features": [1, 2, 3, 4, 5], "mult_key": "secret",
        "rotations": [1, -1],
    }


# ---------------------------------------------------------------- parameters
def test_params_defaults_and_setters():
    p = ckks.CCParamsCKKSRNS()
    assert p.GetMultiplicativeDepth() == 1 and p.GetScalingModSize() == 50
    assert p.GetFirstModSize() == 60 and p.GetRingDim() == 0
    assert p.GetScalingTechnique() == ckks.ScalingTechnique.FLEXIBLEAUTO
    p.SetRingDim(8192)
    p.SetMultiplicativeDepth(7)
    assert p.GetRingDim() == 8192 and p.GetMultiplicativeDepth() == 7
    with pytest.raises(AttributeError):
        p.SetNoSuchThing(1)


def test_num_large_digits_rule():
    assert [ckks._num_large_digits(0, d) for d in (0, 1, 2, 3, 4, 30)] == [1, 2, 2, 2, 3, 3]
    assert ckks._num_large_digits(5, 1) == 5


def _params(**kw):
    p = ckks.CCParamsCKKSRNS()
    for k, v in kw.items():
        getattr(p, "Set" + k)(v)
    return p


def test_select_chain_explicit_ring():
    ring, q, p, dnum = ckks.select_chain(_params(
        RingDim=8192, MultiplicativeDepth=7, ScalingModSize=50, FirstModSize=60,
        SecurityLevel=ckks.SecurityLevel.HEStd_NotSet))
    assert ring == 8192 and len(q) == 8 and dnum == 3
    assert all((x - 1) % (2 * ring) == 0 for x in q + p)
    with pytest.raises(ValueError):  # 8 x ~50-bit + P far above 2^13's 218-bit bound
        ckks.select_chain(_params(RingDim=8192, MultiplicativeDepth=7, ScalingModSize=50))


def test_select_chain_smallest_secure_ring():
    ring, q, p, _ = ckks.select_chain(_params(MultiplicativeDepth=3, ScalingModSize=40,
                                              FirstModSize=50))
    bits = ckks._log2_qp(q, p)
    table = ckks._HE_STD_MAX_LOGQ[ckks.SecurityLevel.HEStd_128_classic]
    assert bits <= table[ring]
    smaller = [r for r in table if r < ring]
    if smaller:  # the next smaller ring would not hold this chain
        r2 = max(smaller)
        try:
            q2, p2 = ckks.gen_moduli(r2.bit_length() - 1, 3, 40, 50, 2)
            assert ckks._log2_qp(q2, p2) > table[r2]
        except Exception:
            pass


def test_select_chain_rejects_unimplemented():
    for kw in ({"ScalingTechnique": ckks.ScalingTechnique.FIXEDMANUAL},
               {"KeySwitchTechnique": ckks.KeySwitchTechnique.BV},
               {"SecretKeyDist": ckks.SecretKeyDist.GAUSSIAN}):
        with pytest.raises(NotImplementedError):
            ckks.select_chain(_params(RingDim=1024, **kw))
    # sparse-ternary secrets use the same chain as uniform-ternary ones
    assert ckks.select_chain(_params(RingDim=1024, SecurityLevel=ckks.SecurityLevel.HEStd_NotSet,
                                     SecretKeyDist=ckks.SecretKeyDist.SPARSE_TERNARY)) == \
        ckks.select_chain(_params(RingDim=1024, SecurityLevel=ckks.SecurityLevel.HEStd_NotSet))
    with pytest.raises(ValueError):
        ckks.select_chain(_params(SecurityLevel=ckks.SecurityLevel.HEStd_NotSet))


@pytest.mark.parametrize("degrees", [(0, 0), (1, 3), (7, 5), (15, 7), (31, 2), (59, 59)])
def test_vector_coefficient_series(degrees):
    """chebyshev_ps_rows (one coefficient per slot) over one shared basis:
    each slot's value equals numpy's Chebyshev series of that slot's
    coefficient column, and the depth ledger equals cheb_ps_depth with the
    shared baby-step size (zero rows are skipped, and a series with no
    term is the constant ciphertext)."""
    from fhemamba_amd.ckks_probes import ChebBasis, chebyshev_ps_rows
    rng = np.random.default_rng(sum(degrees))
    slots = 12
    x = np.linspace(-0.97, 0.97, slots)
    baby = cheb_baby_size(max(max(degrees), 1))
    be = ArrayBackend()
    basis = ChebBasis(be, x)
    for deg in degrees:
        rows = rng.normal(size=(deg + 1, slots))
        rows[:, 3] = 0.0                         # an inactive slot
        if deg >= 2:
            rows[1] = 0.0                        # a zero row is skipped
        got = chebyshev_ps_rows(basis, rows, baby, lambda c, r, k: c * r,
                                lambda c, r: c + r, lambda r: r.copy())
        want = [np.polynomial.chebyshev.chebval(x[s], rows[:, s]) for s in range(slots)]
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)
        assert got[3] == 0.0
    db = DepthBackend()
    dbasis = ChebBasis(db, 0)
    for deg in degrees:
        depth = chebyshev_ps_rows(dbasis, np.ones((deg + 1, 2)), baby,
                                  lambda c, r, k: c + 1, lambda c, r: c, lambda r: 0)
        assert depth == cheb_ps_depth(deg, baby)
