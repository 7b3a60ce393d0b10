"""The OpenFHE-shaped CKKS interface end to end on the GPU: FLEXIBLEAUTO
level / scale bookkeeping, ciphertext and plaintext arithmetic, rotations,
conjugation, the BSGS linear transform and the probe circuits, checked by
decryption against numpy (CKKS precision; the residue-level parity of every
primitive is covered by the oracle tests)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd import ckks  # noqa: E402
from fhemamba_amd.ckks_probes import (CkksPrimitives, build_toy_context,  # noqa: E402
                                      cheb_eval64, cheb_ps_depth)

SLOTS = 64
ROTS = [1, -1, 2, 3, 7, -5, 8, 16, 24]


@pytest.fixture(scope="module")
def env():
    cc, keys = build_toy_context(ring_dimension=1 << 12, batch=SLOTS, depth=10, scale_bits=45,
                                 first_mod_bits=60, rotations=ROTS, seed=1234)
    cc.EvalConjugateKeyGen(keys.secretKey)
    return cc, keys


def enc(cc, keys, v, level=0):
    return cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(v), 1, level))


def dec(cc, keys, ct, n=SLOTS, complex_=False):
    pt = cc.Decrypt(ct, keys.secretKey)
    pt.SetLength(n)
    return np.asarray(pt.GetCKKSPackedValue() if complex_ else pt.GetRealPackedValue())


def vec(seed, n=SLOTS, lo=-1.0, hi=1.0):
    return np.random.default_rng(seed).uniform(lo, hi, n)


TOL = 2e-6


def test_context_shape(env):
    cc, _ = env
    assert cc.GetRingDimension() == 4096 and cc.GetCyclotomicOrder() == 8192
    assert cc.GetBatchSize() == SLOTS
    q, p = cc.GetModuli()
    assert len(q) == 11 and cc.GetScalingFactorReal(0) == float(q[-1])
    # FLEXIBLEAUTO chain: sf[l] = sf[l-1]^2 / q_{L-l}
    for lev in range(1, 5):
        assert cc.GetScalingFactorReal(lev) == pytest.approx(
            cc.GetScalingFactorReal(lev - 1) ** 2 / q[len(q) - lev], rel=1e-15)


def test_roundtrip_real_and_complex(env):
    cc, keys = env
    x = vec(1)
    np.testing.assert_allclose(dec(cc, keys, enc(cc, keys, x)), x, atol=TOL)
    z = vec(2) + 1j * vec(3)
    got = dec(cc, keys, enc(cc, keys, z), complex_=True)
    np.testing.assert_allclose(got, z, atol=TOL)
    short = dec(cc, keys, enc(cc, keys, x[:10]))
    np.testing.assert_allclose(short[:10], x[:10], atol=TOL)
    np.testing.assert_allclose(short[10:], 0, atol=TOL)


def test_arithmetic_and_metadata(env):
    cc, keys = env
    x, y, z = vec(4), vec(5), vec(6)
    cx, cy, cz = enc(cc, keys, x), enc(cc, keys, y), enc(cc, keys, z)
    pz = cc.MakeCKKSPackedPlaintext(list(z))
    cases = {
        "add": (cc.EvalAdd(cx, cy), x + y),
        "sub": (cc.EvalSub(cx, cy), x - y),
        "add_pt": (cc.EvalAdd(cx, pz), x + z),
        "sub_pt": (cc.EvalSub(cx, pz), x - z),
        "pt_sub": (cc.EvalSub(pz, cx), z - x),
        "add_dbl": (cc.EvalAdd(cx, 0.75), x + 0.75),
        "dbl_sub": (cc.EvalSub(0.75, cx), 0.75 - x),
        "neg": (cc.EvalNegate(cx), -x),
        "mul_dbl": (cc.EvalMult(cx, -2.5), -2.5 * x),
        "mul_pt": (cc.EvalMult(cx, pz), x * z),
        "mul": (cc.EvalMult(cx, cy), x * y),
        "square": (cc.EvalSquare(cx), x * x),
        "int": (cc.MultByInteger(cx, -3), -3 * x),
    }
    for name, (ct, want) in cases.items():
        np.testing.assert_allclose(dec(cc, keys, ct), want, atol=TOL, err_msg=name)
    m = cases["mul"][0]
    assert (m.GetLevel(), m.GetNoiseScaleDeg()) == (0, 2)
    r = cc.Rescale(m)
    assert (r.GetLevel(), r.GetNoiseScaleDeg()) == (1, 1)
    assert r.GetScalingFactor() == pytest.approx(cc.GetScalingFactorReal(1), rel=1e-12)
    # degree-2 input is rescaled before the next product
    m2 = cc.EvalMult(m, cz)
    assert (m2.GetLevel(), m2.GetNoiseScaleDeg()) == (1, 2)
    np.testing.assert_allclose(dec(cc, keys, m2), x * y * z, atol=TOL)


def test_level_and_degree_alignment(env):
    cc, keys = env
    x, y, z = vec(7), vec(8), vec(9)
    cx, cy, cz = enc(cc, keys, x), enc(cc, keys, y), enc(cc, keys, z)
    xy = cc.EvalMult(cx, cy)                      # level 0, degree 2
    checks = [
        (cc.EvalAdd(xy, cz), x * y + z),          # same level, degree 2 + 1
        (cc.EvalAdd(cz, xy), z + x * y),
        (cc.EvalSub(cc.Rescale(xy), cz), x * y - z),  # level 1 vs level 0
        (cc.EvalAdd(cz, cc.Rescale(cc.EvalMult(cc.Rescale(xy), cz))), z + x * y * z),
        (cc.EvalMult(cz, cc.Rescale(cc.EvalMult(cc.Rescale(xy), cz))), x * y * z * z),
    ]
    for i, (ct, want) in enumerate(checks):
        np.testing.assert_allclose(dec(cc, keys, ct), want, atol=TOL, err_msg=str(i))
    # a plaintext encoded at level 0 is re-encoded for a degree-2 ciphertext
    pz = cc.MakeCKKSPackedPlaintext(list(z))
    np.testing.assert_allclose(dec(cc, keys, cc.EvalAdd(xy, pz)), x * y + z, atol=TOL)
    # deep chain: x^8 by squaring, then + x at level 0
    p8 = cx
    for _ in range(3):
        p8 = cc.EvalSquare(p8)
    np.testing.assert_allclose(dec(cc, keys, cc.EvalAdd(p8, cx)), x ** 8 + x, atol=TOL)
    # SetLevel / LevelReduce drop limbs and keep the value
    c2 = cx.Clone()
    c2.SetLevel(3)
    assert c2.GetLevel() == 3 and c2.residues().shape[1] == len(cc.GetModuli()[0]) - 3
    lr = cc.LevelReduce(cx, None, 2)
    assert lr.GetLevel() == 2
    np.testing.assert_allclose(dec(cc, keys, c2), x, atol=TOL)


def test_align_to_level(env):
    """AlignToLevel: a shallower or degree-2 ciphertext reaches the target
    level on its standard scale with its value kept, and then meets a
    ciphertext made at that level as EvalAdd's own alignment would; a
    deeper target than the input is refused."""
    cc, keys = env
    x, y = vec(31), vec(32)
    cx = enc(cc, keys, x)
    cy = cc.Rescale(cc.EvalMult(enc(cc, keys, y), 1.0))       # level 1
    for src, want in ((cx, x), (cc.EvalMult(cx, cx), x * x)):
        out = cc.AlignToLevel(src, 4)
        assert out.GetLevel() == 4 and out.GetNoiseScaleDeg() == 1
        assert out.GetScalingFactor() == cc.GetScalingFactorReal(4)
        np.testing.assert_allclose(dec(cc, keys, out), want, atol=TOL)
    same = cc.AlignToLevel(cy, 1)
    assert same.GetLevel() == 1
    np.testing.assert_allclose(dec(cc, keys, same), y, atol=TOL)
    deep = cc.AlignToLevel(cx, 3)
    np.testing.assert_allclose(dec(cc, keys, cc.EvalAdd(deep, cy)), x + y, atol=TOL)
    with pytest.raises(ValueError):
        cc.AlignToLevel(deep, 2)


def test_in_place_forms(env):
    cc, keys = env
    x, y = vec(10), vec(11)
    c = enc(cc, keys, x)
    cc.EvalAddInPlace(c, enc(cc, keys, y))
    cc.EvalMultInPlace(c, 0.5)
    cc.EvalSubInPlace(c, 0.25)
    d = enc(cc, keys, y)
    cc.EvalMultMutableInPlace(c, d)
    cc.RescaleInPlace(c)
    cc.EvalSquareInPlace(c)
    want = ((0.5 * (x + y) - 0.25) * y) ** 2
    np.testing.assert_allclose(dec(cc, keys, c), want, atol=TOL)


def test_rotations(env):
    cc, keys = env
    x = vec(12)
    cx = enc(cc, keys, x)
    for k in ROTS:
        np.testing.assert_allclose(dec(cc, keys, cc.EvalRotate(cx, k)), np.roll(x, -k),
                                   atol=TOL, err_msg=str(k))
    with pytest.raises(KeyError):
        cc.EvalRotate(cx, 5)
    pre = cc.EvalFastRotationPrecompute(cx)
    fast = cc.EvalFastRotation(cx, ROTS, 2 * cc.GetRingDimension(), pre)
    for k, ct in zip(ROTS, fast):
        assert np.array_equal(ct.residues(), cc.EvalRotate(cx, k).residues())
    one = cc.EvalFastRotation(cx, 3, 2 * cc.GetRingDimension(), pre)
    assert np.array_equal(one.residues(), fast[ROTS.index(3)].residues())
    # rotation of a degree-2 ciphertext at a lower level
    m = cc.EvalMult(cx, cx)
    cc.EvalRotateInPlace(m, 2)
    np.testing.assert_allclose(dec(cc, keys, m), np.roll(x * x, -2), atol=TOL)


def test_conjugate(env):
    cc, keys = env
    z = vec(13) + 1j * vec(14)
    got = dec(cc, keys, cc.EvalConjugate(enc(cc, keys, z)), complex_=True)
    np.testing.assert_allclose(got, np.conj(z), atol=TOL)


@pytest.mark.parametrize("bstep,rows", [(8, 64), (4, 10), (1, 3), (16, 16)])
def test_linear_transform_matvec(env, bstep, rows):
    """y = M x over 64 slots with `rows` diagonals:
    diag_k[i] = M[i, (i + k) % n], pre-rotated by the giant step."""
    cc, keys = env
    n = SLOTS
    rng = np.random.default_rng(bstep * 100 + rows)
    M = np.zeros((n, n))
    for k in range(rows):
        for i in range(n):
            M[i, (i + k) % n] = rng.uniform(-1, 1) / rows
    x = vec(15)
    pts = []
    for k in range(rows):
        diag = np.array([M[i, (i + k) % n] for i in range(n)])
        g = (k // bstep) * bstep
        pts.append(cc.MakeCKKSPackedPlaintext(list(np.roll(diag, g))))
    needed = sorted({b for b in range(1, min(bstep, rows))} |
                    ({bstep} if rows > bstep else set()))
    cc.EvalRotateKeyGen(keys.secretKey, needed)
    ct = enc(cc, keys, x)
    cc.LinearTransformInPlace(ct, rows, bstep, pts)
    assert ct.GetNoiseScaleDeg() == 2
    np.testing.assert_allclose(dec(cc, keys, ct), M @ x, atol=1e-5)


def test_probe_circuits_on_gpu(env):
    cc, keys = env
    he = CkksPrimitives(cc, keys, batch=SLOTS)
    x = np.linspace(-0.9, 0.9, SLOTS)
    for degree in (7, 15):
        coeffs = list(np.random.default_rng(degree).normal(size=degree + 1) / 4)
        assert cheb_ps_depth(degree) <= 10
        out = he.eval_chebyshev(he.encrypt(x), coeffs)
        np.testing.assert_allclose(he.decrypt(out), cheb_eval64(coeffs, x), atol=1e-4)
    v = np.linspace(0.5, 2.0, SLOTS)
    y = he.newton_refine(he.encrypt(1.0 / np.sqrt(v) * 1.02), he.encrypt(-0.5 * v), 2)
    np.testing.assert_allclose(he.decrypt(y), 1.0 / np.sqrt(v), atol=1e-4)
    np.testing.assert_allclose(he.decrypt(he.affine_ct(he.encrypt(x), 2.0, 0.5)), 2 * x + 0.5,
                               atol=TOL)
    np.testing.assert_allclose(he.decrypt(he.const_ct(-1.25)), -1.25, atol=TOL)


def test_errors(env):
    cc, keys = env
    with pytest.raises(ValueError):
        cc.MakeCKKSPackedPlaintext([0.0] * (SLOTS + 1))
    with pytest.raises(TypeError):
        cc.EvalAdd(1.0, 2.0)
    p = ckks.CCParamsCKKSRNS()
    p.SetRingDim(1 << 12)
    p.SetMultiplicativeDepth(2)
    p.SetSecurityLevel(ckks.SecurityLevel.HEStd_NotSet)
    c2 = ckks.GenCryptoContext(p, seed=5)
    k2 = c2.KeyGen()
    ct = c2.Encrypt(k2.publicKey, c2.MakeCKKSPackedPlaintext([1.0]))
    with pytest.raises(KeyError):  # no relinearization key yet
        c2.EvalMult(ct, ct)


def test_batched_plaintexts_equal_single(env):
    """MakeCKKSPackedPlaintexts (one batched encode) gives the residues,
    level, degree and scale of MakeCKKSPackedPlaintext per vector, degree 2
    included, for rows of unequal length."""
    cc, _ = env
    rows = [vec(40 + i, n) for i, n in enumerate((SLOTS, 5, SLOTS, 33))]
    for level, deg in ((0, 1), (3, 1), (2, 2)):
        many = cc.MakeCKKSPackedPlaintexts(rows, deg, level, slots=SLOTS)
        for r, p in zip(rows, many):
            one = cc.MakeCKKSPackedPlaintext(list(r), deg, level, None, SLOTS)
            assert np.array_equal(p.poly.numpy(), one.poly.numpy())
            assert (p.level, p.deg, p.scale, p.slots) == (one.level, one.deg, one.scale, one.slots)
    assert cc.MakeCKKSPackedPlaintexts([], 1, 0) == []


def test_mult_many_equals_mult(env):
    """EvalMultMany gives the ciphertexts EvalMult gives, residue for
    residue: products at two levels (two batched relinearizations), a
    square (one operand twice), operands of different levels and degrees
    (aligned as EvalMult aligns them) and a plaintext product; RescaleMany
    gives the ciphertexts Rescale gives."""
    cc, keys = env
    a, b = enc(cc, keys, vec(1)), enc(cc, keys, vec(2))
    c = enc(cc, keys, vec(3), level=2)
    d = cc.EvalMult(enc(cc, keys, vec(4)), enc(cc, keys, vec(5)))   # degree 2
    pt = cc.MakeCKKSPackedPlaintext(list(vec(6)))
    pairs = [(a, b), (a, a), (c, c), (b, c), (d, a), (c, enc(cc, keys, vec(7), level=2)),
             (a, pt), (b, 0.5)]
    got = cc.EvalMultMany(pairs)
    for (x, y), g in zip(pairs, got):
        want = cc.EvalMult(x, y)
        assert (g.GetLevel(), g.GetNoiseScaleDeg()) == (want.GetLevel(), want.GetNoiseScaleDeg())
        assert g.GetScalingFactor() == want.GetScalingFactor()
        assert np.array_equal(g.poly.numpy(), want.poly.numpy())
    deep = [cc.EvalMult(a, b), cc.EvalMult(c, c), d, cc.EvalMult(b, c)]
    for g, x in zip(cc.RescaleMany(deep + [a]), deep + [a]):
        want = cc.Rescale(x)
        assert (g.GetLevel(), g.GetNoiseScaleDeg()) == (want.GetLevel(), want.GetNoiseScaleDeg())
        assert g.GetScalingFactor() == want.GetScalingFactor()
        assert np.array_equal(g.poly.numpy(), want.poly.numpy())
