"""CKKS bootstrapping end to end on the GPU (EvalBootstrapSetup /
EvalBootstrapKeyGen / EvalBootstrap as native/fideslib_stage0/src/
packed_fideslib.cpp:235-270 drives them), checked by decryption against the
input slots.  Tolerances: one pass keeps about 2^-18 absolute on values in
[-1, 1] at these toy parameters (N = 2^12, uniform-ternary secret, K = 128,
59-bit scale over a 60-bit q0, as the reference's bootstrapped chains use);
the test allows 2^-16.  Two passes allow 2^-24."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd.ckks_probes import build_toy_context  # noqa: E402

LOG_N = 12
SLOTS = 1 << (LOG_N - 1)
ONE_PASS_TOL = 2.0 ** -16
TWO_PASS_TOL = 2.0 ** -24


@pytest.fixture(scope="module")
def env():
    cc, keys = build_toy_context(ring_dimension=1 << LOG_N, batch=SLOTS, depth=44,
                                 scale_bits=59, first_mod_bits=60, seed=99)
    cc.EvalBootstrapSetup([3, 3], [0, 0], SLOTS)
    cc.EvalBootstrapKeyGen(keys.secretKey, SLOTS)
    return cc, keys


def enc_at(cc, keys, v, level):
    ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(v)))
    ct.SetLevel(level)
    return ct


def dec(cc, keys, ct, complex_=False):
    pt = cc.Decrypt(ct, keys.secretKey)
    pt.SetLength(SLOTS)
    return np.asarray(pt.GetCKKSPackedValue() if complex_ else pt.GetRealPackedValue())


def test_bootstrap_refreshes_real_slots(env):
    cc, keys = env
    L = len(cc.GetModuli()[0])
    x = np.random.default_rng(1).uniform(-1, 1, SLOTS)
    ct = enc_at(cc, keys, x, L - 2)
    out = cc.EvalBootstrap(ct)
    assert out.GetLevel() == cc.GetBootstrapDepth() < L - 2
    err = np.max(np.abs(dec(cc, keys, out) - x))
    print(f"one-pass bootstrap error 2^{np.log2(err):.1f}", flush=True)
    assert err < ONE_PASS_TOL
    # the refreshed ciphertext multiplies on
    sq = cc.EvalMult(out, out)
    assert np.max(np.abs(dec(cc, keys, sq) - x * x)) < 4 * ONE_PASS_TOL


def test_bootstrap_complex_slots_and_lower_input_levels(env):
    cc, keys = env
    L = len(cc.GetModuli()[0])
    rng = np.random.default_rng(2)
    z = rng.uniform(-1, 1, SLOTS) + 1j * rng.uniform(-1, 1, SLOTS)
    for level in (L - 2, L - 5):
        ct = enc_at(cc, keys, z, level)
        out = cc.EvalBootstrap(ct)
        err = np.max(np.abs(dec(cc, keys, out, complex_=True) - z))
        assert err < ONE_PASS_TOL, (level, err)


def test_bootstrap_with_a_coefficient_bound(env):
    """A public coefficient bound b (random slots: b ~ 2^-5 at 2048 slots)
    lets the ordinary order scale the message down ~3 bits less, so the
    noise, which dominates one pass here, shrinks by about as much; the
    worst case (a constant vector, b = 1) keeps its precision."""
    from fhemamba_amd.bootstrap import coefficient_bound
    cc, keys = env
    L = len(cc.GetModuli()[0])
    boot = cc._bootstrapper()
    rng = np.random.default_rng(11)
    x = rng.uniform(-1, 1, SLOTS)
    b = coefficient_bound(x)
    in_scale, q0 = cc.GetScalingFactorReal(L - 1), float(cc.GetModuli()[0][0])
    c1 = boot.correction_bits(in_scale, q0, cc.GetScalingFactorReal(0))
    cb = boot.correction_bits(in_scale, q0, cc.GetScalingFactorReal(0), b)
    assert c1 - cb >= 2, (c1, cb, b)
    ct = enc_at(cc, keys, x, L - 2)
    err1 = np.max(np.abs(dec(cc, keys, cc.EvalBootstrap(ct)) - x))
    errb = np.max(np.abs(dec(cc, keys, cc.EvalBootstrap(ct, coeff_bound=b)) - x))
    print(f"one pass: c {c1} -> {cb} (b = 2^{np.log2(b):.1f}): "
          f"2^{np.log2(err1):.1f} -> 2^{np.log2(errb):.1f}", flush=True)
    assert errb < err1 / 2
    const = np.full(SLOTS, 0.75)
    assert coefficient_bound(const) == 1.0
    out = cc.EvalBootstrap(enc_at(cc, keys, const, L - 2), coeff_bound=1.0)
    assert np.max(np.abs(dec(cc, keys, out) - const)) < ONE_PASS_TOL
    with pytest.raises(ValueError):
        cc.EvalBootstrap(ct, coeff_bound=0.0)


def test_bootstrap_after_a_multiplication(env):
    """A degree-2 input (unrescaled product) is rescaled first."""
    cc, keys = env
    L = len(cc.GetModuli()[0])
    x = np.random.default_rng(3).uniform(-1, 1, SLOTS)
    ct = enc_at(cc, keys, x, L - 4)
    prod = cc.EvalMult(ct, ct)
    assert prod.GetNoiseScaleDeg() == 2
    out = cc.EvalBootstrap(prod)
    assert np.max(np.abs(dec(cc, keys, out) - x * x)) < ONE_PASS_TOL


def test_two_pass_bootstrap(env):
    cc, keys = env
    L = len(cc.GetModuli()[0])
    x = np.random.default_rng(4).uniform(-1, 1, SLOTS)
    ct = enc_at(cc, keys, x, L - 2)
    out = cc.EvalBootstrap(ct, 2, 15)
    err = np.max(np.abs(dec(cc, keys, out) - x))
    print(f"two-pass bootstrap error 2^{np.log2(err):.1f}", flush=True)
    assert err < TWO_PASS_TOL


def test_bootstrap_input_checks(env):
    cc, keys = env
    x = np.zeros(SLOTS)
    with pytest.raises(ValueError):
        cc.EvalBootstrap(enc_at(cc, keys, x, len(cc.GetModuli()[0]) - 1))
    with pytest.raises(ValueError):
        cc.EvalBootstrapSetup([3, 3], [0, 0], 3)


@pytest.mark.parametrize("slots", [8, 256])
def test_sparse_packing_bootstrap(slots):
    """Sparse packing (slots < N/2), as the reference's packed programs use
    it (batch size = program slots on a larger ring)."""
    cc, keys = build_toy_context(ring_dimension=1 << LOG_N, batch=slots, depth=44,
                                 scale_bits=59, first_mod_bits=60, seed=7 + slots)
    cc.EvalBootstrapSetup([2, 2], [0, 0], slots)
    cc.EvalBootstrapKeyGen(keys.secretKey, slots)
    L = len(cc.GetModuli()[0])
    x = np.random.default_rng(slots).uniform(-1, 1, slots)
    ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(x)))
    ct.SetLevel(L - 2)
    for passes, tol in ((1, ONE_PASS_TOL), (2, TWO_PASS_TOL)):
        out = cc.EvalBootstrap(ct, passes, 15)
        pt = cc.Decrypt(out, keys.secretKey)
        pt.SetLength(slots)
        err = np.max(np.abs(np.asarray(pt.GetRealPackedValue()) - x))
        print(f"sparse {slots} slots, {passes} pass(es): error 2^{np.log2(err):.1f}", flush=True)
        assert err < tol


# ------------------------------------------------------- sparse-ternary secret
def test_sparse_secret_matches_oracle():
    """The library's seeded sparse-ternary sampler equals the oracle's."""
    import oracle as O
    q, p = O.gen_moduli(LOG_N, 6, 45, 60, 3)
    ctx, orc = F.Context(LOG_N, q, p, 3, sampling="seeded"), O.Ctx(LOG_N, q, p, 3)
    for seed, h in ((3, 192), (4, 64), (5, 1 << LOG_N)):
        s = ctx.keygen_secret_sparse(seed, h)
        assert int(np.count_nonzero(s)) == h
        assert np.array_equal(s, orc.secret_sparse(seed, h))
    with pytest.raises(ValueError):
        ctx.keygen_secret_sparse(1, (1 << LOG_N) + 1)


def test_sparse_secret_bootstrap():
    """A SPARSE_TERNARY context (h = 192): K = 64, four double angles, a
    degree-59 cosine, so the bootstrap consumes fewer levels than the
    uniform-ternary one and keeps the one-pass tolerance."""
    from fhemamba_amd import ckks
    cc, keys = build_toy_context(ring_dimension=1 << LOG_N, batch=SLOTS, depth=44,
                                 scale_bits=59, first_mod_bits=60, seed=98,
                                 secret_dist="SPARSE_TERNARY")
    assert int(np.count_nonzero(keys.secretKey.s)) == ckks.SPARSE_HAMMING_WEIGHT
    cc.EvalBootstrapSetup([3, 3], [0, 0], SLOTS)
    cc.EvalBootstrapKeyGen(keys.secretKey, SLOTS)
    boot = cc._bootstrapper()
    assert (boot.cfg.sine.K, boot.cfg.sine.r) == (64, 4)
    L = len(cc.GetModuli()[0])
    x = np.random.default_rng(5).uniform(-1, 1, SLOTS)
    ct = enc_at(cc, keys, x, L - 2)
    out = cc.EvalBootstrap(ct)
    assert out.GetLevel() == cc.GetBootstrapDepth() < L - 2
    err = np.max(np.abs(dec(cc, keys, out) - x))
    print(f"sparse-secret one-pass bootstrap error 2^{np.log2(err):.1f}", flush=True)
    assert err < ONE_PASS_TOL
    out2 = cc.EvalBootstrap(ct, 2)
    err2 = np.max(np.abs(dec(cc, keys, out2) - x))
    print(f"sparse-secret two-pass bootstrap error 2^{np.log2(err2):.1f}", flush=True)
    assert err2 < TWO_PASS_TOL


@pytest.mark.parametrize("real", [False, True])
def test_s2c_first_bootstrap(real):
    """S2C-first ordering (SlotToCoeff on the input, then ModRaise,
    CoeffToSlot, EvalMod): the output keeps the SlotToCoeff levels, the
    input must sit that many levels lower, and the refreshed slots meet
    the one- and two-pass tolerances (complex slots, or real slots with
    one EvalMod).  With real_slots the imaginary part of the input is
    dropped and the output projected onto its real part: its imaginary
    parts hold only the projection's key-switch noise (below 2^-30)."""
    cc, keys = build_toy_context(ring_dimension=1 << LOG_N, batch=SLOTS, depth=44,
                                 scale_bits=59, first_mod_bits=60, seed=11)
    cc.EvalBootstrapSetup([3, 3], [0, 0], SLOTS, s2c_first=True, real_slots=real)
    cc.EvalBootstrapKeyGen(keys.secretKey, SLOTS)
    L = len(cc.GetModuli()[0])
    assert cc.GetBootstrapInputCeiling() == L - 2 - 3
    rng = np.random.default_rng(12)
    z = rng.uniform(-1, 1, SLOTS) + (0 if real else 1j * rng.uniform(-1, 1, SLOTS))
    ct = enc_at(cc, keys, z, L - 5)
    for passes, tol in ((1, ONE_PASS_TOL), (2, TWO_PASS_TOL)):
        out = cc.EvalBootstrap(ct, passes, 15)
        assert out.GetLevel() == cc.GetBootstrapDepth()
        got = dec(cc, keys, out, complex_=True)
        err = np.max(np.abs((got.real if real else got) - z))
        print(f"S2C-first ({'real' if real else 'complex'}) {passes} pass(es): "
              f"error 2^{np.log2(err):.1f}, imaginary 2^{np.log2(np.max(np.abs(got.imag))):.1f}",
              flush=True)
        assert err < tol
        if real:
            assert np.max(np.abs(got.imag)) < 2.0 ** -30
    with pytest.raises(ValueError, match="level"):
        cc.EvalBootstrap(enc_at(cc, keys, z, L - 4))
    with pytest.raises(ValueError, match="full packing"):
        cc.EvalBootstrapSetup([3, 3], [0, 0], SLOTS // 2, s2c_first=True)


@pytest.mark.parametrize("real", [False, True])
def test_bootstrap_many_equals_single(real):
    """EvalBootstrapMany over three ciphertexts in step (S2C-first: shared
    linear-transform, conjugation, rescale and EvalMod launches) gives
    the ciphertexts of one EvalBootstrap each, word for word, for one and
    two passes; the ordinary order refreshes them in turn."""
    cc, keys = build_toy_context(ring_dimension=1 << LOG_N, batch=SLOTS, depth=44,
                                 scale_bits=59, first_mod_bits=60, seed=13)
    cc.EvalBootstrapSetup([3, 3], [0, 0], SLOTS, s2c_first=True, real_slots=real)
    cc.EvalBootstrapKeyGen(keys.secretKey, SLOTS)
    L = len(cc.GetModuli()[0])
    rng = np.random.default_rng(14)
    cts = []
    for i in range(3):
        z = rng.uniform(-1, 1, SLOTS) + (0 if real else 1j * rng.uniform(-1, 1, SLOTS))
        cts.append(enc_at(cc, keys, z, L - 5 - (i == 2)))     # one a level deeper
    for passes in (1, 2):
        singles = [cc.EvalBootstrap(ct, passes, 15, scale=2.0) for ct in cts]
        many = cc.EvalBootstrapMany(cts, passes, 15, scale=2.0)
        for got, want in zip(many, singles):
            assert got.GetLevel() == want.GetLevel()
            assert got.GetScalingFactor() == want.GetScalingFactor()
            assert np.array_equal(got.residues(), want.residues())


@pytest.mark.parametrize("s2c_first", [False, True])
def test_bootstrap_at_ring_2_16(s2c_first):
    """Full packing at N = 2^16 (32768 slots, the decoder's ring) with the
    uniform-ternary secret (K = 512, degree 59, 7 double angles), both
    orderings, level budget (4, 4): one pass within 2^-11, two passes
    within 2^-22 (measured about 2^-12.9 and 2^-25)."""
    n = 1 << 16
    cc, keys = build_toy_context(ring_dimension=n, batch=n // 2, depth=44, scale_bits=59,
                                 first_mod_bits=60, seed=16)
    cc.EvalBootstrapSetup([4, 4], [0, 0], n // 2, s2c_first=s2c_first, real_slots=s2c_first)
    cc.EvalBootstrapKeyGen(keys.secretKey, n // 2)
    x = np.random.default_rng(17).uniform(-1, 1, n // 2)
    ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(x)))
    ct.SetLevel(cc.GetBootstrapInputCeiling())
    for passes, tol in ((1, 2.0 ** -11), (2, 2.0 ** -22)):
        out = cc.EvalBootstrap(ct, passes, 12)
        pt = cc.Decrypt(out, keys.secretKey)
        pt.SetLength(n // 2)
        err = np.max(np.abs(np.asarray(pt.GetRealPackedValue()) - x))
        print(f"N=2^16 {'S2C-first' if s2c_first else 'ordinary'} {passes} pass(es): "
              f"level {out.GetLevel()}, error 2^{np.log2(err):.1f}", flush=True)
        assert out.GetLevel() == cc.GetBootstrapDepth()
        assert err < tol


@pytest.mark.parametrize("order", ["s2c-first", "ordinary"])
def test_bootstrap_command_line(order, capsys):
    """python -m fhemamba_amd.bootstrap at N=2^12: one JSON line with the
    timing, launch count and a refreshed value within 2^-10."""
    import json

    from fhemamba_amd import bootstrap as B
    assert B.main(["--log-n", "12", "--order", order, "--repeat", "1", "--warmup", "0"]) == 0
    rep = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    print(rep, flush=True)
    assert rep["ring_dimension"] == 4096 and rep["order"] == order
    assert rep["launches_per_call"] > 0 and rep["ms_per_call"] > 0
    assert rep["max_abs_err"] < 2.0**-10
