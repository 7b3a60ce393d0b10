"""Hybrid key switching, rotations (single and hoisted), conjugation and
relinearisation on the GPU, bit-exact against the CPU oracle."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd._lib import FheError  # noqa: E402

# (log_n, depth, scale bits, first bits, dnum): config-1-like toy chain and
# a chain with a partial last digit.
PARAMS = [(13, 7, 50, 60, 2), (12, 6, 45, 60, 3), (11, 4, 40, 60, 1)]


@pytest.fixture(scope="module", params=PARAMS)
def setup(request):
    log_n, depth, sb, fb, dnum = request.param
    q, p = O.gen_moduli(log_n, depth, sb, fb, dnum)
    ctx, orc = F.Context(log_n, q, p, dnum, sampling="seeded"), O.Ctx(log_n, q, p, dnum)
    s = orc.secret(11)
    return ctx, orc, s


def test_secret_matches_oracle(setup):
    ctx, orc, s = setup
    assert np.array_equal(ctx.keygen_secret(11), s)


def test_keyswitch_matches_oracle(setup):
    ctx, orc, s = setup
    rng = np.random.default_rng(1)
    key = orc.relin_key(s, 3)
    dkey = ctx.load_key(key)
    for nq in sorted({ctx.L, max(1, ctx.L - 1), ctx.alpha + 1, 1}):
        a = residues(rng, ctx.q[:nq], (1,), ctx.n)
        got = ctx.keyswitch(ctx.upload(a), dkey).numpy()
        assert np.array_equal(got, orc.keyswitch(a[0], key)), nq


def test_modup_moddown_pieces_through_keyswitch_in_place(setup):
    ctx, orc, s = setup
    rng = np.random.default_rng(2)
    key = orc.relin_key(s, 4)
    a = residues(rng, ctx.q, (1,), ctx.n)
    da = ctx.upload(a)
    ctx.keyswitch(da, ctx.load_key(key), out=da)
    assert np.array_equal(da.numpy(), orc.keyswitch(a[0], key))


@pytest.mark.parametrize("step", [1, -1, 7, 2, -16])
def test_rotate_matches_oracle(setup, step):
    ctx, orc, s = setup
    g = O.galois_elt(step, ctx.n)
    assert g == F.galois_element(step, ctx.n)
    key = orc.galois_key(s, g, 20 + step)
    rng = np.random.default_rng(30 + step)
    for nq in (ctx.L, max(1, ctx.L - 2)):
        ct = residues(rng, ctx.q[:nq], (2,), ctx.n)
        got = ctx.rotate(ctx.upload(ct), ctx.load_key(key), g).numpy()
        assert np.array_equal(got, orc.rotate(ct, key, g)), nq


def test_conjugate_matches_oracle(setup):
    ctx, orc, s = setup
    g = F.conjugation_element(ctx.n)
    key = orc.galois_key(s, g, 9)
    ct = residues(np.random.default_rng(9), ctx.q, (2,), ctx.n)
    got = ctx.rotate(ctx.upload(ct), ctx.load_key(key), g).numpy()
    assert np.array_equal(got, orc.rotate(ct, key, g))


def test_hoisted_rotations_equal_single_rotations(setup):
    ctx, orc, s = setup
    steps = [1, -1, 2, -2, 4, 8]
    gal = [O.galois_elt(r, ctx.n) for r in steps]
    keys = [orc.galois_key(s, g, 40 + i) for i, g in enumerate(gal)]
    ct = residues(np.random.default_rng(12), ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    digits = ctx.rotation_precompute(dct)
    assert digits.shape == (orc.num_digits(ctx.L), ctx.L + ctx.K)
    assert np.array_equal(digits.numpy(), orc.modup(ct[1]))
    outs = ctx.rotate_hoisted(dct, digits, [ctx.load_key(k) for k in keys], gal)
    for out, key, g in zip(outs, keys, gal):
        assert np.array_equal(out.numpy(), orc.rotate(ct, key, g))


def test_hoisted_pipelined_set_matches_oracle(setup):
    """15 rotations (more than one pipeline chunk, with a partial last
    chunk; repeated and conjugation elements included): every output equals
    the oracle's single rotation, and the input and digits are untouched."""
    ctx, orc, s = setup
    steps = [1, -1, 2, -2, 3, 5, 7, -7, 16, 1, -3, 9, 11, -16, 6]
    gal = [O.galois_elt(r, ctx.n) for r in steps]
    gal[7] = 2 * ctx.n - 1
    keys = {g: orc.galois_key(s, g, 60 + i) for i, g in enumerate(dict.fromkeys(gal))}
    dkeys = {g: ctx.load_key(k) for g, k in keys.items()}
    ct = residues(np.random.default_rng(15), ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    digits = ctx.rotation_precompute(dct)
    before = digits.numpy()
    outs = ctx.rotate_hoisted(dct, digits, [dkeys[g] for g in gal], gal)
    for out, g in zip(outs, gal):
        assert np.array_equal(out.numpy(), orc.rotate(ct, keys[g], g))
    assert np.array_equal(dct.numpy(), ct)
    assert np.array_equal(digits.numpy(), before)
    # a second call reusing the outputs gives the same words
    again = ctx.rotate_hoisted(dct, digits, [dkeys[g] for g in gal], gal, outs=outs)
    for out, g in zip(again, gal):
        assert np.array_equal(out.numpy(), orc.rotate(ct, keys[g], g))


def test_rotate_many_matches_single_rotations(setup):
    """Five different ciphertexts (one level down), mixed keys, one output
    written over its own input and one over another's: each equals the
    oracle's rotation of the original input."""
    ctx, orc, s = setup
    rng = np.random.default_rng(16)
    nq = ctx.L - 1
    steps = [1, -1, 3, 1, 2 * ctx.n - 1]
    gal = [O.galois_elt(r, ctx.n) for r in steps[:4]] + [steps[4]]
    keys = {g: orc.galois_key(s, g, 80 + i) for i, g in enumerate(dict.fromkeys(gal))}
    dkeys = {g: ctx.load_key(k) for g, k in keys.items()}
    cts = [residues(rng, ctx.q[:nq], (2,), ctx.n) for _ in steps]
    dcts = [ctx.upload(c) for c in cts]
    outs = [ctx.poly(2, nq) for _ in steps]
    outs[1] = dcts[1]          # in place
    outs[3] = dcts[0]          # over another rotation's input
    got = ctx.rotate_many(dcts, [dkeys[g] for g in gal], gal, outs=outs)
    for r, (g, c) in enumerate(zip(gal, cts)):
        assert np.array_equal(got[r].numpy(), orc.rotate(c, keys[g], g)), r


def test_relinearize_matches_oracle(setup):
    ctx, orc, s = setup
    key = orc.relin_key(s, 5)
    rng = np.random.default_rng(13)
    a = residues(rng, ctx.q, (2,), ctx.n)
    b = residues(rng, ctx.q, (2,), ctx.n)
    t = orc.tensor(a, b)
    got = ctx.relinearize(ctx.upload(t), ctx.load_key(key)).numpy()
    assert np.array_equal(got, orc.relinearize(t, key))


def test_relinearize_many_matches_oracle(setup):
    """Several tensors of one level in one batched relinearization
    (fhe_relinearize_many) equal the oracle's relinearization of each, at
    the top level and one limb lower; an output that is one of the tensors
    is refused, and so are tensors of two levels in one call."""
    ctx, orc, s = setup
    key = orc.relin_key(s, 5)
    dkey = ctx.load_key(key)
    rng = np.random.default_rng(19)
    for nl in (ctx.L, ctx.L - 1):
        q = ctx.q[:nl]
        ts = [orc.tensor(residues(rng, q, (2,), ctx.n), residues(rng, q, (2,), ctx.n))
              for _ in range(5)]
        got = ctx.relinearize_many([ctx.upload(t) for t in ts], dkey)
        for r, t in enumerate(ts):
            assert np.array_equal(got[r].numpy(), orc.relinearize(t, key)), (nl, r)
    a = ctx.upload(ts[0])
    with pytest.raises(FheError):
        ctx.relinearize_many([a, ctx.upload(ts[1])], dkey, outs=[a, ctx.poly(2, ctx.L - 1)])
    with pytest.raises(FheError):
        big = orc.tensor(residues(rng, ctx.q, (2,), ctx.n), residues(rng, ctx.q, (2,), ctx.n))
        ctx.relinearize_many([a, ctx.upload(big)], dkey)


def test_rotate_and_relinearize_in_place(setup):
    """An output that aliases the input (rotate, relinearize of a 3-poly
    tensor into itself) takes fresh storage and holds the oracle's result;
    the old storage goes back to the pool and later results stay exact."""
    ctx, orc, s = setup
    rng = np.random.default_rng(41)
    g = O.galois_elt(3, ctx.n)
    gkey = orc.galois_key(s, g, 42)
    ct = residues(rng, ctx.q, (2,), ctx.n)
    d = ctx.upload(ct)
    before = d.data_ptr()
    ctx.rotate(d, ctx.load_key(gkey), g, out=d)
    assert np.array_equal(d.numpy(), orc.rotate(ct, gkey, g))
    assert d.data_ptr() != before
    t = residues(rng, ctx.q, (3,), ctx.n)
    rkey = orc.relin_key(s, 43)
    dt = ctx.upload(t)
    ctx.relinearize(dt, ctx.load_key(rkey), out=dt)
    assert dt.shape == (2, ctx.L)
    assert np.array_equal(dt.numpy(), orc.relinearize(t, rkey))
    # the freed storage is reused by later allocations without corrupting them
    again = ctx.rotate(ctx.upload(ct), ctx.load_key(gkey), g)
    assert np.array_equal(again.numpy(), orc.rotate(ct, gkey, g))


def test_gpu_keygen_matches_oracle_keys(setup):
    """GPU-generated keys equal the oracle's: their key switches agree
    word for word (keys are stored in Montgomery form on the device)."""
    ctx, orc, s = setup
    rng = np.random.default_rng(14)
    a = residues(rng, ctx.q, (1,), ctx.n)
    da = ctx.upload(a)
    rk = ctx.keygen_relin(s, 77)
    assert np.array_equal(ctx.keyswitch(da, rk).numpy(), orc.keyswitch(a[0], orc.relin_key(s, 77)))
    g = O.galois_elt(3, ctx.n)
    gk = ctx.keygen_galois(s, g, 78)
    ct = residues(rng, ctx.q, (2,), ctx.n)
    assert np.array_equal(ctx.rotate(ctx.upload(ct), gk, g).numpy(),
                          orc.rotate(ct, orc.galois_key(s, g, 78), g))
    pk = ctx.keygen_public(s, 79)
    assert np.array_equal(pk.numpy(), orc.public_key(s, 79))


def test_rotation_decrypts_to_rolled_slots(setup):
    ctx, orc, s = setup
    slots = ctx.n // 2
    scale = float(ctx.q[-1])
    x = np.random.default_rng(15).uniform(-1, 1, slots)
    pk = ctx.keygen_public(s, 5)
    ct = ctx.encrypt(pk, ctx.encode(x, slots, scale, ctx.L), 6)
    for step in (1, -5):
        g = F.galois_element(step, ctx.n)
        out = ctx.rotate(ct, ctx.keygen_galois(s, g, 7), g)
        got = ctx.decode(ctx.decrypt(out, s), slots, scale).real
        assert np.abs(got - np.roll(x, -step)).max() < 1e-4
