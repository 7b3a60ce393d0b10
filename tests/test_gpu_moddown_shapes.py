"""Key switching and rescaling at every ring dimension of the fused ModUp /
ModDown / rescale paths
(2^13 .. 2^17: column lengths 128 / 256 / 512 rows, blocked row groups of
32 / 16 / 8) and at the rotation benchmark's shape (N=2^16, 24 limbs,
8 special primes, dnum 3), bit-exact against the oracle."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd._lib import FheError  # noqa: E402

# (log_n, depth, scale bits, first bits, dnum); N=2^13 is covered by
# test_gpu_keyswitch.py.
SHAPES = [(14, 3, 50, 60, 2), (15, 3, 50, 60, 2), (16, 3, 50, 60, 3), (17, 2, 50, 60, 1)]


@pytest.fixture(scope="module", params=SHAPES, ids=lambda p: f"logn{p[0]}")
def setup(request):
    log_n, depth, sb, fb, dnum = request.param
    q, p = O.gen_moduli(log_n, depth, sb, fb, dnum)
    ctx, orc = F.Context(log_n, q, p, dnum, sampling="seeded"), O.Ctx(log_n, q, p, dnum)
    return ctx, orc, orc.secret(21)


def test_keyswitch_every_level(setup):
    ctx, orc, s = setup
    rng = np.random.default_rng(3)
    key = orc.relin_key(s, 6)
    dkey = ctx.load_key(key)
    for nq in range(1, ctx.L + 1):
        a = residues(rng, ctx.q[:nq], (1,), ctx.n)
        got = ctx.keyswitch(ctx.upload(a), dkey).numpy()
        assert np.array_equal(got, orc.keyswitch(a[0], key)), nq


def test_rescale_shapes(setup):
    """Rescale (four-launch form at these ring dimensions) of 1 and 2 polys
    at every level, against the oracle."""
    ctx, orc, s = setup
    rng = np.random.default_rng(11)
    for npoly in (1, 2):
        for nq in range(2, ctx.L + 1):
            a = residues(rng, ctx.q[:nq], (npoly,), ctx.n)
            assert np.array_equal(ctx.rescale(ctx.upload(a)).numpy(), orc.rescale(a)), nq


def test_rescale_many(setup):
    """Rescale of 19 inputs of one shape in shared launches (16 per launch
    set, then 3) equals the oracle's rescale of each, for 2-poly and 1-poly
    inputs; outputs aliasing an input and inputs of two shapes are refused."""
    ctx, orc, s = setup
    rng = np.random.default_rng(12)
    for npoly, nq in ((2, ctx.L), (1, 3)):
        xs = [residues(rng, ctx.q[:nq], (npoly,), ctx.n) for _ in range(19)]
        got = ctx.rescale_many([ctx.upload(x) for x in xs])
        for r, x in enumerate(xs):
            assert np.array_equal(got[r].numpy(), orc.rescale(x)), (npoly, nq, r)
    a = ctx.upload(residues(rng, ctx.q[:2], (2,), ctx.n))
    b = ctx.upload(residues(rng, ctx.q[:3], (2,), ctx.n))
    with pytest.raises(FheError):
        ctx.rescale_many([a, b])
    with pytest.raises(FheError):
        ctx.rescale_many([a], outs=[a])


def test_hoisted_rotations(setup):
    ctx, orc, s = setup
    steps = [1, -3, 64]
    gal = [O.galois_elt(r, ctx.n) for r in steps] + [2 * ctx.n - 1]
    keys = [orc.galois_key(s, g, 90 + i) for i, g in enumerate(gal)]
    ct = residues(np.random.default_rng(4), ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    digits = ctx.rotation_precompute(dct)
    outs = ctx.rotate_hoisted(dct, digits, [ctx.load_key(k) for k in keys], gal)
    for out, key, g in zip(outs, keys, gal):
        assert np.array_equal(out.numpy(), orc.rotate(ct, key, g)), g


def test_benchmark_shape_rotations():
    """Eight hoisted rotations (16 polys x 256 columns: the 4-wave middle
    kernel) and one single rotation one level down (the 8-wave one) at the
    benchmark's parameters."""
    q, p = O.gen_moduli(16, 23, 59, 60, 3)
    ctx, orc = F.Context(16, q, p, 3, sampling="seeded"), O.Ctx(16, q, p, 3)
    assert (ctx.L, ctx.K) == (24, 8)
    s = orc.secret(5)
    gal = [O.galois_elt(r, ctx.n) for r in (1, -4096, 5, 2 * ctx.n - 1)]
    gal = gal + gal[::-1]
    keys = {g: orc.galois_key(s, g, 31 + i) for i, g in enumerate(dict.fromkeys(gal))}
    dkeys = {g: ctx.load_key(k) for g, k in keys.items()}
    rng = np.random.default_rng(6)
    ct = residues(rng, ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    outs = ctx.rotate_hoisted(dct, ctx.rotation_precompute(dct), [dkeys[g] for g in gal], gal)
    want = {g: orc.rotate(ct, keys[g], g) for g in keys}
    for out, g in zip(outs, gal):
        assert np.array_equal(out.numpy(), want[g]), g
    low = residues(rng, ctx.q[:ctx.L - 1], (2,), ctx.n)
    got = ctx.rotate(ctx.upload(low), dkeys[gal[0]], gal[0]).numpy()
    assert np.array_equal(got, orc.rotate(low, keys[gal[0]], gal[0]))


def test_benchmark_step_matches_oracle():
    """The benchmark's whole timed step (bench.py run_rotations) at its
    parameters: the hoisted set {+-2^k, k < 15} of one ciphertext at
    N = 2^16, L = 24, K = 8, dnum 3 (one ModUp, the 30 rotations as one
    key-switch batch) and the rescale of the ciphertext; the ModUp digits,
    every rotation and the rescale equal the oracle word for word (the
    oracle's rotations on all usable cores)."""
    import concurrent.futures as cf
    import os
    steps = [sg * (1 << k) for k in range(15) for sg in (1, -1)]
    q, p = O.gen_moduli(16, 23, 59, 60, 3)
    ctx, orc = F.Context(16, q, p, 3, sampling="seeded"), O.Ctx(16, q, p, 3)
    assert (ctx.L, ctx.K, ctx.dnum) == (24, 8, 3)
    s = ctx.keygen_secret(1)
    gal = [F.galois_element(r, ctx.n) for r in steps]
    keys = [ctx.keygen_galois(s, g, 1000 + i) for i, g in enumerate(gal)]
    ct = residues(np.random.default_rng(7), ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    digits = ctx.rotation_precompute(dct)
    outs = ctx.rotate_hoisted(dct, digits, keys, gal)
    rs = ctx.rescale(dct)
    print(f"[bench step] GPU done; oracle on {len(steps)} rotations", flush=True)
    odig = orc.modup(ct[1])
    assert np.array_equal(digits.numpy(), odig)
    hkeys = [k.numpy() for k in keys]
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    with cf.ThreadPoolExecutor(threads) as ex:
        want = list(ex.map(lambda i: orc.rotate_hoisted(ct, odig, hkeys[i], gal[i]),
                           range(len(steps))))
    for r, out, w in zip(steps, outs, want):
        assert np.array_equal(out.numpy(), w), r
    assert np.array_equal(rs.numpy(), orc.rescale(ct))


@pytest.mark.parametrize("log_n,depth,dnum", [(14, 7, 4), (15, 9, 5), (13, 15, 8),
                                               (16, 7, 4), (16, 9, 5), (16, 11, 6),
                                               (16, 13, 7)])
def test_many_digits(log_n, depth, dnum):
    """More than three digits: the fused ModUp converts four to eight digits
    in one launch; ModDown's first and last passes run the paired kernels up
    to seven digits and the run-time digit-count kernels for eight.  At
    N=2^16 (two digit limbs each) the paired passes run with their radix-8
    block size for four to seven digits."""
    q, p = O.gen_moduli(log_n, depth, 50, 60, dnum)
    ctx, orc = F.Context(log_n, q, p, dnum, sampling="seeded"), O.Ctx(log_n, q, p, dnum)
    s = orc.secret(12)
    rng = np.random.default_rng(13)
    key = orc.relin_key(s, 7)
    dkey = ctx.load_key(key)
    for nq in (ctx.L, ctx.L - 3):
        a = residues(rng, ctx.q[:nq], (1,), ctx.n)
        assert np.array_equal(ctx.keyswitch(ctx.upload(a), dkey).numpy(), orc.keyswitch(a[0], key)), nq
    gal = [O.galois_elt(r, ctx.n) for r in (1, -2)]
    keys = [orc.galois_key(s, g, 40 + i) for i, g in enumerate(gal)]
    ct = residues(rng, ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    outs = ctx.rotate_hoisted(dct, ctx.rotation_precompute(dct), [ctx.load_key(k) for k in keys], gal)
    for out, k, g in zip(outs, keys, gal):
        assert np.array_equal(out.numpy(), orc.rotate(ct, k, g)), g


def test_full_batch_small_ring():
    """32 hoisted rotations at N=2^13 (64 polys x 64 columns: the 4-wave
    middle kernel with two column lines per wavefront)."""
    q, p = O.gen_moduli(13, 7, 50, 60, 2)
    ctx, orc = F.Context(13, q, p, 2, sampling="seeded"), O.Ctx(13, q, p, 2)
    s = orc.secret(8)
    steps = list(range(1, 17)) + [-r for r in range(1, 17)]
    gal = [O.galois_elt(r, ctx.n) for r in steps]
    keys = [orc.galois_key(s, g, 200 + i) for i, g in enumerate(gal)]
    ct = residues(np.random.default_rng(9), ctx.q, (2,), ctx.n)
    dct = ctx.upload(ct)
    outs = ctx.rotate_hoisted(dct, ctx.rotation_precompute(dct),
                              [ctx.load_key(k) for k in keys], gal)
    for out, key, g in zip(outs, keys, gal):
        assert np.array_equal(out.numpy(), orc.rotate(ct, key, g)), g


def test_classical128_chain_key_switch():
    """The reference's audited classical-128 chain (N=2^17, 45 Q + 12 P
    primes, four digits: the golden OpenFHE chain) at the full level and at
    31 limbs: relinearisation key switch and hoisted rotations, word for
    word against the oracle (the fused middle kernel holds the 12 source
    lines of a column in up to 160 KB of LDS per workgroup)."""
    import json
    import os
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                       "openfhe_prime_chain_n131072.json")))
    q, p = gold["primes"][:gold["num_q"]], gold["primes"][gold["num_q"]:]
    print(f"[classical-128] N=2^17 Q={len(q)} P={len(p)} dnum=4", flush=True)
    ctx, orc = F.Context(17, q, p, 4, sampling="seeded"), O.Ctx(17, q, p, 4)
    assert (ctx.L, ctx.K, ctx.dnum) == (45, 12, 4)
    s = orc.secret(17)
    rng = np.random.default_rng(18)
    key = orc.relin_key(s, 19)
    dkey = ctx.load_key(key)
    gal = [O.galois_elt(r, ctx.n) for r in (1, -8, 2, 4, -16, 32, 64, -128, 256)]
    gkeys = [orc.galois_key(s, g, 60 + i) for i, g in enumerate(gal)]
    dgk = [ctx.load_key(k) for k in gkeys]
    # 2 rotations: one 16-wave middle-kernel launch; at 31 limbs also 3
    # (8-wave) and 9 (4-wave), the 12 sources in two groups each time
    for nq, counts in ((45, (2,)), (31, (2, 3, 9))):
        a = residues(rng, ctx.q[:nq], (1,), ctx.n)
        assert np.array_equal(ctx.keyswitch(ctx.upload(a), dkey).numpy(),
                              orc.keyswitch(a[0], key)), nq
        ct = residues(rng, ctx.q[:nq], (2,), ctx.n)
        want = [orc.rotate(ct, k, g) for k, g in zip(gkeys[:max(counts)], gal)]
        dct = ctx.upload(ct)
        pre = ctx.rotation_precompute(dct)
        for m in counts:
            outs = ctx.rotate_hoisted(dct, pre, dgk[:m], gal[:m])
            for i, out in enumerate(outs):
                assert np.array_equal(out.numpy(), want[i]), (nq, m, i)
    ctx.close()


def test_decode_chain_conversion_groups():
    """The decode's N=2^16 chain (45 Q + 15 P primes, dnum 3), whose
    conversions have 15 sources (two groups of at most eight), word for word
    against the oracle in each middle-kernel launch shape: a relinearisation
    key switch (one ciphertext: 16-wave workgroups), 3 hoisted rotations
    (8-wave) and 9 (4-wave), at 45 limbs and at 20 (ModUp digits of 15 and 5
    sources)."""
    q, p = O.gen_moduli(16, 44, 59, 60, 3)
    print(f"[decode chain] N=2^16 Q={len(q)} P={len(p)} dnum=3", flush=True)
    ctx, orc = F.Context(16, q, p, 3, sampling="seeded"), O.Ctx(16, q, p, 3)
    assert (ctx.L, ctx.K, ctx.dnum) == (45, 15, 3)
    s = orc.secret(31)
    rng = np.random.default_rng(32)
    key = orc.relin_key(s, 33)
    dkey = ctx.load_key(key)
    gal = [O.galois_elt(r, ctx.n) for r in (1, -2, 4, 8, -16, 32, 64, -128, 256)]
    gkeys = [orc.galois_key(s, g, 40 + i) for i, g in enumerate(gal)]
    dgk = [ctx.load_key(k) for k in gkeys]
    for nq, counts in ((45, (3,)), (20, (3, 9))):
        a = residues(rng, ctx.q[:nq], (1,), ctx.n)
        assert np.array_equal(ctx.keyswitch(ctx.upload(a), dkey).numpy(),
                              orc.keyswitch(a[0], key)), nq
        ct = residues(rng, ctx.q[:nq], (2,), ctx.n)
        want = [orc.rotate(ct, k, g) for k, g in zip(gkeys[:max(counts)], gal)]
        dct = ctx.upload(ct)
        pre = ctx.rotation_precompute(dct)
        for m in counts:
            outs = ctx.rotate_hoisted(dct, pre, dgk[:m], gal[:m])
            for i, out in enumerate(outs):
                assert np.array_equal(out.numpy(), want[i]), (nq, m, i)
    ctx.close()
