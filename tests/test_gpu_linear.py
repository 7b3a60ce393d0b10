"""BSGS plaintext linear transform on the GPU, bit-exact against the same
composition of oracle rotations, plaintext MACs and additions (babies from
one ModUp, giant steps by Horner's rule with one giant key)."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")

PARAMS = [(12, 5, 45, 60, 2), (11, 4, 40, 60, 3)]


@pytest.fixture(scope="module", params=PARAMS)
def setup(request):
    log_n, depth, sb, fb, dnum = request.param
    q, p = O.gen_moduli(log_n, depth, sb, fb, dnum)
    ctx, orc = F.Context(log_n, q, p, dnum, sampling="seeded"), O.Ctx(log_n, q, p, dnum)
    s = orc.secret(21)
    return ctx, orc, s, {}


def _key(setup, step):
    ctx, orc, s, cache = setup
    if step not in cache:
        g = O.galois_elt(step, ctx.n)
        k = orc.galois_key(s, g, 300 + len(cache))
        cache[step] = (g, k, ctx.load_key(k))
    return cache[step]


def oracle_transform(orc, q, ct, pts, bstep, baby, giant):
    count, nq = len(pts), ct.shape[1]
    qa = np.array(q[:nq], dtype=np.uint64)[None, :, None]
    used = {k % bstep for k in range(count) if pts[k] is not None}
    babies = {0: ct}
    for b in range(1, min(bstep, count)):
        if b in used:
            g, k = baby[b]
            babies[b] = orc.rotate(ct, k, g)

    def inner(g):
        xs, ws = [], []
        for b in range(bstep):
            k = g * bstep + b
            if k < count and pts[k] is not None:
                xs.append(babies[b])
                ws.append(pts[k][:nq])
        if not xs:
            return np.zeros_like(ct)
        return orc.mac(np.stack(xs), np.stack(ws))

    giants = -(-count // bstep)
    acc = inner(giants - 1)
    for g in range(giants - 2, -1, -1):
        r = orc.rotate(acc, giant[1], giant[0])
        acc = (r + inner(g)) % qa
    return acc


CASES = [
    # (count, bstep, stride, null diagonals, in place)
    (7, 3, 1, (4,), False),
    (4, 4, 2, (), False),
    (5, 1, 1, (), False),
    (9, 4, 1, (1, 5, 8), True),
    (1, 1, 1, (), False),
]


@pytest.mark.parametrize("count,bstep,stride,nulls,inplace", CASES)
def test_linear_transform_matches_oracle(setup, count, bstep, stride, nulls, inplace):
    ctx, orc, s, _ = setup
    rng = np.random.default_rng(100 + count * 7 + bstep)
    nq = ctx.L - 1  # one level down: keys and plaintexts carry more limbs
    ct = residues(rng, ctx.q[:nq], (2,), ctx.n)
    pts_host = [None if k in nulls else residues(rng, ctx.q, (), ctx.n)
                for k in range(count)]
    pts_dev = [None if p is None else ctx.upload(p[None]) for p in pts_host]
    baby = {b: _key(setup, b * stride)[:2] for b in range(1, min(bstep, count))}
    baby_dev = [_key(setup, b * stride)[2] for b in range(1, min(bstep, count))]
    baby_gal = [baby[b][0] for b in range(1, min(bstep, count))]
    gk = _key(setup, bstep * stride) if count > bstep else None
    dct = ctx.upload(ct)
    out = dct if inplace else None
    got = ctx.linear_transform(dct, pts_dev, bstep, baby_dev, baby_gal,
                               gk[2] if gk else None, gk[0] if gk else 1, out=out).numpy()
    want = oracle_transform(orc, ctx.q, ct, pts_host, bstep, baby,
                            gk[:2] if gk else None)
    assert np.array_equal(got, want)


def test_linear_transform_rejects_bad_arguments(setup):
    ctx, orc, s, _ = setup
    rng = np.random.default_rng(5)
    ct = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
    pt = ctx.upload(residues(rng, ctx.q, (1,), ctx.n))
    with pytest.raises(ValueError):  # every diagonal null
        ctx.linear_transform(ct, [None, None], 2, [None], [1])
    with pytest.raises(ValueError):  # giant key missing
        ctx.linear_transform(ct, [pt, pt, pt], 2, [_key(setup, 1)[2]], [_key(setup, 1)[0]])
    short = ctx.upload(residues(rng, ctx.q[:2], (1,), ctx.n))
    with pytest.raises(ValueError):  # plaintext with fewer limbs than ct
        ctx.linear_transform(ct, [short], 1, [], [])


def oracle_transform_hoisted(orc, q, ct, pts, bstep, offset_keys, giant_keys):
    """The hoisted schedule: babies ct rotated by offset + b strides (each
    from ct), every giant step's inner sum rotated by its own key, summed."""
    count, nq = len(pts), ct.shape[1]
    qa = np.array(q[:nq], dtype=np.uint64)[None, :, None]
    used = {k % bstep for k in range(count) if pts[k] is not None}
    babies = {}
    for b in used:
        babies[b] = ct if offset_keys.get(b) is None else \
            orc.rotate(ct, offset_keys[b][1], offset_keys[b][0])

    def inner(g):
        xs, ws = [], []
        for b in range(bstep):
            k = g * bstep + b
            if k < count and pts[k] is not None:
                xs.append(babies[b])
                ws.append(pts[k][:nq])
        if not xs:
            return np.zeros_like(ct)
        return orc.mac(np.stack(xs), np.stack(ws))

    giants = -(-count // bstep)
    acc = inner(0)
    for g in range(1, giants):
        gk = giant_keys[g - 1]
        acc = (acc + orc.rotate(inner(g), gk[1], gk[0])) % qa
    return acc


HOISTED = [
    # (count, bstep, stride, offset, null diagonals)
    (9, 3, 1, -4, (4,)),
    (12, 4, 2, -11, ()),
    (7, 4, 1, 0, (2,)),
    (16, 4, 3, 5, (0, 13)),
    # ten giants (inner sums in two passes of at most eight), one all-null
    (40, 4, 1, 0, (8, 9, 10, 11, 30)),
    # eighteen giants (the giant-step sum in pairwise additions past 16)
    (36, 2, 1, 3, (7,)),
    # more babies than one inner-sum pass takes (35 > 32)
    (70, 35, 1, 0, (3, 40)),
]


@pytest.mark.parametrize("count,bstep,stride,offset,nulls", HOISTED)
def test_hoisted_linear_transform_matches_oracle(setup, count, bstep, stride, offset, nulls):
    """fhe_linear_transform_hoisted: the offset folded into the babies'
    shared ModUp and one key per giant step (the giant rotations as one
    batch), bit-exact against the same composition of oracle rotations."""
    check_hoisted(setup, count, bstep, stride, offset, nulls)


@pytest.fixture(scope="module")
def setup16():
    q, p = O.gen_moduli(16, 9, 59, 60, 3)
    ctx, orc = F.Context(16, q, p, 3, sampling="seeded"), O.Ctx(16, q, p, 3)
    return ctx, orc, orc.secret(22), {}


HOISTED16 = [
    # a CoeffToSlot level-budget group of the N = 2^16 bootstrap: four
    # radix-2 stages, 31 diagonals on an arithmetic progression of offsets
    # (stride 2^9 here), baby step 8, four giant steps
    (31, 8, 512, -15 * 512, ()),
    # an in_proj-sized projection of the 130M decoder: 110 diagonals, baby
    # step 10, eleven giant steps (two inner-sum passes of at most eight)
    (110, 10, 1, 0, (5, 57)),
]


@pytest.mark.parametrize("count,bstep,stride,offset,nulls", HOISTED16)
def test_hoisted_linear_transform_at_n65536(setup16, count, bstep, stride, offset, nulls):
    """The hoisted transform (k_mac_giants, the batched giant key switches,
    k_sum) and its Horner form at N = 2^16 with the giant-step counts of
    the bootstrap and of the decoder's projections, bit-exact against the
    oracle composition."""
    print(f"[linear] N=2^16: {count} diagonals, baby step {bstep}", flush=True)
    check_hoisted(setup16, count, bstep, stride, offset, nulls)


def check_hoisted(setup, count, bstep, stride, offset, nulls):
    ctx, orc, s, _ = setup
    rng = np.random.default_rng((300 + count + bstep + offset) % 2**32)
    nq = ctx.L - 1
    ct = residues(rng, ctx.q[:nq], (2,), ctx.n)
    pts_host = [None if k in nulls else residues(rng, ctx.q, (), ctx.n)
                for k in range(count)]
    pts_dev = [None if p is None else ctx.upload(p[None]) for p in pts_host]
    nb = min(bstep, count)
    used = {k % bstep for k in range(count) if pts_host[k] is not None}
    okeys = {b: (_key(setup, offset + b * stride)[:2] if (b or offset) else None)
             for b in used}
    bdev = [(_key(setup, offset + b * stride)[2] if b in used and (b or offset) else None)
            for b in range(nb)]
    bgal = [(_key(setup, offset + b * stride)[0] if b in used and (b or offset) else 1)
            for b in range(nb)]
    giants = -(-count // bstep)
    gks = [_key(setup, g * bstep * stride) for g in range(1, giants)]
    got = ctx.linear_transform_hoisted(ctx.upload(ct), pts_dev, bstep, bdev, bgal,
                                       [k[2] for k in gks], [k[0] for k in gks]).numpy()
    want = oracle_transform_hoisted(orc, ctx.q, ct, pts_host, bstep, okeys,
                                    [k[:2] for k in gks])
    assert np.array_equal(got, want)
    # Horner's rule with the single giant key, through the same entry
    if giants > 2:
        g1 = _key(setup, bstep * stride)
        got1 = ctx.linear_transform_hoisted(ctx.upload(ct), pts_dev, bstep, bdev, bgal,
                                            [g1[2]], [g1[0]]).numpy()
        babies_first = {b: okeys.get(b) for b in used}
        want1 = oracle_transform_horner_from_babies(orc, ctx.q, ct, pts_host, bstep,
                                                    babies_first, g1[:2])
        assert np.array_equal(got1, want1)


def oracle_transform_horner_from_babies(orc, q, ct, pts, bstep, offset_keys, giant):
    count, nq = len(pts), ct.shape[1]
    qa = np.array(q[:nq], dtype=np.uint64)[None, :, None]
    babies = {b: ct if k is None else orc.rotate(ct, k[1], k[0]) for b, k in offset_keys.items()}

    def inner(g):
        xs, ws = [], []
        for b in range(bstep):
            k = g * bstep + b
            if k < count and pts[k] is not None:
                xs.append(babies[b])
                ws.append(pts[k][:nq])
        return orc.mac(np.stack(xs), np.stack(ws)) if xs else np.zeros_like(ct)

    giants = -(-count // bstep)
    acc = inner(giants - 1)
    for g in range(giants - 2, -1, -1):
        acc = (orc.rotate(acc, giant[1], giant[0]) + inner(g)) % qa
    return acc


def test_hoisted_linear_transform_rejects_bad_giant_keys(setup):
    ctx, orc, s, _ = setup
    rng = np.random.default_rng(6)
    ct = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
    pts = [ctx.upload(residues(rng, ctx.q, (1,), ctx.n)) for _ in range(9)]
    k1 = _key(setup, 1)
    with pytest.raises(ValueError):  # three keys for three giant steps (one or two)
        ctx.linear_transform_hoisted(ct, pts, 3, [None, k1[2], k1[2]], [1, k1[0], k1[0]],
                                     [k1[2]] * 3, [k1[0]] * 3)
    with pytest.raises(ValueError):  # no giant key at all
        ctx.linear_transform_hoisted(ct, pts, 3, [None, k1[2], k1[2]], [1, k1[0], k1[0]])


MANY = [
    # (count, bstep, stride, offset, null diagonals)
    (9, 3, 1, -4, (4,)),
    (16, 4, 3, 5, (0, 13)),
    (7, 4, 1, 0, (2,)),
]


@pytest.mark.parametrize("count,bstep,stride,offset,nulls", MANY)
def test_hoisted_linear_transform_many_equals_single(setup, count, bstep, stride, offset, nulls):
    """fhe_linear_transform_hoisted_many over three ciphertexts: each output
    equal to the single entry point's (both giant schedules), the first
    also to the oracle composition; outputs written over the inputs (each
    into another input's handle) give the same polys."""
    ctx, orc, s, _ = setup
    rng = np.random.default_rng((900 + count * 3 + bstep + offset) % 2**32)
    nq = ctx.L - 1
    cts = [residues(rng, ctx.q[:nq], (2,), ctx.n) for _ in range(3)]
    pts_host = [None if k in nulls else residues(rng, ctx.q, (), ctx.n)
                for k in range(count)]
    pts_dev = [None if p is None else ctx.upload(p[None]) for p in pts_host]
    nb = min(bstep, count)
    used = {k % bstep for k in range(count) if pts_host[k] is not None}
    okeys = {b: (_key(setup, offset + b * stride)[:2] if (b or offset) else None)
             for b in used}
    bdev = [(_key(setup, offset + b * stride)[2] if b in used and (b or offset) else None)
            for b in range(nb)]
    bgal = [(_key(setup, offset + b * stride)[0] if b in used and (b or offset) else 1)
            for b in range(nb)]
    giants = -(-count // bstep)
    gks = [_key(setup, g * bstep * stride) for g in range(1, giants)]
    schedules = [([k[2] for k in gks], [k[0] for k in gks])]
    if giants > 2:
        g1 = _key(setup, bstep * stride)
        schedules.append(([g1[2]], [g1[0]]))
    first = None
    for gk, gg in schedules:
        singles = [ctx.linear_transform_hoisted(ctx.upload(c), pts_dev, bstep, bdev, bgal,
                                                gk, gg).numpy() for c in cts]
        first = singles[0] if first is None else first
        got = ctx.linear_transform_hoisted_many([ctx.upload(c) for c in cts], pts_dev, bstep,
                                                bdev, bgal, gk, gg)
        for g, w in zip(got, singles):
            assert np.array_equal(g.numpy(), w)
        dcts = [ctx.upload(c) for c in cts]
        got = ctx.linear_transform_hoisted_many(dcts, pts_dev, bstep, bdev, bgal, gk, gg,
                                                outs=dcts[1:] + dcts[:1])
        for g, w in zip(got, singles):
            assert np.array_equal(g.numpy(), w)
    want = oracle_transform_hoisted(orc, ctx.q, cts[0], pts_host, bstep, okeys,
                                    [k[:2] for k in gks])
    assert np.array_equal(first, want)


def test_linear_transform_many_rejects_bad_arguments(setup):
    ctx, orc, s, _ = setup
    rng = np.random.default_rng(6)
    a = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
    b = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
    short = ctx.upload(residues(rng, ctx.q[:-1], (2,), ctx.n))
    pt = ctx.upload(residues(rng, ctx.q, (1,), ctx.n))
    with pytest.raises(ValueError):  # limb counts differ within the call
        ctx.linear_transform_hoisted_many([a, short], [pt], 1, [None], [1])
    o = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
    with pytest.raises(ValueError):  # one output for two ciphertexts
        ctx.linear_transform_hoisted_many([a, b], [pt], 1, [None], [1], outs=[o, o])
    with pytest.raises(ValueError):  # a diagonal as an output
        ctx.linear_transform_hoisted_many([a, b], [pt], 1, [None], [1], outs=[o, pt])
    with pytest.raises(ValueError):  # no ciphertext
        ctx.linear_transform_hoisted_many([], [pt], 1, [None], [1])
