"""Elementwise RNS ops, MAC, tensor and rescale on the GPU vs the oracle."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")


@pytest.fixture(scope="module", params=[(11, 6), (13, 8), (16, 5)])
def pair(request):
    log_n, depth = request.param
    q, p = O.gen_moduli(log_n, depth, 50, 60, 2)
    return F.Context(log_n, q, p, 2, sampling="seeded"), O.Ctx(log_n, q, p, 2)


def _obj(a):
    return a.astype(object)


def test_add_sub_negate(pair):
    ctx, orc = pair
    rng = np.random.default_rng(1)
    a = residues(rng, ctx.q, (2,), ctx.n)
    b = residues(rng, ctx.q, (2,), ctx.n)
    qv = np.array(ctx.q, dtype=object)[None, :, None]
    da, db = ctx.upload(a), ctx.upload(b)
    assert np.array_equal(ctx.add(da, db).numpy(), ((_obj(a) + _obj(b)) % qv).astype(np.uint64))
    assert np.array_equal(ctx.sub(da, db).numpy(), ((_obj(a) - _obj(b)) % qv).astype(np.uint64))
    assert np.array_equal(ctx.negate(da).numpy(), ((-_obj(a)) % qv).astype(np.uint64))
    # in place: out aliases an input
    ctx.add(da, db, out=da)
    assert np.array_equal(da.numpy(), ((_obj(a) + _obj(b)) % qv).astype(np.uint64))


def test_plain_and_constant_products(pair):
    ctx, orc = pair
    rng = np.random.default_rng(2)
    nq = ctx.L - 1
    a = residues(rng, ctx.q[:nq], (2,), ctx.n)
    w = residues(rng, ctx.q, (1,), ctx.n)  # plaintext may carry more limbs
    qv = np.array(ctx.q[:nq], dtype=object)[None, :, None]
    da, dw = ctx.upload(a), ctx.upload(w)
    got = ctx.mul_plain(da, dw).numpy()
    assert np.array_equal(got, ((_obj(a) * _obj(w[:, :nq])) % qv).astype(np.uint64))
    got = ctx.add_plain(da, dw).numpy()
    want = _obj(a).copy()
    want[0] = (want[0] + _obj(w[0, :nq])) % qv[0]
    assert np.array_equal(got, want.astype(np.uint64))
    c = [int(x) for x in rng.integers(0, 2**40, nq)]
    c = [x % q for x, q in zip(c, ctx.q)]
    cv = np.array(c, dtype=object)[None, :, None]
    assert np.array_equal(ctx.mul_const(da, c).numpy(), ((_obj(a) * cv) % qv).astype(np.uint64))
    got = ctx.add_const(da, c).numpy()
    want = _obj(a).copy()
    want[0] = (want[0] + cv[0]) % qv[0]
    assert np.array_equal(got, want.astype(np.uint64))
    for v in (4096, -3, 0, -(2**62)):
        got = ctx.mul_int(da, v).numpy()
        assert np.array_equal(got, ((_obj(a) * v) % qv).astype(np.uint64)), v


def test_drop_limbs_and_copy(pair):
    ctx, _ = pair
    rng = np.random.default_rng(3)
    a = residues(rng, ctx.q, (2,), ctx.n)
    da = ctx.upload(a)
    assert np.array_equal(ctx.drop_limbs(da, 2).numpy(), a[:, :2])
    cp = da.copy()
    ctx.drop_limbs(da, 3, out=da)
    assert np.array_equal(da.numpy(), a[:, :3])
    assert np.array_equal(cp.numpy(), a)


def test_tensor_and_square(pair):
    ctx, orc = pair
    rng = np.random.default_rng(4)
    a = residues(rng, ctx.q, (2,), ctx.n)
    b = residues(rng, ctx.q, (2,), ctx.n)
    da, db = ctx.upload(a), ctx.upload(b)
    assert np.array_equal(ctx.tensor(da, db).numpy(), orc.tensor(a, b))
    assert np.array_equal(ctx.tensor(da, da).numpy(), orc.tensor(a, a))


@pytest.mark.parametrize("npoly", [1, 2, 3])
def test_rescale(pair, npoly):
    ctx, orc = pair
    rng = np.random.default_rng(5 + npoly)
    for nq in (2, ctx.L):
        a = residues(rng, ctx.q[:nq], (npoly,), ctx.n)
        da = ctx.upload(a)
        assert np.array_equal(ctx.rescale(da).numpy(), orc.rescale(a))
    # in place
    a = residues(rng, ctx.q, (npoly,), ctx.n)
    da = ctx.upload(a)
    ctx.rescale(da, out=da)
    assert np.array_equal(da.numpy(), orc.rescale(a))


def oracle_mod_raise(orc, q, a, nlimb):
    """Limb 0 to coefficients (oracle iNTT), centred mod q0, reduced mod
    each q_j and back through the oracle NTT."""
    out = np.empty((a.shape[0], nlimb, a.shape[2]), dtype=np.uint64)
    for p in range(a.shape[0]):
        c = orc.ntt_inv(a[p, 0].copy(), 0).astype(object)
        c = np.where(c > q[0] // 2, c - q[0], c)
        for j in range(nlimb):
            out[p, j] = orc.ntt_fwd(np.array([int(v) % q[j] for v in c], dtype=np.uint64), j)
    return out


def test_mod_raise(pair):
    ctx, orc = pair
    rng = np.random.default_rng(17)
    for src_limbs, nlimb in ((1, ctx.L), (3, ctx.L - 1), (1, 1)):
        a = residues(rng, ctx.q[:src_limbs], (2,), ctx.n)
        got = ctx.mod_raise(ctx.upload(a), nlimb).numpy()
        assert np.array_equal(got, oracle_mod_raise(orc, ctx.q, a, nlimb))
    # in place, and the centring at the edges (0, q0 // 2, q0 // 2 + 1, q0 - 1)
    c = np.zeros(ctx.n, dtype=np.uint64)
    c[:4] = [0, ctx.q[0] // 2, ctx.q[0] // 2 + 1, ctx.q[0] - 1]
    a = orc.ntt_fwd(c.copy(), 0)[None, None, :].copy()
    da = ctx.upload(a)
    ctx.mod_raise(da, ctx.L, out=da)
    want = oracle_mod_raise(orc, ctx.q, a, ctx.L)
    assert np.array_equal(da.numpy(), want)
    # centred values 0, (q0-1)/2, -(q0-1)/2, -1 reduced mod q1 (q1 < q0/2 here)
    coef = orc.ntt_inv(want[0, 1].copy(), 1)
    q0, q1 = ctx.q[0], ctx.q[1]
    assert [int(x) for x in coef[:4]] == [0, (q0 // 2) % q1, (q0 // 2 + 1 - q0) % q1, q1 - 1]


@pytest.mark.parametrize("count", [1, 5, 40])
def test_mac(pair, count):
    ctx, orc = pair
    rng = np.random.default_rng(6 + count)
    nq = ctx.L
    x = residues(rng, ctx.q, (count, 2), ctx.n)
    w = residues(rng, ctx.q, (count,), ctx.n)
    dx = ctx.upload(x.reshape(count * 2, nq, ctx.n))
    dw = ctx.upload(w)
    acc = ctx.poly(2, nq)
    ctx.mac_dev(dx.data_ptr(), dw.data_ptr(), count, nq, acc.data_ptr())
    assert np.array_equal(acc.numpy(), orc.mac(x, w))


@pytest.mark.parametrize("count", [1, 5, 20])
def test_linear_wsum_matches_big_integer_sum(pair, count):
    """fhe_linear_wsum = sum_i m_i x_i mod q_j exactly (Python integers),
    for terms holding more limbs than the sum, negative weights, weights
    past 64 bits and 20 terms (two launches, the second accumulating)."""
    ctx, _ = pair
    rng = np.random.default_rng(count)
    nq = ctx.L - 1
    xs, hs, ms = [], [], []
    for i in range(count):
        nl = nq + int(rng.integers(0, 2))
        a = residues(rng, ctx.q[:nl], (2,), ctx.n)
        xs.append(a[:, :nq])
        hs.append(ctx.upload(a))
        m = int(rng.integers(-2**62, 2**62)) * (1 if i % 3 else 2**40 + 7)
        ms.append(-m if i % 2 else m)
    ms[0] = -(2**125) + 3
    got = ctx.linear_wsum(hs, ms, nq).numpy()
    qv = np.array(ctx.q[:nq], dtype=object)[None, :, None]
    want = sum(_obj(x) * m for x, m in zip(xs, ms)) % qv
    assert np.array_equal(got, want.astype(np.uint64))
    with pytest.raises(ValueError):
        ctx.linear_wsum(hs, [2**127] * count, nq)


def test_argument_errors_raise(pair):
    ctx, _ = pair
    a = ctx.poly(2, 2)
    b = ctx.poly(2, 3)
    with pytest.raises(ValueError):
        ctx.add(a, b)
    with pytest.raises(ValueError):
        ctx.mul_const(a, [ctx.q[0], 0])  # not reduced
    with pytest.raises(ValueError):
        ctx.rescale(ctx.poly(2, 1))
