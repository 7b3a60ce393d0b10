"""CKKS encode/decode and encryption on the GPU vs the CPU oracle."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")


@pytest.fixture(scope="module", params=[(12, 5, 40), (13, 7, 50), (16, 3, 59), (17, 3, 59)])
def pair(request):
    log_n, depth, sb = request.param
    q, p = O.gen_moduli(log_n, depth, sb, 60, 2)
    return F.Context(log_n, q, p, 2, sampling="seeded"), O.Ctx(log_n, q, p, 2)


@pytest.mark.parametrize("slots_div", [2, 8, 64])
def test_encode_bit_exact_and_decode_within_tolerance(pair, slots_div):
    ctx, orc = pair
    slots = ctx.n // slots_div
    rng = np.random.default_rng(slots)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    scale = float(ctx.q[-1])
    for nq in (1, ctx.L):
        got = ctx.encode(z, slots, scale, nq)
        want = orc.encode(z, slots, scale, nq)
        assert np.array_equal(got.numpy()[0], want)
        dec = ctx.decode(got, slots, scale)
        # decoded slot vectors match within 2^-30 relative to the input range
        assert np.abs(dec - z).max() < 2.0**-30
        assert np.abs(dec - orc.decode(want, slots, scale)).max() < 2.0**-40


def test_encode_real_partial_and_zero(pair):
    ctx, orc = pair
    slots = ctx.n // 2
    x = np.linspace(-3, 3, 17)
    scale = 2.0**40
    assert np.array_equal(ctx.encode(x, slots, scale, 2).numpy()[0],
                          orc.encode(x, slots, scale, 2))
    assert not ctx.encode(np.zeros(4), slots, scale, 1).numpy().any()


def test_encode_range_check_path_and_queued_encodes(pair):
    """An input whose largest slot exceeds 2^62 / scale takes the checked
    path (status read back) and still encodes when its coefficients fit: one
    nonzero slot spreads over 2 slots coefficients of 1/slots its size.
    Then 40 encodes queued without waits (the staging ring's 16 slots
    cycle) all equal the oracle."""
    ctx, orc = pair
    slots = ctx.n // 2
    scale = 2.0**40
    z = np.zeros(slots, dtype=complex)
    z[3] = 1.5 * 2.0**22 + 0.5j * 2.0**22  # |z| scale > 2^62, coefficients < 2^62
    got = ctx.encode(z, slots, scale, 2)
    assert np.array_equal(got.numpy()[0], orc.encode(z, slots, scale, 2))
    rng = np.random.default_rng(11)
    zs = [rng.uniform(-4, 4, slots) for _ in range(40)]
    outs = [ctx.encode(v, slots, scale, 2) for v in zs]
    for v, o in zip(zs, outs):
        assert np.array_equal(o.numpy()[0], orc.encode(v, slots, scale, 2))


def test_encode_out_of_range_raises(pair):
    ctx, _ = pair
    with pytest.raises(OverflowError):
        ctx.encode([2.0**30], 8, 2.0**40, 1)


@pytest.mark.parametrize("nvec,slots_div", [(1, 2), (5, 8), (16, 2), (37, 64)])
def test_encode_many_equals_single_encodes(pair, nvec, slots_div):
    """fhe_encode_many (shared FFT, rounding and NTT launches, outputs
    reached through a device table, sets of 16 rows) writes every row's
    plaintext exactly as one encode per row: complex rows at one and all
    limbs, and short real rows against the oracle."""
    ctx, orc = pair
    slots = ctx.n // slots_div
    rng = np.random.default_rng(nvec * 7 + slots_div)
    scale = float(ctx.q[-1])
    rows = rng.uniform(-1, 1, (nvec, slots)) + 1j * rng.uniform(-1, 1, (nvec, slots))
    for nq in (1, ctx.L):
        got = ctx.encode_many(rows, slots, scale, nq)
        assert len(got) == nvec
        for r, g in zip(rows, got):
            assert np.array_equal(g.numpy()[0], ctx.encode(r, slots, scale, nq).numpy()[0])
    real = rng.uniform(-3, 3, (nvec, 17))
    got = ctx.encode_many(real, slots, 2.0**40, 2)
    for r, g in zip(real[:3], got[:3]):
        assert np.array_equal(g.numpy()[0], orc.encode(r, slots, 2.0**40, 2))
    for r, g in zip(real[3:], got[3:]):
        assert np.array_equal(g.numpy()[0], ctx.encode(r, slots, 2.0**40, 2).numpy()[0])


def test_encode_many_checked_rows_and_errors(pair):
    """A set holding a row over the host bound takes the checked single path:
    rows whose coefficients fit still match the oracle; a row that does not
    fit raises OverflowError; zero rows encode nothing."""
    ctx, orc = pair
    slots = ctx.n // 2
    scale = 2.0**40
    rows = np.zeros((3, slots), dtype=complex)
    rows[0, 5] = 0.25
    rows[1, 3] = 1.5 * 2.0**22 + 0.5j * 2.0**22  # over the bound, coefficients fit
    rows[2, 7] = -0.75
    got = ctx.encode_many(rows, slots, scale, 2)
    for r, g in zip(rows, got):
        assert np.array_equal(g.numpy()[0], orc.encode(r, slots, scale, 2))
    with pytest.raises(OverflowError):
        ctx.encode_many(np.full((2, 8), 2.0**30), 8, scale, 1)
    assert ctx.encode_many(np.zeros((0, 8)), 8, scale, 1) == []


def test_encrypt_decrypt_match_oracle(pair):
    ctx, orc = pair
    s = orc.secret(3)
    pk = orc.public_key(s, 4)
    slots = ctx.n // 2
    x = np.random.default_rng(5).uniform(-1, 1, slots)
    scale = float(ctx.q[-1])
    m = orc.encode(x, slots, scale, ctx.L)
    dpk = ctx.upload(pk)
    ct = ctx.encrypt(dpk, ctx.upload(m), 6)
    assert np.array_equal(ct.numpy(), orc.encrypt(pk, m, 6))
    dm = ctx.decrypt(ct, s)
    assert np.array_equal(dm.numpy()[0], orc.decrypt(ct.numpy(), s))
    assert np.abs(ctx.decode(dm, slots, scale).real - x).max() < 1e-6
