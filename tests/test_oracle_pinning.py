"""Pin the CPU oracle against golden vectors, closed forms and brute force.

Each test names the mistake it is designed to catch.  The oracle is the
checker for every GPU parity test, so it is checked here first.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------- moduli
def test_prime_chain_matches_openfhe_golden_chain():
    """All 57 primes of OpenFHE's N=2^17 chain, in order (catches a wrong
    FirstPrime direction, a swapped alternation or P selection)."""
    with open(os.path.join(GOLDEN, "openfhe_prime_chain_n131072.json")) as fh:
        gold = json.load(fh)
    q, p = O.gen_moduli(17, gold["multiplicative_depth"], gold["scaling_mod_size"],
                        gold["first_mod_size"], gold["num_large_digits"])
    assert len(q) == gold["num_q"] and len(p) == gold["num_p"]
    assert q + p == gold["primes"]


@pytest.mark.parametrize("log_n,depth,dnum", [(13, 7, 2), (16, 23, 3), (16, 4, 3)])
def test_prime_chain_invariants(log_n, depth, dnum):
    q, p = O.gen_moduli(log_n, depth, 59, 60, dnum)
    m = 2 << log_n
    assert len(set(q + p)) == len(q) + len(p)
    for x in q + p:
        assert (x - 1) % m == 0 and O.lib.orc_is_prime(x)
    assert q[0] < 2**60 and all(abs(np.log2(x) - 59) < 0.01 for x in q[1:])


def test_special_prime_count_rule():
    """K = ceil(max digit bits / 60): the L=24, dnum=3 chain needs 8."""
    q, p = O.gen_moduli(16, 23, 59, 60, 3)
    assert len(p) == 8


def test_miller_rabin_against_trial_division():
    rng = np.random.default_rng(5)
    for v in list(range(2, 3000)) + [int(x) for x in rng.integers(2**31, 2**33, 300)]:
        d, prime = 2, v >= 2
        while d * d <= v:
            if v % d == 0:
                prime = False
                break
            d += 1
        assert bool(O.lib.orc_is_prime(v)) == prime, v


def test_root_of_unity_is_smallest_primitive():
    for log_n in (3, 4, 5):
        m = 2 << log_n
        for q in O.ntt_friendly_primes(log_n, 14, 3):
            psi = O.lib.orc_root_of_unity(m, q)
            assert pow(psi, m // 2, q) == q - 1
            roots = [x for x in range(2, q) if pow(x, m, q) == 1 and pow(x, m // 2, q) == q - 1]
            assert psi == min(roots)


# ------------------------------------------------------------- NTT
def _brv(i, bits):
    return int(format(i, f"0{bits}b")[::-1], 2) if bits else 0


@pytest.mark.parametrize("log_n", [1, 4, 8, 10])
def test_ntt_matches_direct_evaluation(log_n):
    """NTT output index i holds a(psi^(2 brv(i)+1)) (catches a wrong
    twiddle order or ordering of the output)."""
    n = 1 << log_n
    q = O.ntt_friendly_primes(log_n, 60, 1)[0]
    psi = O.lib.orc_root_of_unity(2 * n, q)
    rng = np.random.default_rng(log_n)
    a = [int(x) for x in rng.integers(0, q, n, dtype=np.uint64)]
    got = O.u64(a)
    O.lib.orc_ntt_fwd(O.ptr(got), n, q, psi)
    for i in range(n):
        x = pow(psi, 2 * _brv(i, log_n) + 1, q)
        assert int(got[i]) == sum(c * pow(x, j, q) for j, c in enumerate(a)) % q


@pytest.mark.parametrize("log_n,bits", [(6, 60), (9, 50), (10, 31)])
def test_ntt_convolution_theorem_and_inverse(log_n, bits):
    n = 1 << log_n
    q = O.ntt_friendly_primes(log_n, bits, 1)[0]
    psi = O.lib.orc_root_of_unity(2 * n, q)
    rng = np.random.default_rng(bits)
    a, b = (rng.integers(0, q, n, dtype=np.uint64) for _ in range(2))
    want = np.zeros(n, dtype=np.uint64)
    O.lib.orc_negacyclic_schoolbook(O.ptr(O.u64(a)), O.ptr(O.u64(b)), O.ptr(want), n, q)
    fa, fb = O.u64(a).copy(), O.u64(b).copy()
    O.lib.orc_ntt_fwd(O.ptr(fa), n, q, psi)
    O.lib.orc_ntt_fwd(O.ptr(fb), n, q, psi)
    prod = O.u64([(int(x) * int(y)) % q for x, y in zip(fa, fb)])
    O.lib.orc_ntt_inv(O.ptr(prod), n, q, psi)
    assert (prod == want).all()
    O.lib.orc_ntt_inv(O.ptr(fa), n, q, psi)
    assert (fa == a).all()


def test_schoolbook_negacyclic_wraps_with_sign():
    q, n = 97, 4
    a, b = O.u64([0, 0, 0, 1]), O.u64([0, 1, 0, 0])  # X^3 * X = X^4 = -1
    out = np.zeros(4, dtype=np.uint64)
    O.lib.orc_negacyclic_schoolbook(O.ptr(a), O.ptr(b), O.ptr(out), n, q)
    assert list(out) == [96, 0, 0, 0]


# ------------------------------------------------------------- automorphisms
@pytest.mark.parametrize("k", [5, 25, 3, 2 * 64 - 1])
def test_automorphism_eval_permutation_matches_coefficient_map(k):
    n = 64
    q = O.ntt_friendly_primes(6, 60, 1)[0]
    psi = O.lib.orc_root_of_unity(2 * n, q)
    rng = np.random.default_rng(k)
    a = rng.integers(0, q, n, dtype=np.uint64)
    ac = np.zeros(n, dtype=np.uint64)
    O.lib.orc_automorph_coeff(O.ptr(O.u64(a)), O.ptr(ac), n, k, q)
    # closed form X^j -> +-X^{jk mod 2n}
    for j in range(n):
        e = j * k % (2 * n)
        v = int(a[j])
        assert int(ac[e % n]) == (v if e < n else (q - v) % q)
    fa, fac = O.u64(a).copy(), ac.copy()
    O.lib.orc_ntt_fwd(O.ptr(fa), n, q, psi)
    O.lib.orc_ntt_fwd(O.ptr(fac), n, q, psi)
    perm = np.zeros(n, dtype=np.uint64)
    O.lib.orc_automorph_ntt(O.ptr(fa), O.ptr(perm), n, k)
    assert (perm == fac).all()


def test_galois_elements():
    n = 1 << 10
    assert O.galois_elt(1, n) == 5 and O.galois_elt(2, n) == 25
    assert (O.galois_elt(-1, n) * 5) % (2 * n) == 1
    assert O.galois_elt(n // 2, n) == 1


# ------------------------------------------------------------- basis conversion
def test_switch_basis_matches_big_integer_crt():
    """y = x + u*Q_from with 0 <= u < |from| (the uncorrected fast basis
    conversion identity), checked with exact integers."""
    n = 32
    src = O.ntt_friendly_primes(5, 60, 3)
    dst = O.ntt_friendly_primes(5, 59, 4)
    rng = np.random.default_rng(9)
    x = np.stack([rng.integers(0, q, n, dtype=np.uint64) for q in src])
    y = np.zeros((len(dst), n), dtype=np.uint64)
    O.lib.orc_switch_basis(O.ptr(x), O.ptr(O.u64(src)), len(src), O.ptr(y), O.ptr(O.u64(dst)),
                           len(dst), n)
    Q = int(np.prod([int(q) for q in src], dtype=object))
    for c in range(n):
        X = 0
        acc = 0
        for i, q in enumerate(src):
            qh = Q // q
            v = int(x[i, c]) * pow(qh, -1, q) % q
            acc += v * qh
            X = (X + int(x[i, c]) * qh * pow(qh, -1, q)) % Q
        u = (acc - X) // Q
        assert (acc - X) % Q == 0 and 0 <= u < len(src)
        for k, m in enumerate(dst):
            assert int(y[k, c]) == acc % m


# ------------------------------------------------------------- key switching
@pytest.fixture(scope="module")
def tiny_ctx():
    log_n = 5
    q = O.ntt_friendly_primes(log_n, 50, 5)
    p = O.ntt_friendly_primes(log_n, 60, 2, skip=q)
    return O.Ctx(log_n, q, p, 2)


def _crt(residues, mods):
    M = 1
    for m in mods:
        M *= m
    x = 0
    for r, m in zip(residues, mods):
        mh = M // m
        x += int(r) * mh * pow(mh, -1, m)
    return x % M, M


def test_modup_digits_extend_each_digit(tiny_ctx):
    c = tiny_ctx
    rng = np.random.default_rng(2)
    nq = 5
    a = np.stack([rng.integers(0, q, c.n, dtype=np.uint64) for q in c.q])
    digits = c.modup(a)
    coef = lambda poly, idx: c.ntt_inv(poly, idx)  # noqa: E731
    nd = c.num_digits(nq)
    assert nd == 2 and digits.shape == (nd, nq + c.K, c.n)
    for j in range(nd):
        s, e = j * c.alpha, min((j + 1) * c.alpha, nq)
        part = [coef(a[i], i) for i in range(s, e)]
        ext_mods = c.q[:nq] + c.p
        dcoef = [coef(digits[j, i], i if i < nq else c.L + i - nq) for i in range(nq + c.K)]
        for t in range(c.n):
            xj, Qj = _crt([p[t] for p in part], c.q[s:e])
            vals = [int(d[t]) for d in dcoef]
            u = None
            for i, m in enumerate(ext_mods):
                if s <= i < e:
                    assert vals[i] == xj % m
                    continue
                for cand in range(e - s):
                    if (xj + cand * Qj) % m == vals[i]:
                        u = cand if u is None else u
                        break
                else:
                    raise AssertionError("digit residue is not x + u*Q_j")
                assert (xj + u * Qj) % m == vals[i]


def test_moddown_divides_by_p(tiny_ctx):
    """ModDown(x) = floor(x / P) - u, 0 <= u < K, for x in [0, QP)."""
    c = tiny_ctx
    nq = 4
    rng = np.random.default_rng(3)
    mods = c.q[:nq] + c.p
    coefs = np.stack([rng.integers(0, m, c.n, dtype=np.uint64) for m in mods])
    ext = np.stack([c.ntt_fwd(coefs[i], i if i < nq else c.L + i - nq) for i in range(nq + c.K)])
    out = c.moddown(ext)
    outc = [c.ntt_inv(out[i], i) for i in range(nq)]
    P = int(np.prod([int(p) for p in c.p], dtype=object))
    for t in range(c.n):
        x, _ = _crt([coefs[i, t] for i in range(nq + c.K)], mods)
        y, Q = _crt([o[t] for o in outc], c.q[:nq])
        diff = (x // P - y) % Q
        assert diff < c.K


def test_rescale_is_exact_division(tiny_ctx):
    """x = q_l*Y + r with |r| < q_l/2 rescales to exactly Y."""
    c = tiny_ctx
    nq = 4
    rng = np.random.default_rng(4)
    ql = c.q[nq - 1]
    Qr = int(np.prod([int(q) for q in c.q[: nq - 1]], dtype=object))
    Y = [int(v) for v in rng.integers(0, 2**62, c.n)]
    Y = [(v * 1234567 + 99) % Qr for v in Y]
    r = [int(v) for v in rng.integers(-(ql // 2), ql // 2, c.n)]
    X = [ql * y + e for y, e in zip(Y, r)]
    coef = np.stack([O.u64([x % q for x in X]) for q in c.q[:nq]])
    ev = np.stack([c.ntt_fwd(coef[i], i) for i in range(nq)])
    out = c.rescale(ev[None])[0]
    got = [c.ntt_inv(out[i], i) for i in range(nq - 1)]
    for i, q in enumerate(c.q[: nq - 1]):
        assert [int(v) for v in got[i]] == [y % q for y in Y]


@pytest.fixture(scope="module")
def small_scheme():
    log_n = 11
    q, p = O.gen_moduli(log_n, 5, 40, 60, 2)
    c = O.Ctx(log_n, q, p, 2)
    s = c.secret(21)
    return c, s, c.public_key(s, 22)


@pytest.mark.parametrize("step", [1, 7, -3, 256])
def test_rotation_decrypts_to_rolled_message(small_scheme, step):
    c, s, pk = small_scheme
    slots = c.n // 2
    x = np.random.default_rng(step + 50).uniform(-1, 1, slots)
    scale = float(c.q[-1])
    ct = c.encrypt(pk, c.encode(x, slots, scale, c.L), 5)
    g = O.galois_elt(step, c.n)
    out = c.rotate(ct, c.galois_key(s, g, 6), g)
    got = c.decode(c.decrypt(out, s), slots, scale).real
    assert np.abs(got - np.roll(x, -step)).max() < 1e-5


def test_conjugation_decrypts_to_conjugate(small_scheme):
    c, s, pk = small_scheme
    slots = c.n // 2
    rng = np.random.default_rng(8)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    scale = float(c.q[-1])
    ct = c.encrypt(pk, c.encode(z, slots, scale, c.L), 5)
    g = 2 * c.n - 1
    out = c.rotate(ct, c.galois_key(s, g, 6), g)
    got = c.decode(c.decrypt(out, s), slots, scale)
    assert np.abs(got - np.conj(z)).max() < 1e-5


def test_relinearized_product_and_rescale(small_scheme):
    c, s, pk = small_scheme
    slots = c.n // 2
    rng = np.random.default_rng(12)
    x, y = rng.uniform(-1, 1, slots), rng.uniform(-1, 1, slots)
    scale = float(c.q[-1])
    cx = c.encrypt(pk, c.encode(x, slots, scale, c.L), 1)
    cy = c.encrypt(pk, c.encode(y, slots, scale, c.L), 2)
    t = c.tensor(cx, cy)
    # the 3-element tensor decrypts (with s^2) to the product already
    d3 = c.decode(c.decrypt(t, s), slots, scale * scale).real
    assert np.abs(d3 - x * y).max() < 1e-5
    ct = c.rescale(c.relinearize(t, c.relin_key(s, 3)))
    got = c.decode(c.decrypt(ct, s), slots, scale * scale / c.q[-1]).real
    assert np.abs(got - x * y).max() < 1e-5


# ------------------------------------------------------------- encoding
@pytest.mark.parametrize("slots", [1, 2, 8, 64])
def test_special_fft_matches_direct_evaluation(slots):
    """z_j = sum_i w_i * exp(2 pi i 5^j i / (4 slots)) (the canonical
    embedding restricted to the 5-orbit); catches conjugated twiddles or a
    missing bit reversal."""
    rng = np.random.default_rng(slots)
    w = rng.normal(size=slots) + 1j * rng.normal(size=slots)
    got = O.fft_special(w)
    m = 4 * slots
    for j in range(slots):
        xi = np.exp(2j * np.pi * pow(5, j, m) / m)
        want = sum(w[i] * xi**i for i in range(slots))
        assert abs(got[j] - want) < 1e-9 * max(1, abs(want))
    back = O.fft_special_inv(got)
    assert np.abs(back - w).max() < 1e-12


def test_encode_rounds_scaled_coefficients(small_scheme):
    c, _, _ = small_scheme
    slots = 64
    rng = np.random.default_rng(1)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    scale = 2.0**40
    m = c.encode(z, slots, scale, 2)
    coef = c.ntt_inv(m[0], 0)
    qv = c.q[0]
    signed = np.array([int(v) if v <= qv // 2 else int(v) - qv for v in coef], dtype=np.float64)
    w = O.fft_special_inv(z)
    gap = c.n // (2 * slots)
    want = np.zeros(c.n)
    want[0: 2 * slots * gap: gap] = np.concatenate([w.real, w.imag]) * scale
    assert np.abs(signed - want).max() <= 0.5 + 1e-3
    assert int(np.count_nonzero(signed)) <= 2 * slots
    dec = c.decode(m, slots, scale)
    assert np.abs(dec - z).max() < 1e-9


@pytest.mark.parametrize("kind", ["uniform", "gauss", "constant", "spike", "alternating"])
def test_special_inverse_fft_bounded_by_largest_slot(kind):
    """The encoder's asynchronous path relies on this: every coefficient of
    the special inverse FFT (division by slots included) has modulus at most
    the largest slot's, so scale * max|z| < 2^62 rules out the range error.
    A constant vector attains the bound (one coefficient equals it)."""
    slots = 256
    rng = np.random.default_rng(len(kind))
    z = {"uniform": rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots),
         "gauss": rng.normal(0, 3, slots) + 1j * rng.normal(0, 3, slots),
         "constant": np.full(slots, 2.5 - 1.5j),
         "spike": np.eye(1, slots, 7)[0] * (3 + 4j),
         "alternating": np.where(np.arange(slots) % 2, 1.0, -1.0) + 0j}[kind]
    w = O.fft_special_inv(z)
    assert np.abs(w).max() <= np.abs(z).max() * (1 + 1e-12)
    if kind == "constant":
        assert np.isclose(np.abs(w).max(), np.abs(z).max(), rtol=1e-12)


def test_encode_rejects_out_of_range(small_scheme):
    c, _, _ = small_scheme
    with pytest.raises(ValueError):
        c.encode([2.0**30], 8, 2.0**40, 1)


def test_crt_centered_reconstructs_signed_values(small_scheme):
    c, _, _ = small_scheme
    nq = 4
    rng = np.random.default_rng(6)
    vals = [int(v) for v in rng.integers(-(2**62), 2**62, c.n)]
    vals[0], vals[1] = 0, -1
    coef = np.stack([O.u64([v % q for v in vals]) for q in c.q[:nq]])
    got = c.crt_centered(coef)
    assert np.allclose(got, np.array(vals, dtype=np.float64), rtol=1e-15, atol=0)


# ------------------------------------------------------------- sampling
def test_sampling_ranges_and_moments():
    n = 1 << 16
    q = O.ntt_friendly_primes(16, 60, 1)[0]
    u = np.zeros(n, dtype=np.uint64)
    O.lib.orc_sample_uniform(123, q, O.ptr(u), n)
    assert int(u.max()) < q and abs(float(u.astype(np.float64).mean()) / q - 0.5) < 0.01
    t = np.zeros(n, dtype=np.int64)
    O.lib.orc_sample_ternary(5, O.ptr(t), n)
    assert set(np.unique(t)) == {-1, 0, 1}
    e = np.zeros(n, dtype=np.int64)
    O.lib.orc_sample_cbd(6, O.ptr(e), n)
    assert abs(e.var() - 10.5) < 0.5 and abs(e).max() <= 21


@pytest.mark.parametrize("h", [1, 64, 192, 4096])
def test_sparse_ternary_sampler(h):
    """Exactly h coefficients +-1 (h = n gives no zero), deterministic per
    seed; over many seeds every position and both signs are equally likely
    (a partial Fisher-Yates shuffle: no position bias from the modular
    reduction)."""
    n = 4096
    ctx = O.Ctx(12, O.ntt_friendly_primes(12, 50, 1), [], 1)
    s = ctx.secret_sparse(17, h)
    assert int(np.count_nonzero(s)) == h and set(np.unique(s)) <= {-1, 0, 1}
    assert np.array_equal(s, ctx.secret_sparse(17, h))
    if h < n:
        assert not np.array_equal(s, ctx.secret_sparse(18, h))
    if h == 192:
        hits = np.zeros(n)
        signs = 0
        for seed in range(400):
            t = ctx.secret_sparse(1000 + seed, h)
            hits += t != 0
            signs += int(t.sum())
        # 400 * 192 / 4096 = 18.75 expected hits per position
        buckets = hits.reshape(16, 256).sum(axis=1)
        assert np.all(np.abs(buckets / buckets.mean() - 1) < 0.05)
        assert abs(signs) < 4 * np.sqrt(400 * h)


# ------------------------------------------------------------- plaintext MAC
@pytest.mark.parametrize("count", [1, 31, 32, 33, 64, 65, 200])
@pytest.mark.parametrize("extreme", [False, True])
def test_mac_batch_matches_big_integer_sum(count, extreme):
    """acc[b][l][e] = sum_i x[i][b][l][e] * w[i][l][e] mod q_l, checked with
    Python integers.  Counts 31..33 and 64 straddle the oracle's periodic
    reduction of its 128-bit accumulator (every 32 terms); all-(q-1)
    operands at 61-bit primes (the largest the library accepts) give the
    largest partial sums: more than 64 products of (q-1)^2 exceed 2^128
    unless the accumulator is folded (catches a dropped or misplaced reduction, an
    overflowing accumulator, or a poly / limb index mix-up between x and w)."""
    log_n = 3
    n = 1 << log_n
    q = O.ntt_friendly_primes(log_n, 61, 1) + O.ntt_friendly_primes(log_n, 60, 1) + \
        O.ntt_friendly_primes(log_n, 59, 1)
    c = O.Ctx(log_n, q, [], 1)
    rng = np.random.default_rng(count)
    nq = len(q)
    if extreme:
        x = np.stack([np.stack([np.full((nq, n), 0, dtype=np.uint64)] * 2)] * count)
        w = np.zeros((count, nq, n), dtype=np.uint64)
        for l, ql in enumerate(q):
            x[:, :, l, :] = ql - 1
            w[:, l, :] = ql - 1
    else:
        x = np.zeros((count, 2, nq, n), dtype=np.uint64)
        w = np.zeros((count, nq, n), dtype=np.uint64)
        for l, ql in enumerate(q):
            x[:, :, l, :] = rng.integers(0, ql, (count, 2, n), dtype=np.uint64)
            w[:, l, :] = rng.integers(0, ql, (count, n), dtype=np.uint64)
    got = c.mac(x, w)
    for b in range(2):
        for l, ql in enumerate(q):
            for e in range(n):
                want = sum(int(x[i, b, l, e]) * int(w[i, l, e]) for i in range(count)) % ql
                assert int(got[b, l, e]) == want, (b, l, e)


# ------------------------------------------------------------- FLEXIBLEAUTO scale table
def _golden_chain():
    with open(os.path.join(GOLDEN, "openfhe_prime_chain_n131072.json")) as fh:
        gold = json.load(fh)
    return gold["primes"][: gold["num_q"]], gold["primes"][gold["num_q"]:]


def test_flexibleauto_scale_matches_openfhe_record():
    """The reference records OpenFHE's scaling factor of a degree-2
    ciphertext at level 35 of the 45-prime N=2^17 chain:
    results/b300/2026-09-28/long-accuracy/replay-controls-smoke/
    native.json.refresh-replay.json (inputs[0]: level 35, degree 2,
    scaling_factor 3.3230699877697935e+35).  The table must give exactly
    that double, and its neighbours must not (catches an off-by-one-prime
    recursion, which no decryption tolerance can see)."""
    from fhemamba_amd.ckks import flexibleauto_scaling_factors

    q, _ = _golden_chain()
    sf = flexibleauto_scaling_factors(q)
    assert len(sf) == len(q) and sf[0] == float(q[-1])
    recorded = 3.3230699877697935e+35
    assert sf[35] * sf[35] == recorded
    assert sf[34] * sf[34] != recorded and sf[36] * sf[36] != recorded


def test_classical128_audit_matches_openfhe_record():
    """The same run's security audit (native.json `security_audit`):
    ring 131072, q_bits 2656, p_bits 720, qp_bits 3376, 45 Q towers, 12 P
    towers, 4 digits, bound 3523, passed -- as fideslib_security.hpp:33-80
    computes it (exact bit lengths of Q, P and Q*P)."""
    from fhemamba_amd.ckks import SecretKeyDist, SecurityLevel, audit_chain

    q, p = _golden_chain()
    a = audit_chain(131072, q, p, 4, security_level=SecurityLevel.HEStd_128_classic,
                    secret_dist=SecretKeyDist.UNIFORM_TERNARY)
    assert (a["ring_dimension"], a["q_bits"], a["p_bits"], a["qp_bits"]) == (131072, 2656, 720,
                                                                            3376)
    assert (a["q_towers"], a["p_towers"], a["hybrid_digits"]) == (45, 12, 4)
    assert a["guideline_max_qp_bits"] == 3523 and a["passed"] is True
    sparse = audit_chain(131072, q, p, 4, security_level=SecurityLevel.HEStd_128_classic,
                         secret_dist=SecretKeyDist.SPARSE_TERNARY)
    assert sparse["passed"] is False and sparse["uniform_ternary"] is False
    # The same 45 + 12 chain at N=2^16 exceeds the 1747-bit bound.
    small = audit_chain(65536, q, p, 4, security_level=SecurityLevel.HEStd_128_classic,
                        secret_dist=SecretKeyDist.UNIFORM_TERNARY)
    assert small["guideline_max_qp_bits"] == 1747 and small["passed"] is False


def test_hoisted_rotation_equals_single_rotation(small_scheme):
    """A rotation from shared ModUp digits equals the full rotation (the
    precompute only moves the ModUp out of the loop)."""
    c, s = small_scheme[0], small_scheme[1]
    rng = np.random.default_rng(41)
    ct = np.stack([np.stack([rng.integers(0, q, c.n, dtype=np.uint64) for q in c.q])
                   for _ in range(2)])
    digits = c.modup(ct[1])
    for step in (1, -3):
        g = O.galois_elt(step, c.n)
        key = c.galois_key(s, g, 50 + step)
        assert np.array_equal(c.rotate_hoisted(ct, digits, key, g), c.rotate(ct, key, g))


def test_add_matches_big_integer_sum():
    """orc_add (EvalAdd per limb) against Python integers, including the
    largest residues (q - 1 + q - 1) and 61-bit moduli where a + b carries
    past 2^61."""
    q, p = O.gen_moduli(12, 5, 59, 61, 2)
    c = O.Ctx(12, q, p, 2)
    rng = np.random.default_rng(77)
    a = np.stack([np.stack([rng.integers(0, qj, c.n, dtype=np.uint64) for qj in q])
                  for _ in range(2)])
    b = np.stack([np.stack([rng.integers(0, qj, c.n, dtype=np.uint64) for qj in q])
                  for _ in range(2)])
    for j, qj in enumerate(q):
        a[:, j, :4] = qj - 1
        b[:, j, :4] = [qj - 1, 1, 0, qj - 2]
    got = c.add(a, b)
    for k in range(2):
        for j, qj in enumerate(q):
            want = [(int(x) + int(y)) % qj for x, y in zip(a[k, j], b[k, j])]
            assert [int(v) for v in got[k, j]] == want
