"""GPU key generation and encryption with the ChaCha20 sampling family.

Under one fixed 32-byte master key, every key and ciphertext the library
draws equals the oracle's ChaCha20 restatement (whose block function is
pinned to RFC 8439's vectors in test_sampling_security.py), word for word.
A context created without a key draws its master key from OS entropy, so
two contexts give different secrets for the same per-call seed.
"""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

F = pytest.importorskip("fhemamba_amd")

MASTER = bytes(range(200, 232))


@pytest.fixture(scope="module", params=[(12, 3, 2), (13, 5, 3)])
def pair(request):
    log_n, depth, dnum = request.param
    q, p = O.gen_moduli(log_n, depth, 50, 60, dnum)
    ctx = F.Context(log_n, q, p, dnum, sampling="chacha20", sampling_key=MASTER)
    orc = O.Ctx(log_n, q, p, dnum)
    yield ctx, orc
    ctx.close()


@pytest.mark.gpu
def test_chacha20_keys_match_oracle(pair):
    ctx, orc = pair
    with O.sampling_key(MASTER):
        s_o = orc.secret(41)
        sp_o = orc.secret_sparse(42, 64)
        pk_o = orc.public_key(s_o, 43)
        g = F.galois_element(3, ctx.n)
        gk_o = orc.galois_key(s_o, g, 44)
        rk_o = orc.relin_key(s_o, 45)
    s = ctx.keygen_secret(41)
    assert np.array_equal(s, s_o)
    assert np.array_equal(ctx.keygen_secret_sparse(42, 64), sp_o)
    assert np.array_equal(ctx.keygen_public(s, 43).numpy(), pk_o)
    # switching keys live in Montgomery form on the device: compare them
    # through the key switches they perform
    rng = np.random.default_rng(3)
    ct = residues(rng, ctx.q, (2,), ctx.n)
    assert np.array_equal(ctx.rotate(ctx.upload(ct), ctx.keygen_galois(s, g, 44), g).numpy(),
                          orc.rotate(ct, gk_o, g))
    assert np.array_equal(ctx.keyswitch(ctx.upload(ct[1:]), ctx.keygen_relin(s, 45)).numpy(),
                          orc.keyswitch(ct[1], rk_o))
    # the seeded family differs from the secure one for the same seed
    assert not np.array_equal(orc.secret(41), s_o)


@pytest.mark.gpu
def test_chacha20_encryption_matches_oracle(pair):
    ctx, orc = pair
    rng = np.random.default_rng(4)
    m = residues(rng, ctx.q, (), ctx.n)
    with O.sampling_key(MASTER):
        s = orc.secret(51)
        pk = orc.public_key(s, 52)
        want = orc.encrypt(pk, m, 53)
    got = ctx.encrypt(ctx.upload(pk), ctx.upload(m[None]), 53)
    assert np.array_equal(got.numpy(), want)


@pytest.mark.gpu
def test_entropy_keyed_contexts_differ():
    q, p = O.gen_moduli(12, 3, 50, 60, 2)
    a = F.Context(12, q, p, 2)
    b = F.Context(12, q, p, 2)
    sa, sb = a.keygen_secret(7), b.keygen_secret(7)
    assert set(np.unique(sa)) <= {-1, 0, 1} and not np.array_equal(sa, sb)
    # the same context keeps one master key: equal seeds give equal draws
    assert np.array_equal(a.keygen_secret(7), sa)
    a.close()
    b.close()
