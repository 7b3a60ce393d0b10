"""The benchmark configurations at their stated shapes, residues checked
against the oracle.

Config 1 (the reference's toy plumbing case): N=2^13, eight 50-bit Q primes
q = 1 mod 2N and two special primes given explicitly, dnum 2; forward and
inverse NTT, HMult + relinearisation, rescale, rotations by +1 and +7, each
bit-exact.

Config 2 (raw RNS NTT / MAC batch): N=2^16, 24 limbs of 60-bit primes, 64
ciphertexts x 2 polys resident on the device at once (1.61 GB): forward NTT
of the whole batch, plaintext MAC over the 64 ciphertexts, inverse NTT.
The forward NTT is compared with the oracle on a sample of polys and limbs,
the MAC on sampled limbs (all 64 terms), and the inverse NTT of the whole
batch must give back the input word for word (iNTT(NTT(x)) = x over all
128 x 24 limbs).
"""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

pytestmark = pytest.mark.gpu
F = pytest.importorskip("fhemamba_amd")


def test_config1_stated_shape_bit_exact():
    log_n = 13
    q = O.ntt_friendly_primes(log_n, 50, 8)
    p = O.ntt_friendly_primes(log_n, 60, 2, skip=q)
    print(f"[config 1] N=2^13 Q={len(q)}x50-bit P={len(p)} dnum=2", flush=True)
    ctx = F.Context(log_n, q, p, 2, sampling="seeded")
    orc = O.Ctx(log_n, q, p, 2)
    assert (ctx.L, ctx.K, ctx.dnum) == (8, 2, 2)
    rng = np.random.default_rng(101)
    n = ctx.n
    # forward / inverse NTT of a two-poly ciphertext (limb-major [2][8][N])
    a = residues(rng, q, (2,), n)
    dev = ctx.upload(a)
    ctx.ntt_forward_dev(dev.data_ptr(), 2, 8)
    want = np.stack([np.stack([orc.ntt_fwd(a[b, j], j) for j in range(8)]) for b in range(2)])
    assert np.array_equal(dev.numpy(), want)
    ctx.ntt_inverse_dev(dev.data_ptr(), 2, 8)
    assert np.array_equal(dev.numpy(), a)
    # HMult + relinearize, rescale, rotations
    s = orc.secret(7)
    rk = orc.relin_key(s, 8)
    x, y = residues(rng, q, (2,), n), residues(rng, q, (2,), n)
    t3 = ctx.tensor(ctx.upload(x), ctx.upload(y))
    want3 = orc.tensor(x, y)
    assert np.array_equal(t3.numpy(), want3)
    prod = ctx.relinearize(t3, ctx.load_key(rk))
    want_prod = orc.relinearize(want3, rk)
    assert np.array_equal(prod.numpy(), want_prod)
    assert np.array_equal(ctx.rescale(prod).numpy(), orc.rescale(want_prod))
    for step in (1, 7):
        g = O.galois_elt(step, n)
        gk = orc.galois_key(s, g, 20 + step)
        assert np.array_equal(ctx.rotate(ctx.upload(x), ctx.load_key(gk), g).numpy(),
                              orc.rotate(x, gk, g)), step
    ctx.close()


def test_config2_full_batch():
    log_n, L, count = 16, 24, 64
    q = O.ntt_friendly_primes(log_n, 60, L)
    print(f"[config 2] N=2^16 L={L} {count} ciphertexts x 2 polys", flush=True)
    ctx = F.Context(log_n, q, [], 1, sampling="seeded")
    orc = O.Ctx(log_n, q, [], 1)
    n = ctx.n
    rng = np.random.default_rng(202)
    host = residues(rng, q, (2 * count,), n)          # [128][24][N]
    w_host = residues(rng, q, (count,), n)            # [64][24][N]
    x = ctx.upload(host)
    w = ctx.upload(w_host)
    acc = ctx.poly(2, L)
    ctx.ntt_forward_dev(x.data_ptr(), 2 * count, L)
    fx = x.numpy()
    # sampled polys x limbs against the oracle
    for poly in (0, 1, 77, 127):
        for j in (0, 9, 23):
            assert np.array_equal(fx[poly, j], orc.ntt_fwd(host[poly, j], j)), (poly, j)
    ctx.mac_dev(x.data_ptr(), w.data_ptr(), count, L, acc.data_ptr())
    got = acc.numpy()
    fxc = fx.reshape(count, 2, L, n)
    for j in (0, 13, 23):
        # the MAC of limb j alone, by an oracle context whose only modulus is q_j
        sub = O.Ctx(log_n, [q[j]], [], 1)
        want = sub.mac(np.ascontiguousarray(fxc[:, :, j:j + 1, :]),
                       np.ascontiguousarray(w_host[:, j:j + 1, :]))
        assert np.array_equal(got[:, j:j + 1, :], want), j
    ctx.ntt_inverse_dev(x.data_ptr(), 2 * count, L)
    assert np.array_equal(x.numpy(), host)
    ctx.close()
