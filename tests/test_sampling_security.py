"""Sampling streams of key generation and encryption (host, oracle).

* The ChaCha20 block function is pinned to RFC 8439's published test
  vectors; the oracle's ChaCha20 stream family is the checker the GPU
  sampling tests compare against.
* Threat check: with the seeded (parity) family, inverting SplitMix64 on
  one public key's `a` recovers the stream seed and from it the key's error
  `e`; with the ChaCha20 family (the library's default) the same attack
  finds nothing.
"""
import numpy as np
import pytest

import oracle as O

M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15
TAG_PK_A, TAG_PK_E = 2, 3


# ------------------------------------------------------------- RFC 8439 vectors
def test_chacha20_block_rfc8439_section_2_3_2():
    """RFC 8439 2.3.2: key 00..1f, counter 1, nonce 00:00:00:09:00:00:00:4a:00:00:00:00."""
    out = O.chacha20_block(bytes(range(32)), 1, bytes.fromhex("000000090000004a00000000"))
    assert out.hex() == (
        "10f1e7e4d13b5915500fdd1fa32071c4c7d1f4c733c068030422aa9ac3d46c4e"
        "d2826446079faa0914c2d705d98b02a2b5129cd1de164eb9cbd083e8a2503c4e")


def test_chacha20_block_rfc8439_appendix_a1_vector_1():
    """RFC 8439 A.1 test vector #1: all-zero key and nonce, counter 0."""
    out = O.chacha20_block(bytes(32), 0, bytes(12))
    assert out.hex() == (
        "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
        "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586")


def test_chacha20_block_counter_is_the_block_index():
    """The block after the 2.3.2 one (counter 2), as `openssl enc -chacha20`
    (OpenSSL 3.0.2) emits it for the same key and nonce."""
    out = O.chacha20_block(bytes(range(32)), 2, bytes.fromhex("000000090000004a00000000"))
    assert out.hex() == (
        "0a88837739d7bf4ef8ccacb0ea2bb9d69d56c394aa351dfda5bf459f0a2e9fe8"
        "e721f89255f9c486bf21679c683d4f9c5cf2fa27865526005b06ca374c86af3b")


def test_stream_words_follow_the_stated_derivation():
    """word i of stream (seed, tag, index) = little-endian 64-bit word i of
    ChaCha20(K1, nonce (tag, index, 1)) with K1 the first 32 bytes of
    ChaCha20Block(master, 0, (lo32 seed, hi32 seed, 0))."""
    master = bytes(range(100, 132))
    seed, tag, index = 0x0123456789ABCDEF, 0x200000 + (5 << 3) + 6, (2 << 16) | 7
    k1 = O.chacha20_block(master, 0, (seed & 0xFFFFFFFF).to_bytes(4, "little")
                          + (seed >> 32).to_bytes(4, "little") + bytes(4))[:32]
    nonce = tag.to_bytes(4, "little") + index.to_bytes(4, "little") + (1).to_bytes(4, "little")
    want = []
    for b in range(3):
        blk = O.chacha20_block(k1, b, nonce)
        want += [int.from_bytes(blk[8 * i: 8 * i + 8], "little") for i in range(8)]
    with O.sampling_key(master):
        got = [O.lib.orc_stream_word(seed, tag, index, i) for i in range(24)]
    assert got == want
    # outside the block the oracle is back on the seeded family
    assert O.lib.orc_stream_word(seed, tag, index, 0) == O.lib.orc_draw(
        O.lib.orc_stream_key(seed, tag, index), 0)


# ------------------------------------------------------------- inversion attack
def _unxorshift(z, s):
    x = z
    for _ in range(64 // s + 1):
        x = z ^ (x >> s)
    return x & M64


def unmix64(z):
    """Inverse of SplitMix64's finaliser fmix64."""
    z = _unxorshift(z, 31)
    z = (z * pow(0x94D049BB133111EB, -1, 1 << 64)) & M64
    z = _unxorshift(z, 27)
    z = (z * pow(0xBF58476D1CE4E5B9, -1, 1 << 64)) & M64
    return _unxorshift(z, 30)


def fmix64(z):
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _uniform(hi, lo, q):
    return (hi * q + ((lo * q) >> 64)) >> 64


def recover_seed_from_public_a(a0, a1, q):
    """Assume the seeded family: a0, a1 = the first two coefficients of the
    public key's `a` in limb 0 (uniform samples 0 and 1 of stream
    (seed, TAG_PK_A, 0)).  Enumerate the ~2^64 / q hidden words consistent
    with a0, invert fmix64, and keep the stream key that also reproduces
    a1; then invert the stream-key derivation.  None if no candidate fits."""
    lo_hi = (a0 << 64) // q
    hits = []
    for hi in range(max(0, lo_hi - 2), min(M64, lo_hi + (1 << 64) // q + 2) + 1):
        # some lo in [0, 2^64) must give a0 for this hi
        if not (_uniform(hi, 0, q) <= a0 <= _uniform(hi, M64, q)):
            continue
        key = (unmix64(hi) - GAMMA) & M64  # word 0 = fmix64(key + 1 * gamma)
        w2, w3 = fmix64((key + 3 * GAMMA) & M64), fmix64((key + 4 * GAMMA) & M64)
        if _uniform(w2, w3, q) == a1:
            hits.append(key)
    if len(hits) != 1:
        return None
    return unmix64(hits[0]) ^ fmix64((TAG_PK_A << 32) ^ 0 ^ 0x5851F42D4C957F2D)


@pytest.fixture(scope="module")
def scheme():
    log_n = 6
    q = O.ntt_friendly_primes(log_n, 59, 2)
    p = O.ntt_friendly_primes(log_n, 60, 1, skip=q)
    return O.Ctx(log_n, q, p, 2)


def _attack(c, pk_seed):
    s = c.secret(11)
    pk = c.public_key(s, pk_seed)
    a = pk[1]
    seed = recover_seed_from_public_a(int(a[0, 0]), int(a[0, 1]), c.q[0])
    # the key's actual error: b = e - a s, so e = b + a s (evaluation form)
    s_eval = c.signed_to_eval(s, 0, c.L)
    e_eval = np.stack([(pk[0, j].astype(object) + a[j].astype(object) * s_eval[j].astype(object))
                       % qj for j, qj in enumerate(c.q)]).astype(np.uint64)
    if seed is None:
        return None, e_eval
    ec = np.zeros(c.n, dtype=np.int64)
    O.lib.orc_sample_cbd(O.lib.orc_stream_key(seed, TAG_PK_E, 0), O.ptr(ec), c.n)
    return c.signed_to_eval(ec, 0, c.L), e_eval


def test_seeded_family_public_key_reveals_its_error(scheme):
    """The attack works on the seeded family (so the next test's negative
    result means something): one public key gives its seed and its e."""
    got, e_eval = _attack(scheme, pk_seed=0xC0FFEE1234)
    assert got is not None and np.array_equal(got, e_eval)


def test_chacha20_family_public_key_does_not_reveal_its_error(scheme):
    with O.sampling_key(bytes(range(7, 39))):
        got, e_eval = _attack(scheme, pk_seed=0xC0FFEE1234)
    assert got is None or not np.array_equal(got, e_eval)
