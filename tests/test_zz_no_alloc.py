"""fhe_rotate_noalloc through the C ABI: equal to fhe_rotate word for word.

Two calls in a row on one context (the second at a smaller level, so the
library's shared scratch array still holds the first call's data), then the
output-aliases-input form, with the library's allocation counter unchanged
across all of them; calls from two contexts (two streams) on one GPU issued
back to back without a synchronisation between them; then the rejections: a
shape above the scratch limit and a level whose conversion tables were never
built.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd._lib import FheError, call  # noqa: E402

FHE_ERR_ARG, FHE_ERR_STATE = 1, 4


def noalloc(out, ct, key, galois):
    call("fhe_rotate_noalloc", out.handle, ct.handle, key.handle, galois)


def alloc_count() -> int:
    n = ctypes.c_uint64()
    call("fhe_alloc_count", ctypes.byref(n))
    return n.value


@pytest.mark.gpu
@pytest.mark.parametrize("log_n,depth,dnum", [(13, 7, 2), (16, 23, 3)])
def test_noalloc_rotation_equals_fhe_rotate(log_n, depth, dnum):
    q, p = O.gen_moduli(log_n, depth, 59, 60, dnum)
    ctx = F.Context(log_n, q, p, dnum, sampling="seeded")
    print(f"[no-alloc] N=2^{log_n} L={ctx.L} K={ctx.K} dnum={dnum}", flush=True)
    rng = np.random.default_rng(log_n)
    s = ctx.keygen_secret(5)
    g1, g2 = F.galois_element(1, ctx.n), F.galois_element(-7, ctx.n)
    k1, k2 = ctx.keygen_galois(s, g1, 6), ctx.keygen_galois(s, g2, 7)
    big = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
    small_l = ctx.L - 3
    small = ctx.upload(residues(rng, ctx.q[:small_l], (2,), ctx.n))
    # allocating reference results (these also build each level's tables)
    want_big = ctx.rotate(big, k1, g1).numpy()
    want_small = ctx.rotate(small, k2, g2).numpy()
    out_big, out_small = ctx.poly(2, ctx.L), ctx.poly(2, small_l)
    alias = ctx.upload(small.numpy())
    before = alloc_count()
    noalloc(out_big, big, k1, g1)
    noalloc(out_small, small, k2, g2)
    noalloc(alias, alias, k2, g2)  # output aliasing the input
    ctx.sync()
    assert alloc_count() == before, "the no-allocation calls made an allocation request"
    assert np.array_equal(out_big.numpy(), want_big)
    assert np.array_equal(out_small.numpy(), want_small)
    assert np.array_equal(alias.numpy(), want_small)
    # an output of the wrong shape is refused, not reshaped
    with pytest.raises(FheError) as e:
        noalloc(ctx.poly(2, small_l), big, k1, g1)
    assert e.value.code == FHE_ERR_ARG
    ctx.close()


@pytest.mark.gpu
def test_noalloc_calls_from_two_contexts_are_ordered():
    """Two contexts on one GPU, each with its own stream, share the GPU's
    scratch array; their calls, issued back to back with no synchronisation
    between them, must still each equal fhe_rotate."""
    q, p = O.gen_moduli(16, 23, 59, 60, 3)
    ctxs = [F.Context(16, q, p, 3, sampling="seeded") for _ in range(2)]
    print(f"[no-alloc] two contexts, N=2^16 L={ctxs[0].L}", flush=True)
    rng = np.random.default_rng(99)
    cases = []
    for i, ctx in enumerate(ctxs):
        s = ctx.keygen_secret(10 + i)
        g = F.galois_element(2 * i + 1, ctx.n)
        key = ctx.keygen_galois(s, g, 20 + i)
        ct = ctx.upload(residues(rng, ctx.q, (2,), ctx.n))
        want = ctx.rotate(ct, key, g).numpy()
        cases.append((ctx, ct, key, g, want, ctx.poly(2, ctx.L)))
    for ctx, *_ in cases:
        ctx.sync()
    for _ in range(3):
        for ctx, ct, key, g, want, out in cases:
            noalloc(out, ct, key, g)
        for ctx, ct, key, g, want, out in cases:
            ctx.sync()
            assert np.array_equal(out.numpy(), want)
    for ctx, *_ in cases:
        ctx.close()


@pytest.mark.gpu
def test_noalloc_rotation_rejects_what_it_cannot_do():
    # tables never built at this level
    q, p = O.gen_moduli(13, 7, 59, 60, 2)
    ctx = F.Context(13, q, p, 2, sampling="seeded")
    s = ctx.keygen_secret(1)
    g = F.galois_element(3, ctx.n)
    key = ctx.keygen_galois(s, g, 2)
    ct = ctx.upload(residues(np.random.default_rng(1), ctx.q[:5], (2,), ctx.n))
    out = ctx.poly(2, 5)
    with pytest.raises(FheError) as e:
        noalloc(out, ct, key, g)
    assert e.value.code == FHE_ERR_STATE
    ctx.rotate(ct, key, g)
    noalloc(out, ct, key, g)
    ctx.close()
    # a shape above the 128 MiB scratch: N=2^16, 45 limbs, dnum 3
    q, p = O.gen_moduli(16, 44, 59, 60, 3)
    ctx = F.Context(16, q, p, 3, sampling="seeded")
    s = ctx.keygen_secret(1)
    g = F.galois_element(1, ctx.n)
    key = ctx.keygen_galois(s, g, 2)
    ct = ctx.upload(np.zeros((2, ctx.L, ctx.n), dtype=np.uint64))
    ctx.rotate(ct, key, g)
    with pytest.raises(FheError) as e:
        noalloc(ctx.poly(2, ctx.L), ct, key, g)
    assert e.value.code == FHE_ERR_ARG and "scratch" in str(e.value)
    ctx.close()
