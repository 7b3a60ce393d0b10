"""fhe_rotate_noalloc through the C ABI: equal to fhe_rotate word for word.

Two calls in a row on one context (the second at a smaller level, so the
library's shared scratch array still holds the first call's data), then the
output-aliases-input form, then the rejections: a shape above the scratch
limit and a level whose conversion tables were never built.
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
    noalloc(out_big, big, k1, g1)
    noalloc(out_small, small, k2, g2)
    assert np.array_equal(out_big.numpy(), want_big)
    assert np.array_equal(out_small.numpy(), want_small)
    # output aliasing the input
    alias = ctx.upload(small.numpy())
    noalloc(alias, alias, k2, g2)
    assert np.array_equal(alias.numpy(), want_small)
    # an output of the wrong shape is refused, not reshaped
    with pytest.raises(FheError) as e:
        noalloc(ctx.poly(2, small_l), big, k1, g1)
    assert e.value.code == FHE_ERR_ARG
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
