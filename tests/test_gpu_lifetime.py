"""Handle lifetime and argument checks of the C ABI on a device.

* A context handle released (or garbage-collected) before its polys and
  keys: every handle shares ownership of the context, so the later
  finalisers and calls still find it alive.  Regression test for a host
  segfault where a poly's finaliser ran after its context was gone.
* Outputs that alias an input the call still has to read are refused with
  FHE_ERR_ARG before any kernel launch.
"""
import gc

import numpy as np
import pytest

import oracle as O
from gpu_helpers import residues

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd._lib import FheError  # noqa: E402

FHE_ERR_ARG = 1


def _ctx(log_n=12, depth=3, dnum=2):
    q, p = O.gen_moduli(log_n, depth, 40, 60, dnum)
    return F.Context(log_n, q, p, dnum, sampling="seeded"), q


@pytest.mark.gpu
def test_context_released_before_its_polys_and_keys():
    ctx, q = _ctx()
    host = residues(np.random.default_rng(1), q, (2,), ctx.n)
    a = ctx.upload(host)
    s = ctx.keygen_secret(1)
    key = ctx.keygen_relin(s, 2)
    b = ctx.add(a, a)
    ctx.close()
    del ctx
    gc.collect()
    # the polys and the key still hold the context: downloads work
    assert np.array_equal(a.numpy(), host)
    twice = b.numpy()
    for j, qj in enumerate(q):
        assert np.array_equal(twice[:, j], (host[:, j] * 2) % np.uint64(qj))
    del a, b, key
    gc.collect()


@pytest.mark.gpu
def test_context_collected_first_by_the_garbage_collector():
    ctx, q = _ctx()
    polys = [ctx.poly(2, len(q)) for _ in range(4)]
    cycle = {"ctx": ctx, "polys": polys}
    cycle["self"] = cycle  # only the cycle collector frees this
    del ctx, polys, cycle
    gc.collect()
    gc.collect()


@pytest.mark.gpu
def test_hoisted_rotation_rejects_aliased_outputs():
    ctx, q = _ctx()
    rng = np.random.default_rng(2)
    ct = ctx.upload(residues(rng, q, (2,), ctx.n))
    s = ctx.keygen_secret(3)
    g1, g2 = F.galois_element(1, ctx.n), F.galois_element(2, ctx.n)
    k1, k2 = ctx.keygen_galois(s, g1, 4), ctx.keygen_galois(s, g2, 5)
    digits = ctx.rotation_precompute(ct)
    before = digits.numpy()
    with pytest.raises(FheError) as e:
        ctx.rotate_hoisted(ct, digits, [k1], [g1], outs=[digits])
    assert e.value.code == FHE_ERR_ARG
    out = ctx.poly(2, len(q))
    with pytest.raises(FheError) as e:
        ctx.rotate_hoisted(ct, digits, [k1, k2], [g1, g2], outs=[out, out])
    assert e.value.code == FHE_ERR_ARG
    assert np.array_equal(digits.numpy(), before)
    # the same call with distinct outputs works
    o1, o2 = ctx.rotate_hoisted(ct, digits, [k1, k2], [g1, g2])
    assert np.array_equal(o1.numpy(), ctx.rotate(ct, k1, g1).numpy())
    assert np.array_equal(o2.numpy(), ctx.rotate(ct, k2, g2).numpy())


@pytest.mark.gpu
def test_plaintext_ops_reject_plaintext_output_of_another_shape():
    ctx, q = _ctx()
    rng = np.random.default_rng(3)
    ct = ctx.upload(residues(rng, q, (2,), ctx.n))
    pt_host = residues(rng, q, (1,), ctx.n)
    pt = ctx.upload(pt_host)
    for op in (ctx.mul_plain, ctx.add_plain):
        with pytest.raises(FheError) as e:
            op(ct, pt, out=pt)
        assert e.value.code == FHE_ERR_ARG
        assert np.array_equal(pt.numpy(), pt_host)
    # same shape: in place on the plaintext is allowed
    one = ctx.upload(pt_host)
    ctx.mul_plain(one, pt, out=pt)
    want = np.stack([(pt_host[0, j].astype(object) * pt_host[0, j].astype(object)) % qj
                     for j, qj in enumerate(q)]).astype(np.uint64)
    assert np.array_equal(pt.numpy()[0], want)
