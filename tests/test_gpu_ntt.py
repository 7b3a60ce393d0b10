"""NTT / inverse NTT on the GPU, word-for-word against the CPU oracle."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import edge_patterns, residues

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")


@pytest.fixture(scope="module", params=[10, 12, 13, 14, 15, 16, 17])
def pair(request):
    log_n = request.param
    q = O.ntt_friendly_primes(log_n, 60, 3)
    p = O.ntt_friendly_primes(log_n, 59, 2)
    ctx = F.Context(log_n, q, p, 2, sampling="seeded")
    orc = O.Ctx(log_n, q, p, 2)
    return log_n, ctx, orc


def test_forward_inverse_match_oracle(pair):
    log_n, ctx, orc = pair
    n = 1 << log_n
    rng = np.random.default_rng(log_n)
    x = residues(rng, ctx.mods, (2,), n)  # 2 polys x 5 limbs (Q then P moduli)
    dev = ctx.upload(x.reshape(2, -1, n))
    ctx.ntt_forward_dev(dev.data_ptr(), 2, len(ctx.mods), 0)
    got = dev.numpy()
    want = orc.ntt_fwd_batch(x, 0)
    assert np.array_equal(got, want)
    ctx.ntt_inverse_dev(dev.data_ptr(), 2, len(ctx.mods), 0)
    assert np.array_equal(dev.numpy(), x)
    back = orc.ntt_inv_batch(want, 0)
    assert np.array_equal(back, x)


def test_edge_patterns_and_limb_offset(pair):
    log_n, ctx, orc = pair
    n = 1 << log_n
    mods = ctx.mods[2:]  # limbs start at modulus index 2
    x = edge_patterns(mods, n)
    dev = ctx.upload(x)
    ctx.ntt_forward_dev(dev.data_ptr(), 4, len(mods), 2)
    assert np.array_equal(dev.numpy(), orc.ntt_fwd_batch(x, 2))
    ctx.ntt_inverse_dev(dev.data_ptr(), 4, len(mods), 2)
    assert np.array_equal(dev.numpy(), x)


def test_inverse_of_unreduced_style_inputs(pair):
    """Inverse NTT of arbitrary residues matches the oracle (not only of
    forward outputs)."""
    log_n, ctx, orc = pair
    n = 1 << log_n
    rng = np.random.default_rng(100 + log_n)
    x = residues(rng, ctx.mods[:3], (1,), n)
    dev = ctx.upload(x)
    ctx.ntt_inverse_dev(dev.data_ptr(), 1, 3, 0)
    assert np.array_equal(dev.numpy(), orc.ntt_inv_batch(x, 0))
