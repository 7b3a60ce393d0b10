"""Mamba-2 SSM layer step: packing, float64 reference, decay polynomial, and
the encrypted circuit run on a slot-level array backend (host only; the GPU
run is tests/test_gpu_mamba2.py)."""
import itertools
from types import SimpleNamespace

import numpy as np
import pytest

from fhemamba_amd.mamba2 import (DecayPolynomial, EncryptedSSMStep, SSMShape, expand_channels,
                                 expand_heads, expand_states, pack_state, ssm_step_reference,
                                 unpack_state)


class SlotBackend:
    """Slot vectors in place of ciphertexts: the circuit's data movement
    (masks, rotations, replication) without encryption."""

    def __init__(self, slots):
        self.slots = slots
        self.rotations = []

    def _v(self, x):
        return x if isinstance(x, np.ndarray) else np.full(self.slots, float(x))

    def MakeCKKSPackedPlaintext(self, values):  # noqa: N802
        v = np.zeros(self.slots)
        v[: len(values)] = values
        return v

    def Encrypt(self, key, v):  # noqa: N802
        return v.copy()

    def EvalMult(self, a, b):  # noqa: N802
        return self._v(a) * self._v(b)

    def EvalAdd(self, a, b):  # noqa: N802
        return self._v(a) + self._v(b)

    def EvalSub(self, a, b):  # noqa: N802
        return self._v(a) - self._v(b)

    def EvalSquare(self, a):  # noqa: N802
        return a * a

    def EvalRotate(self, a, k):  # noqa: N802
        self.rotations.append(k)
        return np.roll(a, -k)


def model_inputs(shape, seed):
    rng = np.random.default_rng(seed)
    h = rng.normal(0, 0.5, (shape.nheads, shape.headdim, shape.d_state))
    x = np.clip(rng.normal(0, 1, (shape.nheads, shape.headdim)), -8, 8)
    dt = np.log1p(np.exp(rng.normal(0, 1, shape.nheads)))      # softplus
    A = -np.exp(rng.uniform(0, np.log(16), shape.nheads))
    B = rng.normal(0, 0.3, shape.d_state)
    C = rng.normal(0, 0.3, shape.d_state)
    D = rng.normal(0, 1, shape.nheads)
    return h, x, dt, A, B, C, D


SMALL = SSMShape(nheads=8, headdim=8, d_state=16, slots=512)


def test_shape_arithmetic():
    s = SSMShape()
    assert (s.heads_per_ct, s.group_block, s.groups, s.d_inner) == (4, 256, 6, 1536)
    assert (SMALL.heads_per_ct, SMALL.group_block, SMALL.groups) == (4, 32, 2)
    with pytest.raises(ValueError):
        SSMShape(nheads=5, headdim=8, d_state=16, slots=512)


def test_packing_roundtrip_and_layout():
    s = SMALL
    h = np.arange(s.nheads * s.headdim * s.d_state, dtype=float).reshape(
        s.nheads, s.headdim, s.d_state)
    vecs = pack_state(h, s)
    assert np.array_equal(unpack_state(vecs, s), h)
    for g, v in enumerate(vecs):
        for hl, p, n in itertools.product(range(s.heads_per_ct), range(s.headdim),
                                          range(s.d_state)):
            assert v[n * s.group_block + hl * s.headdim + p] == h[g * s.heads_per_ct + hl, p, n]
    x = np.arange(s.nheads * s.headdim, dtype=float).reshape(s.nheads, s.headdim)
    xe = expand_channels(x, s)
    assert xe[1][3 * s.group_block + 2 * s.headdim + 5] == x[s.heads_per_ct + 2, 5]
    de = expand_heads(np.arange(s.nheads), s)
    assert de[1][7 * s.group_block + 3 * s.headdim + 1] == s.heads_per_ct + 3
    be = expand_states(np.arange(s.d_state), s)
    assert be[5 * s.group_block + 17] == 5


def test_reference_matches_loops():
    s = SSMShape(nheads=4, headdim=3, d_state=4, slots=48)
    h, x, dt, A, B, C, D = model_inputs(s, 1)
    h2, y = ssm_step_reference(h, x, dt, A, B, C, D)
    for hh, p, n in itertools.product(range(4), range(3), range(4)):
        want = np.exp(dt[hh] * A[hh]) * h[hh, p, n] + dt[hh] * x[hh, p] * B[n]
        assert h2[hh, p, n] == pytest.approx(want, rel=1e-14, abs=1e-14)
    for hh, p in itertools.product(range(4), range(3)):
        want = sum(h2[hh, p, n] * C[n] for n in range(4)) + D[hh] * x[hh, p]
        assert y[hh, p] == pytest.approx(want, rel=1e-12, abs=1e-12)


def test_decay_polynomial_accuracy():
    d = DecayPolynomial(amax=96.0, squarings=5, degree=13)
    t = np.linspace(-96, 0, 20001)
    assert np.max(np.abs(d.plain(t) - np.exp(t))) < 1e-9
    # the interpolant variable spans [-1, 1] exactly on the domain
    assert d.u_scale() * -96 + 1 == pytest.approx(-1.0)
    assert d.depth() >= 1 + 4 + 5


def test_encrypted_circuit_on_slot_backend():
    s = SMALL
    h, x, dt, A, B, C, D = model_inputs(s, 2)
    be = SlotBackend(s.slots)
    step = EncryptedSSMStep(be, SimpleNamespace(publicKey=None), s, A, D,
                            DecayPolynomial(amax=float(np.max(-A * dt)) + 1, squarings=4,
                                            degree=13))
    xc = np.zeros(s.slots)
    xc[: s.d_inner] = x.reshape(-1)
    new_state, y = step(pack_state(h, s), expand_channels(x, s), expand_heads(dt, s),
                        expand_states(B, s), expand_states(C, s), xc)
    h2, y_ref = ssm_step_reference(h, x, dt, A, B, C, D)
    np.testing.assert_allclose(unpack_state(new_state, s), h2, atol=1e-8)
    np.testing.assert_allclose(y[: s.d_inner].reshape(s.nheads, s.headdim), y_ref, atol=1e-8)
    np.testing.assert_allclose(y[s.d_inner:], 0, atol=1e-12)
    assert sorted(set(step.rotation_indices())) == sorted(set(be.rotations))
