"""Encrypted Mamba-2 SSM layer step on the GPU (small shape: 8 heads x 8
channels x 16 states in 512 slots, two state groups), decrypted and checked
against the float64 reference step."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd.ckks_probes import build_toy_context  # noqa: E402
from fhemamba_amd.mamba2 import (DecayPolynomial, EncryptedSSMStep, SSMShape,  # noqa: E402
                                 expand_channels, expand_heads, expand_states, pack_state,
                                 ssm_step_reference, unpack_state)

from test_mamba2_step import model_inputs  # noqa: E402

SHAPE = SSMShape(nheads=8, headdim=8, d_state=16, slots=512)


def test_encrypted_ssm_step_matches_reference():
    s = SHAPE
    h, x, dt, A, B, C, D = model_inputs(s, 3)
    decay = DecayPolynomial(amax=float(np.max(-A * dt)) * 1.05, squarings=5, degree=13)
    cc, keys = build_toy_context(ring_dimension=1 << 12, batch=s.slots, depth=16,
                                 scale_bits=45, first_mod_bits=60, seed=77)
    step = EncryptedSSMStep(cc, keys, s, A, D, decay)
    cc.EvalRotateKeyGen(keys.secretKey, step.rotation_indices())

    def enc(v):
        return cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(v)))

    xc = np.zeros(s.slots)
    xc[: s.d_inner] = x.reshape(-1)
    state = [enc(v) for v in pack_state(h, s)]
    new_state, y = step(state, [enc(v) for v in expand_channels(x, s)],
                        [enc(v) for v in expand_heads(dt, s)], enc(expand_states(B, s)),
                        enc(expand_states(C, s)), enc(xc))

    def dec(ct):
        pt = cc.Decrypt(ct, keys.secretKey)
        pt.SetLength(s.slots)
        return np.asarray(pt.GetRealPackedValue())

    h2, y_ref = ssm_step_reference(h, x, dt, A, B, C, D)
    got_h = unpack_state([dec(c) for c in new_state], s)
    got_y = dec(y)
    assert np.max(np.abs(got_h - h2)) < 1e-4
    assert np.max(np.abs(got_y[: s.d_inner].reshape(s.nheads, s.headdim) - y_ref)) < 1e-4
    assert y.GetLevel() <= 16
