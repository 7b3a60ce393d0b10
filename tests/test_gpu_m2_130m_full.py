"""The Mamba-2-130M workloads at their full size on the GPU.

* The full encrypted decode of a 24-layer 130M-shaped model (d_model 768,
  d_inner 1536, 24 heads x 64, d_state 128, conv 4; seeded random-init
  weights and calibrated polynomials, mamba2_payload.synthetic_chain), a
  first token from zero state and a second with the carried SSM state and
  conv FIFO, decrypted and compared with the payload's polynomial circuit
  (chain_expected_poly_final) within 1e-3, the reference decoder's pass
  criterion for this payload family:
    - at the audited classical-128 setting (N = 2^17, 65536 slots, depth
      44, 45 Q + 12 P primes, four digits, uniform ternary secret): the
      reference's own classical-128 parameters.  The classical-128 setting
      at N = 2^16 with 24 working limbs has no parameter set (the 2^16
      bound is 1,747 bits of Q*P; 24 limbs of 59 bits plus a bootstrap's
      levels and the special primes need about twice that);
    - at N = 2^16, depth 44, security not set, sparse-ternary secret (the
      reference decoder's ring-65536 campaign setting).
* One encrypted SSM layer step at the 130M shape (24 heads x 64 channels x
  128 states in six 32768-slot state ciphertexts) at N = 2^16 with 24 limbs,
  against the float64 step (mamba2.ssm_step_reference).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd import mamba2_decode as D  # noqa: E402
from fhemamba_amd import mamba2_payload as M  # noqa: E402

from test_mamba2_step import model_inputs  # noqa: E402

TOL = 1e-3


def _decode(tmp_path, seed, **kw):
    print(f"[130m] building the 24-layer payload (seed {seed})", flush=True)
    M.synthetic_chain(str(tmp_path), n_layers=24, n_test_tokens=2, seed=seed)
    report = D.run_payload(str(tmp_path), seed=seed + 1, log=lambda m: None, **kw)
    print(f"[130m] {kw or 'not-set'}: {report['seconds_per_token']} s/token, "
          f"{report['bootstraps']} bootstraps, errors vs polynomial "
          f"{report['per_token_errors_vs_polynomial']}", flush=True)
    assert report["layers"] == 24 and report["tokens"] == 2
    assert len(report["per_token_errors_vs_polynomial"]) == 2
    assert report["max_abs_error_vs_polynomial"] < TOL
    return report


def test_24_layer_decode_classical128(tmp_path):
    report = _decode(tmp_path, 13, security="128-classic")
    a = report["security_audit"]
    assert report["ring_dimension"] == 131072 and report["slots"] == 65536
    assert a["passed"] and a["qp_bits"] == 3376 and a["hybrid_digits"] == 4
    assert report["secret_key_dist"] == "uniform-ternary"


def test_24_layer_decode_n65536(tmp_path):
    report = _decode(tmp_path, 23)
    assert report["ring_dimension"] == 65536 and report["slots"] == 32768
    assert report["secret_key_dist"] == "sparse-ternary"


def test_ssm_layer_step_at_130m_shape():
    from fhemamba_amd.ckks_probes import build_toy_context
    from fhemamba_amd.mamba2 import (DecayPolynomial, EncryptedSSMStep, SSMShape,
                                     expand_channels, expand_heads, expand_states, pack_state,
                                     ssm_step_reference, unpack_state)
    s = SSMShape()
    assert (s.nheads, s.headdim, s.d_state, s.slots) == (24, 64, 128, 32768)
    h, x, dt, A, B, C, Dp = model_inputs(s, 5)
    dt = np.clip(dt, 0.0, 6.0)
    # N = 2^16, 24 limbs (depth 23), 59-bit scale, 60-bit first prime
    cc, keys = build_toy_context(ring_dimension=1 << 16, batch=s.slots, depth=23,
                                 scale_bits=59, first_mod_bits=60, seed=11)
    assert len(cc.GetModuli()[0]) == 24
    step = EncryptedSSMStep(cc, keys, s, A, Dp, DecayPolynomial(amax=96.0, squarings=5,
                                                                degree=13))
    cc.EvalRotateKeyGen(keys.secretKey, step.rotation_indices())

    def enc(v):
        return cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(v)))

    xc = np.zeros(s.slots)
    xc[: s.d_inner] = x.reshape(-1)
    state = [enc(v) for v in pack_state(h, s)]
    assert len(state) == 6
    new_state, y = step(state, [enc(v) for v in expand_channels(x, s)],
                        [enc(v) for v in expand_heads(dt, s)], enc(expand_states(B, s)),
                        enc(expand_states(C, s)), enc(xc))

    def dec(ct):
        pt = cc.Decrypt(ct, keys.secretKey)
        pt.SetLength(s.slots)
        return np.asarray(pt.GetRealPackedValue())

    h2, y_ref = ssm_step_reference(h, x, dt, A, B, C, Dp)
    err_h = np.max(np.abs(unpack_state([dec(c) for c in new_state], s) - h2))
    err_y = np.max(np.abs(dec(y)[: s.d_inner].reshape(s.nheads, s.headdim) - y_ref))
    print(f"[130m] SSM step: state error {err_h:.2e}, output error {err_y:.2e}, "
          f"output level {y.GetLevel()}", flush=True)
    assert err_h < 1e-6 and err_y < 1e-6
    assert y.GetLevel() <= 23
