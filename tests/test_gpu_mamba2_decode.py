"""Encrypted Mamba-2 decode on the GPU at the 130M shape (two layers of a
seeded random-init payload, N = 2^16, 32768 slots, depth 44): three tokens
with carried state (SSM state and conv FIFO ciphertexts), decrypted and
compared with the payload's polynomial-circuit reference.  Tolerance 1e-4
on the final normed hidden (values ~1); measured ~4e-6."""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd import mamba2_decode as D  # noqa: E402
from fhemamba_amd import mamba2_payload as M  # noqa: E402

TOL = 1e-4


def test_two_layer_decode_with_carried_state(tmp_path):
    M.synthetic_chain(str(tmp_path), n_layers=2, n_test_tokens=3, seed=3)
    report = D.run_payload(str(tmp_path), seed=4)
    print(f"decode: {report['seconds_per_token']} s/token, errors "
          f"{report['per_token_errors_vs_polynomial']}", flush=True)
    assert report["max_abs_error_vs_polynomial"] < TOL
    # two-pass refreshes at the precision-critical sites, one pass elsewhere
    r, b = report["logical_refreshes"], report["bootstraps"]
    assert r > 0 and r < b < 2 * r


def test_state_groups_refresh_together(tmp_path, monkeypatch):
    """Two layers decoded over ten tokens: the second layer's carried state
    deepens a level a token until its six groups reach the refresh ceiling
    together (the eighth carried token); they are refreshed by one
    multi-ciphertext bootstrap, and every token stays within the decode
    tolerance."""
    from fhemamba_amd import packed
    sizes = []
    orig = packed.PackedEvaluator.refresh_many

    def refresh_many(self, cts, *a, **k):
        sizes.append(len(cts))
        return orig(self, cts, *a, **k)

    monkeypatch.setattr(packed.PackedEvaluator, "refresh_many", refresh_many)
    M.synthetic_chain(str(tmp_path), n_layers=2, n_test_tokens=10, seed=15)
    report = D.run_payload(str(tmp_path), seed=16)
    print(f"ten-token decode: batched refresh sizes {sizes}, errors "
          f"{report['per_token_errors_vs_polynomial']}", flush=True)
    assert max(sizes, default=0) == 6
    assert report["max_abs_error_vs_polynomial"] < TOL


def test_command_line(tmp_path):
    M.synthetic_chain(str(tmp_path / "p"), n_layers=1, n_test_tokens=1, seed=5)
    res = tmp_path / "r.json"
    assert D.main([str(tmp_path / "p"), str(res), "--tolerance", str(TOL)]) == 0
    rep = json.loads(res.read_text())
    assert rep["passed"] is True and rep["schema"] == "fhemamba-m2-decode-result-v1"
    assert rep["layers"] == 1 and rep["ring_dimension"] == 65536
    assert D.main([str(tmp_path / "missing"), str(res)]) == 2


def test_joint_gate_decode_at_130m_shape(tmp_path):
    """One layer of the 130M shape with joint gates (per-head degree-15 p
    and degree-7 q over a shared basis, write = p^2 q^2, decay = 1 - p^2),
    two tokens with carried state, within the decode tolerance."""
    M.synthetic_chain(str(tmp_path), n_layers=1, n_test_tokens=2, seed=8,
                      joint_degrees=(15, 7))
    report = D.run_payload(str(tmp_path), seed=9)
    print(f"joint decode: {report['seconds_per_token']} s/token, errors "
          f"{report['per_token_errors_vs_polynomial']}", flush=True)
    assert report["max_abs_error_vs_polynomial"] < TOL


def test_classical128_two_layer_decode(tmp_path):
    """Two layers of the 130M-shape payload at the audited classical-128
    setting (N=2^17, 65536 slots, 45 Q + 12 P primes, four digits, uniform
    ternary secret; QP 3376 bits within the 3523-bit bound), two tokens
    with carried state, within the decode tolerance of the polynomial
    circuit."""
    M.synthetic_chain(str(tmp_path), n_layers=2, n_test_tokens=2, seed=6)
    report = D.run_payload(str(tmp_path), seed=7, security="128-classic")
    a = report["security_audit"]
    print(f"classical-128 decode: {report['seconds_per_token']} s/token, errors "
          f"{report['per_token_errors_vs_polynomial']}, audit {a}", flush=True)
    assert report["ring_dimension"] == 131072 and report["slots"] == 65536
    assert a["passed"] and a["qp_bits"] == 3376 and a["hybrid_digits"] == 4
    assert report["secret_key_dist"] == "uniform-ternary"
    assert report["max_abs_error_vs_polynomial"] < 1e-3
