"""Encrypted Mamba-2 decode on the GPU of a payload written by the
reference's own exporter (tests/golden/m2_chain_tiny: export_chain_payload,
src/fhemamba/m1_payload.py:901, on the reference tests' tiny seeded
Mamba-2; two layers, two test tokens with carried state).  Pass criterion
as the exporter states it (m1_payload.py:1067) and the reference decoder
gates it: decrypted final hidden against chain_expected_poly_final within
1e-3 (the decoder's default --tolerance); measured errors are printed."""
import os

import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd import mamba2_decode as D  # noqa: E402

FIX = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny")
TOL = 1e-3


def test_reference_exported_payload_decodes_within_tolerance():
    report = D.run_payload(FIX, seed=31, log=lambda m: None)
    print(f"reference payload: {report['seconds_per_token']} s/token, errors vs polynomial "
          f"{report['per_token_errors_vs_polynomial']}, vs exact "
          f"{report['max_abs_error_vs_exact']:.2e}", flush=True)
    assert report["tokens"] == 2 and report["layers"] == 2
    assert report["max_abs_error_vs_polynomial"] < TOL


def test_reference_scheduled_normalization_payload_decodes():
    """The exporter's scheduled-normalization payload (Goldschmidt schedules
    for the block, gated and final norms) decoded on the GPU, two tokens
    with carried state, against its chain_expected_poly_final."""
    sched = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny_sched")
    report = D.run_payload(sched, seed=32, log=lambda m: None)
    print(f"scheduled payload: {report['seconds_per_token']} s/token, {report['bootstraps']} "
          f"bootstraps, errors vs polynomial {report['per_token_errors_vs_polynomial']}",
          flush=True)
    assert report["max_abs_error_vs_polynomial"] < TOL


@pytest.mark.parametrize("name", ["m2_chain_tiny_joint", "m2_chain_tiny_joint_cheb"])
def test_reference_joint_gate_payload_decodes(name):
    """The exporter's joint-gate payloads (constant gates of the reference
    tests' bundle; per-head degree-7 / degree-5 Chebyshev gates) decoded on
    the GPU, two tokens with carried state, against chain_expected_poly_final."""
    path = os.path.join(os.path.dirname(__file__), "golden", name)
    report = D.run_payload(path, seed=33, log=lambda m: None)
    print(f"{name}: {report['seconds_per_token']} s/token, {report['bootstraps']} bootstraps, "
          f"errors vs polynomial {report['per_token_errors_vs_polynomial']}", flush=True)
    assert report["max_abs_error_vs_polynomial"] < TOL


def test_reference_autoregressive_client_loop():
    """The exporter's client-in-loop assets on the GPU: three server
    evaluations (two prompt tokens, then the client's own greedy choice),
    each final hidden within the tolerance of the exporter's polynomial
    trace, and the client selects the exporter's greedy ids."""
    path = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny_ar")
    report = D.run_payload(path, seed=34, autoregressive=True, log=lambda m: None)
    print(f"client loop: selected {report['autoregressive_selected_ids']} expected "
          f"{report['autoregressive_expected_ids']}, errors vs polynomial "
          f"{report['per_token_errors_vs_polynomial']}", flush=True)
    assert report["tokens"] == 3
    assert report["autoregressive_tokens_match"]
    assert report["max_abs_error_vs_polynomial"] < TOL
