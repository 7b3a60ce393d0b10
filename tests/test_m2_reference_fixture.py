"""The Mamba-2 chain reader and plain decode against a payload written by the
reference's own exporter (tests/golden/m2_chain_tiny, made by
tests/golden/make_m2_chain_fixture.py: export_chain_payload,
src/fhemamba/m1_payload.py:901, on the reference tests' tiny seeded
Mamba-2).

* The payload reads (format, dims, polynomial kinds, carried bounds).
* Decoding its embeddings with the payload's polynomials reproduces the
  exporter's polynomial-circuit references: every layer's output and
  recurrent state (test_layer_output_poly, test_state_output_poly) and the
  final normed hidden (chain_expected_poly_final, the FHE pass criterion,
  m1_payload.py:1067).
* Decoding with the exact functions reproduces the exact-model references
  (chain_expected_final, test_layer_output, test_state_output) to float32
  precision of the exporter's torch forward.
"""
import json
import os

import numpy as np
import pytest

from fhemamba_amd import mamba2_payload as M

FIX = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny")


@pytest.fixture(scope="module")
def chain():
    return M.read_chain_payload(FIX)


def _layer_ref(i, name):
    d = os.path.join(FIX, f"layer_{i:02d}")
    meta = json.load(open(os.path.join(d, "meta.json")))
    return np.fromfile(os.path.join(d, name + ".bin"), dtype="<f4").reshape(
        meta["tensors"][name]).astype(np.float64)


def test_reads_reference_export(chain):
    assert chain.n_layers == 2 and chain.n_test_tokens == 2
    lay = chain.layers[0]
    assert (lay.d_model, lay.d_inner, lay.num_heads, lay.head_dim, lay.state_size,
            lay.conv_kernel) == (32, 64, 4, 16, 8, 4)
    assert {k: v.kind for k, v in lay.polys.items()} == {
        "conv_silu": "cheb", "gate_silu": "cheb", "dt_softplus": "cheb-squared",
        "decay_exp": "cheb-resquared", "rms_invsqrt": "poly-newton",
        "gated_rms_invsqrt": "sq-poly-newton"}
    assert chain.expected_poly_final is not None
    assert set(lay.bounds) >= {"residual", "proj", "y", "output"}


def _run(chain, polynomial):
    states = [M.zero_state(lay) for lay in chain.layers]
    layer_out = [[] for _ in chain.layers]
    layer_state = [[] for _ in chain.layers]
    finals = []
    for e in chain.input_embeddings:
        h = e
        for i, lay in enumerate(chain.layers):
            h, states[i] = M.layer_step(lay, h, states[i], polynomial)
            layer_out[i].append(h)
            layer_state[i].append(states[i].ssm)
        finals.append(M.final_norm(chain, h, polynomial))
    return np.array(finals), layer_out, layer_state


def _rel(got, want):
    return float(np.max(np.abs(np.asarray(got) - want)) / max(np.max(np.abs(want)), 1e-30))


def test_polynomial_circuit_matches_exporter(chain):
    finals, outs, sts = _run(chain, polynomial=True)
    assert _rel(finals, chain.expected_poly_final) < 1e-5
    for i in range(chain.n_layers):
        assert _rel(outs[i], _layer_ref(i, "test_layer_output_poly")[: chain.n_test_tokens]) < 1e-5
        assert _rel(sts[i], _layer_ref(i, "test_state_output_poly")[: chain.n_test_tokens]) < 1e-4


def test_exact_decode_matches_exporter(chain):
    finals, outs, sts = _run(chain, polynomial=False)
    assert _rel(finals, chain.expected_final) < 1e-5
    for i in range(chain.n_layers):
        assert _rel(outs[i], _layer_ref(i, "test_layer_output")[: chain.n_test_tokens]) < 1e-5
        assert _rel(sts[i], _layer_ref(i, "test_state_output")[: chain.n_test_tokens]) < 1e-4


def test_decoder_circuit_on_slots_meets_exporter_criterion(chain):
    """The encrypted decoder's operation sequence on the slot-level stand-in
    (tests/packed_builder.py) over the exporter's payload, two tokens with
    carried state: each final hidden equals chain_expected_poly_final."""
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
    from packed_builder import SlotContext, SlotKeys
    dec = EncryptedMamba2Decoder(SlotContext(1024), SlotKeys(), chain)
    states = dec.initial_states()
    for k, e in enumerate(chain.input_embeddings):
        ct, states = dec.step(e, states)
        got = dec.decrypt(ct)
        assert _rel(got, chain.expected_poly_final[k]) < 1e-5, k


# ------------------------------------------------------------- variants
SCHED = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny_sched")
JOINT = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny_joint")


def _ref(directory, name):
    meta = json.load(open(os.path.join(directory, "chain.json")))
    return np.fromfile(os.path.join(directory, name + ".bin"), dtype="<f4").reshape(
        meta["tensors"][name]).astype(np.float64)


def test_scheduled_normalization_payload():
    """The exporter's scheduled-normalization payload (the reference tests'
    plan_invsqrt bundle): block, gated and final norms read as
    scaled-goldschmidt-invsqrt-v1 recipes, the final norm from chain.json's
    final_norm_poly, and the polynomial decode reproduces the exporter's
    circuit (chain_expected_poly_final)."""
    ch = M.read_chain_payload(SCHED)
    for lay in ch.layers:
        assert lay.polys["rms_invsqrt"].kind == "scaled-goldschmidt-invsqrt-v1"
        assert lay.polys["gated_rms_invsqrt"].kind == "scaled-goldschmidt-invsqrt-v1"
    assert ch.final_norm_poly is not None and ch.final_norm_poly.hi == 200
    finals, _ = M.decode_tokens(ch, ch.input_embeddings, True)
    assert _rel(finals, ch.expected_poly_final) < 1e-5
    exact, _ = M.decode_tokens(ch, ch.input_embeddings, False)
    assert _rel(exact, ch.expected_final) < 1e-5


def test_scheduled_recipe_matches_inverse_square_root():
    """Each schedule meets its own relative-error target on its interval
    (the certificate's claim, normalization.py:173-210)."""
    ch = M.read_chain_payload(SCHED)
    spec = ch.final_norm_poly
    v = np.geomspace(spec.lo, spec.hi, 2001)
    assert np.max(np.abs(spec(v) * np.sqrt(v) - 1)) < spec.tolerance * 1.01


def test_scheduled_decoder_circuit_on_slots():
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
    from packed_builder import SlotContext, SlotKeys
    ch = M.read_chain_payload(SCHED)
    dec = EncryptedMamba2Decoder(SlotContext(1024), SlotKeys(), ch)
    states = dec.initial_states()
    for k, e in enumerate(ch.input_embeddings):
        ct, states = dec.step(e, states)
        assert _rel(dec.decrypt(ct), ch.expected_poly_final[k]) < 1e-5, k


def test_joint_gate_payload_is_refused():
    """The exporter's joint-gate payload (fhemamba-m2-chain-joint-v1 with
    fhemamba-m1-joint-v1 layers: shared-dissipation-factor gates in place of
    dt_softplus and decay_exp) is refused by format, not misread."""
    meta = json.load(open(os.path.join(JOINT, "chain.json")))
    assert meta["format"] == "fhemamba-m2-chain-joint-v1"
    with pytest.raises(ValueError, match="format"):
        M.read_chain_payload(JOINT)
    with pytest.raises(ValueError, match="joint"):
        M.read_layer_payload(os.path.join(JOINT, "layer_00"))
