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


def test_out_proj_diagonals_encoded_at_one_level(chain, monkeypatch):
    """The carried state deepens the gated norm's input a level a token;
    aligned to one level before out_proj, its diagonals are looked up at
    that level on every token (encoded once), while the slot-level values
    stay equal to the exporter's polynomial circuit."""
    from fhemamba_amd import packed
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
    from packed_builder import SlotContext, SlotKeys
    seen: dict = {}
    orig = packed.PlaintextCache.get

    def get(self, key):
        if isinstance(key, tuple) and len(key) == 3 and key[1] == "replicated":
            seen.setdefault(key[0][0], set()).add(key[2])
        return orig(self, key)

    monkeypatch.setattr(packed.PlaintextCache, "get", get)
    dec = EncryptedMamba2Decoder(SlotContext(1024), SlotKeys(), chain)
    states = dec.initial_states()
    state_levels = []
    for k, e in enumerate(chain.input_embeddings):
        ct, states = dec.step(e, states)
        state_levels.append(max(s.ssm[0].GetLevel() for s in states if s.ssm))
        assert _rel(dec.decrypt(ct), chain.expected_poly_final[k]) < 1e-5, k
    assert len(chain.input_embeddings) >= 2 and len(set(state_levels)) > 1
    assert seen["out_proj"] == {dec.ev.refresh_ceiling - 4}


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


JOINT_CHEB = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny_joint_cheb")


def _layer_ref_in(directory, i, name):
    d = os.path.join(directory, f"layer_{i:02d}")
    meta = json.load(open(os.path.join(d, "meta.json")))
    return np.fromfile(os.path.join(d, name + ".bin"), dtype="<f4").reshape(
        meta["tensors"][name]).astype(np.float64)


@pytest.mark.parametrize("directory", [JOINT, JOINT_CHEB], ids=["constant", "chebyshev"])
def test_joint_gate_payload_decodes_like_exporter(directory):
    """The exporter's joint-gate payloads (fhemamba-m2-chain-joint-v1 with
    fhemamba-m1-joint-v1 layers: shared-dissipation-factor gates in place of
    dt_softplus and decay_exp): the gates read degree-major, head-minor, and
    the polynomial decode reproduces every layer's output and state and the
    final hidden of the exporter's own circuit; the exact decode its
    exact-model references."""
    meta = json.load(open(os.path.join(directory, "chain.json")))
    assert meta["format"] == "fhemamba-m2-chain-joint-v1"
    ch = M.read_chain_payload(directory)
    for lay in ch.layers:
        assert lay.joint is not None and lay.joint.heads == lay.num_heads
        assert np.allclose(lay.joint.rates, np.exp(lay.t("a_log")), rtol=2e-7)
    finals, outs, sts = _run(ch, polynomial=True)
    assert _rel(finals, ch.expected_poly_final) < 1e-5
    for i in range(ch.n_layers):
        assert _rel(outs[i], _layer_ref_in(directory, i, "test_layer_output_poly")) < 1e-5
        assert _rel(sts[i], _layer_ref_in(directory, i, "test_state_output_poly")) < 1e-4
    exact, _, _ = _run(ch, polynomial=False)
    assert _rel(exact, ch.expected_final) < 1e-5


def test_constant_joint_gate_values():
    """The reference tests' constant gate bundle (p = 0.5, q = 0.75 on every
    head) gives write 0.140625 and decay 0.75 for any input, the values the
    reference's own test asserts (tests/test_scheduled_payload.py:95-102)."""
    gate = M.read_chain_payload(JOINT).layers[0].joint
    write, decay = gate(np.array([[0.0] * 4, [-3.0, 1.0, 7.5, -20.0]]))
    assert np.array_equal(write, np.full((2, 4), 0.140625))
    assert np.array_equal(decay, np.full((2, 4), 0.75))


def test_chebyshev_joint_gate_against_power_series():
    """The degree-7 / degree-5 gates evaluated through the power basis
    (numpy's cheb2poly, then Horner) at points inside and outside each
    head's domain: the Chebyshev evaluation and the head-minor layout agree;
    decay = 1 - p^2 stays in [0, 1] on the domain (|p| <= sum |p_k| <= 1)."""
    gate = M.read_chain_payload(JOINT_CHEB).layers[1].joint
    rng = np.random.default_rng(5)
    z = gate.lo + (gate.hi - gate.lo) * rng.uniform(-0.2, 1.2, (64, gate.heads))
    write, decay = gate(z)
    t = (2 * z - (gate.lo + gate.hi)) / (gate.hi - gate.lo)
    for h in range(gate.heads):
        p = np.polyval(np.polynomial.chebyshev.cheb2poly(gate.p[:, h])[::-1], t[:, h])
        q = np.polyval(np.polynomial.chebyshev.cheb2poly(gate.q[:, h])[::-1], t[:, h])
        np.testing.assert_allclose(write[:, h], p * p * q * q, rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(decay[:, h], 1 - p * p, rtol=1e-9, atol=1e-12)
    inside = (t >= -1) & (t <= 1)
    assert np.all((decay[inside] >= 0) & (decay[inside] <= 1))
    assert np.all(np.abs(gate.p).sum(axis=0) <= 1)


@pytest.mark.parametrize("directory", [JOINT, JOINT_CHEB], ids=["constant", "chebyshev"])
def test_joint_decoder_circuit_on_slots(directory):
    """The encrypted decoder's joint-gate circuit (per-head affine map, the
    vector-coefficient Paterson-Stockmeyer p and q over one basis, write and
    decay) on the slot-level stand-in, two tokens with carried state,
    against chain_expected_poly_final."""
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
    from packed_builder import SlotContext, SlotKeys
    ch = M.read_chain_payload(directory)
    dec = EncryptedMamba2Decoder(SlotContext(1024), SlotKeys(), ch)
    states = dec.initial_states()
    for k, e in enumerate(ch.input_embeddings):
        ct, states = dec.step(e, states)
        assert _rel(dec.decrypt(ct), ch.expected_poly_final[k]) < 1e-5, k


def _copy_with(tmp_path, edit_layer=None, edit_chain=None):
    import shutil
    dst = tmp_path / "p"
    shutil.copytree(JOINT_CHEB, dst)
    if edit_layer:
        path = dst / "layer_00" / "meta.json"
        meta = json.loads(path.read_text())
        edit_layer(meta)
        path.write_text(json.dumps(meta))
    if edit_chain:
        path = dst / "chain.json"
        meta = json.loads(path.read_text())
        edit_chain(meta)
        path.write_text(json.dumps(meta))
    return str(dst)


def _set(d, key, value):
    d[key] = value


@pytest.mark.parametrize("edit, match", [
    (lambda m: _set(m["joint_gates"], "kind", "other"), "recipe"),
    (lambda m: _set(m["joint_gates"], "coefficient_layout", "head-major"), "recipe"),
    (lambda m: _set(m["joint_gates"], "p", m["joint_gates"]["p"][:-1]), "matrix shape"),
    (lambda m: _set(m["joint_gates"], "lo", m["joint_gates"]["hi"]), "domain"),
    (lambda m: _set(m["joint_gates"], "rates", [2 * r for r in m["joint_gates"]["rates"]]),
     "rates"),
    (lambda m: _set(m["joint_gates"], "rates", m["joint_gates"]["rates"][:2]), "per head"),
    (lambda m: _set(m["joint_gates"], "q", ["x"] + m["joint_gates"]["q"][1:]), "numeric"),
    (lambda m: _set(m["polys"]["decay_exp"], "head_mask", [1, 0, 1, 1]), "retain all heads"),
    (lambda m: _set(m, "format", "fhemamba-m1-v1"), "versioned joint format"),
    (lambda m: m.pop("joint_gates"), "recipe"),
])
def test_joint_gate_payload_checks(tmp_path, edit, match):
    """Malformed joint payloads are refused with the reference reader's
    reasons (stage1_joint_gates.hpp:51-66, stage1_mamba2_payload.cpp:208-230,
    :293-317; rates against the layer's A as ops.py:557-560)."""
    with pytest.raises(ValueError, match=match):
        M.read_chain_payload(_copy_with(tmp_path, edit_layer=edit))


def test_unknown_chain_format_is_refused(tmp_path):
    with pytest.raises(ValueError, match="format"):
        M.read_chain_payload(_copy_with(tmp_path, edit_chain=lambda m: _set(
            m, "format", "fhemamba-m3-chain-v1")))


def test_synthetic_joint_chain_round_trip(tmp_path):
    """The synthetic writer's joint payloads (per-head fits of the exact
    gates) read back to the same gates and format, and their polynomial
    decode stays near the exact model's."""
    ch = M.synthetic_chain(str(tmp_path), n_layers=2, n_test_tokens=2, seed=3, d_model=64,
                           d_inner=128, num_heads=8, head_dim=16, state_size=16,
                           joint_degrees=(15, 7))
    meta = json.load(open(tmp_path / "chain.json"))
    assert meta["format"] == "fhemamba-m2-chain-joint-v1"
    g = ch.layers[1].joint
    assert g.p.shape == (16, 8) and g.q.shape == (8, 8)
    again = M.read_chain_payload(str(tmp_path)).layers[1].joint
    assert np.array_equal(again.p, g.p) and np.array_equal(again.lo, g.lo)
    assert _rel(ch.expected_poly_final, ch.expected_final) < 1e-3


# ------------------------------------------------------------- client loop
AR = os.path.join(os.path.dirname(__file__), "golden", "m2_chain_tiny_ar")


def test_autoregressive_assets_read():
    """The exporter's client-in-loop assets (tests/test_scheduled_payload.py's
    export: two prompt tokens, two generated): protocol, counts, untied
    lm_head, tensor shapes."""
    ar = M.read_chain_payload(AR).autoregressive
    assert (ar.prompt_tokens, ar.generate_tokens, ar.server_evaluations) == (2, 2, 3)
    assert ar.vocab == 97 and ar.lm_head_w is not None and ar.lm_head_b is None
    assert ar.embeddings.shape == (3, 32) and len(ar.expected_ids) == 2
    # the evaluated embeddings are the table's rows of the evaluated ids
    meta = json.load(open(os.path.join(AR, "chain.json")))["autoregressive"]
    for k, tok in enumerate(meta["poly_evaluated_ids"]):
        assert np.array_equal(ar.embeddings[k], ar.embedding_w[tok])


@pytest.mark.parametrize("polynomial", [True, False])
def test_autoregressive_plain_loop_selects_exporter_ids(polynomial):
    """The plain client loop reproduces the exporter's traces: the final
    hiddens of the polynomial (exact) circuit and the greedy ids it chose."""
    ch = M.read_chain_payload(AR)
    ar = ch.autoregressive
    finals, ids = M.autoregressive_decode(ch, polynomial)
    meta = json.load(open(os.path.join(AR, "chain.json")))["autoregressive"]
    want = ar.expected_poly_final if polynomial else ar.expected_exact_final
    assert _rel(finals, want) < 1e-5
    assert ids == meta["poly_generated_ids" if polynomial else "exact_generated_ids"]


def test_autoregressive_client_loop_on_slots():
    """The decoder's token loop with the client in it, on the slot-level
    stand-in: every server evaluation matches the polynomial trace and the
    client selects the exporter's ids (the third input is the client's own
    choice, not a stored embedding)."""
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder, token_loop
    from packed_builder import SlotContext, SlotKeys
    ch = M.read_chain_payload(AR)
    dec = EncryptedMamba2Decoder(SlotContext(1024), SlotKeys(), ch)
    out = token_loop(dec, ch, ch.autoregressive.server_evaluations, ch.autoregressive,
                     log=lambda m: None)
    assert out["selected"] == ch.autoregressive.expected_ids
    assert max(out["errors_poly"]) < 1e-5


def test_autoregressive_selection_rules():
    """Greedy choice: first maximal logit, bias added, tied head uses the
    embedding table, non-finite logits refused; a missing client choice is
    refused."""
    emb = np.array([[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]])
    mk = lambda head, bias: M.AutoregressiveAssets(  # noqa: E731
        1, 2, 2, [0], [2, 2], emb, head, bias, emb[:2], emb[:2], emb[:2])
    assert mk(None, None).select([1.0, 1.0]) == 2
    assert mk(None, np.array([0.0, 0.0, -1.0])).select([1.0, 1.0]) == 0   # tie: first
    assert mk(emb[::-1].copy(), None).select([1.0, 0.0]) == 0
    with pytest.raises(ValueError, match="non-finite"):
        mk(None, None).select([np.inf, 0.0])
    with pytest.raises(ValueError, match="missing"):
        mk(None, None).input_for(1, [])


@pytest.mark.parametrize("edit, match", [
    (lambda m: _set(m["autoregressive"], "protocol", "sampled"), "protocol"),
    (lambda m: _set(m["autoregressive"], "server_evaluations", 4), "evaluation count"),
    (lambda m: _set(m["autoregressive"], "poly_generated_ids", [85]), "shape"),
    (lambda m: _set(m["autoregressive"], "poly_generated_ids", [85, 97]), "shape"),
])
def test_autoregressive_payload_checks(tmp_path, edit, match):
    import shutil
    dst = tmp_path / "p"
    shutil.copytree(AR, dst)
    meta = json.loads((dst / "chain.json").read_text())
    edit(meta)
    (dst / "chain.json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match=match):
        M.read_chain_payload(str(dst))


def test_autoregressive_command_line_refusals(tmp_path):
    """--autoregressive-client-loop on a payload without assets, or with a
    truncated chain, exits 2 before any device work."""
    from fhemamba_amd import mamba2_decode as D
    res = str(tmp_path / "r.json")
    assert D.main([FIX, res, "--autoregressive-client-loop"]) == 2
    assert D.main([AR, res, "--autoregressive-client-loop", "--layers", "1"]) == 2
    assert D.main([AR, res, "--autoregressive-client-loop", "--tokens", "4"]) == 2
    assert D.main([FIX, res, "--tokens", "3"]) == 2


def test_s2c_first_decoder_circuit_on_slots(chain):
    """With S2C-first refreshes the ceiling is the SlotToCoeff levels lower
    and refreshed values come back that much higher; the decoder's level
    planning still reaches the exporter's circuit."""
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
    from packed_builder import SlotContext, SlotKeys
    dec = EncryptedMamba2Decoder(SlotContext(1024), SlotKeys(), chain, s2c_first=True)
    assert dec.ev.refresh_ceiling == 45 - 3 - 4
    states = dec.initial_states()
    for k, e in enumerate(chain.input_embeddings):
        ct, states = dec.step(e, states)
        assert _rel(dec.decrypt(ct), chain.expected_poly_final[k]) < 1e-5, k
