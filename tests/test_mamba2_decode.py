"""Mamba-2 chain payloads and the encrypted decoder's circuit on the CPU:
payload write / read round trip and validation, the polynomial kinds against
the functions they approximate, the plain decode, and the decoder's
homomorphic operation sequence on a slot-level stand-in for the CKKS
context against the payload's polynomial-circuit reference."""
import json
import os

import numpy as np
import pytest

from fhemamba_amd import mamba2_payload as M
from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
from packed_builder import SlotContext, SlotKeys

SMALL = dict(d_model=64, d_inner=128, num_heads=4, head_dim=32, state_size=16)


@pytest.fixture(scope="module")
def chain(tmp_path_factory):
    d = tmp_path_factory.mktemp("chain")
    return str(d), M.synthetic_chain(str(d), n_layers=2, n_test_tokens=3, seed=1, **SMALL)


def test_payload_round_trip(chain):
    d, ch = chain
    again = M.read_chain_payload(d)
    assert again.n_layers == 2 and len(again.layers) == 2
    lay = again.layers[0]
    assert lay.proj_dim == 2 * 128 + 2 * 16 + 4 and lay.t("in_proj_w").shape == (292, 64)
    assert set(lay.polys) == set(M.SITES)
    assert lay.polys["decay_exp"].kind == "cheb-resquared"
    assert np.array_equal(again.input_embeddings, ch.input_embeddings)
    # the stored references are what the stored weights give (float32 storage)
    out, _ = M.decode_tokens(again, again.input_embeddings, True)
    assert np.max(np.abs(out - again.expected_poly_final)) < 1e-6


def test_polynomials_track_their_functions(chain):
    _, ch = chain
    lay = ch.layers[0]
    P = lay.polys
    for site, fn in (("conv_silu", M.silu), ("gate_silu", M.silu)):
        x = np.linspace(P[site].lo, P[site].hi, 1001)
        assert np.max(np.abs(P[site](x) - fn(x))) < 1e-6, site
    sp = P["dt_softplus"]
    x = np.linspace(sp.lo, sp.hi, 1001)
    assert np.max(np.abs(sp(x) - M.softplus(x)) / M.softplus(x)) < 1e-6
    de = P["decay_exp"]
    x = np.linspace(de.lo * 2 ** de.squarings, 0, 1001)
    assert np.max(np.abs(de(x) - np.exp(x))) < 1e-8
    rn = P["rms_invsqrt"]
    v = np.linspace(rn.lo * 2, rn.hi / 2, 1001)
    assert np.max(np.abs(rn(v) * np.sqrt(v) - 1)) < 1e-9


def test_plain_decode_polynomial_close_to_exact(chain):
    _, ch = chain
    assert np.max(np.abs(ch.expected_poly_final - ch.expected_final)) < 1e-5


def test_reader_rejects_bad_payloads(tmp_path, chain):
    d, _ = chain
    meta_path = os.path.join(d, "layer_00", "meta.json")
    meta = json.load(open(meta_path))
    bad = tmp_path / "bad"
    import shutil
    shutil.copytree(d, bad)
    for change, msg in ((("format", "fhemamba-m1-joint-v1"), "joint"),
                        (("format", "other"), "unexpected")):
        m = dict(meta)
        m[change[0]] = change[1]
        json.dump(m, open(bad / "layer_00" / "meta.json", "w"))
        with pytest.raises(ValueError, match=msg):
            M.read_chain_payload(str(bad))
    m = dict(meta)
    m["polys"] = dict(meta["polys"], rms_invsqrt={"kind": "scaled-goldschmidt-invsqrt-v1"})
    json.dump(m, open(bad / "layer_00" / "meta.json", "w"))
    # a scheduled recipe without its schedule is refused (the reference's check)
    with pytest.raises(ValueError, match="recipe"):
        M.read_chain_payload(str(bad))
    json.dump(meta, open(bad / "layer_00" / "meta.json", "w"))
    (bad / "layer_00" / "conv_b.bin").write_bytes(b"\0" * 12)
    with pytest.raises(ValueError, match="size mismatch"):
        M.read_chain_payload(str(bad))


def test_decoder_circuit_on_slots(chain):
    """Three tokens with carried state through the decoder's operation
    sequence (levels, refreshes and rotation keys checked by the stand-in)."""
    _, ch = chain
    cc = SlotContext(1024)
    dec = EncryptedMamba2Decoder(cc, SlotKeys(), ch)
    states = dec.initial_states()
    for k, e in enumerate(ch.input_embeddings):
        ct, states = dec.step(e, states)
        got = dec.decrypt(ct)
        assert np.max(np.abs(got - ch.expected_poly_final[k])) < 1e-6, k
    assert dec.ev.stats["logical_refreshes"] > 0
    assert all(len(s.ssm) == dec.groups and len(s.fifo) == 3 for s in states)
    # the state groups' rotate-sums ran in lockstep batches
    assert dec.groups > 1 and getattr(cc, "rotate_many_calls", 0) > 0


def test_decoder_rejects_shapes_that_do_not_pack(chain):
    _, ch = chain
    with pytest.raises(ValueError):
        EncryptedMamba2Decoder(SlotContext(256), SlotKeys(), ch)
