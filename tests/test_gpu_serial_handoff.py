"""Wire-format round trips on the GPU and the process-separated decode end
to end.

* Context, public key, secret key, ciphertext, multiplication key and
  rotation keys written and read back into a context rebuilt from the file:
  every residue equal, and operations with the loaded keys (relinearised
  product, rotation, conjugation) bit-exact against the originals.
* fhe_key_download is the inverse of fhe_key_load (standard form).
* The three roles (client-init, server-eval, client-decrypt) on the
  reference exporter's tiny payload at N = 2^12: the server loads no
  secret, the decrypted outputs meet the decode tolerance (1e-3) against
  chain_expected_poly_final, and a secret-named file under server/ fails
  the run."""
import json
import os
import stat

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd import ckks, serial as S  # noqa: E402
from fhemamba_amd import handoff as H  # noqa: E402
from fhemamba_amd import mamba2_decode as D  # noqa: E402
from fhemamba_amd.ckks_probes import build_toy_context  # noqa: E402

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_round_trips_into_a_rebuilt_context(tmp_path):
    cc, keys = build_toy_context(ring_dimension=1 << 12, batch=2048, depth=8, scale_bits=50,
                                 first_mod_bits=60, seed=5)
    cc.EvalRotateKeyGen(keys.secretKey, [1, -3, 17])
    cc.EvalConjugateKeyGen(keys.secretKey)
    x = np.random.default_rng(1).uniform(-1, 1, 2048)
    ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(x)))
    ct = cc.EvalMult(ct, ct)                               # degree 2, level 0
    p = {k: str(tmp_path / k) for k in ("cc", "pk", "sk", "ct", "mult", "rot")}
    assert ckks.SerializeToFile(p["cc"], cc) and ckks.SerializeToFile(p["pk"], keys.publicKey)
    assert ckks.SerializeToFile(p["sk"], keys.secretKey) and ckks.SerializeToFile(p["ct"], ct)
    assert cc.SerializeEvalMultKey(p["mult"]) and cc.SerializeEvalAutomorphismKey(p["rot"])
    cc2, ok = ckks.DeserializeCryptoContext(p["cc"])
    assert ok and cc2 is not cc and cc2.GetModuli() == cc.GetModuli()
    pk2, ok1 = ckks.DeserializePublicKey(p["pk"])
    sk2, ok2 = ckks.DeserializePrivateKey(p["sk"])
    ct2, ok3 = ckks.DeserializeCiphertext(p["ct"])
    assert ok1 and ok2 and ok3 and ct2.cc is cc2
    assert cc2.DeserializeEvalMultKey(p["mult"]) and cc2.DeserializeEvalAutomorphismKey(p["rot"])
    assert np.array_equal(pk2.poly.numpy(), keys.publicKey.poly.numpy())
    assert np.array_equal(sk2.s, keys.secretKey.s)
    assert np.array_equal(ct2.residues(), ct.residues())
    assert (ct2.GetLevel(), ct2.GetNoiseScaleDeg(), ct2.GetScalingFactor(), ct2.GetSlots()) == \
        (ct.GetLevel(), ct.GetNoiseScaleDeg(), ct.GetScalingFactor(), ct.GetSlots())
    assert sorted(cc2._galois) == sorted(cc._galois)
    for g in cc._galois:
        assert np.array_equal(cc2._galois[g].numpy(), cc._galois[g].numpy())
    # operations with the loaded keys in the rebuilt context: bit-exact
    a = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(x)))
    assert ckks.SerializeToFile(p["ct"], a)
    a2, _ = ckks.DeserializeCiphertext(p["ct"])
    pairs = [(cc.EvalMult(a, a), cc2.EvalMult(a2, a2)),
             (cc.EvalRotate(a, -3), cc2.EvalRotate(a2, -3)),
             (cc.EvalConjugate(a), cc2.EvalConjugate(a2))]
    for u, v in pairs:
        assert np.array_equal(u.residues(), v.residues())
    pt = cc2.Decrypt(cc2.EvalRotate(a2, 17), sk2)
    pt.SetLength(2048)
    assert np.max(np.abs(np.asarray(pt.GetRealPackedValue()) - np.roll(x, -17))) < 1e-6
    # a ciphertext of another context is refused by fingerprint
    other, _ = build_toy_context(ring_dimension=1 << 12, batch=2048, depth=6, scale_bits=50,
                                 first_mod_bits=60, seed=6)
    ct3, ok = ckks.DeserializeCiphertext(p["ct"], cc=other)
    assert ct3 is None and not ok and "another crypto context" in S.last_error()


def test_key_download_inverts_key_load():
    from fhemamba_amd.core import Context
    import oracle as O
    q = O.ntt_friendly_primes(12, 50, 4)
    p = O.ntt_friendly_primes(12, 60, 2, skip=q)
    ctx = Context(12, q, p, 2, sampling="seeded")
    rng = np.random.default_rng(3)
    mods = np.array(q + p, dtype=np.uint64)
    host = (rng.integers(0, 2 ** 63, size=(2, 2, 6, 4096), dtype=np.uint64) %
            mods[None, None, :, None])
    assert np.array_equal(ctx.load_key(host).numpy(), host)
    ctx.close()


def test_process_separated_decode(tmp_path):
    fix = os.path.join(GOLD, "m2_chain_tiny")
    root = str(tmp_path / "handoff")
    res = {r: str(tmp_path / f"{r}.json") for r in ("init", "eval", "dec")}
    common = ["--handoff-dir", root, "--ring-dim", "4096"]
    print("[handoff] client-init", flush=True)
    assert D.main([fix, res["init"], "--process-role", "client-init"] + common) == 0
    init = json.load(open(res["init"]))
    paths = H.HandoffPaths(root)
    assert sorted(os.listdir(paths.server)) == ["context.bin", "eval-mult.bin",
                                                "eval-rotation.bin", "handoff.json",
                                                "public-key.bin"]
    assert stat.S_IMODE(os.stat(os.path.join(paths.client, "secret-key.bin")).st_mode) == 0o600
    print(f"[handoff] server-eval ({init['automorphism_keys']} keys)", flush=True)
    assert D.main([fix, res["eval"], "--process-role", "server-eval", "--handoff-dir",
                   root]) == 0
    ev = json.load(open(res["eval"]))
    assert ev["server_secret_key_files"] == 0 and ev["encrypted_outputs_written"] == 2
    assert ev["measurement_scope"]["server_secret_key_loaded"] is False
    print("[handoff] client-decrypt", flush=True)
    assert D.main([fix, res["dec"], "--process-role", "client-decrypt", "--handoff-dir",
                   root]) == 0
    dec = json.load(open(res["dec"]))
    print(f"handoff: server {ev['seconds_per_token']} s/token, errors "
          f"{dec['per_token_max_abs_error']}", flush=True)
    assert dec["passed"] and dec["max_abs_error"] < 1e-3 and dec["per_token_decrypt_ok"] == [1, 1]
    # a secret-named file on the server side fails the client's verdict
    open(os.path.join(paths.server, "leaked-secret.bin"), "w").close()
    assert D.main([fix, res["dec"], "--process-role", "client-decrypt", "--handoff-dir",
                   root]) == 1
    assert json.load(open(res["dec"]))["server_secret_key_files"] == 1
