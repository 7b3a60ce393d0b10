"""Wire format and handoff-directory rules on the host (no device work):
the file layout's round trip and its integrity checks, the parameter set's
JSON form, the handoff directory rules of the reference
(src/stage1_mamba2_process.cpp:28-79) and the decoder's role checks
(stage1_mamba2_config.cpp:253-277), and the key plan against the rotations
the decoder actually requests."""
import json
import os
import stat

import numpy as np
import pytest

from fhemamba_amd import ckks, handoff as H, serial as S
from fhemamba_amd import mamba2_decode as D
from fhemamba_amd import mamba2_payload as M

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_file_layout_round_trip_and_checks(tmp_path):
    a = np.arange(24, dtype=np.uint64).reshape(2, 3, 4) * np.uint64(2 ** 59 + 7)
    b = np.array([-1, 0, 1, 1], dtype=np.int64)
    path = str(tmp_path / "x.bin")
    S._write(path, {"kind": "thing", "note": "é", "arrays": [S._spec(a.shape),
                                                             S._spec(b.shape, "int64")]},
             iter([a, b]))
    with S._Reader(path) as r:
        assert r.kind("thing")["note"] == "é"
        assert np.array_equal(r.array(), a) and np.array_equal(r.array(), b)
        with pytest.raises(S.SerialError, match="fewer arrays"):
            r.array()
    with S._Reader(path) as r, pytest.raises(S.SerialError, match="not a ciphertext"):
        r.kind("ciphertext")
    raw = bytearray(open(path, "rb").read())
    raw[-3] ^= 1                                   # a flipped bit in the data
    open(path, "wb").write(raw)
    with S._Reader(path) as r, pytest.raises(S.SerialError, match="checksum"):
        r.array(), r.array()
    open(path, "wb").write(bytes(raw[:-9]))        # truncated
    with S._Reader(path) as r, pytest.raises(S.SerialError, match="truncated|checksum"):
        r.array(), r.array()
    open(path, "wb").write(b"NOTAFILE" + bytes(16))
    with pytest.raises(S.SerialError, match="not an fhecore"):
        S._Reader(path)
    with pytest.raises(S.SerialError, match="match its header"):
        S._write(path, {"kind": "t", "arrays": [S._spec((2,))]}, [np.zeros(3, np.uint64)])


def test_parameter_set_json_round_trip():
    p = ckks.CCParamsCKKSRNS()
    p.SetMultiplicativeDepth(44)
    p.SetSecretKeyDist(ckks.SecretKeyDist.SPARSE_TERNARY)
    p.SetSecurityLevel(ckks.SecurityLevel.HEStd_NotSet)
    p.SetRingDim(1 << 12)

    class CC:
        _params = p
    d = json.loads(json.dumps(S._params_json(CC())))
    q = S._params_from_json(d)
    assert q._v == p._v
    d["SecretKeyDist"]["name"] = "NOPE"
    with pytest.raises(S.SerialError):
        S._params_from_json(d)
    with pytest.raises(S.SerialError):
        S._params_from_json({"Bogus": 1})


def test_only_binary_is_provided(tmp_path):
    with pytest.raises(S.SerialError, match="BINARY"):
        S.DeserializeCiphertext(str(tmp_path / "x"), S.JSON)
    ct, ok = S.DeserializeCiphertext(str(tmp_path / "missing.ct"))
    assert ct is None and ok is False and "missing.ct" in S.last_error()


def test_handoff_directory_rules(tmp_path):
    paths = H.HandoffPaths(str(tmp_path / "h"))
    H.prepare_client_handoff(paths)
    for d in (paths.root, paths.client, paths.server, paths.exchange):
        assert stat.S_IMODE(os.stat(d).st_mode) == 0o700
    open(os.path.join(paths.client, "x"), "w").close()
    with pytest.raises(ValueError, match="non-empty"):
        H.prepare_client_handoff(paths)
    assert H.count_server_secret_files(paths) == 0
    os.makedirs(os.path.join(paths.server, "sub"))
    open(os.path.join(paths.server, "sub", "My-SECRET.bin"), "w").close()
    assert H.count_server_secret_files(paths) == 1
    with pytest.raises(ValueError, match="secret"):
        H.require_server_has_no_secret_files(paths)
    f = tmp_path / "file"
    f.write_text("x")
    with pytest.raises(ValueError, match="not a directory"):
        H.prepare_client_handoff(H.HandoffPaths(str(f)))


def test_role_checks(tmp_path):
    fix = os.path.join(GOLD, "m2_chain_tiny")
    res = str(tmp_path / "r.json")
    assert D.main([fix, res, "--process-role", "server-eval"]) == 2
    assert D.main([fix, res, "--process-role", "client-init", "--handoff-dir",
                   str(tmp_path / "h"), "--autoregressive-client-loop"]) == 2
    # a server that finds a secret-named file refuses before loading anything
    paths = H.HandoffPaths(str(tmp_path / "h2"))
    H.prepare_client_handoff(paths)
    open(os.path.join(paths.server, "secret-key.bin"), "w").close()
    assert D.main([fix, res, "--process-role", "server-eval", "--handoff-dir",
                   paths.root]) == 2
    with pytest.raises(SystemExit):
        D.main([fix, res, "--process-role", "bogus"])


@pytest.mark.parametrize("name", ["m2_chain_tiny", "m2_chain_tiny_joint_cheb"])
@pytest.mark.parametrize("s2c", [False, True])
def test_key_plan_equals_requested_rotations(name, s2c):
    """The dry run's rotation set equals the rotations the decoder requests
    when it runs the payload's tokens on the slot-level stand-in."""
    from fhemamba_amd.keyplan import plan_decoder_rotations
    from fhemamba_amd.mamba2_decode import EncryptedMamba2Decoder
    from packed_builder import SlotContext, SlotKeys
    ch = M.read_chain_payload(os.path.join(GOLD, name))
    cc = SlotContext(1024, L=45, boot_depth=21)
    dec = EncryptedMamba2Decoder(cc, SlotKeys(), ch, s2c_first=s2c)
    st = dec.initial_states()
    for e in ch.input_embeddings:
        _, st = dec.step(e, st)
    plan = plan_decoder_rotations(ch, slots=1024, ring_dim=2048, limbs=45,
                                  boot_level=21 - 4 * s2c, boot_ceiling=43 - 4 * s2c,
                                  s2c_first=s2c)
    assert plan == cc.keys and len(plan) > 10
