"""Process-separated Mamba-2 decode: a client that holds the secret key
and a server that never sees it, exchanging files in a handoff directory
(the reference decoder's --process-role client-init | server-eval |
client-decrypt with --handoff-dir, native/fideslib_stage0/src/
stage1_mamba2_decode_fideslib.cpp:879-962, :1248-1275, :1446-1512,
:4646-4700; directory rules of src/stage1_mamba2_process.cpp:28-79).

Layout under the handoff root (each directory owner-only):
  client/   context.bin, secret-key.bin (owner read/write only)
  server/   context.bin, public-key.bin, eval-mult.bin, eval-rotation.bin,
            handoff.json (the slot count, refresh order and passes the keys
            were made for)
  exchange/ input_t<k>.ct (client-init), output_t<k>.ct (server-eval)
Files are in this library's wire format (fhemamba_amd.serial).  The server
refuses to run while any file under server/ has "secret" in its name, and
client-decrypt fails the run if one is there.

client-init builds the context and keys, generates every rotation key the
server's circuit will ask for (fhemamba_amd.keyplan, a dry run of the
decoder) plus the bootstrapping and conjugation keys, writes the server's
files and encrypts the payload's test embeddings.  server-eval loads the
context, the public key and the evaluation keys, decodes the encrypted
embeddings with carried state and writes the encrypted outputs.
client-decrypt decrypts them and compares them with the payload's
polynomial-circuit references (exact references if the payload has none).
"""
from __future__ import annotations

import json
import os
import shutil
import stat
import time

import numpy as np

LEVEL_BUDGET = (4, 4)


class HandoffPaths:
    def __init__(self, root: str):
        self.root = root
        self.client = os.path.join(root, "client")
        self.server = os.path.join(root, "server")
        self.exchange = os.path.join(root, "exchange")

    def input(self, k: int) -> str:
        return os.path.join(self.exchange, f"input_t{k}.ct")

    def output(self, k: int) -> str:
        return os.path.join(self.exchange, f"output_t{k}.ct")


def _owner_only(path: str) -> None:
    os.chmod(path, stat.S_IRWXU)


def prepare_client_handoff(paths: HandoffPaths) -> None:
    """A fresh (absent or empty) root with client/, server/ and exchange/,
    each owner-only."""
    if os.path.exists(paths.root):
        if not os.path.isdir(paths.root):
            raise ValueError(f"handoff root exists but is not a directory: {paths.root}")
        if os.listdir(paths.root):
            raise ValueError(f"refusing to reuse non-empty handoff root: {paths.root}")
    for d in (paths.client, paths.server, paths.exchange):
        os.makedirs(d, exist_ok=True)
    for d in (paths.root, paths.client, paths.server, paths.exchange):
        _owner_only(d)


def count_server_secret_files(paths: HandoffPaths) -> int:
    """Files under server/ whose name contains "secret" (any case)."""
    if not os.path.isdir(paths.server):
        return 0
    return sum(1 for _, _, files in os.walk(paths.server) for f in files
               if "secret" in f.lower())


def require_server_has_no_secret_files(paths: HandoffPaths) -> None:
    n = count_server_secret_files(paths)
    if n:
        raise ValueError(f"server handoff contains {n} secret-key-named file(s)")


def _check(ok: bool, what: str) -> None:
    from . import serial
    if not ok:
        raise ValueError(f"failed to {what}: {serial.last_error()}")


def _scope(**kw) -> dict:
    return {"client_server_process_separation": True, "server_secret_key_loaded": False, **kw}


def client_init(payload_dir: str, handoff_dir: str, *, tokens: int = 0,
                bootstrap_passes: int = 2, transient_passes: int | None = None, seed=None,
                secret_key_dist=None,
                security: str = "not-set", layers: int = 0, s2c_first: bool = True,
                ring_dim: int = 0, log=print) -> dict:
    from . import ckks
    from .keyplan import decoder_rotations
    from .mamba2_decode import _build, _decode_setup, _truncate, default_transient_passes
    paths = HandoffPaths(handoff_dir)
    chain, classical, dist, slots, extra = _decode_setup(payload_dir, security,
                                                         secret_key_dist, ring_dim)
    if transient_passes is None:
        transient_passes = default_transient_passes(dist, bootstrap_passes)
    _truncate(chain, layers)
    n_tok = tokens or chain.n_test_tokens
    if n_tok > chain.n_test_tokens:
        raise ValueError("tokens exceeds the payload's n_test_tokens")
    prepare_client_handoff(paths)
    t0 = time.perf_counter()
    cc, keys = _build(slots, seed, dist, extra)
    cc.EvalBootstrapSetup(list(LEVEL_BUDGET), [0, 0], slots, s2c_first=s2c_first,
                          real_slots=True)
    cc.EvalBootstrapKeyGen(keys.secretKey, slots)
    rot = sorted(decoder_rotations(cc, chain, s2c_first=s2c_first,
                                   bootstrap_passes=bootstrap_passes))
    cc.EvalRotateKeyGen(keys.secretKey, rot)
    keygen = time.perf_counter() - t0
    log(f"client-init: {len(rot)} circuit rotation keys, {len(cc._galois)} automorphism keys")
    ctx_client = os.path.join(paths.client, "context.bin")
    _check(ckks.SerializeToFile(ctx_client, cc), "serialize the context")
    shutil.copyfile(ctx_client, os.path.join(paths.server, "context.bin"))
    _check(ckks.SerializeToFile(os.path.join(paths.server, "public-key.bin"), keys.publicKey),
           "serialize the public key")
    sk_path = os.path.join(paths.client, "secret-key.bin")
    _check(ckks.SerializeToFile(sk_path, keys.secretKey), "serialize the secret key")
    os.chmod(sk_path, stat.S_IRUSR | stat.S_IWUSR)
    _check(cc.SerializeEvalMultKey(os.path.join(paths.server, "eval-mult.bin")),
           "serialize the multiplication key")
    _check(cc.SerializeEvalAutomorphismKey(os.path.join(paths.server, "eval-rotation.bin")),
           "serialize the rotation / bootstrapping keys")
    with open(os.path.join(paths.server, "handoff.json"), "w") as f:
        json.dump({"slots": slots, "s2c_first": bool(s2c_first),
                   "bootstrap_passes": int(bootstrap_passes),
                   "transient_passes": int(transient_passes),
                   "level_budget": list(LEVEL_BUDGET), "tokens": n_tok,
                   "layers": chain.n_layers}, f)
    for k in range(n_tok):
        v = np.zeros(slots)
        v[: chain.layers[0].d_model] = chain.input_embeddings[k]
        ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(v, 1, 0, slots=slots))
        _check(ckks.SerializeToFile(paths.input(k), ct), f"serialize input {k}")
    return {"schema": "fhemamba-m2-decode-result-v1", "process_role": "client-init",
            "passed": True, "tokens": n_tok, "layers": chain.n_layers,
            "ring_dimension": cc.GetRingDimension(), "slots": slots, "security": security,
            "secret_key_dist": dist, "s2c_first": bool(s2c_first),
            "encrypted_inputs_written": n_tok, "circuit_rotation_keys": len(rot),
            "automorphism_keys": len(cc._galois), "keygen_seconds": keygen,
            "measurement_scope": _scope(
                full_model_correctness_claimed=False,
                claim="client key generation and encrypted input serialization for the "
                      "process-separated decode; no server evaluation is claimed by this "
                      "phase")}


def server_eval(payload_dir: str, handoff_dir: str, *, tokens: int = 0, layers: int = 0,
                log=print) -> dict:
    """The server: no secret key is read or present."""
    from . import ckks
    from .mamba2_decode import EncryptedMamba2Decoder, _truncate
    from .mamba2_payload import read_chain_payload
    paths = HandoffPaths(handoff_dir)
    require_server_has_no_secret_files(paths)
    with open(os.path.join(paths.server, "handoff.json")) as f:
        plan = json.load(f)
    chain = read_chain_payload(payload_dir)
    _truncate(chain, layers)
    n_tok = tokens or int(plan["tokens"])
    if n_tok > int(plan["tokens"]) or chain.n_layers != int(plan["layers"]):
        raise ValueError("tokens / layers differ from what client-init prepared")
    t0 = time.perf_counter()
    cc, ok = ckks.DeserializeCryptoContext(os.path.join(paths.server, "context.bin"))
    _check(ok, "deserialize the server context")
    pk, ok = ckks.DeserializePublicKey(os.path.join(paths.server, "public-key.bin"))
    _check(ok, "deserialize the public key")
    _check(cc.DeserializeEvalMultKey(os.path.join(paths.server, "eval-mult.bin")),
           "deserialize the multiplication key")
    _check(cc.DeserializeEvalAutomorphismKey(os.path.join(paths.server, "eval-rotation.bin")),
           "deserialize the rotation / bootstrapping keys")
    if cc.GetBatchSize() != int(plan["slots"]):
        raise ValueError("the server context's batch size differs from the handoff plan")
    keys = ckks.KeyPair(pk, None)
    dec = EncryptedMamba2Decoder(cc, keys, chain, bootstrap_passes=int(plan["bootstrap_passes"]),
                                 transient_passes=int(plan.get("transient_passes", 1)),
                                 s2c_first=bool(plan["s2c_first"]), log=log)
    setup = time.perf_counter() - t0
    log("server key load done secret_key_loaded=false")
    states = dec.initial_states()
    steps = []
    t_eval = time.perf_counter()
    for k in range(n_tok):
        ct, ok = ckks.DeserializeCiphertext(paths.input(k))
        _check(ok, f"deserialize input {k}")
        cc.device.sync()
        t = time.perf_counter()
        out, states = dec.step_ct(ct, states)
        cc.device.sync()
        steps.append(time.perf_counter() - t)
        _check(ckks.SerializeToFile(paths.output(k), out), f"serialize output {k}")
        log(f"server token {k}: {steps[-1]:.2f}s")
    s = dec.ev.stats
    return {"schema": "fhemamba-m2-decode-result-v1", "process_role": "server-eval",
            "passed": True, "tokens": n_tok, "layers": chain.n_layers,
            "encrypted_outputs_written": n_tok,
            "server_secret_key_files": count_server_secret_files(paths),
            "setup_seconds": setup, "eval_seconds": time.perf_counter() - t_eval,
            "seconds_per_token": steps,
            "carried_token_seconds": (sum(steps[1:]) / (n_tok - 1)) if n_tok > 1 else None,
            "bootstraps": s["bootstraps"], "rotations": s["rotations"],
            "ct_ct_mul": s["ct_ct"], "ct_pt_mul": s["ct_pt"],
            "measurement_scope": _scope(
                encrypted_full_layer_chain_evaluated=True, full_model_correctness_claimed=False,
                claim="secret-key-free server evaluation and encrypted output serialization; "
                      "correctness is established only by the separate client-decrypt phase")}


def client_decrypt(payload_dir: str, handoff_dir: str, *, tokens: int = 0, layers: int = 0,
                   tolerance: float = 1e-3, log=print) -> dict:
    from . import ckks, serial
    from .mamba2_decode import _truncate
    from .mamba2_payload import read_chain_payload
    paths = HandoffPaths(handoff_dir)
    chain = read_chain_payload(payload_dir)
    full = not layers or layers == chain.n_layers
    _truncate(chain, layers)
    with open(os.path.join(paths.server, "handoff.json")) as f:
        n_tok = tokens or int(json.load(f)["tokens"])
    cc, ok = ckks.DeserializeCryptoContext(os.path.join(paths.client, "context.bin"))
    _check(ok, "deserialize the client context")
    sk, ok = ckks.DeserializePrivateKey(os.path.join(paths.client, "secret-key.bin"))
    _check(ok, "deserialize the secret key")
    want = chain.expected_poly_final if chain.expected_poly_final is not None \
        else chain.expected_final
    d = chain.layers[0].d_model
    errors, decrypted = [], []
    for k in range(n_tok):
        ct, ok = ckks.DeserializeCiphertext(paths.output(k))
        if not ok:
            log(f"client decrypt token {k} failed: {serial.last_error()}")
            errors.append(float("inf"))
            decrypted.append(0)
            continue
        pt = cc.Decrypt(ct, sk)
        pt.SetLength(d)
        got = np.asarray(pt.GetRealPackedValue())
        e = float(np.max(np.abs(got - want[k])))
        errors.append(e if np.isfinite(e) else float("inf"))
        decrypted.append(1)
    n_secret = count_server_secret_files(paths)
    worst = max(errors) if errors else float("inf")
    passed = bool(worst <= tolerance and n_secret == 0)
    return {"schema": "fhemamba-m2-decode-result-v1", "process_role": "client-decrypt",
            "passed": passed, "tokens": n_tok, "layers": chain.n_layers, "tolerance": tolerance,
            "max_abs_error": worst, "per_token_max_abs_error": errors,
            "per_token_decrypt_ok": decrypted, "server_secret_key_files": n_secret,
            "reference": "chain_expected_poly_final" if chain.expected_poly_final is not None
            else "chain_expected_final",
            "measurement_scope": _scope(
                full_model_correctness_claimed=full,
                claim="client-only decryption and correctness check of the ciphertext "
                      "outputs of the process-separated server")}
