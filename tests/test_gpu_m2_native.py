"""The Mamba-2 decode drop-in run as the reference runner runs its decode
binary (src/fhemamba/models/mamba2.py:219-262): the executable
fhe-mamba_amd/stage1_mamba2_decode with the campaign's argv
(tests/golden/m2_decode_cli.json, ring 65536, depth 44, security not-set,
level budget 5/5, client loop on) plus the runner's identity flags, in a
working directory whose `payload` is the reference exporter's autoregressive
tiny chain (tests/golden/m2_chain_tiny_ar, two layers, two prompt tokens,
two generated).  Its native.json must pass the runner's gates
(tests/m2_gates.py) with the exporter's greedy ids."""
import hashlib
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

from m2_gates import acceptance_issues, generation_checks, runner_gate  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "..", "fhe-mamba_amd", "stage1_mamba2_decode")
FIX = json.load(open(os.path.join(HERE, "golden", "m2_decode_cli.json")))
CHAIN = os.path.join(HERE, "golden", "m2_chain_tiny_ar")


def test_runner_invocation_passes_the_runner_gates(tmp_path):
    chain = json.load(open(os.path.join(CHAIN, "chain.json")))
    ar = chain["autoregressive"]
    layers, tokens = chain["n_layers"], ar["server_evaluations"]
    os.symlink(CHAIN, tmp_path / "payload")
    with open(EXE, "rb") as f:
        identity = hashlib.sha256(f.read()).hexdigest()
    out = tmp_path / "out"
    out.mkdir()
    argv = [sys.executable, EXE]
    for flag, value in FIX["runner_argv"]:
        argv += [flag, value.format(layers=layers, tokens=tokens)]
    argv += ["--artifact-version", "0.5.0", "--repo-commit", "working-tree",
             "--binary-sha256", identity, "--output-json", str(out / "native.json")]
    print(f"running the decode drop-in: {layers} layers, {tokens} evaluations", flush=True)
    proc = subprocess.run(argv, cwd=tmp_path, capture_output=True, text=True, timeout=900)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    native = json.loads((out / "native.json").read_text())
    m = native["measurements"]
    print(f"native.json: passed {native['passed']}, errors {m.get('per_token_max_abs_error')}, "
          f"ids {m.get('autoregressive_selected_ids')}, timing {m.get('timing')}", flush=True)
    assert proc.returncode == 0
    runner_gate(native, identity)
    request = {"prompt_tokens": ar["prompt_tokens"], "generate_tokens": ar["generate_tokens"],
               "n_layers": layers, "server_evaluations": tokens}
    checks = generation_checks(native, request, ar["poly_generated_ids"],
                               vocab=chain["tensors"]["client_embedding_w"][0])
    assert all(checks.values()), checks
    acceptance = dict(FIX["acceptance"], layers=layers, tokens=tokens)
    assert acceptance_issues(acceptance, native) == []
    assert native["parameters"]["bootstrap_level_budget"] == [5, 5]
