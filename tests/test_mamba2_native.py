"""The Mamba-2 decode drop-in (fhemamba_amd.mamba2_native) against the
reference decoder's command-line contract, on the CPU.

The contract is pinned by tests/golden/m2_decode_cli.json, extracted from the
reference's sources by tests/golden/make_m2_decode_cli_fixture.py: the flag
set and Config defaults of stage1_mamba2_config.{hpp,cpp}, its error
messages, and the argv the reference runner passes
(src/fhemamba/models/mamba2.py:40-75, 219-236).  The result is checked with
the runner's own gates restated in tests/m2_gates.py (models/mamba2.py:255-262,
generation.py:108-156, benchmarks/acceptance.py), on a result built from a
stubbed decode; the GPU decode itself is tests/test_gpu_m2_native.py."""
import json
import os

import pytest

from fhemamba_amd import mamba2_native as N
from m2_gates import acceptance_issues, generation_checks, runner_gate

FIX = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "m2_decode_cli.json")))
SHA = "ab" * 32


def runner_argv(layers, tokens, output="out/native.json"):
    argv = []
    for flag, value in FIX["runner_argv"]:
        argv += [flag, value.format(layers=layers, tokens=tokens)]
    return argv + ["--artifact-version", "0.5.0", "--repo-commit", "working-tree",
                   "--binary-sha256", SHA, "--output-json", output]


def test_flags_and_defaults_are_the_reference_decoders():
    assert sorted(N.FLAGS) == FIX["flags"]
    c = N.Config()
    got = {name: (sorted(v) if isinstance(v, set) else v) for name, v in vars(c).items()}
    assert got == FIX["defaults"]


def test_runner_argv_parses():
    c = N.parse_args(runner_argv(24, 5))
    assert c.input_chain == "payload" and c.max_layers == 24 and c.tokens == 5
    assert (c.ring_dim, c.multiplicative_depth, c.scaling_mod_size, c.first_mod_size) == \
        (65536, 44, 59, 60)
    assert c.security == "not-set" and c.fideslib_sync_profile == "full"
    assert c.autoregressive_client_loop and c.binary_sha256 == SHA
    assert c.meta_bts_residual_layers == {21, 22, 23} and c.bootstrap_before_token == set()
    assert c.tolerance == 0.05


BAD = [
    ([], "exactly one of --input or --input-chain is required"),
    (["--input", "a", "--input-chain", "b"], "exactly one of --input or --input-chain is required"),
    (["--input-chain", "p", "--tokens"], "missing value for --tokens"),
    (["--input-chain", "p", "--nope", "1"], "unknown argument: --nope"),
    (["--input-chain", "p", "--process-role", "server"],
     "process-role must be inline, client-init, server-eval, or client-decrypt"),
    (["--input-chain", "p", "--process-role", "server-eval"],
     "non-inline process-role requires --handoff-dir"),
    (["--input-chain", "p", "--process-role", "server-eval", "--handoff-dir", "h"],
     "non-inline process-role requires --output-json"),
    (["--input-chain", "p", "--ring-dim", "1000"], "ring-dim must be a positive power of two"),
    (["--input-chain", "p", "--tokens", "0"], "invalid CKKS parameters"),
    (["--input-chain", "p", "--tokens", "3", "--bootstrap-before-token", "3"],
     "bootstrap-before-token must be in [1, tokens-1]"),
    (["--input-chain", "p", "--security", "192"], "security must be not-set or 128-classic"),
    (["--input-chain", "p", "--secret-key-dist", "gaussian"],
     "secret-key-dist must be sparse-ternary, uniform-ternary, or sparse-encapsulated"),
    (["--input-chain", "p", "--binary-sha256", "xyz"],
     "binary-sha256 must be unknown or 64 hexadecimal characters"),
    (["--input-chain", "p", "--pt-cache", "huge"], "pt-cache must be auto, full, masks, or off"),
    (["--input-chain", "p", "--streams", "3"], "streams must be a positive power of two"),
    (["--input-chain", "p", "--streams", "2"], "streams > 1 requires --input (single-layer mode)"),
    (["--input-chain", "p", "--meta-bts-alpha", "41"], "meta-bts-alpha must be in [0, 40]"),
    (["--input-chain", "p", "--replicated-true-bsgs", "1"],
     "replicated-true-bsgs requires replicated layout"),
    (["--input-chain", "p", "--fideslib-sync-profile", "x"],
     "fideslib-sync-profile must be unspecified, full, bootstrap-lifetime, lifetime, or none"),
    (["--input-chain", "p", "--debug-recurrence-token", "1"],
     "debug-recurrence-token and debug-recurrence-layer must be set together"),
    (["--input", "p", "--autoregressive-client-loop", "1"],
     "autoregressive-client-loop requires --input-chain"),
]


@pytest.mark.parametrize("argv,message", BAD)
def test_rejections_use_the_reference_messages(argv, message):
    with pytest.raises(ValueError) as e:
        N.parse_args(argv)
    assert str(e.value) == message
    if not message.startswith(("missing value", "unknown argument")):
        assert message in FIX["messages"]


@pytest.mark.parametrize("flag,value", [("--tokens", "5x"), ("--tokens", "99999999999"),
                                        ("--tolerance", "nan"), ("--tolerance", "1e-3 "),
                                        ("--meta-bts", "yes")])
def test_value_parsing_is_strict(flag, value):
    with pytest.raises(ValueError):
        N.parse_args(["--input-chain", "p", flag, value])


def test_value_parsing_accepts_what_stoi_stod_accept():
    c = N.parse_args(["--input-chain", "p", "--tokens", " +7", "--tolerance", "5e-2",
                      "--bootstrap-before-token", "1,,3,", "--meta-bts", "true"])
    assert c.tokens == 7 and c.tolerance == 0.05 and c.bootstrap_before_token == {1, 3}
    assert c.meta_bts is True


def fake_decode(n_layers, n_tok, errs, selected, expected):
    def run_payload(path, **kw):
        return {"autoregressive_selected_ids": selected, "autoregressive_expected_ids": expected,
                "autoregressive_tokens_match": selected == expected,
                "autoregressive_client_seconds": 0.1, "tokens": n_tok, "layers": n_layers,
                "n_layers_total": n_layers, "slots": 32768, "ring_dimension": 65536,
                "security_audit": None, "s2c_first": True,
                "secret_key_dist": kw["secret_key_dist"], "setup_seconds": 1.0,
                "seconds_per_token": [2.0] * n_tok, "carried_token_seconds": 2.0,
                "max_abs_error_vs_polynomial": max(errs), "per_token_errors_vs_polynomial": errs,
                "per_token_errors_vs_exact": [e * 10 for e in errs], "bootstraps": 8,
                "logical_refreshes": 4, "bootstrap_seconds": 0.5, "rotations": 100,
                "ct_ct_mul": 10, "ct_pt_mul": 20, "rotation_keys_generated": 30,
                "keygen_seconds": 0.3, "per_token_bootstraps": [2] * n_tok,
                "decrypt_seconds": 0.01, "token0_samples": {"decrypted": [0.0],
                                                            "expected": [0.0], "exact": [0.0]},
                "level_budget": list(kw["level_budget"]), "multiplicative_depth": 44,
                "refresh_passes": [kw["bootstrap_passes"], 1],
                "dims": {"d_model": 64, "d_inner": 128, "num_heads": 8, "head_dim": 16,
                         "state_size": 16, "conv_kernel": 4, "conv_dim": 160, "proj_dim": 296,
                         "n_groups": 1, "state_group_count": 1}}
    return run_payload


class FakeAssets:
    prompt_tokens, generate_tokens = 2, 2


class FakeChain:
    n_layers = 2
    autoregressive = FakeAssets()


@pytest.fixture
def stubbed(monkeypatch):
    from fhemamba_amd import mamba2_decode, mamba2_payload
    monkeypatch.setattr(mamba2_payload, "read_chain_payload", lambda p, *a, **k: FakeChain())

    def install(errs, selected, expected):
        monkeypatch.setattr(mamba2_decode, "run_payload",
                            fake_decode(2, 3, errs, selected, expected))
    return install


def test_result_passes_the_runner_gates(stubbed, tmp_path):
    stubbed([1e-4, 2e-4, 3e-4], [7, 9], [7, 9])
    out = tmp_path / "native.json"
    assert N.main(runner_argv(2, 3, str(out))) == 0
    native = json.loads(out.read_text())
    runner_gate(native, SHA)
    request = {"prompt_tokens": 2, "generate_tokens": 2, "n_layers": 2, "server_evaluations": 3}
    checks = generation_checks(native, request, [7, 9], vocab=100)
    assert all(checks.values()), checks
    acceptance = dict(FIX["acceptance"], layers=2, tokens=3)
    assert acceptance_issues(acceptance, native) == []
    assert native["parameters"]["bootstrap_level_budget"] == [5, 5]
    assert native["parameters"]["recorded_options"]["rotation_keys"] == "balanced"


def test_failing_decode_fails_the_gates(stubbed, tmp_path):
    stubbed([1e-4, 0.2, 3e-4], [7, 8], [7, 9])
    out = tmp_path / "native.json"
    assert N.main(runner_argv(2, 3, str(out))) == 1
    native = json.loads(out.read_text())
    runner_gate(native, SHA)
    assert native["passed"] is False and native["status"] == "failed"
    request = {"prompt_tokens": 2, "generate_tokens": 2, "n_layers": 2, "server_evaluations": 3}
    checks = generation_checks(native, request, [7, 9], vocab=100)
    assert not checks["matches_polynomial_tokens"] and not checks["all_errors_within_0_05"]
    assert "error" in acceptance_issues(dict(FIX["acceptance"], layers=2, tokens=3), native)


def test_unsupported_option_writes_a_failure_result(tmp_path):
    out = tmp_path / "native.json"
    argv = runner_argv(2, 3, str(out))
    argv[argv.index("--debug-decrypt") + 1] = "1"
    assert N.main(argv) == 1
    native = json.loads(out.read_text())
    assert native["passed"] is False and native["failure_phase"] == "runtime"
    assert "diagnostics" in native["error_message"]
    assert native["binary_sha256"] == SHA and native["parameters"]["security"] == "not-set"


def test_parse_error_exits_without_a_result(tmp_path, capsys):
    out = tmp_path / "native.json"
    assert N.main(["--input-chain", "p", "--output-json", str(out), "--tokens", "x"]) == 1
    assert not out.exists()
    assert "invalid integer for --tokens" in capsys.readouterr().err


def test_launcher_is_an_executable_script():
    path = os.path.join(os.path.dirname(__file__), "..", "fhe-mamba_amd", "stage1_mamba2_decode")
    assert os.access(path, os.X_OK)
    with open(path) as f:
        assert "fhemamba_amd.mamba2_native" in f.read()
