"""The reference runner's gates on a Mamba-2 decode result, restated for
the tests (shared by the CPU and GPU tests of the decode drop-in).  These
are checks a result must pass, not an implementation of anything the
library runs."""


def runner_gate(native, identity):
    """models/mamba2.py:255-262."""
    for section in ("parameters", "measurements", "measurement_scope"):
        assert isinstance(native.get(section), dict), section
    assert native.get("binary_sha256") == identity
    assert native["parameters"].get("security") == "not-set"


def generation_checks(native, request, poly_ids, vocab):
    """generation.py:108-156 (the checks dictionary)."""
    p = native["parameters"]
    expected = {"autoregressive_client_loop": True,
                "autoregressive_prompt_tokens": request["prompt_tokens"],
                "autoregressive_generate_tokens": request["generate_tokens"],
                "n_layers_loaded": request["n_layers"], "tokens": request["server_evaluations"],
                "final_norm_applied": True}
    assert all(p.get(k) == v for k, v in expected.items()), \
        {k: (p.get(k), v) for k, v in expected.items()}
    m, scope = native["measurements"], native["measurement_scope"]
    selected = m["autoregressive_selected_ids"]
    assert all(type(v) is int and 0 <= v < vocab for v in selected)
    checks = {
        "native_passed": native.get("passed") is True,
        "encrypted_full_chain": native.get("encrypted") is True and all(
            scope.get(k) is True for k in (
                "fideslib_encrypted_execution", "full_layer_chain",
                "multi_token_ciphertext_state_carry", "ciphertext_conv_fifo",
                "per_token_fresh_embedding_encryption",
                "client_output_decrypts_are_protocol_boundary")),
        "complete_generation": len(selected) == request["generate_tokens"],
        "matches_polynomial_tokens": selected == poly_ids,
        "all_outputs_decrypt": len(m["per_token_decrypt_ok"]) == request["server_evaluations"]
        and all(m["per_token_decrypt_ok"]),
        "all_errors_within_0_05": len(m["per_token_max_abs_error"]) ==
        request["server_evaluations"] and all(0 <= v <= 0.05 for v in m["per_token_max_abs_error"]),
        "no_intermediate_diagnostic_decrypts": scope.get("zero_intermediate_decrypts") is True,
        "client_output_decrypts": scope.get("autoregressive_client_output_decrypt_count") ==
        request["generate_tokens"],
    }
    return checks


def acceptance_issues(acceptance, native):
    """benchmarks/acceptance.py evaluate_acceptance, one artifact."""
    issues = []
    if not (native.get("status") == "passed" and native.get("passed") is True):
        issues.append("not passed")
    p, scope, m = native["parameters"], native["measurement_scope"], native["measurements"]
    layers = p.get("n_layers_loaded", scope.get("layers_loaded"))
    if acceptance.get("layers") is not None and layers != acceptance["layers"]:
        issues.append("layers")
    tokens = p.get("tokens", scope.get("tokens"))
    if acceptance.get("tokens") is not None and tokens != acceptance["tokens"]:
        issues.append("tokens")
    if m.get("max_abs_error") is None or m["max_abs_error"] > acceptance["max_abs_error_lte"]:
        issues.append("error")
    ok = m.get("per_token_decrypt_ok")
    if acceptance.get("all_tokens_decrypt") and not (ok and all(v == 1 for v in ok) and
                                                      len(ok) == acceptance.get("tokens")):
        issues.append("decrypt")
    if acceptance.get("autoregressive_tokens_match") and not (
            m.get("autoregressive_tokens_match") is True and m["autoregressive_selected_ids"]
            and m["autoregressive_selected_ids"] == m["autoregressive_expected_ids"]):
        issues.append("ids")
    if acceptance.get("zero_intermediate_decrypts") and \
            scope.get("zero_intermediate_decrypts") is not True:
        issues.append("decrypts")
    if p.get("fideslib_sync_profile") != acceptance.get("required_sync_profile"):
        issues.append("sync profile")
    return issues
