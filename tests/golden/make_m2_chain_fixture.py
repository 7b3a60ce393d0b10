"""Write the Mamba-2 chain payload fixtures with the reference's own exporter.

Runs `export_chain_payload` (src/fhemamba/m1_payload.py:901) of the
reference tree at /root/reference on the tiny seeded Hugging Face Mamba-2
that the reference's own tests build (tests/conftest.py:9-34: vocab 97,
hidden 32, state 8, 2 layers, conv 4, expand 2, 4 heads x 16, 1 group,
chunk 8, torch seed 19) with the reference tests' tokenizer stand-in
(tests/conftest.py:37-50), the prompt "The capital of France is" and two
test tokens:
  m2_chain_tiny/        the default payload (fhemamba-m1-v1 layers);
  m2_chain_tiny_sched/  scheduled normalization: the bundle the reference's
                        tests build (tests/test_scheduled_payload.py:18-33,
                        plan_invsqrt(1e-6, hi) for every block, gated and
                        final norm), 16 calibration tokens;
  m2_chain_tiny_joint/  the same plus shared-factor joint gates from the
                        gate bundle of tests/test_scheduled_payload.py:42-67
                        (fhemamba-m1-joint-v1 / fhemamba-m2-chain-joint-v1);
                        that bundle's gates are constants (degree 0);
  m2_chain_tiny_joint_cheb/  joint gates of degree 7 (p) and 5 (q) per head:
                        on each head's public domain (the exporter's own
                        public_gate_domains), p interpolates
                        sqrt(1 - exp(-softplus(z) rate)) (scaled so that
                        sum |p_k| <= 0.999, which the exporter's gate
                        certificate requires) and q interpolates
                        sqrt(softplus(z) / (1 - exp(-softplus(z) rate))).
  m2_chain_tiny_ar/     the scheduled-normalization payload plus the
                        client-in-loop greedy assets, as the reference's
                        test exports them (tests/test_scheduled_payload.py:
                        autoregressive_prompt_tokens 2,
                        autoregressive_generate_tokens 2: client embedding
                        table, the embeddings of the evaluated tokens, the
                        polynomial and exact final hiddens and the greedy ids).
Only the payloads it writes (float32 tensors and JSON) are kept: nothing of
the reference is copied, and nothing here runs at test time.

    python tests/golden/make_m2_chain_fixture.py [REFERENCE_ROOT [NAME ...]]
"""
import os
import shutil
import sys
import tempfile
from types import SimpleNamespace

HERE = os.path.dirname(os.path.abspath(__file__))


class Tokenizer:
    """Character tokenizer of the reference tests (ids ord(c) % 90 + 3)."""

    def __init__(self, limit=64):
        self.limit = limit

    def __call__(self, text, return_tensors=None):
        import torch
        ids = torch.tensor([[ord(c) % 90 + 3 for c in text[: self.limit]]])
        return SimpleNamespace(input_ids=ids)


def tiny_mamba2(seed=19):
    import torch
    import transformers
    torch.manual_seed(seed)
    config = transformers.Mamba2Config(vocab_size=97, hidden_size=32, state_size=8,
                                       num_hidden_layers=2, conv_kernel=4, expand=2,
                                       num_heads=4, head_dim=16, n_groups=1, chunk_size=8)
    return transformers.Mamba2ForCausalLM(config).float().eval()


def normalization_bundle(path):
    """The reference tests' schedule bundle (tests/test_scheduled_payload.py:18-33)."""
    import json
    from fhemamba.normalization import plan_invsqrt
    bundle = {
        "format": "fhemamba-normalization-schedules-v1",
        "operators": [
            {"layer": layer, "site": site, "recipe": plan_invsqrt(1e-6, hi).recipe()}
            for layer, site, hi in ((0, "rms_invsqrt", 50), (0, "gated_rms_invsqrt", 100),
                                    (1, "rms_invsqrt", 50), (1, "gated_rms_invsqrt", 100),
                                    (2, "rms_invsqrt", 200))
        ],
    }
    with open(path, "w") as f:
        json.dump(bundle, f)


def gate_bundle(path, model):
    """The reference tests' joint-gate bundle (tests/test_scheduled_payload.py:42-67)."""
    import json
    import numpy as np
    from fhemamba.payload_surrogate import public_gate_domains
    arrays = {}
    for layer, block in enumerate(model.backbone.layers):
        lo, hi = public_gate_domains(block)
        for name, value in {"lo": lo, "hi": hi, "p": np.full((1, len(lo)), 0.5),
                            "q": np.full((1, len(lo)), 0.75),
                            "rates": block.mixer.A_log.detach().exp().double().numpy()}.items():
            arrays[f"layer_{layer}_{name}"] = value
    arrays["manifest"] = np.array(json.dumps({"format": "dissipative-mamba2-gates-v1",
                                              "layers": [0, 1],
                                              "input_payload_sha256": "0" * 64}))
    np.savez(path, **arrays)


def cheb_gate_bundle(path, model, degree_p=7, degree_q=5):
    """Per-head Chebyshev joint gates (p: degree_p, q: degree_q) on the
    exporter's public domains."""
    import json
    import numpy as np
    from fhemamba.payload_surrogate import public_gate_domains
    arrays = {}
    for layer, block in enumerate(model.backbone.layers):
        lo, hi = public_gate_domains(block)
        rates = block.mixer.A_log.detach().exp().double().numpy()
        p = np.zeros((degree_p + 1, len(lo)))
        q = np.zeros((degree_q + 1, len(lo)))
        for h in range(len(lo)):
            def dt(t, h=h):
                return np.logaddexp(0.0, lo[h] + (t + 1.0) * 0.5 * (hi[h] - lo[h]))

            def keep(t, h=h):
                return -np.expm1(-dt(t) * rates[h])
            ph = np.polynomial.chebyshev.chebinterpolate(lambda t: np.sqrt(keep(t)), degree_p)
            ph *= min(1.0, 0.999 / np.abs(ph).sum())
            p[:, h] = ph
            q[:, h] = np.polynomial.chebyshev.chebinterpolate(
                lambda t: np.sqrt(dt(t) / keep(t)), degree_q)
        for name, value in {"lo": lo, "hi": hi, "p": p, "q": q, "rates": rates}.items():
            arrays[f"layer_{layer}_{name}"] = value
    arrays["manifest"] = np.array(json.dumps({"format": "dissipative-mamba2-gates-v1",
                                              "layers": [0, 1],
                                              "input_payload_sha256": "0" * 64}))
    np.savez(path, **arrays)


def main(reference_root="/root/reference", *names):
    sys.path.insert(0, os.path.join(reference_root, "src"))
    from fhemamba.m1_payload import export_chain_payload
    model = tiny_mamba2()
    with tempfile.TemporaryDirectory() as tmp:
        norms, gates = os.path.join(tmp, "norms.json"), os.path.join(tmp, "gates.npz")
        cheb_gates = os.path.join(tmp, "cheb_gates.npz")
        normalization_bundle(norms)
        gate_bundle(gates, model)
        cheb_gate_bundle(cheb_gates, model)
        runs = {
            "m2_chain_tiny": dict(),
            "m2_chain_tiny_sched": dict(cal_tokens=16, normalization_bundle=norms),
            "m2_chain_tiny_joint": dict(cal_tokens=16, normalization_bundle=norms,
                                        stabilized_gate_bundle=gates),
            "m2_chain_tiny_ar": dict(cal_tokens=16, normalization_bundle=norms,
                                     autoregressive_prompt_tokens=2,
                                     autoregressive_generate_tokens=2),
            "m2_chain_tiny_joint_cheb": dict(cal_tokens=16, normalization_bundle=norms,
                                             stabilized_gate_bundle=cheb_gates),
        }
        for name, kw in runs.items():
            if names and name not in names:
                continue
            out = export_chain_payload(model, Tokenizer(), os.path.join(tmp, name),
                                       n_test_tokens=2, **kw)
            dest = os.path.join(HERE, name)
            if os.path.isdir(dest):
                shutil.rmtree(dest)
            shutil.copytree(out, dest)
            print(dest)


if __name__ == "__main__":
    main(*sys.argv[1:])
