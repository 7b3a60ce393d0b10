"""Write tests/golden/m2_chain_tiny/ with the reference's own chain exporter.

Runs `export_chain_payload` (src/fhemamba/m1_payload.py:901) of the
reference tree at /root/reference on the tiny seeded Hugging Face Mamba-2
that the reference's own tests build (tests/conftest.py:9-34: vocab 97,
hidden 32, state 8, 2 layers, conv 4, expand 2, 4 heads x 16, 1 group,
chunk 8, torch seed 19) with the reference tests' tokenizer stand-in
(tests/conftest.py:37-50), the prompt "The capital of France is" and two
test tokens.  Only the payload it writes (float32 tensors and JSON) is kept:
nothing of the reference is copied, and nothing here runs at test time.

    python tests/golden/make_m2_chain_fixture.py [REFERENCE_ROOT]
"""
import os
import shutil
import sys
import tempfile
from types import SimpleNamespace

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "m2_chain_tiny")


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


def main(reference_root="/root/reference"):
    sys.path.insert(0, os.path.join(reference_root, "src"))
    from fhemamba.m1_payload import export_chain_payload
    model = tiny_mamba2()
    with tempfile.TemporaryDirectory() as tmp:
        out = export_chain_payload(model, Tokenizer(), os.path.join(tmp, "chain"),
                                   n_test_tokens=2)
        if os.path.isdir(OUT):
            shutil.rmtree(OUT)
        shutil.copytree(out, OUT)
    print(OUT)


if __name__ == "__main__":
    main(*sys.argv[1:])
