"""Writes the committed golden fixtures under tests/golden/ from the reference's own test data.

Run in a container that has the reference at /root/reference (it never runs on the GPU box):

    python tests/golden/make_fixtures.py

What it takes, all data (no source text):
  * hf_tiny/<model>/ for llama, qwen2, qwen3 and gemma3: the tiny HF checkpoints with their golden
    logits (transformers), AttnLRP relevance (LXT 2.1) and the gradient x input negative control
    (LXT's patches off) -- copied byte for byte from tests/fixtures/hf_tiny/.
  * lxt_values.json: the float vectors pasted into tests/lrp_reference_test.cpp (kMhaLogits,
    kMhaRelevance, kBlockLogits, kBlockRelevance), parsed out of the file's array literals.
  * zennit_values.json: the same file's Zennit 1.0.0 MLP input relevance (kMlpEpsilon1e6,
    kMlpEpsilon025, kMlpZPlus, kMlpAlphaBeta21, kMlpGamma025, kMlpEpsilonPlus,
    kMlpEpsilonAlpha2Beta1, kMlpEpsilonGammaBox).
  * hf_attention_values.json: the Hugging Face LlamaAttention / Qwen2Attention / Qwen3Attention
    forward outputs and input gradients pasted into tests/attention_reference_test.cpp (kLlamaOutput,
    kLlamaInputGrad, kQwen2Output, kQwen2InputGrad, kQwen3Output, kQwen3InputGrad).
  * legacy_block_values.json: the independent NumPy AttnLRP block of tests/transformer_block_test.cpp
    (ValidatesAgainstIndependentAttnLRPReference): its gains and weights as the test sets them, the
    input, the output relevance, and the expected output and input relevance.
"""
import json
import os
import re
import shutil

REF = os.environ.get("PULSATRIX_REF", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))

MODELS = ("llama", "qwen2", "qwen3", "gemma3")
FILES = ("config.json", "golden.safetensors", "attnlrp.safetensors", "gradient_x_input.safetensors",
         "model.safetensors", "model.safetensors.index.json", "model-00001-of-00002.safetensors",
         "model-00002-of-00002.safetensors")


def copy_hf_tiny():
    for m in MODELS:
        src = os.path.join(REF, "tests", "fixtures", "hf_tiny", m)
        dst = os.path.join(HERE, "hf_tiny", m)
        os.makedirs(dst, exist_ok=True)
        for f in FILES:
            p = os.path.join(src, f)
            if os.path.exists(p):
                shutil.copyfile(p, os.path.join(dst, f))
                os.chmod(os.path.join(dst, f), 0o644)


def extract_vectors(names, filename, source="lrp_reference_test.cpp"):
    text = open(os.path.join(REF, "tests", source)).read()
    out = {}
    for name in names:
        m = re.search(r"const std::vector<float> %s = \{([^}]*)\};" % name, text)
        if m is None:
            raise RuntimeError("missing " + name)
        out[name] = [float(v.strip().rstrip("f")) for v in m.group(1).split(",") if v.strip()]
    with open(os.path.join(HERE, filename), "w") as f:
        json.dump(out, f, indent=1)


def extract_lxt_values():
    extract_vectors(("kMhaLogits", "kMhaRelevance", "kBlockLogits", "kBlockRelevance"), "lxt_values.json")


def extract_zennit_values():
    extract_vectors(("kMlpEpsilon1e6", "kMlpEpsilon025", "kMlpZPlus", "kMlpAlphaBeta21", "kMlpGamma025",
                     "kMlpEpsilonPlus", "kMlpEpsilonAlpha2Beta1", "kMlpEpsilonGammaBox"), "zennit_values.json")


def extract_hf_attention_values():
    extract_vectors(("kLlamaOutput", "kLlamaInputGrad", "kQwen2Output", "kQwen2InputGrad", "kQwen3Output",
                     "kQwen3InputGrad"), "hf_attention_values.json", "attention_reference_test.cpp")


def floats(literal):
    return [float(v.strip().rstrip("f")) for v in literal.split(",") if v.strip()]


def extract_legacy_block_values():
    text = open(os.path.join(REF, "tests", "transformer_block_test.cpp")).read()
    body = text[text.index("ValidatesAgainstIndependentAttnLRPReference"):]
    body = body[:body.index("\nTEST")]
    setters = {
        "norm1": r"block\.norm1\(\)\.set_gamma\(\{([^}]*)\}\)",
        "q": r"block\.mha\(\)\.q_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "k": r"block\.mha\(\)\.k_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "v": r"block\.mha\(\)\.v_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "out": r"block\.mha\(\)\.out_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "norm2": r"block\.norm2\(\)\.set_gamma\(\{([^}]*)\}\)",
        "gate": r"block\.swiglu\(\)\.gate_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "up": r"block\.swiglu\(\)\.up_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "down": r"block\.swiglu\(\)\.down_proj\(\)\.set_weight\(\{([^}]*)\}\)",
        "x": r"Tensor x\(Shape\(\{1, 2, 4\}\), &backend,\s*\{([^}]*)\}\)",
        "relevance_out": r"Tensor relevance_out\(Shape\(\{1, 2, 4\}\), &backend,\s*\{([^}]*)\}\)",
        "expected_y": r"expected_y2\{([^}]*)\}",
        "expected_r_x": r"expected_r_x\{([^}]*)\}",
    }
    m = re.search(r"TransformerBlock block\((\d+), (\d+), (\d+), &backend", body)
    out = {"d_model": int(m.group(1)), "heads": int(m.group(2)), "d_ff": int(m.group(3))}
    for key, pat in setters.items():
        found = re.search(pat, body)
        if found is None:
            raise RuntimeError("missing " + key)
        out[key] = floats(found.group(1))
    with open(os.path.join(HERE, "legacy_block_values.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    copy_hf_tiny()
    extract_lxt_values()
    extract_zennit_values()
    extract_hf_attention_values()
    extract_legacy_block_values()
    print("fixtures written under", HERE)
