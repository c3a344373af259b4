"""Shared cases for the KV-cached decode tests: the oracle's greedy decode (a full forward over the
whole sequence at every step, as MakeNextTokenLogits does, generation.cpp:160-187) and the configs.

Test infrastructure only.
"""
import numpy as np

import oracle_ctypes as oc
from test_oracle import gemma_config


def oracle_greedy(cfg, params, prompts, new_tokens):
    """(ids (n, P + T), picked logits (n, T), smallest top-2 margin relative to max(1, max|logit|))."""
    lm = oc.oracle().lm(cfg, params)
    ids = np.asarray(prompts, dtype=np.int64)
    picked, margin = [], np.inf
    for _ in range(new_tokens):
        last = lm.forward(ids)[:, -1]
        nxt = last.argmax(-1)  # the first maximum, as Generate's greedy step takes it
        top2 = np.sort(last, -1)[:, -2:]
        margin = min(margin, float(((top2[:, 1] - top2[:, 0]) / np.maximum(1.0, np.abs(last).max(-1))).min()))
        picked.append(last[np.arange(len(nxt)), nxt])
        ids = np.concatenate([ids, nxt[:, None]], axis=1)
    return ids, np.stack(picked, 1), margin


def llama_decode_config():
    return oc.model_config(vocab_size=500, hidden_size=64, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
                           intermediate_size=96, rms_norm_eps=1e-5, rope_theta=100000.0)


def gemma_decode_config():
    """Gemma 3 variants with a window of 5 on layers 0 and 2: the decode runs past the window."""
    return gemma_config(vocab_size=300)


def qwen3_decode_config():
    """Qwen3-style: QK-Norm without sandwich norms, SiLU, GQA 4 / 2, llama3 RoPE scaling (the decode
    runs past its original context of 8)."""
    return gemma_config(vocab_size=257, hidden_size=64, num_heads=4, num_kv_heads=2, head_dim=16, hidden_act=0,
                        qk_norm=1, post_norms=0, norm_weight_offset=0.0, embed_scale=0.0, query_pre_attn_scalar=0.0,
                        sliding_window=0, sliding_layers=0, rope_local_base=0.0, rope_scaling=2, rope_factor=8.0,
                        rope_low_freq_factor=1.0, rope_high_freq_factor=4.0, rope_original_max_position=8)


CASES = {
    # name: (config factory, param seed, param std, prompt seed, n, prompt, new tokens)
    "llama": (llama_decode_config, 41, 0.2, 1, 3, 7, 12),
    "gemma": (gemma_decode_config, 43, 0.05, 2, 2, 6, 11),
    "qwen3": (qwen3_decode_config, 47, 0.1, 3, 3, 5, 12),
}


def case(name):
    make, pseed, std, iseed, n, prompt, new = CASES[name]
    cfg = make()
    params = oc.synthetic_params(cfg, pseed, std=std)
    prompts = np.random.RandomState(iseed).randint(0, cfg.vocab_size, size=(n, prompt))
    return cfg, params, prompts, new
