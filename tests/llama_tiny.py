"""A tiny Llama-shaped model (weights as oracle/llama_oracle.py takes them)
for the CPU tests of the decoder oracle; the LM head is the embedding, as in
the reference forward it is pinned against."""
import types

import numpy as np


def tiny_config():
    return types.SimpleNamespace(vocab_size=64, hidden_size=32, num_layers=2, num_q_heads=4,
                                 num_kv_heads=2, head_dim=8, ffn_size=48, rms_eps=1e-5,
                                 rope_theta=10000.0)


def tiny_weights(cfg, seed):
    rng = np.random.default_rng(seed)
    v, h, f = cfg.vocab_size, cfg.hidden_size, cfg.ffn_size
    nqkv = (cfg.num_q_heads + 2 * cfg.num_kv_heads) * cfg.head_dim
    n = lambda *s: (0.3 * rng.standard_normal(s)).astype(np.float32)
    norm = lambda: (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    w = {"embed": n(v, h), "final_norm": norm(), "layers": []}
    w["lm_head"] = w["embed"]
    for _ in range(cfg.num_layers):
        w["layers"].append({"attn_norm": norm(), "ffn_norm": norm(), "w_qkv": n(nqkv, h),
                            "w_o": n(h, cfg.num_q_heads * cfg.head_dim),
                            "w_gate_up": n(2 * f, h), "w_down": n(h, f)})
    return w
