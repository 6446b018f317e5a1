"""Pins the composition of oracle/llama_oracle.py (the CPU decoder used by
the config-5 greedy-token test) against the reference's own CPU model
forward, src/model/forward_cpu.cpp:58-174: live through oracle/_ref where
the reference tree was built, and through the committed fixture
tests/golden/ref_forward_tiny.npz (written by tests/golden/make_golden_llama.py
from that build) everywhere.  Checked: the prompt's logits, and the K/V-cached
decode path (one new token per call) against the reference's full causal
re-run of the same prefix.  Tiny Llama-shaped model, zero projection biases,
LM head tied to the embedding as in the reference.
"""
import os

import numpy as np
import pytest

from llama_oracle import LlamaOracle, ref_flat_weights, ref_forward_available, ref_forward_cpu
from llama_tiny import tiny_config, tiny_weights

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_forward_tiny.npz")
# Both sides run the same fp32/fp64 operations; the cached decode path
# reorders nothing but the attention over the cache, so agreement is to fp32
# rounding.
TOL = 2e-5


def _cached_logits(cfg, w, prompt, n_prefill):
    """Logits after each prefix length n_prefill..len(prompt): one prefill
    call, then one decode call per remaining token."""
    o = LlamaOracle(cfg, w, nthreads=2)
    rows = [o.forward(prompt[:n_prefill])]
    for t in prompt[n_prefill:]:
        rows.append(o.forward([int(t)]))
    return np.stack(rows)


def _check(cfg, w, prompt, ref_logits):
    scale = float(np.abs(ref_logits).max())
    full = LlamaOracle(cfg, w, nthreads=2).forward(prompt)
    assert np.abs(full - ref_logits[-1]).max() <= TOL * scale
    got = _cached_logits(cfg, w, prompt, 3)
    assert np.abs(got - ref_logits[2:]).max() <= TOL * scale
    assert np.argmax(got[-1]) == np.argmax(ref_logits[-1])


def test_llama_oracle_matches_reference_forward_golden():
    g = np.load(GOLDEN)
    cfg = tiny_config()
    w = tiny_weights(cfg, seed=31)
    assert np.array_equal(ref_flat_weights(w, cfg), g["flat_weights"]), "fixture weights moved"
    _check(cfg, w, g["prompt"], g["logits"])


@pytest.mark.skipif(not ref_forward_available(), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("seed", [1, 2])
def test_llama_oracle_matches_reference_forward_live(seed):
    cfg = tiny_config()
    w = tiny_weights(cfg, seed=seed)
    prompt = np.random.default_rng(100 + seed).integers(0, cfg.vocab_size, 9).astype(np.int64)
    _check(cfg, w, prompt, ref_forward_cpu(prompt, cfg, w))


def test_llama_oracle_planted_mistake_is_caught(monkeypatch):
    """A plausible composition slip planted in the oracle -- RoPE positions
    restarting at 0 on every call instead of continuing after the cache --
    must fail the same check."""
    import llama_oracle
    g = np.load(GOLDEN)
    cfg = tiny_config()
    w = tiny_weights(cfg, seed=31)
    rope = llama_oracle.oracle.apply_rope
    monkeypatch.setattr(llama_oracle.oracle, "apply_rope",
                        lambda q, k, hq, hkv, d, start, theta: rope(q, k, hq, hkv, d, 0, theta))
    got = _cached_logits(cfg, w, g["prompt"], 3)
    scale = float(np.abs(g["logits"]).max())
    assert np.abs(got[0] - g["logits"][2]).max() <= TOL * scale   # the prefill is unaffected
    assert np.abs(got[1:] - g["logits"][3:]).max() > 100 * TOL * scale
