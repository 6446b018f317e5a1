"""Write tests/golden/ref_forward_tiny.npz from the reference's own CPU model
forward (src/model/forward_cpu.cpp compiled where it lies by
`make -C oracle ref` into oracle/_ref/libref_forward.so; this container
only).  A tiny Llama-shaped model (2 layers, 4 q / 2 kv heads of 8, FFN 48,
vocab 64) with seeded weights; the fixture stores the weights, a 7-id prompt
and the reference's logits for every prefix, so oracle/llama_oracle.py can
be pinned where the reference tree is absent.

    python tests/golden/make_golden_llama.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))
import llama_oracle  # noqa: E402

sys.path.insert(0, os.path.dirname(HERE))
from llama_tiny import tiny_config, tiny_weights  # noqa: E402


def main():
    if not llama_oracle.ref_forward_available():
        raise SystemExit("oracle/_ref/libref_forward.so missing: run `make -C oracle ref` first")
    cfg = tiny_config()
    w = tiny_weights(cfg, seed=31)
    prompt = np.random.default_rng(32).integers(0, cfg.vocab_size, 7).astype(np.int64)
    logits = llama_oracle.ref_forward_cpu(prompt, cfg, w)
    out = {"prompt": prompt, "logits": logits, "flat_weights": llama_oracle.ref_flat_weights(w, cfg)}
    path = os.path.join(HERE, "ref_forward_tiny.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
