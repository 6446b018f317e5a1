"""CPU restatement of the reference's decoder forward, for the config-5 parity test.

TEST INFRASTRUCTURE ONLY: loaded by tests/ (never by the product path).

Restates src/model/forward_cpu.cpp:58-174 layer by layer with this
directory's restated ops (RMSNorm ops.cpp:26-51, matmul with double
accumulation :53-114, RoPE :165-221, causal GQA :223-284, SwiGLU :286-297),
all in fp32 over the fp16 weights read back from the GPU model.  Two changes
of form, not of arithmetic: the model is Llama-style (no projection biases,
untied LM head, fused q/k/v and gate/up weights that are split here), and
the K/V of earlier positions are cached so that each new position costs one
row -- every row's attention only sees keys up to its own position, and the
decode rows use the restated decode attention, which is pinned to equal the
last causal row (tests/test_oracle.py).
"""
import numpy as np

import oracle


class LlamaOracle:
    def __init__(self, cfg, weights, nthreads=8):
        """cfg: object with the kvhp_llama_config fields; weights: dict with
        float32 'embed' [V][H], 'lm_head' [V][H], 'final_norm' [H] and
        'layers': list of dicts 'attn_norm', 'ffn_norm', 'w_qkv', 'w_o',
        'w_gate_up', 'w_down' (row-major [out][in])."""
        self.c = cfg
        self.w = weights
        self.nt = nthreads
        self.pos = 0
        hkv, d = cfg.num_kv_heads, cfg.head_dim
        self.kc = [np.zeros((0, hkv, d), np.float32) for _ in range(cfg.num_layers)]
        self.vc = [np.zeros((0, hkv, d), np.float32) for _ in range(cfg.num_layers)]

    def _mm(self, a, w):
        return oracle.matmul_transB(a, w, nthreads=self.nt)

    def forward(self, tokens):
        """Run the new token ids at positions pos.. ; returns the fp32 logits
        of the last one."""
        c, w = self.c, self.w
        hq, hkv, d, f = c.num_q_heads, c.num_kv_heads, c.head_dim, c.ffn_size
        ids = np.asarray(tokens, np.int64)
        s = ids.size
        start = self.pos
        h = w["embed"][ids].astype(np.float32)                       # [s][H]
        for li, lw in enumerate(w["layers"]):
            xn = oracle.rmsnorm(h, lw["attn_norm"], c.rms_eps)
            qkv = self._mm(xn, lw["w_qkv"])
            q = qkv[:, :hq * d]
            k = qkv[:, hq * d:(hq + hkv) * d]
            v = qkv[:, (hq + hkv) * d:]
            q, k = oracle.apply_rope(q, k, hq, hkv, d, start, c.rope_theta)
            kc = np.concatenate([self.kc[li], k.reshape(s, hkv, d)])
            vc = np.concatenate([self.vc[li], v.reshape(s, hkv, d)])
            self.kc[li], self.vc[li] = kc, vc
            if start == 0:
                attn = oracle.causal_gqa(q.reshape(s, hq, d), kc, vc, hq, hkv, d,
                                         nthreads=self.nt).reshape(s, hq * d)
            else:
                rows = []
                for i in range(s):
                    n = start + i + 1
                    kk = np.ascontiguousarray(kc[:n].transpose(1, 0, 2))[None]
                    vv = np.ascontiguousarray(vc[:n].transpose(1, 0, 2))[None]
                    rows.append(oracle.decode_attention(q[i].reshape(1, hq, d), kk, vv,
                                                        np.array([n], np.int32), hq, hkv, d)
                                .reshape(hq * d))
                attn = np.stack(rows)
            h = h + self._mm(attn, lw["w_o"])
            xn = oracle.rmsnorm(h, lw["ffn_norm"], c.rms_eps)
            gu = self._mm(xn, lw["w_gate_up"])
            act = oracle.swiglu(np.ascontiguousarray(gu[:, :f]), np.ascontiguousarray(gu[:, f:]))
            h = h + self._mm(act, lw["w_down"])
        self.pos += s
        last = oracle.rmsnorm(h[-1:], w["final_norm"], c.rms_eps)
        return self._mm(last, w["lm_head"])[0]


def top2_margin(logits):
    """Top-1 minus top-2 logit (the reference's near-tie measure,
    docs/GATES.md)."""
    two = np.partition(logits, -2)[-2:]
    return float(two.max() - two.min())
