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

    def forward(self, tokens, logit_rows=None):
        """Run the new token ids at positions pos.. ; returns the fp32 logits
        of the last one, or [len(logit_rows)][V] for those rows of this call
        (teacher forcing: one causal pass over a prompt and the tokens a model
        generated gives every generated position's logits)."""
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
        if logit_rows is None:
            last = oracle.rmsnorm(h[-1:], w["final_norm"], c.rms_eps)
            return self._mm(last, w["lm_head"])[0]
        rows = oracle.rmsnorm(h[np.asarray(logit_rows, np.int64)], w["final_norm"], c.rms_eps)
        return self._mm(rows, w["lm_head"])


def top2_margin(logits):
    """Top-1 minus top-2 logit (the reference's near-tie measure,
    docs/GATES.md)."""
    two = np.partition(logits, -2)[-2:]
    return float(two.max() - two.min())


# ---------------------------------------------------------------------------
# The reference's own CPU model forward (src/model/forward_cpu.cpp, compiled
# where it lies by `make -C oracle ref` into _ref/libref_forward.so), used by
# tests to pin LlamaOracle's composition.  Absent where the reference tree is.
import ctypes  # noqa: E402
import os  # noqa: E402

REF_FORWARD_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref",
                               "libref_forward.so")
_ref_fwd = None


def ref_forward_available():
    return os.path.exists(REF_FORWARD_LIB)


def ref_flat_weights(weights, cfg):
    """Pack LlamaOracle weights in ref_forward_shim.cpp's order: embed,
    final_norm, then per layer input/post-attention norms, q, k, v, o, gate,
    up, down (fused q|k|v and gate|up split back into their parts)."""
    hq, hkv, d, f = cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.ffn_size
    parts = [weights["embed"], weights["final_norm"]]
    for lw in weights["layers"]:
        qkv = lw["w_qkv"]
        parts += [lw["attn_norm"], lw["ffn_norm"], qkv[:hq * d], qkv[hq * d:(hq + hkv) * d],
                  qkv[(hq + hkv) * d:], lw["w_o"], lw["w_gate_up"][:f], lw["w_gate_up"][f:],
                  lw["w_down"]]
    return np.ascontiguousarray(np.concatenate([np.ravel(p) for p in parts]), np.float32)


def ref_forward_cpu(ids, cfg, weights):
    """Logits [S][V] of the reference forward over `ids` (biases zero, LM
    head = embedding, as the reference ties them)."""
    global _ref_fwd
    if _ref_fwd is None:
        lib = ctypes.CDLL(REF_FORWARD_LIB)
        f = lib.ref_forward_cpu
        f.restype = ctypes.c_int
        f.argtypes = [np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS"), ctypes.c_int64] + \
            [ctypes.c_int] * 7 + [ctypes.c_float] * 2 + \
            [np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")] * 2
        _ref_fwd = f
    ids = np.ascontiguousarray(ids, np.int64)
    out = np.zeros((ids.size, cfg.vocab_size), np.float32)
    rc = _ref_fwd(ids, ids.size, cfg.vocab_size, cfg.hidden_size, cfg.ffn_size, cfg.num_layers,
                  cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.rms_eps, cfg.rope_theta,
                  ref_flat_weights(weights, cfg), out)
    if rc != 0:
        raise ValueError("ref_forward_cpu: num_q_heads * head_dim must equal hidden_size")
    return out
