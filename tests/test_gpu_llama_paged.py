"""Batched serving over caller-owned pages (kvhp_llama_prefill_paged /
kvhp_llama_decode_paged): the reference runner contract
(docs/runner_interface.md:18-53) with the page pool and block tables in the
caller's hands.

Several sequences live in one pool whose pages are dealt out in a seeded
random order.  One of them shares another's first two full pages ("share"
prefix mode: its prefill writes go through a table in which the shared
pages are -1).  Each is checked against a batch-1 model with the same seed
(same weights) fed the same tokens:
  * prefill logits are bit-identical (the same kernels run on the same
    prompt; only the page placement and the skipped shared-page writes
    differ);
  * batched decode logits agree to 2% of the logit scale (B-row GEMMs
    against the batch-1 GEMVs: fp16 activations rounded in another order),
    and a greedy token may differ only where the batch-1 logits' gap between
    the two tokens is at most twice the measured max |logit diff| (the only
    flips that difference can cause);
  * one sequence's decode logits also against the CPU restatement of the
    reference forward (oracle/llama_oracle.py), same bound;
  * the shared pages keep the first sequence's K/V bit for bit through the
    second's prefill and every decode step, and pages no table names stay
    zero (an idle batch row, position -1 and no pages, writes nothing).
    Whether the skipped writes would have changed any bit is left to the
    C++ engine test, which recomputes the shared prefix with other K/V.
"""
import numpy as np
import pytest

import kvhp
from llama_oracle import LlamaOracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

PAGE = 16


def _cfg(ffn=1024):
    return kvhp.LlamaConfig(2048, 512, 3, 8, 2, 64, ffn, 1e-5, 10000.0, 0)


def _weights(model, cfg):
    f32 = lambda a: a.astype(np.float32)
    v, h, f = cfg.vocab_size, cfg.hidden_size, cfg.ffn_size
    nqkv = (cfg.num_q_heads + 2 * cfg.num_kv_heads) * cfg.head_dim
    w = {"embed": f32(model.tensor(-1, kvhp.LLAMA_EMBED)).reshape(v, h),
         "lm_head": f32(model.tensor(-1, kvhp.LLAMA_LM_HEAD)).reshape(v, h),
         "final_norm": f32(model.tensor(-1, kvhp.LLAMA_FINAL_NORM)), "layers": []}
    for li in range(cfg.num_layers):
        w["layers"].append({
            "attn_norm": f32(model.tensor(li, kvhp.LLAMA_ATTN_NORM)),
            "ffn_norm": f32(model.tensor(li, kvhp.LLAMA_FFN_NORM)),
            "w_qkv": f32(model.tensor(li, kvhp.LLAMA_W_QKV)).reshape(nqkv, h),
            "w_o": f32(model.tensor(li, kvhp.LLAMA_W_O)).reshape(h, h),
            "w_gate_up": f32(model.tensor(li, kvhp.LLAMA_W_GATE_UP)).reshape(2 * f, h),
            "w_down": f32(model.tensor(li, kvhp.LLAMA_W_DOWN)).reshape(h, f)})
    return w


def _close(got, ref, what):
    scale = max(float(np.abs(ref).max()), 1.0)
    diff = float(np.abs(got - ref).max())
    assert diff < 0.02 * scale, f"{what}: max |logit diff| {diff:.4f} (scale {scale:.2f})"
    tok, rtok = int(np.argmax(got)), int(np.argmax(ref))
    if tok != rtok:
        gap = float(ref[rtok] - ref[tok])
        print(f"{what}: token {tok} != {rtok}, gap {gap:.5f}, max |logit diff| {diff:.5f}")
        assert gap <= 2 * diff, f"{what}: token {tok} != {rtok} with gap {gap:.5f} > 2 x {diff:.5f}"
    return diff


def test_paged_runner_matches_batch1_runner_and_oracle():
    cfg = _cfg()
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    seed, max_ctx, steps = 21, 128, 5
    P, max_pages = 48, 8
    rng = np.random.default_rng(4242)
    dev = "cuda"

    model = kvhp.LlamaModel(cfg, seed=seed, max_ctx=max_ctx)
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device=dev)

    # sequences 0-2 own their pages; sequence 3 shares sequence 0's first
    # two (full) pages and continues with its own suffix
    lens = [37, 21, 50]
    prompts = [rng.integers(0, V, n).astype(np.int32) for n in lens]
    prompts.append(np.concatenate([prompts[0][:32], rng.integers(0, V, 9).astype(np.int32)]))
    order = rng.permutation(P).tolist()
    tables = np.full((5, max_pages), -1, np.int32)      # row 4: an idle batch row
    refs = np.zeros(P, np.int32)

    def take(n):
        out = [order.pop() for _ in range(n)]
        refs[out] += 1
        return out

    for s in range(3):
        tables[s, :(lens[s] + steps + PAGE - 1) // PAGE] = take((lens[s] + steps + PAGE - 1) // PAGE)
    tables[3, :2] = tables[0, :2]
    refs[tables[0, :2]] += 1
    n3 = (len(prompts[3]) + steps + PAGE - 1) // PAGE
    tables[3, 2:n3] = take(n3 - 2)
    write_tables = np.where((tables >= 0) & (refs[np.maximum(tables, 0)] > 1), -1, tables)
    bt = torch.from_numpy(tables).to(dev)
    wbt = torch.from_numpy(write_tables).to(dev)
    assert write_tables[3, 0] == -1 and write_tables[0, 0] == -1 and write_tables[3, 2] >= 0

    # references: one batch-1 model per sequence, same seed = same weights
    singles = [kvhp.LlamaModel(cfg, seed=seed, max_ctx=max_ctx) for _ in range(4)]
    first, prefill_logits = [], []
    pool5 = pool.view(L, 2, Hkv, P, PAGE, D)
    for s in range(4):
        # sequence 0 writes its shared pages itself (it owns them first): its
        # prefill goes through the block table, the others through the write
        # table.  Prefill attends the recomputed prompt, so even sequence 3
        # matches its batch-1 model bit for bit.
        row = bt[0] if s == 0 else wbt[s]
        tok, lg = model.prefill_paged(prompts[s], pool, P, row, max_pages)
        rtok, rlg = singles[s].prefill(prompts[s])
        assert np.array_equal(lg, rlg), f"sequence {s}: prefill logits differ"
        assert tok == rtok
        first.append(tok)
        prefill_logits.append(lg)
        if s == 0:   # sequence 0's prompt K/V on the pages sequence 3 will share
            torch.cuda.synchronize()
            k0 = [pool5[:, :, :, int(tables[0, i])].clone() for i in range(2)]

    oracle = LlamaOracle(cfg, _weights(model, cfg), nthreads=8)
    _close(prefill_logits[1], oracle.forward(prompts[1]), "sequence 1 prefill vs oracle")

    B = 5
    cur = list(first) + [0]
    seq = [len(p) for p in prompts] + [0]
    logits = torch.empty(B, V, dtype=torch.float32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    diffs = []
    for st in range(steps):
        # bump, then write at num_tokens - 1; the idle row gets position -1, 0 keys
        pos = np.array([seq[b] if b < 4 else -1 for b in range(B)], np.int32)
        sl = np.array([seq[b] + 1 if b < 4 else 0 for b in range(B)], np.int32)
        model.decode_paged(torch.tensor(cur, dtype=torch.int32, device=dev), pool, P, bt,
                           max_pages, torch.from_numpy(pos).to(dev), torch.from_numpy(sl).to(dev),
                           int(sl.max()), logits, nxt)
        torch.cuda.synchronize()
        got = logits.cpu().numpy()
        toks = nxt.cpu().numpy()
        for b in range(4):
            assert toks[b] == int(np.argmax(got[b])), "device argmax != host argmax of its logits"
            _, rlg = singles[b].decode_step(int(cur[b]))   # teacher-forced, same token
            diffs.append(_close(got[b], rlg, f"step {st} sequence {b}"))
        olg = oracle.forward([int(cur[1])])
        diffs.append(_close(got[1], olg, f"step {st} sequence 1 vs oracle"))
        cur = [int(t) for t in toks[:4]] + [0]
        seq = [x + 1 for x in seq[:4]] + [0]
    print(f"max |logit diff| batched vs batch-1 / oracle: {max(diffs):.4f}")

    # shared pages unchanged by sequence 3's prefill and every decode step;
    # pages in no table never written
    for i in range(2):
        assert torch.equal(pool5[:, :, :, int(tables[0, i])], k0[i])
    unused = sorted(set(range(P)) - set(tables[tables >= 0].tolist()))
    assert unused and all(bool((pool5[:, :, :, p] == 0).all()) for p in unused)
    for m in singles:
        m.close()
    model.close()


@pytest.mark.parametrize("ffn", [1024, 5632])
def test_paged_runner_large_batch_path_matches_fused_path(ffn):
    """Batches above 32 run on library GEMMs with separate norm / RoPE /
    SwiGLU launches; up to 32 on the fused batched projections.  One step
    of 40 sequences on one copy of the pool against the same step as two
    calls of 20 on another copy: logits within 2% of the scale, tokens equal
    outside near-ties, and the appended K/V rows within fp16 rounding.  With
    the config-5 FFN width (5632) the calls of 20 split the down projection
    over K (kvhp_gemv_residual_rows_ws with the model's own partials)."""
    cfg = _cfg(ffn)
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    B, plen, max_pages = 40, 9, 2
    P = B * max_pages
    model = kvhp.LlamaModel(cfg, seed=8, max_ctx=64)
    rng = np.random.default_rng(99)
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
    bt = torch.from_numpy(rng.permutation(P).astype(np.int32).reshape(B, max_pages)).cuda()
    toks = []
    for b in range(B):
        t, _ = model.prefill_paged(rng.integers(0, V, plen).astype(np.int32), pool, P, bt[b],
                                   max_pages)
        toks.append(t)
    toks = torch.tensor(toks, dtype=torch.int32, device="cuda")
    pos = torch.full((B,), plen, dtype=torch.int32, device="cuda")
    sl = pos + 1
    pool2 = pool.clone()
    lg_a = torch.empty(B, V, dtype=torch.float32, device="cuda")
    nx_a = torch.empty(B, dtype=torch.int32, device="cuda")
    model.decode_paged(toks, pool, P, bt, max_pages, pos, sl, plen + 1, lg_a, nx_a)
    lg_b = torch.empty_like(lg_a)
    nx_b = torch.empty_like(nx_a)
    for h in (slice(0, 20), slice(20, 40)):
        model.decode_paged(toks[h].contiguous(), pool2, P, bt[h].contiguous(), max_pages,
                           pos[h].contiguous(), sl[h].contiguous(), plen + 1, lg_b[h], nx_b[h])
    torch.cuda.synchronize()
    a, b = lg_a.cpu().numpy(), lg_b.cpu().numpy()
    for r in range(B):
        _close(a[r], b[r], f"row {r}")
    diff = (pool.float() - pool2.float()).abs()
    assert float(diff.max()) <= 0.05 * float(pool.float().abs().max())
    model.close()


def test_paged_runner_single_sequence_step_is_the_batch1_step():
    """A batch of one runs the batch-1 step's kernels: with the same split
    plan (max_seq_len = the batch-1 model's context) its logits equal the
    batch-1 model's bit for bit, over a pool and block table of its own."""
    cfg = _cfg()
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    max_ctx, P, max_pages = 96, 40, 6
    rng = np.random.default_rng(5150)
    prompt = rng.integers(0, V, 45).astype(np.int32)
    model = kvhp.LlamaModel(cfg, seed=17, max_ctx=max_ctx)
    single = kvhp.LlamaModel(cfg, seed=17, max_ctx=max_ctx)
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
    bt = torch.from_numpy(rng.permutation(P)[:max_pages].astype(np.int32)).cuda()
    tok, lg = model.prefill_paged(prompt, pool, P, bt, max_pages)
    rtok, rlg = single.prefill(prompt)
    assert tok == rtok and np.array_equal(lg, rlg)
    logits = torch.empty(1, V, dtype=torch.float32, device="cuda")
    nxt = torch.empty(1, dtype=torch.int32, device="cuda")
    seq = len(prompt)
    for step in range(4):
        pos = torch.tensor([seq], dtype=torch.int32, device="cuda")
        model.decode_paged(torch.tensor([tok], dtype=torch.int32, device="cuda"), pool, P,
                           bt.view(1, -1), max_pages, pos, pos + 1, max_ctx, logits, nxt)
        rtok, rlg = single.decode_step(tok)
        torch.cuda.synchronize()
        assert np.array_equal(logits.cpu().numpy()[0], rlg), f"step {step}: logits differ"
        assert int(nxt.item()) == rtok
        tok, seq = rtok, seq + 1
    single.close()
    model.close()


@pytest.mark.parametrize("suffix", [1, 7, 32, 33, 70])
def test_cached_prefix_prefill_matches_full_prefill(suffix):
    """kvhp_llama_prefill_cached over a prefix whose K/V another prefill
    wrote: up to 32 suffix rows run as one batched decode step (one row on
    the batch-1 kernels), longer suffixes layer by layer with a batched
    decode-attention call; either way the last position's logits match the
    whole-prompt prefill within 2 % of the scale (near-tie rule for the
    token), the prefix pages keep their bytes and the suffix K/V land in the
    following pages."""
    cfg = _cfg()
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    cached, max_pages = 48, 10
    n = cached + suffix
    P = 2 * max_pages
    model = kvhp.LlamaModel(cfg, seed=77, max_ctx=160)
    rng = np.random.default_rng(suffix)
    prompt = rng.integers(0, V, n).astype(np.int32)
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
    pool5 = pool.view(L, 2, Hkv, P, PAGE, D)
    perm = rng.permutation(P).astype(np.int32)
    bt_a = torch.from_numpy(perm[:max_pages]).cuda()             # whole-prompt sequence
    bt_b = torch.from_numpy(np.concatenate([perm[:3], perm[max_pages:2 * max_pages - 3]])).cuda()
    _, ref = model.prefill_paged(prompt, pool, P, bt_a, max_pages)
    torch.cuda.synchronize()
    prefix = pool5[:, :, :, perm[:3]].clone()
    wt = bt_b.clone()
    wt[:3] = -1                                                   # shared prefix pages
    tok, lg = model.prefill_cached(prompt, cached, pool, P, bt_b, max_pages, write_table=wt)
    torch.cuda.synchronize()
    _close(lg, ref, f"suffix {suffix}")
    assert torch.equal(pool5[:, :, :, perm[:3]], prefix)
    # the suffix K/V: B's pages against A's, position by position
    for t in range(cached, n, max(1, suffix // 5)):
        a = pool5[:, :, :, int(bt_a[t // PAGE]), t % PAGE].float()
        b = pool5[:, :, :, int(bt_b[t // PAGE]), t % PAGE].float()
        assert float((a - b).abs().max()) <= 0.02 * max(float(a.abs().max()), 1.0), t
    model.close()


def test_paged_runner_qwen_shapes_use_the_fallback_projections():
    """The reference runner's own model shapes (docs/runner_interface.md:
    hidden 896, 14 query / 2 KV heads -- G = 7 --, head_dim 64; here 2
    layers, FFN 4864, vocab 3000): hidden 896 is not a multiple of 256, so
    batches of 2..32 take the library-GEMM path and a batch of one the
    generic batch-1 GEMVs.  Three sequences, prefill and four decode steps,
    against batch-1 models of the same weights (2 % of the logit scale,
    near-tie rule)."""
    cfg = kvhp.LlamaConfig(3000, 896, 2, 14, 2, 64, 4864, 1e-6, 1000000.0, 0)
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    P, max_pages = 24, 6
    rng = np.random.default_rng(896)
    model = kvhp.LlamaModel(cfg, seed=9, max_ctx=96)
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
    bt = torch.from_numpy(rng.permutation(P)[:3 * max_pages].astype(np.int32).reshape(3, max_pages)).cuda()
    prompts = [rng.integers(0, V, n).astype(np.int32) for n in (30, 17, 52)]
    singles = [kvhp.LlamaModel(cfg, seed=9, max_ctx=96) for _ in prompts]
    toks = []
    for i, pr in enumerate(prompts):
        tok, lg = model.prefill_paged(pr, pool, P, bt[i], max_pages)
        rtok, rlg = singles[i].prefill(pr)
        assert tok == rtok and np.array_equal(lg, rlg), f"prefill {i}"
        toks.append(tok)
    seq = [len(p) for p in prompts]
    for B in (3, 1):                      # library GEMMs, then the batch-1 kernels
        for step in range(2):
            logits = torch.empty(B, V, dtype=torch.float32, device="cuda")
            nxt = torch.empty(B, dtype=torch.int32, device="cuda")
            pos = torch.tensor(seq[:B], dtype=torch.int32, device="cuda")
            model.decode_paged(torch.tensor(toks[:B], dtype=torch.int32, device="cuda"), pool, P,
                               bt[:B].contiguous(), max_pages, pos, pos + 1, max(seq[:B]) + 1,
                               logits, nxt)
            torch.cuda.synchronize()
            got = logits.cpu().numpy()
            for b in range(B):
                _, rlg = singles[b].decode_step(toks[b])
                _close(got[b], rlg, f"B={B} step {step} sequence {b}")
                toks[b] = int(nxt[b].item())
                seq[b] += 1
    for m in singles:
        m.close()
    model.close()


def test_decode_paged_graph_capture_needs_reserve():
    """kvhp_llama_decode_paged under HIP graph capture: without
    kvhp_llama_reserve its first call cannot size the model's buffers and
    returns KVHP_ERR_WORKSPACE (nothing allocated, the capture stays valid);
    after reserve(16, ...) a captured 16-row step (with the config-5 FFN
    width, so the down projection's K-split partials are used) replays with
    logits and appended K/V bit-identical to the same step run eagerly on a
    copy of the pool -- also after eager calls in between, one of which
    grows the buffers past the reservation (earlier buffers stay allocated,
    so the graph's addresses stay valid)."""
    cfg = _cfg(5632)
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    B, plen, max_pages = 16, 9, 2
    P = 2 * B * max_pages
    rng = np.random.default_rng(4242)
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
    bt = torch.from_numpy(rng.permutation(P).astype(np.int32).reshape(2 * B, max_pages)).cuda()
    model = kvhp.LlamaModel(cfg, seed=12, max_ctx=64)
    toks = []
    for b in range(2 * B):
        t, _ = model.prefill_paged(rng.integers(0, V, plen).astype(np.int32), pool, P, bt[b],
                                   max_pages)
        toks.append(t)
    toks = torch.tensor(toks, dtype=torch.int32, device="cuda")
    pos = torch.full((2 * B,), plen, dtype=torch.int32, device="cuda")
    sl = pos + 1
    lg = torch.empty(2 * B, V, dtype=torch.float32, device="cuda")
    nx = torch.empty(2 * B, dtype=torch.int32, device="cuda")
    cap_len = plen + 1

    def step(n, pl, out_lg, out_nx):
        model.decode_paged(toks[:n], pl, P, bt[:n], max_pages, pos[:n], sl[:n], cap_len,
                           out_lg[:n], out_nx[:n])

    torch.cuda.synchronize()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    g0 = torch.cuda.CUDAGraph()
    err = None
    pool_try = pool.clone()
    torch.cuda.synchronize()
    with torch.cuda.stream(cs):
        g0.capture_begin()
        try:
            step(B, pool_try, lg, nx)
        except kvhp.KVHPError as e:
            err = e
        finally:
            g0.capture_end()
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    del g0
    assert err is not None and err.code == kvhp.KVHP_ERR_WORKSPACE, err

    model.reserve(B, cap_len)
    pool_g = pool.clone()
    g = torch.cuda.CUDAGraph()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cs):
        step(B, pool_g, lg, nx)
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    pool_e = pool.clone()
    lg_e = torch.empty_like(lg)
    nx_e = torch.empty_like(nx)
    step(B, pool_e, lg_e, nx_e)              # eager reference of the captured step
    torch.cuda.synchronize()
    lg_ref, nx_ref, pool_ref = lg_e[:B].clone(), nx_e[:B].clone(), pool_e.clone()
    scratch = pool.clone()
    for i, between in enumerate((None, 4, 2 * B)):
        if between:
            # eager calls on another pool copy: a smaller batch (reserved), then
            # a larger one, which grows the buffers past the reservation
            step(between, scratch, lg_e, nx_e)
            torch.cuda.synchronize()
        pool_g.copy_(pool)
        lg.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(lg[:B], lg_ref), f"replay {i}: logits differ from the eager step"
        assert torch.equal(nx[:B], nx_ref), f"replay {i}: tokens differ"
        assert torch.equal(pool_g, pool_ref), f"replay {i}: appended K/V differ"
    del g
    model.close()


@pytest.mark.parametrize("shape,B,plen,ragged", [("d64", 3, 13, False), ("d64", 17, 13, False),
                                                 ("d128", 2, 4190, False), ("d32", 5, 20, False),
                                                 ("d64", 26, 700, True), ("d64", 9, 300, True)])
def test_batched_step_is_the_exported_operators(shape, B, plen, ragged):
    """The runner's batched step keeps its hidden state, attention output
    and SwiGLU output row-tiled between launches; the exported operators
    take row-major activations.  One step of B sequences through
    kvhp_llama_decode_paged against the same step composed from the
    exported calls (embedding, kvhp_rmsnorm_qkv_rope_append_rows_tiled,
    kvhp_decode_attention, kvhp_gemv_residual_rows_tiled for o and down,
    the SwiGLU and LM-head projections) on weights tiled with
    kvhp_rows_tile_weights: logits, greedy tokens and the appended K/V bit
    for bit.  Every attention kernel that writes the tiled output runs:
    d64 (FFN 5632) B = 3 one split per sequence, written by the split
    kernel (fixed chunks, four waves per split), B = 17 balanced splits
    and the per-KV-head merge, with the down projection split over K and
    15 padding rows; d128 B = 2 at 4191 keys 33 fixed splits and the
    per-query-head merge; d32 the generic kernel.  Ragged: prompt lengths
    drawn from 1..plen (balanced splits of different counts per sequence,
    one-split and many-split sequences in one launch) and one idle row
    (position -1, no keys: zero attention output, no page write)."""
    cfg = {"d64": _cfg(5632),
           "d128": kvhp.LlamaConfig(2048, 1024, 2, 8, 2, 128, 1024, 1e-5, 10000.0, 0),
           "d32": kvhp.LlamaConfig(2048, 256, 2, 8, 2, 32, 512, 1e-5, 10000.0, 0)}[shape]
    L, Hq, Hkv, D, V = (cfg.num_layers, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim,
                        cfg.vocab_size)
    H, F, eps, theta = cfg.hidden_size, cfg.ffn_size, cfg.rms_eps, cfg.rope_theta
    max_pages = (plen + 1 + PAGE - 1) // PAGE
    P = B * max_pages
    rng = np.random.default_rng(777 + B)
    model = kvhp.LlamaModel(cfg, seed=31, max_ctx=max(64, plen + 1))
    pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
    bt = torch.from_numpy(rng.permutation(P).astype(np.int32).reshape(B, max_pages)).cuda()
    lens = rng.integers(1, plen + 1, B) if ragged else np.full(B, plen)
    idle = B - 1 if ragged else -1
    toks = torch.tensor([model.prefill_paged(rng.integers(0, V, int(lens[b])).astype(np.int32),
                                             pool, P, bt[b], max_pages)[0] if b != idle else 0
                         for b in range(B)], dtype=torch.int32, device="cuda")
    pos = torch.tensor([int(lens[b]) if b != idle else -1 for b in range(B)], dtype=torch.int32,
                       device="cuda")
    sl = torch.tensor([int(lens[b]) + 1 if b != idle else 0 for b in range(B)], dtype=torch.int32,
                      device="cuda")
    max_len = plen + 1

    pool_r = pool.clone()
    lg_r = torch.empty(B, V, dtype=torch.float32, device="cuda")
    nx_r = torch.empty(B, dtype=torch.int32, device="cuda")
    model.decode_paged(toks, pool_r, P, bt, max_pages, pos, sl, max_len, lg_r, nx_r)

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def tiled(kind, W, N, K):
        out = torch.empty(kvhp.rows_tiled_bytes(kind, N, K, Hq, Hkv, D) // 2,
                          dtype=torch.float16, device="cuda")
        kvhp.rows_tile_weights(kind, dev(W), N, K, out, Hq, Hkv, D)
        return out

    pool_e = pool.clone()
    pools = pool_e.view(L, 2, Hkv, P, PAGE, D)
    x = torch.empty(B, H, dtype=torch.float16, device="cuda")
    kvhp.embedding(toks, dev(model.tensor(-1, kvhp.LLAMA_EMBED)), x, B, H, V)
    q = torch.empty(B, Hq * D, dtype=torch.float16, device="cuda")
    attn = torch.empty(B, Hq * D, dtype=torch.float16, device="cuda")
    act = torch.empty(B, F, dtype=torch.float16, device="cuda")
    ws = torch.empty(max(kvhp.decode_workspace_bytes(B, Hq, Hkv, D, max_len), 16),
                     dtype=torch.uint8, device="cuda")
    part = torch.empty(max(kvhp.gemv_rows_workspace_bytes(H, F, B), 16), dtype=torch.uint8,
                       device="cuda")
    assert (kvhp.gemv_rows_workspace_bytes(H, F, B) > 0) == (B * F > 81920)
    if shape == "d128":   # 33 splits of 128 keys: the per-query-head merge (>= 64 KB of partials)
        assert kvhp.decode_workspace_bytes(B, Hq, Hkv, D, max_len) == 4 * B * Hq * 33 * (D + 2)
    for li in range(L):
        w = lambda which: model.tensor(li, which)
        kvhp.rmsnorm_qkv_rope_append_rows_tiled(
            tiled(kvhp.ROWS_QKV, w(kvhp.LLAMA_W_QKV), 0, H), x, dev(w(kvhp.LLAMA_ATTN_NORM)), eps,
            pos, theta, q, pools[li, 0], pools[li, 1], bt, Hq, Hkv, D, H, B)
        kvhp.decode_attention(q, kvhp.paged_view(pools[li, 0], bt), kvhp.paged_view(pools[li, 1], bt),
                              sl, attn, Hq, Hkv, D, max_len, 0, ws)
        kvhp.gemv_residual_rows_tiled(tiled(kvhp.ROWS_PLAIN, w(kvhp.LLAMA_W_O), H, Hq * D), attn,
                                      x, x, H, Hq * D, B)
        kvhp.rmsnorm_gemv_swiglu_rows_tiled(tiled(kvhp.ROWS_SWIGLU, w(kvhp.LLAMA_W_GATE_UP), F, H),
                                            x, dev(w(kvhp.LLAMA_FFN_NORM)), eps, act, F, H, B)
        kvhp.gemv_residual_rows_tiled(tiled(kvhp.ROWS_PLAIN, w(kvhp.LLAMA_W_DOWN), H, F), act, x, x,
                                      H, F, B, workspace=part)
    lg_e = torch.empty(B, V, dtype=torch.float32, device="cuda")
    kvhp.rmsnorm_gemv_rows_tiled(tiled(kvhp.ROWS_PLAIN, model.tensor(-1, kvhp.LLAMA_LM_HEAD), V, H),
                                 x, dev(model.tensor(-1, kvhp.LLAMA_FINAL_NORM)), eps, V, H, B,
                                 y32=lg_e)
    torch.cuda.synchronize()
    assert torch.equal(lg_r, lg_e), "runner logits differ from the exported operators'"
    assert torch.equal(nx_r.long(), lg_e.argmax(dim=1)), "greedy tokens"
    assert torch.equal(pool_r, pool_e), "appended K/V differ"
    model.close()


def test_batched_steps_see_rewritten_weights_after_reserve():
    """Batched steps (2..32 rows) read the model's tiled copies of the four
    projections and the LM head, built on the first batched step.  Weights
    rewritten through kvhp_llama_tensor after that leave a batched step's
    logits bit-identical to before (the copies are what the step reads);
    after kvhp_llama_reserve rebuilds the copies, its logits equal those of
    a fresh model that was given the same weights before its first batched
    step, bit for bit, and differ from the old ones."""
    cfg = _cfg(5632)
    L, Hkv, D, V = cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size
    B, plen, max_pages = 6, 11, 2
    P = B * max_pages
    rng = np.random.default_rng(2718)
    prompts = [rng.integers(0, V, plen).astype(np.int32) for _ in range(B)]
    bt = torch.from_numpy(rng.permutation(P).astype(np.int32).reshape(B, max_pages)).cuda()
    pos = torch.full((B,), plen, dtype=torch.int32, device="cuda")

    def prefill(model):
        pool = torch.zeros(L * 2 * Hkv * P * PAGE * D, dtype=torch.float16, device="cuda")
        toks = [model.prefill_paged(prompts[b], pool, P, bt[b], max_pages)[0] for b in range(B)]
        return pool, torch.tensor(toks, dtype=torch.int32, device="cuda")

    def step(model, pool, toks):
        lg = torch.empty(B, V, dtype=torch.float32, device="cuda")
        nx = torch.empty(B, dtype=torch.int32, device="cuda")
        model.decode_paged(toks, pool.clone(), P, bt, max_pages, pos, pos + 1, plen + 1, lg, nx)
        torch.cuda.synchronize()
        return lg.cpu().numpy()

    # each kind of tiled tensor (in one layer or another) and the LM head,
    # negated and scaled by 3/4; both models get the same fp16 values
    edits = [(0, kvhp.LLAMA_W_QKV), (1, kvhp.LLAMA_W_O), (2, kvhp.LLAMA_W_GATE_UP),
             (0, kvhp.LLAMA_W_DOWN), (-1, kvhp.LLAMA_LM_HEAD)]
    model = kvhp.LlamaModel(cfg, seed=61, max_ctx=64)
    pool, toks = prefill(model)
    before = step(model, pool, toks)            # first batched step: builds the copies
    new = {e: (model.tensor(*e).astype(np.float32) * -0.75).astype(np.float16) for e in edits}
    for e in edits:
        model.set_tensor(*e, new[e])
    assert np.array_equal(step(model, pool, toks), before), "batched step read the new weights"
    model.reserve(B, plen + 1)
    after = step(model, pool, toks)

    fresh = kvhp.LlamaModel(cfg, seed=61, max_ctx=64)
    fpool, ftoks = prefill(fresh)
    assert torch.equal(fpool, pool) and torch.equal(ftoks, toks)
    for e in edits:
        fresh.set_tensor(*e, new[e])
    ref = step(fresh, fpool, ftoks)
    assert np.array_equal(after, ref), "rebuilt copies differ from a fresh model's"
    assert not np.array_equal(after, before)
    fresh.close()
    model.close()


def test_paged_runner_argument_errors():
    cfg = _cfg()
    model = kvhp.LlamaModel(cfg, seed=3, max_ctx=32)
    pool = torch.zeros(cfg.num_layers * 2 * cfg.num_kv_heads * 4 * PAGE * cfg.head_dim,
                       dtype=torch.float16, device="cuda")
    bt = torch.arange(4, dtype=torch.int32, device="cuda")
    with pytest.raises(kvhp.KVHPError):
        model.prefill_paged(np.zeros(33, np.int32), pool, 4, bt, 4)    # > max_ctx rows
    with pytest.raises(kvhp.KVHPError):
        model.prefill_paged(np.zeros(20, np.int32), pool, 4, bt, 1)    # > 16 * max_pages
    t = torch.zeros(33, dtype=torch.int32, device="cuda")
    out = torch.empty(33, cfg.vocab_size, dtype=torch.float32, device="cuda")
    with pytest.raises(kvhp.KVHPError):                                 # batch > max_ctx
        model.decode_paged(t, pool, 4, bt, 4, t, t, 16, out, t)
    model.close()
