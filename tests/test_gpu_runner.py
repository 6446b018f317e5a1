"""The runner contract end to end on the GPU (serving-engine_amd/runner.py,
reference docs/runner_interface.md): a minimal scheduler loop owns the
block allocator -- it allocates the prompt blocks, forks the blocks of a
cached prefix (the third sequence reuses the first one's two full prompt
blocks, num_cached_tokens = 32; the fourth is exactly those 32 tokens),
allocates the next block when a sequence fills its last one, and is the
only writer of generated_ids / last_token_id (post_step) -- while the Runner
prefills and decodes, in both prefix modes: "share" recomputes every prompt
(flash prefill; shared blocks' writes dropped), "full" forwards only the
uncached suffix, attending to the cached prefix from the pages.  Every
sequence is checked against a batch-1 model of the same weights fed the
same tokens: prefill logits bit-identical where the same kernels run (every
"share" prefill, "full" prefills without a cached prefix), within 2 % of the
logit scale otherwise; decode logits within 2 %; a greedy token may differ
only where the batch-1 logits' gap between the two tokens is at most twice
the measured max |logit diff|.  Shared
blocks keep their bytes throughout, and freeing every sequence returns
every block."""
import numpy as np
import pytest

import kvhp
from llama_oracle import top2_margin

import runner as rc

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

def _close(got, ref, what):
    """Logits within 2 % of the scale; a greedy token may differ only where
    the reference logits' gap between the two tokens is at most twice the
    measured max |logit diff|."""
    scale = max(float(np.abs(ref).max()), 1.0)
    diff = float(np.abs(got - ref).max())
    assert diff < 0.02 * scale, f"{what}: max |logit diff| {diff:.4f} (scale {scale:.2f})"
    tok, rtok = int(np.argmax(got)), int(np.argmax(ref))
    if tok != rtok:
        gap = float(ref[rtok] - ref[tok])
        assert gap <= 2 * diff, f"{what}: token {tok} != {rtok} with gap {gap:.5f} > 2 x {diff:.5f}"


@pytest.mark.parametrize("mode", ["share", "full"])
def test_runner_with_prefix_sharing_matches_batch1_models(mode):
    cfg = kvhp.LlamaConfig(2048, 512, 3, 8, 2, 64, 1024, 1e-5, 10000.0, 0)
    seed, max_ctx, steps = 33, 128, 20
    model = kvhp.LlamaModel(cfg, seed=seed, max_ctx=max_ctx)
    run = rc.Runner(model, num_blocks=40, prefix_mode=mode)
    alloc = rc.BlockAllocator(40)
    rng = np.random.default_rng(808)
    p0 = rng.integers(0, cfg.vocab_size, 37).tolist()
    p1 = rng.integers(0, cfg.vocab_size, 21).tolist()
    p2 = p0[:32] + rng.integers(0, cfg.vocab_size, 9).tolist()
    p3 = p0[:32]
    seqs = [rc.Sequence(prompt_ids=p) for p in (p0, p1, p2, p3)]

    # scheduler: prompt blocks; sequences 2 and 3 hit sequence 0's cached prefix
    for i, s in enumerate(seqs):
        n = len(s.prompt_ids)
        if i >= 2:
            s.block_table.physical_block_ids = [alloc.fork(b) for b in
                                                seqs[0].block_table.physical_block_ids[:2]]
            s.num_cached_tokens = 32
        while len(s.block_table.physical_block_ids) * rc.BLOCK_SIZE < n:
            s.block_table.physical_block_ids.append(alloc.allocate())
        s.block_table.num_tokens = n
    shared = seqs[0].block_table.physical_block_ids[:2]
    assert all(alloc.ref_counts[b] == 3 for b in shared)

    singles = [kvhp.LlamaModel(cfg, seed=seed, max_ctx=max_ctx) for _ in seqs]
    pool = run.pool_view()
    for i, s in enumerate(seqs):
        tok = run.step(rc.ScheduledBatch(rc.BatchType.PREFILL, [s]))[0]
        rtok, rlg = singles[i].prefill(np.array(s.prompt_ids, np.int32))
        if mode == "share" or s.num_cached_tokens == 0:
            assert tok == rtok and np.array_equal(s.last_logits.numpy(), rlg), f"prefill {i}"
        else:
            _close(s.last_logits.numpy(), rlg, f"cached-prefix prefill {i}")
            tok = rtok   # continue both sides from the same token
        assert s.block_table.num_tokens == len(s.prompt_ids)    # the runner leaves it
        s.generated_ids.append(tok)                             # post_step
        s.last_token_id = tok
        if i == 0:
            torch.cuda.synchronize()
            kept = [pool[:, :, :, b].clone() for b in shared]

    for st in range(steps):
        for s in seqs:                                          # scheduler: next block
            if s.block_table.num_tokens % rc.BLOCK_SIZE == 0:
                s.block_table.physical_block_ids.append(alloc.allocate())
        toks = run.step(rc.ScheduledBatch(rc.BatchType.DECODE, seqs))
        for i, s in enumerate(seqs):
            _, rlg = singles[i].decode_step(s.last_token_id)    # same input token
            _close(s.last_logits.numpy(), rlg, f"step {st} sequence {i}")
            assert abs(s.last_logit_margin - top2_margin(s.last_logits.numpy())) < 1e-6
            assert s.block_table.num_tokens == len(s.prompt_ids) + st + 1
            s.generated_ids.append(toks[i])                     # post_step
            s.last_token_id = toks[i]
    torch.cuda.synchronize()
    for b, k in zip(shared, kept):
        assert torch.equal(pool[:, :, :, b], k), f"shared block {b} changed"

    for s in seqs:                                              # scheduler frees
        for b in s.block_table.physical_block_ids:
            alloc.free(b)
    assert alloc.num_free() == 40 and not alloc.ref_counts.any()
    for m in singles:
        m.close()
    model.close()


def test_serving_simulation_with_arrivals_departures_and_prefix_hits():
    """A continuous-batching loop in miniature: each step may admit a new
    sequence (a third of them reuse the full blocks of a live sequence's
    prompt prefix, in the "full" prefix mode) and retire finished ones, then
    decodes every live sequence in one batch whose membership changes from
    step to step.  Every logit vector is checked against that sequence's own
    batch-1 model fed the same tokens; blocks are freed as sequences finish
    and none leak."""
    cfg = kvhp.LlamaConfig(1024, 256, 2, 4, 2, 64, 512, 1e-5, 10000.0, 0)
    seed, num_blocks = 44, 96
    model = kvhp.LlamaModel(cfg, seed=seed, max_ctx=160)
    run = rc.Runner(model, num_blocks=num_blocks, prefix_mode="full")
    alloc = rc.BlockAllocator(num_blocks)
    rng = np.random.default_rng(2024)
    live, singles, budget = [], {}, {}
    admitted = 0
    for step in range(30):
        if admitted < 10 and rng.random() < 0.5:
            prompt = rng.integers(0, cfg.vocab_size, int(rng.integers(5, 60))).tolist()
            s = rc.Sequence(prompt_ids=prompt)
            donors = [d for d in live if len(d.prompt_ids) >= 16]
            if donors and admitted % 3 == 2:          # prefix hit on a live sequence
                d = donors[int(rng.integers(len(donors)))]
                nb = len(d.prompt_ids) // 16
                s.prompt_ids = d.prompt_ids[:16 * nb] + prompt[:int(rng.integers(0, 20))]
                s.block_table.physical_block_ids = [alloc.fork(b) for b in
                                                    d.block_table.physical_block_ids[:nb]]
                s.num_cached_tokens = 16 * nb
            n = len(s.prompt_ids)
            while len(s.block_table.physical_block_ids) * 16 < n:
                s.block_table.physical_block_ids.append(alloc.allocate())
            s.block_table.num_tokens = n
            ref = kvhp.LlamaModel(cfg, seed=seed, max_ctx=160)
            tok = run.prefill(s)
            rtok, rlg = ref.prefill(np.array(s.prompt_ids, np.int32))
            _close(s.last_logits.numpy(), rlg, f"admit {admitted} at step {step}")
            s.generated_ids.append(rtok)
            s.last_token_id = rtok
            singles[id(s)] = ref
            budget[id(s)] = int(rng.integers(3, 15))
            live.append(s)
            admitted += 1
        if not live:
            continue
        for s in live:
            if s.block_table.num_tokens % 16 == 0:
                s.block_table.physical_block_ids.append(alloc.allocate())
        toks = run.decode_step(live, alloc)
        for s, t in zip(live, toks):
            _, rlg = singles[id(s)].decode_step(s.last_token_id)
            _close(s.last_logits.numpy(), rlg, f"step {step}")
            s.generated_ids.append(t)
            s.last_token_id = t
            budget[id(s)] -= 1
        for s in [s for s in live if budget[id(s)] <= 0]:   # retire
            for b in s.block_table.physical_block_ids:
                alloc.free(b)
            singles.pop(id(s)).close()
            live.remove(s)
    for s in live:
        for b in s.block_table.physical_block_ids:
            alloc.free(b)
        singles.pop(id(s)).close()
    assert admitted >= 6
    assert alloc.num_free() == num_blocks and not alloc.ref_counts.any()
    model.close()
