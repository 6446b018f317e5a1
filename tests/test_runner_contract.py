"""The runner contract's host side (serving-engine_amd/runner.py, following
the reference's docs/runner_interface.md): block reference counts, and the
runner's own checks, which fire before any GPU work -- a prefill whose
length the scheduler did not set, too few blocks, and a decode write into a
shared block (:51), after which nothing has changed.  CPU only: the model
is a stand-in carrying a configuration, and the pool a CPU tensor."""
import types

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import runner as rc


def _runner(num_blocks=8):
    cfg = types.SimpleNamespace(num_layers=2, num_kv_heads=2, head_dim=64, vocab_size=100)
    model = types.SimpleNamespace(config=cfg)
    return rc.Runner(model, num_blocks, device="cpu")


def test_block_allocator_reference_counts():
    a = rc.BlockAllocator(4)
    b0, b1 = a.allocate(), a.allocate()
    assert (b0, b1) == (0, 1) and a.num_free() == 2
    a.fork(b0)
    assert a.ref_counts[b0] == 2
    a.free(b0)
    assert a.ref_counts[b0] == 1 and a.num_free() == 2      # still held once
    a.free(b0)
    assert a.num_free() == 3 and a.allocate() == b0          # back on the free list
    with pytest.raises(ValueError):
        a.free(3)                                            # never allocated
    with pytest.raises(ValueError):
        a.fork(3)
    a.allocate(), a.allocate()
    with pytest.raises(RuntimeError):
        a.allocate()                                         # out of blocks


def test_pool_layout():
    r = _runner(num_blocks=5)
    assert tuple(r.pool_view().shape) == (2, 2, 2, 5, rc.BLOCK_SIZE, 64)
    assert r.pool.dtype == torch.float16


def test_prefill_preconditions():
    r = _runner()
    s = rc.Sequence(prompt_ids=list(range(20)))
    s.block_table.physical_block_ids = [0, 1]
    with pytest.raises(AssertionError, match="num_tokens"):
        r.prefill(s)                                         # num_tokens not set
    s.block_table.num_tokens = 20
    s.block_table.physical_block_ids = [0]
    with pytest.raises(AssertionError, match="blocks"):
        r.prefill(s)                                         # 20 tokens need 2 blocks


def test_decode_refuses_a_write_into_a_shared_block():
    r = _runner()
    a = rc.BlockAllocator(8)
    owner = rc.Sequence(prompt_ids=list(range(20)))
    owner.block_table = rc.BlockTable([a.allocate(), a.allocate()], 20)
    # a second sequence shares the owner's first block and ends inside it
    other = rc.Sequence(prompt_ids=list(range(5)))
    other.block_table = rc.BlockTable([a.fork(owner.block_table.physical_block_ids[0])], 5)
    with pytest.raises(AssertionError, match="last_token_id"):
        r.decode_step([owner], a)                            # no token to feed yet
    owner.last_token_id = other.last_token_id = 7
    with pytest.raises(AssertionError, match="shared"):
        r.decode_step([owner, other], a)
    assert owner.block_table.num_tokens == 20 and other.block_table.num_tokens == 5
    # a sequence at a block boundary without its next block
    edge = rc.Sequence(prompt_ids=list(range(16)), last_token_id=3)
    edge.block_table = rc.BlockTable([a.allocate()], 16)
    with pytest.raises(AssertionError, match="blocks"):
        r.decode_step([edge], a)
    assert edge.block_table.num_tokens == 16
    assert r.decode_step([], a) == []
