"""Model runner contract over the MI355X KV-cache path.

Mirrors the runner interface of the reference serving engine
(docs/runner_interface.md): the scheduler owns the block allocator, the
sequences and their block tables; the runner owns the physical page pool
and runs the forward passes.  Names and argument meaning follow that
document:

* ``BlockAllocator`` (:9-10, :81-84): free list and per-block reference
  counts; ``allocate()`` is for the scheduler only; ``fork()`` shares a
  block with another sequence (prefix caching); ``free()`` drops one
  reference.
* ``BlockTable`` / ``Sequence``: ``physical_block_ids``, ``num_tokens``,
  ``num_cached_tokens``, ``last_token_id``, ``generated_ids``,
  ``last_logits``, ``last_logit_margin``.
* ``Runner.prefill(seq, allocator=None)`` (:20-35): K/V go into
  ``physical_block_ids[skip_blocks:]`` with ``skip_blocks =
  num_cached_tokens // block_size``; the blocks before are shared and keep
  their cached K/V.  ``prefix_mode="share"`` recomputes the whole prompt
  (flash prefill) and skips the shared blocks' writes; ``"full"`` forwards
  only the uncached suffix, which attends to the cached prefix from the
  pages (when the whole prompt is cached, its last token is forwarded, its
  write into the shared block dropped).  Never allocates, never changes
  ``num_tokens``.  Returns the greedy first token.
* ``Runner.decode_step(seqs, allocator=None)`` (:37-55): bumps every
  sequence's ``num_tokens`` by one, writes its new K/V at
  ``num_tokens - 1``, asserts that the block written is not shared
  (``allocator.ref_counts[block] > 1`` fails), and returns one greedy token
  per sequence.  Block tables go to the device as int32
  ``[batch, max_blocks]`` padded with 0, lengths as int32 ``[batch]``
  including the decoded token (:94-97).
* ``Runner.step(batch)`` (:57-61): dispatch on ``batch.batch_type``.

The pool differs from the reference's layout on purpose: one fp16 tensor
``[num_layers][2][num_kv_heads][num_blocks][16][head_dim]`` (a page is 16
tokens x head_dim of one KV head, contiguous) instead of per-layer
``[num_blocks][16][num_kv_heads][head_dim]`` -- the decode kernels stream a
page of one head as 4 KiB of contiguous bytes.  Block ids index it the same
way.

The model is the library's decoder (``kvhp.LlamaModel``, synthetic
weights); the forward passes are ``kvhp_llama_prefill_paged`` and
``kvhp_llama_decode_paged``.  Host bookkeeping here is plain Python; every
tensor the kernels touch is a torch tensor on the GPU.  Without the HIP
library nothing runs (``kvhp.load()`` raises).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

import kvhp

BLOCK_SIZE = kvhp.PAGE_SIZE


class BlockAllocator:
    """Physical block ids with reference counts (the scheduler's side)."""

    def __init__(self, num_blocks: int):
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        self.num_blocks = num_blocks
        self.ref_counts = np.zeros(num_blocks, np.int32)
        self._free = list(range(num_blocks - 1, -1, -1))   # pop() hands out 0 first

    def num_free(self) -> int:
        return len(self._free)

    def allocate(self) -> int:
        if not self._free:
            raise RuntimeError("BlockAllocator: out of blocks")
        b = self._free.pop()
        self.ref_counts[b] = 1
        return b

    def fork(self, block: int) -> int:
        """One more sequence holds `block` (a shared prefix block)."""
        if self.ref_counts[block] <= 0:
            raise ValueError(f"BlockAllocator: block {block} is not allocated")
        self.ref_counts[block] += 1
        return block

    def free(self, block: int) -> None:
        if self.ref_counts[block] <= 0:
            raise ValueError(f"BlockAllocator: block {block} freed twice")
        self.ref_counts[block] -= 1
        if self.ref_counts[block] == 0:
            self._free.append(block)


@dataclass
class BlockTable:
    physical_block_ids: List[int] = field(default_factory=list)
    num_tokens: int = 0


@dataclass
class Sequence:
    prompt_ids: List[int]
    block_table: BlockTable = field(default_factory=BlockTable)
    num_cached_tokens: int = 0
    generated_ids: List[int] = field(default_factory=list)
    last_token_id: int = -1
    last_logits: Optional[object] = None       # torch.Tensor (CPU, fp32)
    last_logit_margin: float = 0.0

    @property
    def cur_len(self) -> int:
        return self.block_table.num_tokens


class BatchType(enum.Enum):
    PREFILL = 0
    DECODE = 1


@dataclass
class ScheduledBatch:
    batch_type: BatchType
    sequences: List[Sequence]


def _margin(logits: np.ndarray) -> float:
    top2 = np.partition(logits, -2)[-2:]
    return float(top2[1] - top2[0])


class Runner:
    """Runner.prefill / decode_step / step over a page pool this object owns."""

    def __init__(self, model: "kvhp.LlamaModel", num_blocks: int, device: str = "cuda",
                 prefix_mode: str = "share"):
        import torch
        if prefix_mode not in ("share", "full"):
            raise ValueError(f"prefix_mode must be 'share' or 'full', not {prefix_mode!r}")
        self.prefix_mode = prefix_mode
        self._torch = torch
        c = model.config
        self.model = model
        self.num_blocks = num_blocks
        self.block_size = BLOCK_SIZE
        self.pool = torch.zeros(c.num_layers * 2 * c.num_kv_heads * num_blocks * BLOCK_SIZE *
                                c.head_dim, dtype=torch.float16, device=device)
        self.device = device

    def pool_view(self):
        """The pool as [num_layers][2][num_kv_heads][num_blocks][16][head_dim]."""
        c = self.model.config
        return self.pool.view(c.num_layers, 2, c.num_kv_heads, self.num_blocks, BLOCK_SIZE,
                              c.head_dim)

    def _check_blocks(self, seq: Sequence, tokens: int, what: str) -> None:
        need = (tokens + BLOCK_SIZE - 1) // BLOCK_SIZE
        ids = seq.block_table.physical_block_ids
        if len(ids) < need:
            raise AssertionError(f"{what}: {tokens} tokens need {need} blocks, the scheduler "
                                 f"allocated {len(ids)}")
        for b in ids[:need]:
            if not 0 <= b < self.num_blocks:
                raise AssertionError(f"{what}: block id {b} outside the pool")

    def prefill(self, seq: Sequence, allocator: Optional[BlockAllocator] = None) -> int:
        torch = self._torch
        n = len(seq.prompt_ids)
        if seq.block_table.num_tokens != n:
            raise AssertionError(f"prefill: num_tokens {seq.block_table.num_tokens} != prompt "
                                 f"length {n} (the scheduler sets it)")
        self._check_blocks(seq, n, "prefill")
        skip = seq.num_cached_tokens // BLOCK_SIZE
        ids = seq.block_table.physical_block_ids
        table = np.array(ids, np.int32)
        write = table.copy()
        write[:skip] = -1                       # shared blocks: not overwritten
        prompt = np.asarray(seq.prompt_ids, np.int32)
        with torch.inference_mode():
            wrow = torch.from_numpy(write).to(self.device)
            if self.prefix_mode == "full" and skip > 0:
                first = min(skip * BLOCK_SIZE, n - 1)
                tok, logits = self.model.prefill_cached(
                    prompt, first, self.pool, self.num_blocks,
                    torch.from_numpy(table).to(self.device), len(ids), write_table=wrow)
            else:
                tok, logits = self.model.prefill_paged(prompt, self.pool, self.num_blocks, wrow,
                                                       len(ids))
        seq.last_logits = torch.from_numpy(logits)
        seq.last_logit_margin = _margin(logits)
        return tok

    def decode_step(self, seqs: List[Sequence],
                    allocator: Optional[BlockAllocator] = None) -> List[int]:
        torch = self._torch
        if not seqs:
            return []
        B = len(seqs)
        # every sequence is checked before any is bumped, so a failed
        # assertion leaves the batch as it was
        for s in seqs:
            if s.last_token_id < 0 and not s.generated_ids:
                raise AssertionError("decode_step: a sequence without last_token_id or "
                                     "generated_ids (the previous step's token)")
            write_pos = s.block_table.num_tokens     # = the bumped num_tokens - 1
            self._check_blocks(s, write_pos + 1, "decode_step")
            blk = s.block_table.physical_block_ids[write_pos // BLOCK_SIZE]
            if allocator is not None and allocator.ref_counts[blk] > 1:
                raise AssertionError(f"decode_step: block {blk} is shared "
                                     f"(ref count {allocator.ref_counts[blk]}); a sequence must "
                                     f"never mutate a shared block during decode")
        for s in seqs:
            s.block_table.num_tokens += 1            # bump, then write at num_tokens - 1
        max_blocks = max(len(s.block_table.physical_block_ids) for s in seqs)
        tables = np.zeros((B, max_blocks), np.int32)          # padded with 0
        for i, s in enumerate(seqs):
            ids = s.block_table.physical_block_ids
            tables[i, :len(ids)] = ids
        seq_lens = np.array([s.block_table.num_tokens for s in seqs], np.int32)
        tokens = np.array([s.last_token_id if s.last_token_id >= 0 else s.generated_ids[-1]
                           for s in seqs], np.int32)
        V = self.model.config.vocab_size
        with torch.inference_mode():
            d = lambda a: torch.from_numpy(a).to(self.device)
            lens_d = d(seq_lens)
            logits = torch.empty((B, V), dtype=torch.float32, device=self.device)
            nxt = torch.empty(B, dtype=torch.int32, device=self.device)
            self.model.decode_paged(d(tokens), self.pool, self.num_blocks, d(tables), max_blocks,
                                    lens_d - 1, lens_d, int(seq_lens.max()), logits, nxt)
            host = logits.cpu()
            out = nxt.cpu().numpy().tolist()
        for i, s in enumerate(seqs):
            s.last_logits = host[i]
            s.last_logit_margin = _margin(host[i].numpy())
        return [int(t) for t in out]

    def step(self, batch: ScheduledBatch) -> List[int]:
        if batch.batch_type == BatchType.PREFILL:
            return [self.prefill(batch.sequences[0])]
        if batch.batch_type == BatchType.DECODE:
            return self.decode_step(batch.sequences)
        raise ValueError(f"unknown batch type {batch.batch_type}")
