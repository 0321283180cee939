"""Decode steps captured as HIP graphs, one per power-of-two batch bucket
(reference: GraphRunner, qwen3/graph_runner.py:26-209).

The reference's contract is kept: placeholder handles with reserved pages
and seq_len 1 are used at capture; a dummy row (its own page, seq_len 0)
pads a bucket's unused slots; replay(input_ids, positions, rows) copies the
step's inputs into the captured tensors, picks the smallest bucket that
holds them and returns that bucket's logits (b, 1, V).  Capture goes
through torch.cuda.graph on torch's current stream, which is the stream
every kernel of this package launches on.

Two optional stages, used by the batching engine, ride in the same graph:
  greedy=True    the step ends in the greedy choice instead of logits (the
                 model's decode_greedy: final norm, lm_head and argmax in one
                 pass over the tied embedding on the fused path) written
                 straight into the captured input ids, so the next step's
                 inputs are already in place and only the tokens come back
                 to the host (replay_greedy; such a runner has no logits);
  advance=True   the resident seq_lens of the batch's rows are advanced by
                 one on the device (the dummy row excepted), replacing the
                 host's per-request writes of advance_seq_len.
With positions_from_lengths=True RoPE uses seq_lens[row] (the reference's
drivers always pass those positions), so nothing but the ids and rows of a
changed batch needs a host->device copy.
"""
from __future__ import annotations

import torch

from .kernels.model_ops import advance_seq_lens

__all__ = ["GraphRunner", "pow2_buckets"]


def pow2_buckets(max_batch: int) -> tuple:
    """1, 2, 4, ... up to the first power of two >= max_batch (the
    reference's bucket rule, bench_batched.py:282-286)."""
    b = [1]
    while b[-1] < max_batch:
        b.append(b[-1] * 2)
    return tuple(b)


class GraphRunner:
    def __init__(self, model, pool, caches, buckets=(1, 2, 4, 8), reserve_pages=64, *,
                 greedy: bool = False, advance: bool = False,
                 positions_from_lengths: bool = False):
        self.model = model
        self.pool = pool
        self.buckets = tuple(sorted(set(buckets)))
        self.max_batch = max(self.buckets)
        self.greedy = greedy
        self.advance = advance
        self.positions_from_lengths = positions_from_lengths
        assert len(caches) >= self.max_batch, \
            f"{len(caches)} placeholder handles, need >= max bucket {self.max_batch}"

        # Placeholders: pages reserved before capture (no allocation inside a
        # graph) and seq_len 1, so the captured step is a decode step.
        for c in caches:
            while c.num_pages < reserve_pages:
                c._allocate_block()
            c.seq_len = 1
            pool.seq_lens[c.row_id] = 1

        # Dummy row for unused slots: seq_len 0, one mapped page, so the
        # kernels attend one slot of a real page and write into it.
        self.dummy_row = pool.alloc_row()
        self._dummy_phys = pool.alloc(1)[0]
        pool.block_table_2d[self.dummy_row, 0] = self._dummy_phys

        model.reserve_decode_workspace(self.max_batch, pool)
        self._pool_handle = torch.cuda.graph_pool_handle()
        self.graphs = {}
        self._capture_all(caches)

    def _step(self, t, caches):
        pos = None if self.positions_from_lengths else t["pos"]
        if self.greedy:
            ids = t["input"].view(-1)
            self.model.decode_greedy(ids, t["rows"], self.pool,
                                     None if pos is None else pos.view(-1), out=ids)
            return None
        return self.model.forward_decode(t["input"], pos, t["rows"], caches)

    @torch.no_grad()
    def _capture_all(self, caches):
        device = self.pool.k_buffer.device
        for b in self.buckets:
            t = {
                "input": torch.zeros((b, 1), dtype=torch.long, device=device),
                "pos": torch.zeros((b, 1), dtype=torch.long, device=device),
                "rows": torch.tensor([c.row_id for c in caches[:b]], dtype=torch.int32,
                                     device=device),
            }
            for _ in range(3):  # warm-up outside the graph: library heuristics, allocator
                self._step(t, caches[:b])
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self._pool_handle):
                t["logits"] = self._step(t, caches[:b])
                if self.advance:
                    advance_seq_lens(self.pool.seq_lens, t["rows"], skip_row=self.dummy_row)
            torch.cuda.synchronize()
            self.graphs[b] = (g, t)

    def bucket_for(self, k: int) -> int:
        return min(x for x in self.buckets if x >= k)

    def replay(self, input_ids, positions, rows):
        """Reference entry (qwen3/graph_runner.py:165-200): input_ids,
        positions (k, 1) int64 and rows (k,) int32 of this step; returns the
        bucket's logits (b, 1, V), the first k rows valid."""
        assert not self.greedy, "a greedy runner returns tokens: use replay_greedy"
        k = input_ids.shape[0]
        b = self.bucket_for(k)
        g, t = self.graphs[b]
        t["input"][:k].copy_(input_ids)
        if positions is not None:
            t["pos"][:k].copy_(positions)
        t["rows"][:k].copy_(rows)
        if k < b:
            t["rows"][k:].fill_(self.dummy_row)
        g.replay()
        return t["logits"]

    def replay_greedy(self, k: int, input_ids=None, rows=None):
        """Engine entry (greedy=True): replays the bucket of k rows.  With
        input_ids / rows None the captured tensors already hold them (the
        previous replay of this bucket wrote its tokens there and the batch
        is unchanged).  Returns the bucket's (b, 1) int64 token tensor, the
        first k rows valid."""
        assert self.greedy
        b = self.bucket_for(k)
        g, t = self.graphs[b]
        if input_ids is not None:
            t["input"][:k].copy_(input_ids.view(k, 1))
        if rows is not None:
            t["rows"][:k].copy_(rows)
            if k < b:
                t["rows"][k:].fill_(self.dummy_row)
        g.replay()
        return t["input"]

    def free(self):
        """Returns the dummy row's page and row (qwen3/graph_runner.py:202-209)."""
        self.pool.free([self._dummy_phys])
        self.pool.free_row(self.dummy_row)
