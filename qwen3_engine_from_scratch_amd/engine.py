"""Continuous-batching generation loop over the HIP model steps.

Scheduling policy is the reference's (qwen3/scheduler.py:56-97): while the
running set has free slots and requests wait, the step is a prefill of as
many waiting requests as fit; otherwise it is a decode step of every running
request.  A request finishes after max_new_tokens tokens (the first comes
from its prefill) or on its eos token, and returns its pages.

What differs from the reference's driver (bench_batched.py:139-203) is where
the per-step state lives:
  - prefill packs the prompts (varlen kernel, no padding) and computes
    logits only for each prompt's last token;
  - decode steps replay a captured graph per power-of-two bucket whose
    greedy tokens are written straight into the next step's inputs and
    whose resident seq_lens advance on the device, so an unchanged batch
    needs no host->device copy at all; a changed batch copies its ids and
    rows once;
  - pages for the next token are reserved for the whole batch with one
    asynchronous copy and one launch that maps and zeroes them (PageIn);
  - the host reads back only the B new token ids per step, and does so
    after it has launched the next step (whose inputs are already on the
    device), so its bookkeeping overlaps the GPU.  A request's count limit
    is known without the read-back; an eos seen one step late drops the one
    token computed past it (its page writes land beyond its final length).
Greedy decoding only (temperature 0), as the reference's benchmark runs.
"""
from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

from .PagedKVcache import PageIn, PagedKVCache, set_seq_lens_bulk
from .graph_runner import GraphRunner, pow2_buckets
from .kernels.model_ops import argmax

__all__ = ["GenRequest", "Engine"]


@dataclass
class GenRequest:
    """One generation request (the data half of qwen3/request.py:44-206)."""
    request_id: int
    prompt: list
    max_new_tokens: int
    eos_token_id: int | None = None
    output_ids: list = field(default_factory=list)
    cache: PagedKVCache | None = None
    finished: bool = False
    finish_time: float = 0.0
    inflight: int = 0        # decode steps launched whose token has not been read back
    eos_hit: bool = False

    def is_finished(self) -> bool:
        """Reference rule (qwen3/request.py:121-137): max_new_tokens reached
        or the last token is eos."""
        return len(self.output_ids) >= self.max_new_tokens or self.eos_hit

    def schedulable(self) -> bool:
        """May take part in another decode step: counts the steps in flight,
        so the count limit needs no read-back."""
        return not self.eos_hit and len(self.output_ids) + self.inflight < self.max_new_tokens


class Engine:
    def __init__(self, model, pool, max_batch: int = 64, use_graph: bool = True,
                 batch_invariant: bool = False, max_prefill_batch: int | None = None):
        """batch_invariant: decode attention on the batch-invariant kernel,
        so a request's decode tokens do not depend on what else is batched
        with it.  max_prefill_batch: prompts per prefill step (None: as many
        as there are free rows); 1 prefills every prompt alone, as a
        request running by itself would be (the library GEMMs of the
        prefill pick kernels by row count, so a prompt's prefill bits depend
        on the rows batched with it)."""
        self.model = model
        self.pool = pool
        self.max_batch = max_batch
        self.max_prefill_batch = max_prefill_batch
        model.decode_batch_invariant = batch_invariant
        self.device = pool.k_buffer.device
        self.runner = None
        self._placeholders = []
        if use_graph:
            buckets = pow2_buckets(max_batch)
            self._placeholders = [PagedKVCache(pool) for _ in range(max(buckets))]
            self.runner = GraphRunner(model, pool, self._placeholders, buckets, reserve_pages=1,
                                      greedy=True, advance=True, positions_from_lengths=True)
        else:
            model.reserve_decode_workspace(max_batch, pool)
        # two pinned landing buffers: a step's tokens are read back while the
        # next step's copy is already queued
        self._tok_host = [torch.empty(max(max_batch, 1), dtype=torch.int64, pin_memory=True)
                          for _ in range(2)]
        self._flip = 0
        max_pages = pool.block_table_2d.shape[1]
        self._pages = PageIn(pool, max(max_batch * max_pages, 64))
        self._pending = None     # (requests, host view, event) of the last decode launch
        self._last_batch = None  # (bucket, request ids) of the last graph replay

    # ---- steps -------------------------------------------------------------

    def _prefill(self, reqs) -> None:
        dev = self.device
        lens = [len(r.prompt) for r in reqs]
        for r in reqs:
            r.cache = PagedKVCache(self.pool)
        self._pages.reserve([r.cache for r in reqs], lens)
        n = len(reqs)
        cu = np.zeros(n + 1, dtype=np.int64)
        cu[1:] = np.cumsum(lens)
        T = int(cu[-1])
        bs = self.pool.block_size
        # one host buffer, one copy: ids | positions | slots | last rows | cu
        buf = np.empty(3 * T + 2 * n + 1, dtype=np.int64)
        buf[:T] = np.concatenate([np.asarray(r.prompt, dtype=np.int64) for r in reqs])
        buf[T:2 * T] = np.concatenate([np.arange(L, dtype=np.int64) for L in lens])
        slots = buf[2 * T:3 * T]
        for r, a, L in zip(reqs, cu[:-1], lens):
            p = np.arange(L, dtype=np.int64)
            table = np.asarray(r.cache.block_table, dtype=np.int64)
            slots[a:a + L] = table[p // bs] * bs + p % bs
        buf[3 * T:3 * T + n] = cu[1:] - 1
        buf[3 * T + n:] = cu
        d = torch.from_numpy(buf).to(dev)
        logits = self.model.prefill_logits(d[:T], d[3 * T + n:].to(torch.int32), max(lens),
                                           d[T:2 * T], d[2 * T:3 * T], self.pool,
                                           d[3 * T:3 * T + n])
        toks = argmax(logits).cpu().tolist()
        for r, L, tok in zip(reqs, lens, toks):
            r.cache.seq_len = L
            self._take(r, int(tok))
        set_seq_lens_bulk([r.cache for r in reqs])

    @staticmethod
    def _take(r, tok: int) -> None:
        if r.eos_hit or len(r.output_ids) >= r.max_new_tokens:
            return  # a step launched before the stop was known: its token is dropped
        r.output_ids.append(tok)
        if r.eos_token_id is not None and tok == r.eos_token_id:
            r.eos_hit = True

    def _drain(self) -> None:
        """Reads back the tokens of the decode step in flight."""
        if self._pending is None:
            return
        reqs, host, ev = self._pending
        self._pending = None
        ev.synchronize()
        for r, tok in zip(reqs, host.tolist()):
            r.inflight -= 1
            self._take(r, int(tok))

    def _decode(self, reqs) -> None:
        """Launches one decode step for `reqs` and then reads back the tokens
        of the step before it, so the host's bookkeeping overlaps the GPU."""
        k = len(reqs)
        dev = self.device
        if self.runner is not None:
            b = self.runner.bucket_for(k)
            key = (b, tuple(r.request_id for r in reqs))
            if key != self._last_batch:
                # a changed batch takes its input tokens from the host
                self._drain()
        else:
            self._drain()
        caches = [r.cache for r in reqs]
        # the token of this step lands at position seq_len: reserve its page
        self._pages.reserve(caches, [c.seq_len + 1 for c in caches])
        if self.runner is not None:
            if key == self._last_batch:
                out = self.runner.replay_greedy(k)
            else:
                ids = torch.tensor([r.output_ids[-1] for r in reqs], dtype=torch.int64)
                rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32)
                out = self.runner.replay_greedy(k, ids.to(dev), rows.to(dev))
                self._last_batch = key
            toks = out.view(-1)[:k]
        else:
            ids = torch.tensor([r.output_ids[-1] for r in reqs], dtype=torch.int64).to(dev)
            rows = torch.tensor([c.row_id for c in caches], dtype=torch.int32).to(dev)
            toks = self.model.decode_greedy(ids, rows, self.pool)
        host = self._tok_host[self._flip][:k]
        self._flip ^= 1
        host.copy_(toks, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dev))
        for r in reqs:
            r.inflight += 1
        for c in caches:
            c.seq_len += 1
        if self.runner is None:
            set_seq_lens_bulk(caches)
        self._drain()
        self._pending = (list(reqs), host, ev)

    # ---- loop --------------------------------------------------------------

    @torch.no_grad()
    def generate(self, requests: list) -> dict:
        """Runs every request to completion; returns timing and counts.
        Timing: prefill_s / decode_s are host wall time per kind of step
        (a decode step's read-back overlaps the next launch)."""
        waiting = deque(requests)
        running: list = []
        self._pending = None
        self._last_batch = None
        t0 = time.perf_counter()
        prefill_s = decode_s = 0.0
        n_prefill = n_decode = 0
        while waiting or running:
            ts = time.perf_counter()
            if waiting and len(running) < self.max_batch:
                self._drain()
                n_take = min(self.max_batch - len(running), len(waiting))
                if self.max_prefill_batch:
                    n_take = min(n_take, self.max_prefill_batch)
                take = [waiting.popleft() for _ in range(n_take)]
                self._prefill(take)
                running.extend(take)
                prefill_s += time.perf_counter() - ts
                n_prefill += 1
            else:
                batch = [r for r in running if r.schedulable()][:self.max_batch]
                if batch:
                    self._decode(batch)
                    n_decode += 1
                else:
                    self._drain()
                decode_s += time.perf_counter() - ts
            done = [r for r in running if r.inflight == 0 and r.is_finished()]
            if done:
                now = time.perf_counter() - t0
                for r in done:
                    r.finished = True
                    r.finish_time = now
                    r.cache.free()
                    r.cache = None
                running = [r for r in running if not r.finished]
        self._drain()
        total = time.perf_counter() - t0
        n_tok = sum(len(r.output_ids) for r in requests)
        return {"total_s": total, "output_tokens": n_tok, "tokens_per_s": n_tok / total,
                "prefill_s": prefill_s, "decode_s": decode_s, "prefill_steps": n_prefill,
                "decode_steps": n_decode}

    def close(self):
        self._drain()
        if self.runner is not None:
            self.runner.free()
        for c in self._placeholders:
            c.free()
